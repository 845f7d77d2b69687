/*
 * busfill -- MI355X (gfx950) batched int4-block-weight x fp16-activation GEMM.
 *
 * C-ABI drop-in for the reference kernel's call surface
 *   extern "C" __global__ void busfill_q4(const __half* A, const uint8_t* Wq,
 *                                        const __half* Ws, float* C,
 *                                        int Bsz, int K, int N)
 *   (kernels/busfill_v1a.cu:41-46, launched <<<N/32,128>>> at :151,154,169).
 * The reference has no library or FFI: its harness main() launches that symbol
 * directly.  Every entry point below replaces that launch (or, for the Q4_K and
 * llama.cpp-block formats, the dequantize-then-matmul the reference only
 * describes in RESULTS.md:84-96) with a host-callable function.
 *
 * Conventions
 *   - All pointers are DEVICE pointers owned by the caller.  Two kernels
 *     exchange partial sums between workgroups and need a workspace: the
 *     K-split kernel (BF_ALGO_SPLIT, which bf_gemm picks for 9-32 batch rows
 *     per launch when the activations do not fit in LDS) and the dense kernel
 *     (BF_ALGO_DENSE, above 32 rows, and from 9 or 17 rows on matrices of
 *     3 * 2^24 weights or more).  Three ways to provide it:
 *       * bf_gemm_ws / bf_gemm_batched_ws / bf_busfill_q4_ws: the caller owns
 *         it (size from bf_gemm_workspace_bytes / bf_gemm_batched_workspace_bytes);
 *         the library allocates nothing and keeps no state between calls.
 *       * bf_gemm_noalloc: a fixed array in device memory per GPU.
 *       * bf_gemm, bf_gemm_batched, bf_busfill_q4, bf_ffn_swiglu: the
 *         library's workspace for the (device, stream) -- per host thread for
 *         hipStreamPerThread -- allocated by the first call on the stream that
 *         needs it and grown by a later call that needs more (each region that
 *         is too small to at least twice its size).  A replaced buffer is
 *         retired, never freed before the process ends, so launches already
 *         queued, graphs captured earlier and calls racing on the same stream
 *         from other host threads keep valid memory.  Nothing is allocated
 *         while the stream is being captured into a graph: a call that would
 *         need to returns BF_ERR_UNSUPPORTED and enqueues nothing; make one
 *         uncaptured call of the largest shape on the stream first, or use a
 *         caller-owned workspace.  The one-launch feed-forward block
 *         (bf_ffn_swiglu_ex, BF_FFN_ONE_LAUNCH) keeps its hand-over words in
 *         the same workspace.  A captured graph holds the buffer of the
 *         stream it was captured on: replaying it while other exchanging work
 *         that uses that buffer runs (on another stream, or another replay)
 *         races.
 *     Every call plans all its launches and secures their workspace before
 *     it enqueues the first, so a call that fails enqueues nothing.  A call
 *     whose launches share workspace (a kernel and its second-launch sum, a
 *     slot fill and its kernel, the ggml hook's staging and its GEMMs)
 *     enqueues them under a lock per (device, stream), so calls from several
 *     host threads on one stream never interleave their launches.
 *   - fp16 values travel as uint16_t bit patterns.
 *   - A is [M][lda] row-major fp16, C is [M][ldc] row-major (fp32 or fp16),
 *     W is [N][K] in the chosen block format: C = A . dequant(W)^T.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Calls only enqueue
 *     work; they are asynchronous with respect to the host.
 *   - Shapes, alignments and pointers are validated before anything is
 *     enqueued; a rejected call returns BF_ERR_INVALID and touches nothing.
 *   - Global state: the thread-local text of the last error (bf_last_error),
 *     per-device records that a kernel's LDS limit has been raised and of the
 *     device's XCD and CU counts, the workspaces above, the per-stream
 *     enqueue locks, and the per-GPU address of bf_gemm_noalloc's scratch
 *     array.
 */
#ifndef BUSFILL_H
#define BUSFILL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    BF_OK = 0,
    BF_ERR_INVALID = 1,      /* bad shape, pointer, alignment or enum */
    BF_ERR_UNSUPPORTED = 2,  /* valid request this build cannot serve */
    BF_ERR_HIP = 3           /* the HIP runtime reported an error on launch */
} bf_status;

typedef enum {
    BF_Q4_0 = 0,         /* llama.cpp block_q4_0: {fp16 d; u8 qs[16]} = 18 B / 32 weights,
                            elem j = qs[j] & 0xF, elem j+16 = qs[j] >> 4, value (q-8)*d     */
    BF_Q4_0_PLANES = 1,  /* reference layout (kernels/busfill_v0.cu:42-44,119-123):
                            Wq[N][K/2] u8, byte j = elems 2j (lo) and 2j+1 (hi);
                            Ws[N][K/32] fp16 (passed as W_aux); value (q-8)*d              */
    BF_Q4_K = 2          /* llama.cpp block_q4_K: {fp16 d, dmin; u8 scales[12]; u8 qs[128]}
                            = 144 B / 256 weights; value (d*sc)*q - dmin*m                 */
} bf_qtype;

typedef enum { BF_OUT_F32 = 0, BF_OUT_F16 = 1 } bf_otype;

typedef enum {
    BF_ALGO_AUTO = 0,    /* pick by shape and M                                        */
    BF_ALGO_MFMA = 1,    /* v_mfma_f32_16x16x32_f16 over 16-row batch tiles            */
    BF_ALGO_DOT2 = 2,    /* v_dot2_f32_f16 lanes + cross-lane reduction (small M)      */
    BF_ALGO_SIMPLE = 3,  /* one thread per output; any legal shape (slow, for odd K)   */
    BF_ALGO_LDS = 4,     /* direct-to-LDS staged weights + MFMA (M <= 8; M <= 16 when A
                            fits in LDS; weight steps and A segments cycle through
                            rings when they do not fit)                               */
    BF_ALGO_SLAB = 5,    /* weights and activation slabs through an LDS ring (M <= 32) */
    BF_ALGO_SPLIT = 6,   /* K split over workgroups, all operands resident in LDS (M <= 32);
                            uses a per-stream workspace allocated on first use          */
    BF_ALGO_DENSE = 7    /* all batch rows per workgroup, the weights streamed once
                            (M <= 128 per launch; the default above 32 rows and on
                            large matrices from 9 rows); one workgroup per CU over
                            equal shares of the row groups' K, split row groups
                            summed by a second launch through the same workspace      */
} bf_algo;

/* Reference-compatible entry: Q4_0 planes, fp32 output, C[Bsz][N] overwritten.
 * Replaces the busfill_q4<<<N/32,128>>> launch of kernels/busfill_v1a.cu:154,169
 * (same argument meaning and order, plus the stream).  Unlike the reference it
 * checks its preconditions (K % 32 == 0, Bsz >= 1, non-null pointers) and has no
 * Bsz <= 32 limit (kernels/busfill_v1a.cu:55-56 silently dropped rows >= 32). */
bf_status bf_busfill_q4(const uint16_t* A, const uint8_t* Wq, const uint16_t* Ws, float* C,
                        int Bsz, int K, int N, void* stream);

/* General GEMM: C[M][N] (ldc) = A[M][K] (lda) . dequant(W)^T.
 * W_aux is Ws for BF_Q4_0_PLANES and must be NULL otherwise.
 * Requirements: M, N >= 1; K % 32 == 0 (K % 256 == 0 for BF_Q4_K); lda >= K;
 * ldc >= N.  Fast paths additionally use 16-byte aligned A with lda % 8 == 0,
 * 16-byte aligned W and K % 256 == 0; other legal inputs run BF_ALGO_SIMPLE.
 * Replaces the reference's fused dequant+mma kernel (kernels/busfill_v1a.cu:41-104)
 * and, for Q4_K, its described dequantize-then-matmul (RESULTS.md:84-96). */
bf_status bf_gemm(bf_qtype qtype, const void* W, const void* W_aux,
                  const uint16_t* A, int lda, void* C, int ldc, bf_otype otype,
                  int M, int N, int K, void* stream);

/* bf_gemm with an explicit kernel family (for tests and the crossover sweep).
 * Returns BF_ERR_UNSUPPORTED if that family cannot serve the shape. */
bf_status bf_gemm_ex(bf_qtype qtype, const void* W, const void* W_aux,
                     const uint16_t* A, int lda, void* C, int ldc, bf_otype otype,
                     int M, int N, int K, bf_algo algo, void* stream);

/* bf_gemm that allocates nothing, for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference, whose kernel needs no scratch.
 * Same arguments, kernels and results as bf_gemm, bit for bit; where bf_gemm's
 * cross-workgroup exchanges (the K-split kernel at 9-32 batch rows per launch
 * when the activations do not fit in LDS, the dense kernel above 32 rows and
 * on large matrices) use
 * the workspace it allocates per stream, this call uses a 34 MiB scratch
 * array in device memory that each GPU holds for the life of the process.  It
 * calls no hipMalloc or hipFree; its first call on a device looks up that
 * device's array (hipGetSymbolAddress).  Every call on one GPU shares the
 * array: calls that overlap on one GPU (concurrent streams, or a captured
 * graph replayed while another such call runs) race and may return wrong
 * results.  Each K-split launch that exchanges partials in the kernel first
 * marks its slots free with a small kernel on the stream (no memset node in a
 * captured graph).  Returns
 * BF_ERR_INVALID, enqueueing nothing, for a shape whose launches need more
 * than 34 MiB of scratch (K-split partials of S splits x N x M rows in fp32,
 * 11 MB at the 27B-class layer's largest shapes at M = 32; dense partials of
 * 256 workgroups x 2 x 128 x M rows, 32 MiB at M = 128). */
bf_status bf_gemm_noalloc(bf_qtype qtype, const void* W, const void* W_aux,
                          const uint16_t* A, int lda, void* C, int ldc, bf_otype otype,
                          int M, int N, int K, void* stream);

/* Bytes of caller-owned workspace bf_gemm_ws needs for a GEMM of this format,
 * output type and shape (0: none); computed for lda = K and ldc = N with
 * 16-byte aligned operands, the case that runs the exchanging kernels.
 * The same bytes serve bf_busfill_q4_ws (BF_Q4_0_PLANES, BF_OUT_F32, M = Bsz).
 * No counterpart in the reference, whose kernel needs no scratch
 * (kernels/busfill_v1a.cu:41-46). */
size_t bf_gemm_workspace_bytes(bf_qtype qtype, bf_otype otype, int M, int N, int K);

/* bf_gemm with a caller-owned workspace: the call allocates nothing and the
 * library keeps no state between calls (each launch that exchanges partials
 * in the kernel first marks its slots free with a small kernel on the
 * stream).  workspace: 256-byte aligned device memory
 * of workspace_bytes >= bf_gemm_workspace_bytes(...) (NULL and 0 when that is
 * 0); BF_ERR_INVALID, enqueueing nothing, when it is too small.  The result is
 * bit-identical to bf_gemm's.  Calls that overlap in time (other streams, or
 * graph replays) must not share a workspace; calls in one stream may.
 * Replaces the busfill_q4 launch (kernels/busfill_v1a.cu:154,169) for
 * callers that own every device allocation, as the reference's caller does
 * (kernels/busfill_v1a.cu:140-145). */
bf_status bf_gemm_ws(bf_qtype qtype, const void* W, const void* W_aux,
                     const uint16_t* A, int lda, void* C, int ldc, bf_otype otype,
                     int M, int N, int K, void* workspace, size_t workspace_bytes, void* stream);

/* bf_busfill_q4 with a caller-owned workspace (as bf_gemm_ws).  Replaces the
 * busfill_q4<<<N/32,128>>> launch of kernels/busfill_v1a.cu:154,169 with the
 * reference's argument order and meaning, plus the workspace and the stream. */
bf_status bf_busfill_q4_ws(const uint16_t* A, const uint8_t* Wq, const uint16_t* Ws, float* C,
                           int Bsz, int K, int N, void* workspace, size_t workspace_bytes, void* stream);

/* One GEMM of a batch: bf_gemm's arguments C[0:M][0:N] = A[0:M][0:K] . dequant(W)^T. */
typedef struct {
    const void* W;
    const void* W_aux;
    const uint16_t* A;
    int lda;
    void* C;
    int ldc;
    int M, N, K;
} bf_gemm_desc;

/* `count` independent GEMMs of one format and one output type on `stream`,
 * with the results of calling bf_gemm for each (bit-identical).  No GEMM's
 * output may overlap another one's inputs or output: they may run
 * concurrently.  The GEMMs are grouped by the kernel bf_gemm would give each:
 * those on the LDS-staged kernel (batch 1-8, per batch size), those on the
 * K-split kernel (9-32 rows whose activations do not fit in LDS; 9-16 and
 * 17-32 rows apart) and those on the dense kernel (above 32 rows or from 9
 * rows on large matrices, per batch size) each share one launch per eight
 * GEMMs (the dense ones one sum launch too), so one GEMM's tail overlaps the next one's weight stream and
 * launch gaps go away (a decoder layer's linears); any other GEMM runs as one
 * bf_gemm call.  No counterpart in the reference, whose only entry point is
 * the single-GEMM kernel (kernels/busfill_v1a.cu:41-46). */
bf_status bf_gemm_batched(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs, void* stream);

/* Bytes of caller-owned workspace bf_gemm_batched_ws needs for these GEMMs (0:
 * none; 0 also for invalid descriptors, which bf_gemm_batched_ws rejects). */
size_t bf_gemm_batched_workspace_bytes(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs);

/* bf_gemm_batched with a caller-owned workspace, as bf_gemm_ws: the call
 * allocates nothing, keeps no state between calls and gives bf_gemm_batched's
 * bits.  No counterpart in the reference (kernels/busfill_v1a.cu:41-46 is its
 * only entry point). */
bf_status bf_gemm_batched_ws(bf_qtype qtype, bf_otype otype, int count, const bf_gemm_desc* descs,
                             void* workspace, size_t workspace_bytes, void* stream);

/* Bit-exact fp16 dequant: W_f16[N][K] = RN_fp16(value), value computed in fp32
 * exactly as kernels/busfill_v0.cu:74,78-81 ((q-8)*fp32(d)) for the Q4_0
 * formats and as ggml dequantize_row_q4_K ((d*sc)*q - dmin*m) for Q4_K. */
bf_status bf_dequant_f16(bf_qtype qtype, const void* W, const void* W_aux,
                         uint16_t* W_f16, int N, int K, void* stream);

/* The down projection of a SwiGLU feed-forward block with the activation
 * fused in: C = (SiLU(G) * U) . dequant(W)^T, where gate_up[M][ld] holds the
 * fused gate|up projection's output, G = columns 0..K-1 and U = K..2K-1 (ld >=
 * 2K, rows 16-byte aligned).  Each product is rounded to fp16 as
 * bf_swiglu_f16 rounds it, so the result is bit-identical to bf_swiglu_f16
 * followed by bf_gemm, without the second launch or the intermediate
 * buffer.  Batch 1-2 (decode), with the activations resident in LDS
 * (K <= 17408 at batch 2); other shapes return BF_ERR_UNSUPPORTED.  No
 * counterpart in the reference, which launches only the GEMM
 * (kernels/busfill_v1a.cu:41-46). */
bf_status bf_gemm_swiglu(bf_qtype qtype, const void* W, const void* W_aux,
                         const uint16_t* gate_up, int ld, void* C, int ldc, bf_otype otype,
                         int M, int N, int K, void* stream);

/* out[m][k] = RN_fp16(SiLU(g) * u) for g = gate_up[m][k], u = gate_up[m][K + k],
 * computed in fp32 as g / (1 + e^-g) * u.  K % 8 == 0; rows 16-byte aligned.
 * out may be gate_up itself (ldo = ld): the results then replace the gate half. */
bf_status bf_swiglu_f16(const uint16_t* gate_up, int ld, uint16_t* out, int ldo,
                        int M, int K, void* stream);

/* The weights of one linear: W, and for BF_Q4_0_PLANES its scale plane
 * (NULL for the other formats). */
typedef struct {
    const void* W;
    const void* W_aux;
} bf_qweights;

/* A SwiGLU feed-forward block, C[M][N] = (SiLU(A . Wg^T) * (A . Wu^T)) . Wd^T,
 * with gate and up [F][K] and down [N][F] in one format.  gate_up[M][ldgu]
 * (ldgu >= 2F, rows 16-byte aligned) is the caller's fp16 buffer for the
 * intermediate: the gate projection goes to columns 0..F-1 and the up
 * projection to F..2F-1, each rounded to fp16 as bf_gemm rounds an fp16
 * output, and SiLU(g) * u is rounded as bf_swiglu_f16 rounds it, so C is
 * bit-identical to bf_gemm (gate), bf_gemm (up), bf_swiglu_f16, bf_gemm
 * (down), whichever form runs:
 *   BF_FFN_TWO_LAUNCHES: batch 1-2 with the down projection's activations
 *     resident in LDS (as bf_gemm_swiglu): the gate and up GEMMs in one
 *     launch (bf_gemm_batched), then the down projection with SiLU(g) * u
 *     formed as its activations are loaded.  gate_up holds the two
 *     projections on return.
 *   BF_FFN_ONE_LAUNCH: batch 1-2 where every GEMM takes the LDS-staged
 *     kernel's batch-1 or all-of-A form: one launch, the down projection's
 *     workgroups streaming their weights while the gate and up workgroups
 *     finish and loading their activations once the last of those has
 *     stored its rows (device-scope stores, a count and release flags in the
 *     stream's workspace, described at the top of this file: allocated on
 *     the first such call, BF_ERR_UNSUPPORTED when that call is captured).
 *     Measured slower than two launches at every size tried (7-150 MB of
 *     weights: the in-launch hand-over costs more serial memory round trips
 *     than a kernel boundary); kept for comparison.  gate_up as above.
 *   BF_FFN_CALLS: any batch: the gate and up GEMMs, SiLU(g) * u in place over
 *     the gate half of gate_up, the down GEMM (gate_up then holds SiLU(g) * u
 *     and the up projection).
 *   BF_FFN_AUTO (bf_ffn_swiglu): two launches where they apply, else calls.
 * gate_up must not overlap A, C or the weights.  No counterpart in the
 * reference, whose only entry point is the single-GEMM kernel
 * (kernels/busfill_v1a.cu:41-46) and whose end-to-end runs drive a dense
 * Q4_K_M model through llama.cpp (RESULTS.md:66-68); in a 27B-class decoder
 * layer this block holds 150 MB of the linears' 186 MB of weights. */
typedef enum {
    BF_FFN_AUTO = 0,
    BF_FFN_ONE_LAUNCH = 1,
    BF_FFN_TWO_LAUNCHES = 2,
    BF_FFN_CALLS = 3
} bf_ffn_form;

bf_status bf_ffn_swiglu(bf_qtype qtype, bf_qweights gate, bf_qweights up, bf_qweights down,
                        const uint16_t* A, int lda, uint16_t* gate_up, int ldgu,
                        void* C, int ldc, bf_otype otype, int M, int K, int F, int N, void* stream);

/* bf_ffn_swiglu in a chosen form; BF_ERR_UNSUPPORTED when that form does not
 * serve the shape (nothing enqueued). */
bf_status bf_ffn_swiglu_ex(bf_qtype qtype, bf_qweights gate, bf_qweights up, bf_qweights down,
                           const uint16_t* A, int lda, uint16_t* gate_up, int ldgu,
                           void* C, int ldc, bf_otype otype, int M, int K, int F, int N,
                           bf_ffn_form form, void* stream);

/* ---------------------------------------------------------------- integer-dot path
 * Activations quantized to int8 per 32 values, multiplied in with integer
 * dots over the 4-bit codes (int8 MFMA per 32-weight block from 3 batch rows,
 * a 4-way dot per four weights below).  No counterpart in the reference's kernels;
 * its results (RESULTS.md:72-77, 93-96) credit llama.cpp's quantized GEMM
 * (quantize_q8_1 + dp4a vec-dots) with this activation form.  Not bit-equal
 * to bf_gemm: each activation moves by at most half its block's step d/2
 * (d = amax/127), so |C_q8 - C_fp16| <= sum_k |W[n][k]| * d_blk(k) / 2. */

/* Bytes of the quantized-activation buffer for M rows of K (K % 32 == 0):
 * q[M][K] int8, then d[M][K/32] fp32, then s[M][K/32] int32, contiguous.
 * Returns 0 for an invalid shape. */
size_t bf_q8_bytes(int M, int K);

/* Aq = quantize(A[M][lda] fp16) per 32-value block, as llama.cpp's
 * quantize_q8_1: d = amax/127, q = round(x/d) half away from zero (all zero
 * for an all-zero block), s = sum of the block's q (an exact integer; this
 * build keeps d in fp32).  A rows and Aq 16-byte aligned. */
bf_status bf_quantize_q8(const uint16_t* A, int lda, void* Aq, int M, int K, void* stream);

/* C[M][N] = sum over 32-blocks b of d_b * (scale * dot_b - offset * s_b), the
 * integer dots exact, over the weights in place (any of the three formats).
 * M = 1..16, K % 64 == 0, W and Aq 16-byte aligned; other shapes return
 * BF_ERR_UNSUPPORTED.  Aq must be bf_quantize_q8's output for the same M and
 * K: its d and s regions start at offsets that depend on M (bf_q8_bytes), so
 * to multiply the first rows of a larger batch, quantize those rows alone. */
bf_status bf_gemm_q8(bf_qtype qtype, const void* W, const void* W_aux, const void* Aq, void* C, int ldc,
                     bf_otype otype, int M, int N, int K, void* stream);

/* ---------------------------------------------------------------- GGUF files
 * A reader of llama.cpp's model files (GGUF versions 2 and 3, public
 * specification), memory-mapped.  Q4_0 and Q4_K tensors are stored in the
 * block layouts bf_gemm takes, so their bytes go to the device unchanged (no
 * repack).  The file is treated as untrusted input: every length and offset
 * is checked against the file size.  No counterpart in the reference, which
 * names the format (kernels/q4k_batched.py:7-8) but reads no file. */
typedef struct bf_gguf bf_gguf;

typedef struct {
    const char* name;      /* NUL-terminated; valid until bf_gguf_close */
    uint32_t ggml_type;    /* ggml type code: 0 F32, 1 F16, 2 Q4_0, 12 Q4_K, ... */
    int32_t qtype;         /* the matching bf_qtype (BF_Q4_0, BF_Q4_K), or -1 */
    uint32_t n_dims;
    uint64_t dims[4];      /* dims[0] = weights per row (K), dims[1] = rows (N); unused dims are 1 */
    uint64_t offset;       /* byte offset of the data in the file */
    uint64_t nbytes;       /* 0 when the type's size is unknown to the reader */
    const void* data;      /* host address of the mapped data (NULL when nbytes is 0) */
} bf_gguf_tensor;

bf_status bf_gguf_open(const char* path, bf_gguf** out);
void bf_gguf_close(bf_gguf* g);
int64_t bf_gguf_tensor_count(const bf_gguf* g);
bf_status bf_gguf_tensor_at(const bf_gguf* g, int64_t index, bf_gguf_tensor* out);
bf_status bf_gguf_find(const bf_gguf* g, const char* name, bf_gguf_tensor* out);
/* Metadata: a non-negative integer value of any integer type (or bool), or a
 * string (not NUL-terminated: *len bytes at *out, inside the mapping). */
bf_status bf_gguf_get_u64(const bf_gguf* g, const char* key, uint64_t* out);
bf_status bf_gguf_get_str(const bf_gguf* g, const char* key, const char** out, uint64_t* len);
/* Copies a tensor's bytes to device memory dst (t->nbytes bytes) on stream and
 * waits for the copy. */
bf_status bf_gguf_upload(const bf_gguf* g, const bf_gguf_tensor* t, void* dst, void* stream);

/* ggml mul_mat hook: the branch an engine built on ggml's HIP backend adds to
 * its mul_mat dispatch (ggml-cuda.cu's ggml_cuda_mul_mat) for quantized
 * weights.  No counterpart in the reference, whose end-to-end figures come
 * from a patched llama.cpp that it does not ship (RESULTS.md:66-68).
 *
 * A tensor as ggml describes it: ggml's type code, the device address, and
 * ggml_tensor's ne[4] (elements per dimension, ne[0] innermost) and nb[4]
 * (byte strides), with the meaning those fields have in ggml. */
typedef enum {
    BF_GGML_F32 = 0,
    BF_GGML_F16 = 1,
    BF_GGML_Q4_0 = 2,    /* block_q4_0 rows: BF_Q4_0 */
    BF_GGML_Q4_K = 12    /* block_q4_K rows: BF_Q4_K */
} bf_ggml_type;

typedef struct {
    int32_t type;        /* a bf_ggml_type code */
    void* data;          /* device address (read only for src0 and src1) */
    int64_t ne[4];
    uint64_t nb[4];
} bf_ggml_tensor;

/* dst = ggml_mul_mat(src0, src1) on `stream`, with ggml's semantics:
 *   dst[i3][i2][i1][i0] = sum_k dequant(src0)[i3 / r3][i2 / r2][i0][k] * src1[i3][i2][i1][k],
 * r2 = src1.ne[2] / src0.ne[2], r3 = src1.ne[3] / src0.ne[3] (src0 broadcast
 * over src1's outer dimensions, as ggml_can_mul_mat allows), dst.ne =
 * {src0.ne[1], src1.ne[1], src1.ne[2], src1.ne[3]}.  src1 is F32 or F16 with
 * any strides: it is rounded to fp16 (round to nearest even, as ggml's own
 * conversion) into a staging buffer unless it is already fp16 rows the GEMM
 * can read in place (16-byte aligned, row stride a multiple of 16 bytes), or
 * one or two 16-byte aligned F32 rows on the small-batch kernel whose compute
 * waves load all of A, which rounds them as it loads them (no staging launch);
 * each (i2, i3) slice is then one GEMM of bf_gemm_batched, with bf_gemm's bits
 * for the fp16 activations.
 * Serves src0 Q4_0 / Q4_K with whole rows (nb[0] the block size, nb[1] the
 * row's bytes), dst F32 with nb[0] = 4 and slices that do not overlap; any
 * other type or layout returns BF_ERR_UNSUPPORTED (the engine keeps its own
 * kernels for it), shapes ggml_mul_mat would reject BF_ERR_INVALID; both
 * before anything is enqueued.  The staging buffer is the library's, one per
 * (device, stream) as for bf_gemm's workspace. */
bf_status bf_ggml_mul_mat(const bf_ggml_tensor* src0, const bf_ggml_tensor* src1, const bf_ggml_tensor* dst,
                          void* stream);

/* Bytes of caller-owned workspace bf_ggml_mul_mat_ws needs (staging buffer
 * and the GEMMs' workspace; 0: none, also for requests bf_ggml_mul_mat_ws
 * rejects). */
size_t bf_ggml_mul_mat_workspace_bytes(const bf_ggml_tensor* src0, const bf_ggml_tensor* src1,
                                       const bf_ggml_tensor* dst);

/* bf_ggml_mul_mat with a caller-owned workspace (an engine's memory pool), as
 * bf_gemm_ws: allocates nothing, keeps no state, the same bits. */
bf_status bf_ggml_mul_mat_ws(const bf_ggml_tensor* src0, const bf_ggml_tensor* src1, const bf_ggml_tensor* dst,
                             void* workspace, size_t workspace_bytes, void* stream);

/* Static text for a status code. */
const char* bf_status_str(bf_status status);

/* Detail text for the calling thread's most recent non-OK status ("" if none). */
const char* bf_last_error(void);

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int bf_version(void);

#ifdef __cplusplus
}
#endif
#endif /* BUSFILL_H */
