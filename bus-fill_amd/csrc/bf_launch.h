// Host-side interface between the C-ABI front end (bf_api.hip) and the kernel
// families.  Arguments are validated by the front end before any of these runs.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bf_host.h"

namespace bf {

struct GemmArgs {
    int qtype;                 // QT_Q4_0 / QT_PLANES / QT_Q4_K
    const uint8_t* W;          // block bytes, or the Wq code plane
    const uint8_t* Waux;       // Ws scale plane (planes layout) or nullptr
    const uint16_t* A;         // [M][lda] fp16
    int lda;
    void* C;                   // [M][ldc] fp32 or fp16
    int ldc;
    int out_f16;
    int M, N, K;               // M <= 128 per launch (the front end slices larger M)
    int a_f32 = 0;             // A is fp32 rows, lda in floats (rounded to fp16 as loaded: lds_f32_supports)
};

// Device memory a call may use for the K-split kernel's workspace instead of
// the library's own (bytes == 0 never happens: a null Scratch* means "use the
// library's workspace for the stream").
struct Scratch {
    uint8_t* base;             // 256-byte aligned
    size_t bytes;
};

hipError_t gemm_mfma(const GemmArgs& g, hipStream_t st);
hipError_t gemm_dot2(const GemmArgs& g, hipStream_t st);
hipError_t gemm_simple(const GemmArgs& g, hipStream_t st);
hipError_t gemm_lds(const GemmArgs& g, hipStream_t st);
// g with a_f32 set: the LDS kernel of bf_gemm's plan for g's shape in a form
// whose compute waves load all of A (batch 1, and batch 2 where A fits), then
// rounding the fp32 rows to fp16 as they load them.
bool lds_f32_supports(const GemmArgs& g);
bool lds_supports(const GemmArgs& g);
// Independent GEMMs that all take the same LDS-staged kernel shape (batch 1,
// or G = 4 at batch 2-8), in launches of up to eight.
hipError_t gemm_lds_batched(const GemmArgs* gs, int n, hipStream_t st);
bool lds_batched_supports(const GemmArgs* gs, int n);
hipError_t gemm_slab(const GemmArgs& g, hipStream_t st);
bool slab_supports(const GemmArgs& g);
// XCDs of the current device (the workgroup round robin the XCD-local
// exchanges lay their grids out for), 0 if unknown.
int device_xcds();
// CUs of the current device, 0 if unknown.
int device_cus();
// Bytes of the library's per-stream workspace a launch needs, per region:
// counters (kept zero between launches), partial slots (kept free between
// launches) and partials.
struct WsNeed {
    size_t c = 0, s = 0, p = 0;
    void merge(const WsNeed& o) {
        c = c > o.c ? c : o.c;
        s = s > o.s ? s : o.s;
        p = p > o.p ? p : o.p;
    }
};
// Makes the stream's workspace at least `need` (allocating it now unless it
// already is; hipErrorStreamCaptureUnsupported while the stream is
// capturing), so that the launches that follow on the stream allocate
// nothing.
hipError_t reserve_workspace(hipStream_t st, const WsNeed& need);
// Counters and partials of a cross-workgroup exchange: carved out of `scratch`
// (its counters cleared by a kernel on the stream first) or the library's
// workspace for the stream (allocated on first use; never while the stream is
// capturing: hipErrorStreamCaptureUnsupported).  hipErrorInvalidValue when
// scratch is too small.
hipError_t split_workspace(const Scratch* scratch, hipStream_t st, size_t cbytes, size_t pbytes,
                           unsigned** counters, float** parts);

// The K-split kernel.  With S > 1 splits it needs a workspace (counters and
// partials): from `scratch` when given (its counters are cleared by a kernel
// on the stream first), else the library's per-stream workspace, allocated on
// first use and never while the stream is capturing (then the call returns
// hipErrorStreamCaptureUnsupported).  hipErrorInvalidValue when scratch is too
// small.
hipError_t gemm_split(const GemmArgs& g, const Scratch* scratch, hipStream_t st);
bool split_supports(const GemmArgs& g);
// The K-split plan takes more than one round of one workgroup per CU.
bool split_multi_round(const GemmArgs& g);
size_t split_scratch_bytes(const GemmArgs& g);      // 0 when the plan does not split K
WsNeed split_ws_need(const GemmArgs& g);            // of a launch on the library's workspace
// Independent GEMMs of one format, one output type and one side of M = 16, in
// launches of up to eight (their grids back to back).
hipError_t gemm_split_batched(const GemmArgs* gs, int n, const Scratch* scratch, hipStream_t st);
bool split_batched_supports(const GemmArgs* gs, int n);
size_t split_batched_scratch_bytes(const GemmArgs* gs, int n);
WsNeed split_batched_ws_need(const GemmArgs* gs, int n);
bool dot2_supports(const GemmArgs& g);
// The dense kernel (33-128 batch rows per launch, the weights streamed once):
// 64 weight rows x all batch rows per workgroup, K split with the exchange
// above when that balances the grid.
hipError_t gemm_dense(const GemmArgs& g, const Scratch* scratch, hipStream_t st);
bool dense_supports(const GemmArgs& g);
// Workspace bytes of the dense plan's partial pieces (0 when no row group is
// split between workgroups).
size_t dense_scratch_bytes(const GemmArgs& g);
WsNeed dense_ws_need(const GemmArgs& g);
// Independent dense-kernel GEMMs of one format, one batch size and one output
// type, in launches of up to eight (their grids back to back, each with the
// ranges of a launch of its own) and one sum launch each.
hipError_t gemm_dense_batched(const GemmArgs* gs, int n, const Scratch* scratch, hipStream_t st);
bool dense_batched_supports(const GemmArgs* gs, int n);
size_t dense_batched_scratch_bytes(const GemmArgs* gs, int n);
WsNeed dense_batched_ws_need(const GemmArgs* gs, int n);

hipError_t dequant_f16(int qtype, const uint8_t* W, const uint8_t* Waux, uint16_t* out,
                       int N, int K, hipStream_t st);

// ggml mul_mat hook: the rows of a strided fp32 (f32 = 1) or fp16 tensor
// (ne[4] elements, nb[4] byte strides, as ggml's ne / nb) rounded to fp16
// (nearest even) into dst[(i3 ne[2] + i2) ne[1] + i1][0:ne[0]] (ne[0] % 8 == 0,
// dst 16-byte aligned); and the stream's staging buffer for them (the
// library's, one per (device, stream) as its workspace; grown on demand, a
// replaced one retired, never freed; hipErrorStreamCaptureUnsupported when it
// would have to grow while the stream is capturing).
hipError_t stage_rows_f16(const void* src, int f32, const int64_t ne[4], const uint64_t nb[4], uint16_t* dst,
                          hipStream_t st);
hipError_t staging_buffer(hipStream_t st, size_t bytes, uint16_t** out);
// A = SiLU(A[:, 0:K]) * A[:, K:2K] formed while loading (batch 1-2 plans that
// load A through the compute waves), and the standalone elementwise kernel.
hipError_t gemm_lds_swiglu(const GemmArgs& g, hipStream_t st);
bool lds_swiglu_supports(const GemmArgs& g);
hipError_t swiglu_f16(const uint16_t* gu, int ld, uint16_t* out, int ldo, int M, int K, hipStream_t st);
// The SwiGLU feed-forward block in one launch (gs[0] gate and gs[1] up into
// the two halves of one fp16 gate|up buffer, gs[2] the down projection whose A
// is that buffer, SiLU(gate) * up formed as it is loaded): batch 1-2 where
// every GEMM takes the LDS kernel's batch-1 form or its all-of-A form.  Two
// counters in the stream's workspace (allocated on first use, never while
// the stream is capturing: hipErrorStreamCaptureUnsupported).
hipError_t ffn_lds(const GemmArgs* gs, hipStream_t st);
bool ffn_lds_supports(const GemmArgs* gs);

// Integer-dot activation path: int8 activations per 32 values (q | d | s
// regions of one buffer of q8_bytes(M, K)) and the v_dot4_i32_i8 GEMM.
struct Q8Args {
    int qtype;
    const uint8_t* W;
    const uint8_t* Waux;
    const void* Aq;            // q8_bytes(M, K) bytes from quantize_q8
    void* C;
    int ldc;
    int out_f16;
    int M, N, K;               // M <= 16, K % 64 == 0
};
size_t q8_bytes(int M, int K);
hipError_t quantize_q8(const uint16_t* A, int lda, void* Aq, int M, int K, hipStream_t st);
bool q8_supports(int M, int K);
hipError_t gemm_q8(const Q8Args& g, hipStream_t st);

}  // namespace bf
