// Bench host: the timed loops that drive libbusfill through its C-ABI.
//
// Restates the reference harness's timing (kernels/busfill_v1a.cu:168-175:
// cudaEvent around back-to-back launches, tok/s = B/t) with two changes the
// MI355X needs: the loop cycles through a caller-provided set of DISTINCT
// weight matrices (>= 1 GB, so the 256 MB Infinity Cache cannot serve them),
// and it can replay the same launch sequence as a captured HIP graph.
// Events are recorded on the stream the kernels run on.
//
// Also holds two plain memory kernels used as yardsticks: a 128-bit streaming
// read (the achievable HBM read rate) and a 128-bit copy (the calibration
// kernel for FETCH_SIZE / WRITE_SIZE counters).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

#include "busfill.h"

namespace {

thread_local hipError_t g_err = hipSuccess;
thread_local bf_status g_bf = BF_OK;

#define HCK(x)                                  \
    do {                                        \
        hipError_t e_ = (x);                    \
        if (e_ != hipSuccess) {                 \
            g_err = e_;                         \
            return -1;                          \
        }                                       \
    } while (0)

struct Launch {
    int qtype;
    const void* W;
    const void* W_aux;
    const uint16_t* A;
    int lda;
    void* C;
    int ldc;
    int M, N, K;
};

int issue(const Launch& l, int otype, int algo, hipStream_t st) {
    bf_status s = bf_gemm_ex((bf_qtype)l.qtype, l.W, l.W_aux, l.A, l.lda, l.C, l.ldc, (bf_otype)otype, l.M, l.N,
                             l.K, (bf_algo)algo, st);
    if (s != BF_OK) {
        g_bf = s;
        return -1;
    }
    return 0;
}

// `group` consecutive GEMMs from seq (cyclically) in one bf_gemm_batched call.
int issue_group(const std::vector<Launch>& seq, size_t first, int group, int otype, hipStream_t st) {
    std::vector<bf_gemm_desc> d(group);
    for (int j = 0; j < group; j++) {
        const Launch& l = seq[(first + j) % seq.size()];
        d[j] = bf_gemm_desc{l.W, l.W_aux, l.A, l.lda, l.C, l.ldc, l.M, l.N, l.K};
    }
    bf_status s = bf_gemm_batched((bf_qtype)seq[first % seq.size()].qtype, (bf_otype)otype, group, d.data(), st);
    if (s != BF_OK) {
        g_bf = s;
        return -1;
    }
    return 0;
}

// Runs `warmup` then `steps` GEMMs taken cyclically from seq, one launch call
// per GEMM (group 1) or one bf_gemm_batched call per `group` GEMMs; returns ms.
// The timed GEMMs continue the rotation where the warmup stopped (GEMM i of the
// run uses seq[i % n], i counting from the first warmup GEMM), so with a
// rotation larger than the caches no timed GEMM finds its weights left there
// by the warmup.
int time_seq(const std::vector<Launch>& seq, int otype, int algo, int warmup, int steps, int use_graph,
             hipStream_t st, double* ms_out, int group = 1) {
    const size_t n = seq.size();
    auto issue = [&](int i) -> int {
        if (group > 1) return (i % group) ? 0 : issue_group(seq, (size_t)i, group, otype, st);
        return ::issue(seq[(size_t)i % n], otype, algo, st);
    };
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    float ms = 0.f;
    if (!use_graph) {
        for (int i = 0; i < warmup; i++)
            if (issue(i)) return -1;
        HCK(hipStreamSynchronize(st));
        HCK(hipEventRecord(e0, st));
        for (int i = warmup; i < warmup + steps; i++)
            if (issue(i)) return -1;
        HCK(hipEventRecord(e1, st));
        HCK(hipEventSynchronize(e1));
        HCK(hipEventElapsedTime(&ms, e0, e1));
    } else {
        auto capture = [&](int first, int count, hipGraphExec_t* exec) -> int {
            hipGraph_t g;
            HCK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            for (int i = first; i < first + count; i++)
                if (issue(i)) {
                    hipGraph_t dead;
                    (void)hipStreamEndCapture(st, &dead);
                    return -1;
                }
            HCK(hipStreamEndCapture(st, &g));
            HCK(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
            HCK(hipGraphDestroy(g));
            return 0;
        };
        // one uncaptured call first, so that the stream's workspace exists
        // before the capture (the library allocates none while capturing)
        if (issue(0)) return -1;
        HCK(hipStreamSynchronize(st));
        hipGraphExec_t gw = nullptr, gs = nullptr;
        if (warmup > 0 && capture(0, warmup, &gw)) return -1;
        if (capture(warmup, steps, &gs)) return -1;
        if (gw) HCK(hipGraphLaunch(gw, st));
        HCK(hipStreamSynchronize(st));
        HCK(hipEventRecord(e0, st));
        HCK(hipGraphLaunch(gs, st));
        HCK(hipEventRecord(e1, st));
        HCK(hipEventSynchronize(e1));
        HCK(hipEventElapsedTime(&ms, e0, e1));
        if (gw) HCK(hipGraphExecDestroy(gw));
        HCK(hipGraphExecDestroy(gs));
    }
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    *ms_out = ms;
    return 0;
}

// Times `steps` calls of call(i) (i continuing from the `warmup` untimed
// ones), issued on st directly or captured into a graph and replayed.  One
// uncaptured call comes first, so that any workspace the calls use exists
// before a capture.
template <class Call>
int time_calls(Call call, int warmup, int steps, int use_graph, hipStream_t st, double* ms_out) {
    if ((g_bf = call(0)) != BF_OK) return -1;
    HCK(hipStreamSynchronize(st));
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    float ms = 0.f;
    if (!use_graph) {
        for (int i = 0; i < warmup; i++)
            if ((g_bf = call(i)) != BF_OK) return -1;
        HCK(hipStreamSynchronize(st));
        HCK(hipEventRecord(e0, st));
        for (int i = warmup; i < warmup + steps; i++)
            if ((g_bf = call(i)) != BF_OK) return -1;
        HCK(hipEventRecord(e1, st));
    } else {
        auto capture = [&](int first, int count, hipGraphExec_t* exec) -> int {
            hipGraph_t g;
            HCK(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
            for (int i = first; i < first + count; i++)
                if ((g_bf = call(i)) != BF_OK) {
                    hipGraph_t dead;
                    (void)hipStreamEndCapture(st, &dead);
                    return -1;
                }
            HCK(hipStreamEndCapture(st, &g));
            HCK(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
            HCK(hipGraphDestroy(g));
            return 0;
        };
        hipGraphExec_t gw = nullptr, gs = nullptr;
        if (warmup > 0 && capture(0, warmup, &gw)) return -1;
        if (capture(warmup, steps, &gs)) return -1;
        if (gw) HCK(hipGraphLaunch(gw, st));
        HCK(hipStreamSynchronize(st));
        HCK(hipEventRecord(e0, st));
        HCK(hipGraphLaunch(gs, st));
        HCK(hipEventRecord(e1, st));
        HCK(hipEventSynchronize(e1));
        if (gw) HCK(hipGraphExecDestroy(gw));
        HCK(hipGraphExecDestroy(gs));
    }
    HCK(hipEventSynchronize(e1));
    HCK(hipEventElapsedTime(&ms, e0, e1));
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    *ms_out = ms;
    return 0;
}

__global__ __launch_bounds__(1024) void k_stream_read(const uint4* __restrict__ src, size_t n16,
                                                     unsigned* __restrict__ sink) {
    unsigned acc = 0;
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
        uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;   // keeps the loads live; practically never taken
}

// No memory access at all (the condition is on an argument the host never
// sets): back-to-back launches of it time a stream's per-kernel floor.
__global__ __launch_bounds__(1024) void k_empty(unsigned* __restrict__ sink, int never) {
    if (never == 0x5EED && threadIdx.x == 0) sink[0] = 1u;
}

__global__ __launch_bounds__(256) void k_stream_copy(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                     size_t n16) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

}  // namespace

extern "C" {

// Times `steps` GEMMs (after `warmup` untimed ones) cycling through `count`
// weight matrices W[i] (W_aux[i] for the planes layout), same A and C.
int bfb_time_gemms(int qtype, const void* const* W, const void* const* W_aux, int count, const uint16_t* A,
                   int lda, void* C, int ldc, int otype, int M, int N, int K, int algo, int warmup, int steps,
                   int use_graph, void* stream, double* ms_out) {
    std::vector<Launch> seq;
    for (int i = 0; i < count; i++) seq.push_back(Launch{qtype, W[i], W_aux ? W_aux[i] : nullptr, A, lda, C, ldc, M, N, K});
    return time_seq(seq, otype, algo, warmup, steps, use_graph, (hipStream_t)stream, ms_out);
}

// Times `steps` launches cycling through a heterogeneous list of n GEMMs
// (e.g. the linears of decoder layers).
int bfb_time_sequence(int n, const int* qtype, const void* const* W, const void* const* W_aux,
                      const uint16_t* const* A, const int* lda, void* const* C, const int* ldc, const int* M,
                      const int* N, const int* K, int otype, int algo, int warmup, int steps, int use_graph,
                      void* stream, double* ms_out) {
    std::vector<Launch> seq;
    for (int i = 0; i < n; i++)
        seq.push_back(Launch{qtype[i], W[i], W_aux ? W_aux[i] : nullptr, A[i], lda[i], C[i], ldc[i], M[i], N[i], K[i]});
    return time_seq(seq, otype, algo, warmup, steps, use_graph, (hipStream_t)stream, ms_out);
}

// The same list issued as bf_gemm_batched calls of `group` consecutive GEMMs
// (warmup and steps count GEMMs and must be multiples of group).
int bfb_time_sequence_batched(int n, int group, const int* qtype, const void* const* W, const void* const* W_aux,
                              const uint16_t* const* A, const int* lda, void* const* C, const int* ldc,
                              const int* M, const int* N, const int* K, int otype, int warmup, int steps,
                              int use_graph, void* stream, double* ms_out) {
    if (group < 1 || n % group || warmup % group || steps % group) {
        g_err = hipErrorInvalidValue;
        return -1;
    }
    std::vector<Launch> seq;
    for (int i = 0; i < n; i++)
        seq.push_back(Launch{qtype[i], W[i], W_aux ? W_aux[i] : nullptr, A[i], lda[i], C[i], ldc[i], M[i], N[i], K[i]});
    return time_seq(seq, otype, 0, warmup, steps, use_graph, (hipStream_t)stream, ms_out, group);
}

// Streaming 128-bit read of `bytes` at `src`, `reps` times; returns ms.
int bfb_read_peak(const void* src, size_t bytes, int reps, void* sink, void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    const size_t n16 = bytes / 16;
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    hipLaunchKernelGGL(k_stream_read, dim3(2048), dim3(256), 0, st, (const uint4*)src, n16, (unsigned*)sink);
    HCK(hipGetLastError());
    HCK(hipEventRecord(e0, st));
    for (int r = 0; r < reps; r++)
        hipLaunchKernelGGL(k_stream_read, dim3(2048), dim3(256), 0, st, (const uint4*)src, n16, (unsigned*)sink);
    HCK(hipGetLastError());
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

// The down projection of a SwiGLU block, cycling through `count` weight
// matrices: fused (bf_gemm_swiglu) or SiLU*up by bf_swiglu_f16 into a_tmp
// then bf_gemm; `steps` calls timed after `warmup`.
int bfb_time_swiglu(int qtype, const void* const* W, const void* const* W_aux, int count, const uint16_t* gate_up,
                    int ld, uint16_t* a_tmp, void* C, int M, int N, int K, int fused, int warmup, int steps,
                    void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    auto call = [&](int r) -> bf_status {
        const void* w = W[r % count];
        const void* aux = W_aux ? W_aux[r % count] : nullptr;
        if (fused) return bf_gemm_swiglu((bf_qtype)qtype, w, aux, gate_up, ld, C, N, BF_OUT_F32, M, N, K, st);
        bf_status s2 = bf_swiglu_f16(gate_up, ld, a_tmp, K, M, K, st);
        if (s2 != BF_OK) return s2;
        return bf_gemm((bf_qtype)qtype, w, aux, a_tmp, K, C, N, BF_OUT_F32, M, N, K, st);
    };
    for (int r = 0; r < warmup; r++)
        if ((g_bf = call(r)) != BF_OK) return -1;
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    HCK(hipEventRecord(e0, st));
    for (int r = warmup; r < warmup + steps; r++)
        if ((g_bf = call(r)) != BF_OK) {
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
            return -1;
        }
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

// SwiGLU feed-forward blocks (bf_ffn_swiglu_ex in one form), cycling through
// `count` blocks' weights (gate Wg[i], up Wu[i], down Wd[i]; planes scale
// planes in the *_aux arrays or NULL), same A, gate_up and C.
int bfb_time_ffn(int qtype, const void* const* Wg, const void* const* Wg_aux, const void* const* Wu,
                 const void* const* Wu_aux, const void* const* Wd, const void* const* Wd_aux, int count,
                 const uint16_t* A, uint16_t* gate_up, void* C, int M, int K, int F, int N, int form, int warmup,
                 int steps, int use_graph, void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    auto call = [&](int r) -> bf_status {
        const int i = r % count;
        const bf_qweights g{Wg[i], Wg_aux ? Wg_aux[i] : nullptr}, u{Wu[i], Wu_aux ? Wu_aux[i] : nullptr},
            d{Wd[i], Wd_aux ? Wd_aux[i] : nullptr};
        return bf_ffn_swiglu_ex((bf_qtype)qtype, g, u, d, A, K, gate_up, 2 * F, C, N, BF_OUT_F32, M, K, F, N,
                                (bf_ffn_form)form, st);
    };
    return time_calls(call, warmup, steps, use_graph, st, ms_out);
}

// The integer-dot path against the fp16 GEMM over the same weight rotation:
// mode 0 = bf_gemm on fp16 A, 1 = bf_quantize_q8 + bf_gemm_q8 (the whole
// q8 path per GEMM), 2 = bf_gemm_q8 alone on Aq quantized beforehand.
int bfb_time_q8(int qtype, const void* const* W, const void* const* W_aux, int count, const uint16_t* A,
                void* Aq, void* C, int M, int N, int K, int mode, int warmup, int steps, void* stream,
                double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    auto call = [&](int r) -> bf_status {
        const void* w = W[r % count];
        const void* aux = W_aux ? W_aux[r % count] : nullptr;
        if (mode == 0) return bf_gemm((bf_qtype)qtype, w, aux, A, K, C, N, BF_OUT_F32, M, N, K, st);
        if (mode == 1) {
            bf_status s2 = bf_quantize_q8(A, K, Aq, M, K, st);
            if (s2 != BF_OK) return s2;
        }
        return bf_gemm_q8((bf_qtype)qtype, w, aux, Aq, C, N, BF_OUT_F32, M, N, K, st);
    };
    if (mode == 2 && (g_bf = bf_quantize_q8(A, K, Aq, M, K, st)) != BF_OK) return -1;
    for (int r = 0; r < warmup; r++)
        if ((g_bf = call(r)) != BF_OK) return -1;
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    HCK(hipEventRecord(e0, st));
    for (int r = warmup; r < warmup + steps; r++)
        if ((g_bf = call(r)) != BF_OK) {
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
            return -1;
        }
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

// The ggml mul_mat hook over the rotation (src0 Q4_0 / Q4_K rows, one matrix
// per call, dst [M][N] F32): mode 0 bf_gemm on fp16 activations A16 (the hook's
// GEMM alone), 1 bf_ggml_mul_mat with F32 src1 A32 (staged to fp16 first),
// 2 bf_ggml_mul_mat with F16 src1 A16 (read in place).
int bfb_time_ggml(int qtype, const void* const* W, int count, const float* A32, const uint16_t* A16, float* C,
                  int M, int N, int K, int mode, int warmup, int steps, void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    const int blk = qtype == BF_Q4_K ? 256 : 32, bb = qtype == BF_Q4_K ? 144 : 18;
    bf_ggml_tensor s0 = {}, s1 = {}, d = {};
    s0.type = qtype == BF_Q4_K ? BF_GGML_Q4_K : BF_GGML_Q4_0;
    s1.type = mode == 1 ? BF_GGML_F32 : BF_GGML_F16;
    d.type = BF_GGML_F32;
    const int64_t ne0[4] = {K, N, 1, 1}, ne1[4] = {K, M, 1, 1}, ned[4] = {N, M, 1, 1};
    const uint64_t es = mode == 1 ? 4 : 2, rb = (uint64_t)K / blk * bb;
    const uint64_t nb0[4] = {(uint64_t)bb, rb, rb * N, rb * N}, nb1[4] = {es, es * K, es * K * M, es * K * M},
                   nbd[4] = {4, 4ull * N, 4ull * N * M, 4ull * N * M};
    for (int i = 0; i < 4; i++) {
        s0.ne[i] = ne0[i], s0.nb[i] = nb0[i];
        s1.ne[i] = ne1[i], s1.nb[i] = nb1[i];
        d.ne[i] = ned[i], d.nb[i] = nbd[i];
    }
    s1.data = mode == 1 ? (void*)A32 : (void*)A16;
    d.data = C;
    auto call = [&](int r) -> bf_status {
        const void* w = W[r % count];
        if (mode == 0) return bf_gemm((bf_qtype)qtype, w, nullptr, A16, K, C, N, BF_OUT_F32, M, N, K, st);
        s0.data = (void*)w;
        return bf_ggml_mul_mat(&s0, &s1, &d, st);
    };
    for (int r = 0; r < warmup; r++)
        if ((g_bf = call(r)) != BF_OK) return -1;
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    HCK(hipEventRecord(e0, st));
    for (int r = warmup; r < warmup + steps; r++)
        if ((g_bf = call(r)) != BF_OK) {
            (void)hipEventDestroy(e0);
            (void)hipEventDestroy(e1);
            return -1;
        }
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

// `steps` back-to-back launches of k_empty (blocks x threads) after `warmup`:
// the time per launch that any kernel of that grid takes on the stream.
int bfb_empty_launches(int blocks, int threads, int warmup, int steps, void* sink, void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    if (blocks < 1 || threads < 64 || threads > 1024 || threads % 64) {
        g_err = hipErrorInvalidValue;
        return -1;
    }
    for (int r = 0; r < warmup; r++)
        hipLaunchKernelGGL(k_empty, dim3(blocks), dim3(threads), 0, st, (unsigned*)sink, 0);
    HCK(hipGetLastError());
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    HCK(hipEventRecord(e0, st));
    for (int r = 0; r < steps; r++)
        hipLaunchKernelGGL(k_empty, dim3(blocks), dim3(threads), 0, st, (unsigned*)sink, 0);
    HCK(hipGetLastError());
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

// Streaming reads of `bytes` per launch cycling through `count` buffers src[i]
// (the weight rotation): the time one launch of that size takes to read its
// bytes from HBM with nothing else to do.  Grid blocks x threads.
int bfb_read_slices(const void* const* src, int count, size_t bytes, int blocks, int threads, int warmup,
                    int steps, void* sink, void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    const size_t n16 = bytes / 16;
    if (count < 1 || blocks < 1 || threads < 64 || threads > 1024 || threads % 64) {
        g_err = hipErrorInvalidValue;
        return -1;
    }
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    for (int r = 0; r < warmup; r++)
        hipLaunchKernelGGL(k_stream_read, dim3(blocks), dim3(threads), 0, st, (const uint4*)src[r % count], n16,
                           (unsigned*)sink);
    HCK(hipGetLastError());
    HCK(hipEventRecord(e0, st));
    for (int r = warmup; r < warmup + steps; r++)
        hipLaunchKernelGGL(k_stream_read, dim3(blocks), dim3(threads), 0, st, (const uint4*)src[r % count], n16,
                           (unsigned*)sink);
    HCK(hipGetLastError());
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

// 128-bit copy of `bytes` (the known-size calibration kernel for HBM counters).
int bfb_copy(const void* src, void* dst, size_t bytes, int reps, void* stream, double* ms_out) {
    hipStream_t st = (hipStream_t)stream;
    const size_t n16 = bytes / 16;
    hipEvent_t e0, e1;
    HCK(hipEventCreate(&e0));
    HCK(hipEventCreate(&e1));
    HCK(hipEventRecord(e0, st));
    for (int r = 0; r < reps; r++)
        hipLaunchKernelGGL(k_stream_copy, dim3(2048), dim3(256), 0, st, (const uint4*)src, (uint4*)dst, n16);
    HCK(hipGetLastError());
    HCK(hipEventRecord(e1, st));
    HCK(hipEventSynchronize(e1));
    float ms;
    HCK(hipEventElapsedTime(&ms, e0, e1));
    *ms_out = ms;
    HCK(hipEventDestroy(e0));
    HCK(hipEventDestroy(e1));
    return 0;
}

const char* bfb_last_error(void) {
    static thread_local char buf[512];
    if (g_bf != BF_OK) snprintf(buf, sizeof buf, "%s: %s", bf_status_str(g_bf), bf_last_error());
    else snprintf(buf, sizeof buf, "%s", hipGetErrorString(g_err));
    return buf;
}

}  // extern "C"
