// Slab-streamed MFMA GEMM for batches of 9 to 32 rows (k_gemm_slab).
//
//   C[m][n] = sum_k A[m][k] * dequant(W)[n][k]      (fp32 accumulation)
//
// At these batch sizes the activations are what costs: every workgroup needs
// all of A (328 KB at M = 32, K = 5120), and reading it in the MFMA fragment
// pattern (16 rows x 64 scattered bytes per instruction) reaches only ~5.6 TB/s
// from L2, against 15-27 TB/s for contiguous 1 KB loads.  So:
//
// * One workgroup per CU: the N/16 row tiles are spread over 256 workgroups
//   (N = 5120: 64 workgroups of two tiles, 192 of one), each tile with the full
//   K, so A is read once per CU and no cross-workgroup reduction exists.
// * Loader waves stream, per super-group step e, the workgroup's weights
//   (nt x 16 rows x 144 bytes) and the activation slab A[0:M][256e, 256e+256)
//   into one slot of an LDS ring, with direct-to-LDS loads (1 KB per
//   instruction; the slab's rows are 512-byte runs), then a one-dword marker
//   load into the step's flag (a wave's loads return in order, so a visible
//   marker means the step has landed).  Before reusing a slot, the loader waits
//   for the "consumed" flag of the step that last used it.
// * Compute waves take steps c, c + NC, ...: they read the step's weight images
//   and activation fragments from LDS (bank-conflict-free strides), release the
//   slot, then decode and run nt x MT x 8 MFMAs, accumulating in registers.  At
//   the end each compute wave parks its accumulators in LDS; the last one to
//   finish (an LDS counter) adds them in wave order and stores C, so results
//   do not depend on timing.
#include <atomic>

#include "bf_launch.h"
#include "bf_lds.h"

namespace bf {
namespace {

constexpr int kSlabFlags = 2048;         // ready[e] at 64 + 4e, consumed[e] at 1024 + 4e, counter at 4
constexpr int kSlabPoison = 3;           // flags[3]: a bounded wait gave up (results become NaN)
constexpr int kSlabMaxSteps = (1024 - 64) / 4;

template <int QT, int MT, int NTMAX, int NC, int NL, int D>
__global__ __launch_bounds__(64 * (NC + NL))
void k_gemm_slab(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux,
                 const uint16_t* __restrict__ A, int lda, void* __restrict__ C, int ldc, int out_f16,
                 int M, int N, int K, int tiles, int w_slot, int a_slot) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsg = K >> 8;
    const int t0 = (int)((int64_t)tiles * blockIdx.x / gridDim.x);
    const int t1 = (int)((int64_t)tiles * (blockIdx.x + 1) / gridDim.x);
    const int nt = t1 - t0;                            // 1 .. NTMAX row tiles of 16
    int* const flags = (int*)lds;
    const int slot_bytes = w_slot + a_slot;
    uint8_t* const ring = lds + kSlabFlags;
    float* const parts = (float*)(ring + D * slot_bytes);
    const uint32_t lds0 = lds_addr(lds);

    if (wave == 0) {
        for (int i = lane; i < kSlabFlags / 4; i += 64) flags[i] = 0;
    }
    barrier_lds();

    if (wave >= NC) {
        // ------------------------------------------------------------ loader wave
        __builtin_amdgcn_s_setprio(3);
        const int j = wave - NC;
        const int nIw = (nt * 144 + 63) >> 6;          // instructions of the weight part
        const int nIa = (M * 33 + 63) >> 6;            // instructions of the activation slab
        for (int e = j; e < nsg; e += NL) {
            if (e >= D) wait_flag(&flags[256 + e - D], flags + kSlabPoison);   // the slot's previous step is consumed
            const uint32_t slot = lds0 + (uint32_t)(kSlabFlags + (e % D) * slot_bytes);
            for (int i = 0; i < nIw; i++) {
                const int P = 64 * i + lane;           // piece of the weight part: tile, row, part
                const int tt = P / 144, q = P - 144 * tt, n = q / 9, c = q - 9 * n;
                const int64_t row = min((int64_t)(t0 + min(tt, nt - 1)) * 16 + n, (int64_t)N - 1);
                if (P < nt * 144) dma16(w_piece<QT>(W, Waux, row, e, c, K), slot + (uint32_t)(i << 10));
            }
            for (int i = 0; i < nIa; i++) {
                // LDS piece P of the slab is row m = P / 33, 16-byte part c = P % 33 (part 32 is the
                // row's bank padding and is not loaded): rows sit 528 bytes apart
                const int P = 64 * i + lane;
                const int m = P / 33, c = P - 33 * m;
                if (P < M * 33 && c < 32)
                    dma16(A + (int64_t)m * lda + 256 * e + 8 * c, slot + (uint32_t)(w_slot + (i << 10)));
            }
            dma_marker(g_marker_src + lane, lds0 + 64 + 4 * e, lane);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---------------------------------------------------------------- compute wave
    const int c = wave;
    const Magic mg = make_magic();
    const int r = lane & 15, kg = lane >> 4;
    f4 acc[NTMAX][MT];
#pragma unroll
    for (int tt = 0; tt < NTMAX; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[tt][mt] = f4{0.f, 0.f, 0.f, 0.f};
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = min(16 * mt + r, M - 1) * 528 + 128 * kg;

    for (int e = c; e < nsg; e += NC) {
        wait_flag(&flags[16 + e], flags + kSlabPoison);
        const uint8_t* slot = ring + (e % D) * slot_bytes;
        Raw<QT> raw[NTMAX] = {};
#pragma unroll
        for (int tt = 0; tt < NTMAX; tt++)
            if (tt < nt) lds_raw<QT>(raw[tt], slot + tt * kStep + r * 144, kg);
        h8 a[MT][8];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 8; i++) a[mt][i] = *(const h8*)(slot + w_slot + arow[mt] + 16 * i);
        // every LDS read of this step has returned: release the slot
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[256 + e])), "v"(1) : "memory");
#pragma unroll
        for (int tt = 0; tt < NTMAX; tt++) {
            if (tt < nt) {
                const auto sc = scales(raw[tt], kg);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const h8 b = weights(mg, raw[tt], sc, i);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) acc[tt][mt] = mfma16x16x32(a[mt][i], b, acc[tt][mt]);
                }
            }
        }
    }

    // park this wave's sums; the last compute wave adds them in wave order and stores
    constexpr int PER = NTMAX * MT * 4;                // floats per lane
    float* mine = parts + (c * 64 + lane) * PER;
#pragma unroll
    for (int tt = 0; tt < NTMAX; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) mine[(tt * MT + mt) * 4 + i] = acc[tt][mt][i];
    int old = 0;
    if (lane == 0)
        asm volatile("s_waitcnt lgkmcnt(0)\n\tds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                     : "=v"(old) : "v"(lds_addr(&flags[1])), "v"(1) : "memory");
    if (__builtin_amdgcn_readfirstlane(old) != NC - 1) return;
    const bool bad = poisoned(flags + kSlabPoison);
#pragma unroll
    for (int tt = 0; tt < NTMAX; tt++) {
        if (tt >= nt) break;
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float v = 0.f;
                for (int w2 = 0; w2 < NC; w2++) v += parts[(w2 * 64 + lane) * PER + (tt * MT + mt) * 4 + i];
                if (bad) v = __builtin_nanf("");
                const int m = 16 * mt + 4 * kg + i;
                const int64_t n = (int64_t)(t0 + tt) * 16 + r;
                if (m < M && n < N) {
                    if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)v;
                    else ((float*)C)[(int64_t)m * ldc + n] = v;
                }
            }
        }
    }
}

constexpr int kSlabNC = 8, kSlabNL = 4, kSlabD = 5;

struct SlabPlan {
    int MT, NTMAX, grid, tiles, w_slot, a_slot, lds;
};

bool plan_slab(const GemmArgs& g, SlabPlan& p) {
    if (g.qtype == QT_PLANES) return false;            // block formats only (one weight pointer)
    const int nsg = g.K / 256;
    if (nsg > kSlabMaxSteps || g.M > 32) return false;
    p.MT = g.M <= 16 ? 1 : 2;
    p.tiles = (g.N + 15) / 16;
    p.grid = p.tiles < 256 ? p.tiles : 256;
    int per = (p.tiles + p.grid - 1) / p.grid;
    if (per > 2) {                                      // at most two tiles per workgroup
        p.grid = (p.tiles + 1) / 2;
        per = 2;
    }
    p.NTMAX = per;
    p.w_slot = (per * kStep + 1023) / 1024 * 1024;
    p.a_slot = (g.M * 528 + 1023) / 1024 * 1024;
    const int64_t lds = kSlabFlags + (int64_t)kSlabD * (p.w_slot + p.a_slot) +
                        (int64_t)kSlabNC * 64 * p.NTMAX * p.MT * 4 * 4;
    if (lds > kMaxLds) return false;
    p.lds = (int)lds;
    return true;
}

template <int QT, int MT, int NTMAX>
hipError_t launch_slab(const GemmArgs& g, const SlabPlan& p, hipStream_t st) {
    auto k = k_gemm_slab<QT, MT, NTMAX, kSlabNC, kSlabNL, kSlabD>;
    static std::atomic<uint64_t> attr_set{0};          // one bit per device: LDS limit raised
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(attr_set.load(std::memory_order_acquire) & bit)) {
        e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
        if (e != hipSuccess) return e;
        attr_set.fetch_or(bit, std::memory_order_acq_rel);
    }
    hipLaunchKernelGGL(k, dim3(p.grid), dim3(64 * (kSlabNC + kSlabNL)), p.lds, st, g.W, g.Waux, g.A, g.lda, g.C,
                       g.ldc, g.out_f16, g.M, g.N, g.K, p.tiles, p.w_slot, p.a_slot);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_slab(const GemmArgs& g, const SlabPlan& p, hipStream_t st) {
    if (p.MT == 1) return p.NTMAX == 1 ? launch_slab<QT, 1, 1>(g, p, st) : launch_slab<QT, 1, 2>(g, p, st);
    return p.NTMAX == 1 ? launch_slab<QT, 2, 1>(g, p, st) : launch_slab<QT, 2, 2>(g, p, st);
}

}  // namespace

bool slab_supports(const GemmArgs& g) {
    SlabPlan p;
    return plan_slab(g, p);
}

hipError_t gemm_slab(const GemmArgs& g, hipStream_t st) {
    SlabPlan p;
    if (!plan_slab(g, p)) return hipErrorInvalidValue;
    if (g.qtype == QT_Q4_K) return dispatch_slab<QT_Q4_K>(g, p, st);
    return dispatch_slab<QT_Q4_0>(g, p, st);
}

}  // namespace bf
