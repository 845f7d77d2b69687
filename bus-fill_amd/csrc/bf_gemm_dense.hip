// Dense MFMA GEMM for large batches (33-128 rows per launch): every weight is
// streamed from HBM once per launch, whatever the batch (k_gemm_dense).
//
//   C[m][n] = sum_k A[m][k] * dequant(W)[n][k]      (fp32 accumulation)
//
// At 64-128 batch rows the GEMM is a dense contraction (455 flop per weight
// byte at M = 128): the batch rows are the MFMA's m-tiles, all of them in one
// workgroup, so each weight tile is decoded once per launch and multiplied
// against every batch row.  (Slicing the batch in launches of 32 rows, as the
// K-split kernel must, streams the weights once per slice.)
//
// * Workgroup (row group rg, split s): 128 weight rows (8 tiles of 16) x all
//   M batch rows x the super-groups [s * U, (s + 1) * U).
// * Two loader waves stream two kinds of units through two LDS rings with
//   direct-to-LDS loads (1 KB per instruction; per-lane addresses computed
//   once, advanced per unit): per super-group, the eight tiles' 144-byte
//   weight images (a ring of DW slots), and per half super-group the
//   activation half-slab A[0:M] at the columns the MFMA k-steps 4h .. 4h+3 of
//   the super-group read (64 kg + 32 h + 0..31 for kg = 0..3; rows 272 bytes
//   apart: 16 bytes of bank padding) (a ring of DA slots), in the order
//   W(sg), A(sg, 0), A(sg, 1), W(sg + 1), ...  A loader ends its share of a
//   unit with a one-dword marker load (a wave's loads return in order); before
//   reusing a slot it waits until the four compute waves have counted the unit
//   that held it as consumed.  Half-slabs keep three activation units in the
//   ring at 128 rows (35 KB each): more bytes in flight than a ring of two
//   whole slabs.
// * Compute wave c owns weight tiles 2c and 2c + 1 and every batch m-tile: per
//   super-group it reads its two tiles' weight images (and releases the
//   weight slot), then per 32-k step decodes its two weight fragments in
//   registers (the fp16 weights of bf_formats.h, bit-exact with the oracle's
//   fp16 dequant) and multiplies each activation fragment it reads from LDS
//   against both, so every activation read feeds two MFMAs.  The waves own
//   disjoint outputs: no reduction inside the workgroup.
// * With S > 1 splits the tile sums go to a workspace and the split that
//   finishes last (a counter per row group) adds them in split order and
//   writes C -- the K-split kernel's exchange, with all S splits of a row
//   group on one XCD (bid % nx) so the partials stay in that XCD's L2.
// * Bounded waits poison the workgroup's results to NaN if a producer were
//   ever missing (bf_lds.h).
#include <algorithm>
#include <atomic>

#include "bf_launch.h"
#include "bf_lds.h"

namespace bf {
namespace {

// LDS: [0, 3072) flags: owners-done counter at 4, is-last word at 8, poison at
// 12; per super-group sg: weight-unit marker of loader j at 64 + 8 sg + 4 j,
// consumed count at 704 + 4 sg; per activation unit u = 2 sg + h: marker of
// loader j at 1024 + 8 u + 4 j, consumed count at 2304 + 4 u.  Then the
// weight ring (DW slots of 8 x 2304 bytes), then the activation ring (DA slots
// of M x 272 bytes).
constexpr int kDnFlags = 3072;
constexpr int kDnPoison = 3;
constexpr int kDnWReady = 16, kDnWCons = 176, kDnAReady = 256, kDnACons = 576, kDnMaxSg = 80;
constexpr int kDnNC = 4, kDnNL = 2;      // compute and loader waves per workgroup
constexpr int kDnNT = 8;                 // weight tiles of 16 rows per workgroup (two per compute wave)
constexpr int kDnWSlot = kDnNT * 2304;   // bytes of one weight unit
constexpr int kDnARow = 272;             // LDS bytes of one activation row of a half-slab (256 + 16)
constexpr int kDnAQS = 17, kDnWQS = 9;   // instruction slots per loader: activation / weight unit
constexpr int kDnCounterStride = 64;     // one row-group counter per 256-byte line
constexpr unsigned kDnPoisonCount = 1u << 16;
constexpr int kCoherentDn = 16;          // sc1: device-scope loads (miss the L1)

__device__ __forceinline__ int xcc_id_dn() {
    int x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xF;
}

// One workgroup per CU (the rings fill the LDS), so at most two waves per SIMD:
// the compiler may spend 256 VGPRs per wave on keeping reads in flight.
template <int QT, int MT>
__global__ __launch_bounds__(64 * (kDnNC + kDnNL)) __attribute__((amdgpu_waves_per_eu(1, 2)))
void k_gemm_dense(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux, const uint16_t* __restrict__ A,
                  int lda, void* __restrict__ C, int ldc, int out_f16, int M, int N, int K, int S, int U, int DW,
                  int DA, float* __restrict__ ws, unsigned* __restrict__ counters, int nx) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    constexpr int NC = kDnNC, NL = kDnNL, ROWS = 16 * kDnNT;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int bid = (int)blockIdx.x;
    int rg, s;
    if (nx > 0) {
        // XCD x = bid % nx holds row groups x, x + nx, ..., each as S consecutive workgroups
        const int x = bid % nx, jx = bid / nx, q = jx / S;
        rg = x + nx * q;
        s = jx - q * S;
        if ((int64_t)rg * ROWS >= N) return;               // padding of the last XCD round
        if (S > 1 && nx > 1 && xcc_id_dn() != x) {
            // not on the XCD the exchange assumes: poison this workgroup's rows
            for (int v = threadIdx.x; v < ROWS * M; v += blockDim.x) {
                const int m = v / ROWS;
                const int64_t n = (int64_t)rg * ROWS + (v - m * ROWS);
                if (n < N) {
                    if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)__builtin_nanf("");
                    else ((float*)C)[(int64_t)m * ldc + n] = __builtin_nanf("");
                }
            }
            return;
        }
    } else {
        rg = bid / S;
        s = bid - rg * S;
    }
    const int sg0 = s * U;
    int* const flags = (int*)lds;
    const uint32_t lds0 = lds_addr(lds);
    const int a_slot = M * kDnARow;
    uint8_t* const w_ring = lds + kDnFlags;
    uint8_t* const a_ring = w_ring + DW * kDnWSlot;
    const int PA = M * 17, IA = (PA + 63) >> 6;       // activation pieces and instructions of a half-slab
    constexpr int PW = kDnNT * 144, IW = (PW + 63) >> 6;
    const int Mp = (M + 3) & ~3;                       // workspace rows, whole quads

    auto clear_flags_and_meet = [&]() {
        static_assert((kDnNC + kDnNL) * 128 == kDnFlags / 4, "each wave clears 128 flags");
        flags[128 * wave + lane] = 0;
        flags[128 * wave + 64 + lane] = 0;
        barrier_lds();
    };

    if (wave >= NC) {
        // ------------------------------------------------------------ loader wave
        __builtin_amdgcn_s_setprio(3);
        const int j = wave - NC;
        // activation instruction q = j + NL * slot covers pieces 64 q + lane of a
        // half-slab: row m, 16-byte part c (part 16 is the row's bank padding),
        // columns 64 (c / 4) + 32 h + 8 (c % 4) of the super-group; the unit
        // u = 2 sg + h adds 512 sg + 64 h bytes to every address
        const uint8_t* asrc[kDnAQS];
        bool aon[kDnAQS];
#pragma unroll
        for (int q2 = 0; q2 < kDnAQS; q2++) {
            const uint32_t P = 64u * (j + NL * q2) + lane;
            const uint32_t m = P / 17u, c = P - 17u * m;
            aon[q2] = P < (uint32_t)PA && c < 16;
            asrc[q2] = (const uint8_t*)(A + (int64_t)min((int)m, M - 1) * lda + 256 * sg0 + 64 * (min((int)c, 15) >> 2) +
                                        8 * (c & 3));
        }
        // weight instruction q = j + NL * slot: tile t, row n of the tile, part c
        // of its 144-byte image; the next super-group is `step` bytes further
        const uint8_t* wsrc[kDnWQS];
        uint32_t wstep[kDnWQS];
#pragma unroll
        for (int q2 = 0; q2 < kDnWQS; q2++) {
            const uint32_t P = 64u * (j + NL * q2) + lane;
            wsrc[q2] = W;
            wstep[q2] = 0;
            if (P < (uint32_t)PW) {
                const uint32_t t = P / 144u, rem = P - 144u * t, n = rem / 9u, c = rem - 9u * n;
                const int64_t row = min((int64_t)(rg * kDnNT + (int)t) * 16 + (int)n, (int64_t)N - 1);
                wsrc[q2] = w_piece<QT>(W, Waux, row, sg0, (int)c, K);
                wstep[q2] = QT == QT_PLANES ? (c == 0 ? 16u : 128u) : 144u;
            }
        }
        for (int sg = 0; sg < U; sg++) {
            // the weight slot's previous unit must be consumed by every compute wave
            if (sg >= DW) wait_count(&flags[kDnWCons + sg - DW], NC, flags + kDnPoison);
            const uint32_t wb = lds0 + (uint32_t)(kDnFlags + (sg % DW) * kDnWSlot);
#pragma unroll
            for (int q2 = 0; q2 < kDnWQS; q2++) {
                const int q = j + NL * q2;
                if (q >= IW) break;
                if (wstep[q2]) dma16(wsrc[q2] + (uint32_t)sg * wstep[q2], wb + (uint32_t)(q << 10));
            }
            if (sg == 0) clear_flags_and_meet();
            dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kDnWReady + 2 * sg + j)), lane);
            for (int h = 0; h < 2; h++) {
                const int u = 2 * sg + h;
                if (u >= DA) wait_count(&flags[kDnACons + u - DA], NC, flags + kDnPoison);
                const uint32_t ab = lds0 + (uint32_t)(kDnFlags + DW * kDnWSlot + (u % DA) * a_slot);
                const uint32_t off = 512u * (uint32_t)sg + 64u * (uint32_t)h;
#pragma unroll
                for (int q2 = 0; q2 < kDnAQS; q2++) {
                    const int q = j + NL * q2;
                    if (q >= IA) break;
                    if (aon[q2]) dma16(asrc[q2] + off, ab + (uint32_t)(q << 10));
                }
                dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kDnAReady + 2 * u + j)), lane);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---------------------------------------------------------------- compute wave
    clear_flags_and_meet();
    const int c = wave;
    const Magic mg = make_magic();
    const int r = lane & 15, kg = lane >> 4;
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = min(mt * 16 + r, M - 1) * kDnARow + 64 * kg;   // pad rows reread M-1
    f4 acc[2][MT];
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[tt][mt] = f4{0.f, 0.f, 0.f, 0.f};

    for (int sg = 0; sg < U; sg++) {
        wait_flags(flags + kDnWReady + 2 * sg, NL, lane, flags + kDnPoison);
        const uint8_t* wunit = w_ring + (sg % DW) * kDnWSlot;
        Raw<QT> raw0, raw1;
        lds_raw<QT>(raw0, wunit + (2 * c) * 2304 + r * 144, kg);
        lds_raw<QT>(raw1, wunit + (2 * c + 1) * 2304 + r * 144, kg);
        // the weight images are in registers: release the slot
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnWCons + sg])), "v"(1) : "memory");
        const auto sc0 = scales(raw0, kg);
        const auto sc1 = scales(raw1, kg);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int u = 2 * sg + h;
            wait_flags(flags + kDnAReady + 2 * u, NL, lane, flags + kDnPoison);
            const uint8_t* aunit = a_ring + (u % DA) * a_slot;
            // The k-step's activation fragments of every m-tile are read together,
            // the next k-step's before this one's MFMAs, so the LDS latency is paid
            // once per k-step, not once per MFMA (the scheduling barrier keeps the
            // scheduler from moving each read next to its use).
            h8 a[2][MT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) a[0][mt] = *(const h8*)(aunit + arow[mt]);
#pragma unroll
            for (int i2 = 0; i2 < 4; i2++) {
                if (i2 < 3) {
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) a[(i2 + 1) & 1][mt] = *(const h8*)(aunit + arow[mt] + 16 * (i2 + 1));
                }
                __builtin_amdgcn_sched_barrier(0);
                const h8 b0 = weights(mg, raw0, sc0, 4 * h + i2);
                const h8 b1 = weights(mg, raw1, sc1, 4 * h + i2);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    acc[0][mt] = mfma16x16x32(a[i2 & 1][mt], b0, acc[0][mt]);
                    acc[1][mt] = mfma16x16x32(a[i2 & 1][mt], b1, acc[1][mt]);
                }
            }
            // every LDS read of the half-slab has completed: count it consumed
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnACons + u])), "v"(1) : "memory");
        }
    }

    if (poisoned(flags + kDnPoison)) {
#pragma unroll
        for (int tt = 0; tt < 2; tt++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++) acc[tt][mt] = f4{1.f, 1.f, 1.f, 1.f} * __builtin_nanf("");
    }
    if (S > 1) {
        // workspace [s][n][Mp]: this lane's four rows of an m-tile are one 16-byte store
        const __amdgpu_buffer_rsrc_t wr =
            __builtin_amdgcn_make_buffer_rsrc(ws, (short)0, (int)((int64_t)S * N * Mp * 4), 0x00020000);
#pragma unroll
        for (int tt = 0; tt < 2; tt++) {
            const int64_t n = (int64_t)(rg * kDnNT + 2 * c + tt) * 16 + r;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const int m4 = mt * 16 + 4 * kg;
                if (m4 < Mp && n < N) {
                    const int off = (int)((((int64_t)s * N + n) * Mp + m4) * 4);
                    if (nx > 0) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[tt][mt]), wr, off, 0, 0);
                    else __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, acc[tt][mt]), wr, off, 0,
                                                                kCoherentDn);
                }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[1])), "v"(1) : "memory");

        // --------------------------------------------------- cross-split sum
        if (c == 0) {
            wait_flags(&flags[1], 1, lane, flags + kDnPoison, NC);
            const unsigned add = poisoned(flags + kDnPoison) ? 1u + kDnPoisonCount : 1u;
            unsigned old = 0;
            unsigned* const cnt = counters + rg * kDnCounterStride;
            if (lane == 0) old = __hip_atomic_fetch_add(cnt, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __builtin_amdgcn_readfirstlane(old);
            const int last = (old & (kDnPoisonCount - 1)) == (unsigned)(S - 1);
            if (last && lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // 1: last and clean, 3: last with a poisoned split, 2: not last
            const int word = !last ? 2 : (old >= kDnPoisonCount || add > 1u) ? 3 : 1;
            if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[2])), "v"(word) : "memory");
        }
        wait_flags(&flags[2], 1, lane, flags + kDnPoison);
        const int word = flags[2];
        if (word != 1 && word != 3) return;
        const bool bad = word == 3 || poisoned(flags + kDnPoison);
        // each lane takes one quad (one row n, rows m4 .. m4+3) at a time, its S partial loads issued first
        const int nq = ROWS * (Mp / 4);
        const int64_t n0 = (int64_t)rg * ROWS;
        for (int v = c * 64 + lane; v < nq; v += NC * 64) {
            const int nl = v / (Mp / 4), m4 = 4 * (v - nl * (Mp / 4));
            if (n0 + nl >= N) continue;
            const int off = (int)(((n0 + nl) * Mp + m4) * 4);
            f4 sum = f4{0.f, 0.f, 0.f, 0.f};
            for (int s0 = 0; s0 < S; s0 += 4) {
                f4 x[4];
#pragma unroll
                for (int k = 0; k < 4; k++)
                    x[k] = s0 + k < S ? __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                   wr, off + (int)((int64_t)(s0 + k) * N * Mp * 4), 0,
                                                                   kCoherentDn))
                                      : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int k = 0; k < 4; k++)
                    if (s0 + k < S) sum += x[k];              // splits in order
            }
            const int64_t n = n0 + nl;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (m4 + i >= M) break;
                const float y = bad ? __builtin_nanf("") : sum[i];
                if (out_f16) ((_Float16*)C)[(int64_t)(m4 + i) * ldc + n] = (_Float16)y;
                else ((float*)C)[(int64_t)(m4 + i) * ldc + n] = y;
            }
        }
        return;
    }
#pragma unroll
    for (int tt = 0; tt < 2; tt++) {
        const int64_t n = (int64_t)(rg * kDnNT + 2 * c + tt) * 16 + r;
        if (n >= N) continue;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = mt * 16 + 4 * kg + i;
                if (m < M) {
                    if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + n] = (_Float16)acc[tt][mt][i];
                    else ((float*)C)[(int64_t)m * ldc + n] = acc[tt][mt][i];
                }
            }
    }
}

struct DensePlan {
    int MT, S, U, DW, DA, grid, rgs, lds, nx;
};

// Workspace bytes of S splits over rgs row groups (0 without a split).
size_t dense_ws_bytes(const GemmArgs& g, int S, int rgs) {
    return S > 1 ? (size_t)rgs * kDnCounterStride * 4 + (((size_t)S * g.N * ((g.M + 3) & ~3) * 4 + 255) & ~(size_t)255)
                 : 0;
}

// Rings: two weight slots, as many activation slots as fit (up to 6).  The
// K-split keeps the fewest rounds of 256 workgroups busy, counting the
// partials' round trip as one more super-group per 10 MB of them; only splits
// whose workspace fits in max_ws bytes.
bool plan_dense(const GemmArgs& g, DensePlan& p, int nx, size_t max_ws = ~(size_t)0) {
    if (g.M < 1 || g.M > 128 || g.K % 256) return false;
    const int nsg = g.K / 256;
    const int need_mt = (g.M + 15) / 16;
    const int MT = need_mt <= 4 ? 4 : need_mt <= 6 ? 6 : 8;
    if ((g.M * 17 + 63) / 64 > kDnNL * kDnAQS || (kDnNT * 144 + 63) / 64 > kDnNL * kDnWQS) return false;
    const int DW = 2, a_slot = g.M * kDnARow;
    const int DA = std::min(6, (kMaxLds - kDnFlags - DW * kDnWSlot) / a_slot);
    if (DA < 2) return false;
    const int rgs = (g.N + 16 * kDnNT - 1) / (16 * kDnNT);
    const int Mp = (g.M + 3) & ~3;
    double best = 1e300;
    for (int S = 1; S <= nsg; S++) {
        if (nsg % S) continue;
        const int U = nsg / S;
        if (U > kDnMaxSg) continue;
        if ((int64_t)S * g.N * Mp * 4 >= (1LL << 31)) continue;   // partials addressed by 32-bit offsets
        if (dense_ws_bytes(g, S, rgs) > max_ws) continue;
        const int sx = S > 1 && nx > 0 ? nx : 0;
        const int grid = (sx ? (rgs + sx - 1) / sx * sx : rgs) * S;
        const double partial_mb = S > 1 ? 2.0 * S * g.N * Mp * 4 / 1e6 : 0.0;
        const double est = (double)((grid + 255) / 256) * U + partial_mb / 10.0 + (S > 1 ? 1.0 : 0.0);
        if (est < best) {
            best = est;
            p = DensePlan{MT, S, U, DW, DA, grid, rgs, kDnFlags + DW * kDnWSlot + DA * a_slot, sx};
        }
    }
    return best < 1e300;
}

size_t dense_counter_bytes(const DensePlan& p) { return p.S > 1 ? (size_t)p.rgs * kDnCounterStride * 4 : 0; }
size_t dense_partial_bytes(const GemmArgs& g, const DensePlan& p) {
    return p.S > 1 ? ((size_t)p.S * g.N * ((g.M + 3) & ~3) * 4 + 255) & ~(size_t)255 : 0;
}

template <int QT, int MT>
hipError_t launch_dense(const GemmArgs& g, const DensePlan& p, const Scratch* scratch, hipStream_t st) {
    auto k = k_gemm_dense<QT, MT>;
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
    unsigned* counters = nullptr;
    float* parts = nullptr;
    if (p.S > 1) {
        e = split_workspace(scratch, st, dense_counter_bytes(p), dense_partial_bytes(g, p), &counters, &parts);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(k, dim3(p.grid), dim3(64 * (kDnNC + kDnNL)), p.lds, st, g.W, g.Waux, g.A, g.lda, g.C, g.ldc,
                       g.out_f16, g.M, g.N, g.K, p.S, p.U, p.DW, p.DA, parts, counters, p.nx);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_dense(const GemmArgs& g, const DensePlan& p, const Scratch* scratch, hipStream_t st) {
    if (p.MT == 4) return launch_dense<QT, 4>(g, p, scratch, st);
    if (p.MT == 6) return launch_dense<QT, 6>(g, p, scratch, st);
    return launch_dense<QT, 8>(g, p, scratch, st);
}

}  // namespace

bool dense_supports(const GemmArgs& g) {
    DensePlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return plan_dense(g, p, device_xcds());
}

size_t dense_scratch_bytes(const GemmArgs& g, size_t limit) {
    DensePlan p;
    if (!plan_dense(g, p, device_xcds(), limit)) return ~(size_t)0;
    return dense_counter_bytes(p) + dense_partial_bytes(g, p);
}

hipError_t gemm_dense(const GemmArgs& g, const Scratch* scratch, hipStream_t st) {
    DensePlan p;
    if (!plan_dense(g, p, device_xcds(), scratch ? scratch->bytes : ~(size_t)0)) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_dense<QT_Q4_K>(g, p, scratch, st);
        case QT_PLANES: return dispatch_dense<QT_PLANES>(g, p, scratch, st);
        default: return dispatch_dense<QT_Q4_0>(g, p, scratch, st);
    }
}

}  // namespace bf
