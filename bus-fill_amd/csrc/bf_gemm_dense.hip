// Dense MFMA GEMM for large batches (up to 128 rows per launch): every weight
// is streamed from HBM once per launch, whatever the batch (k_gemm_dense).
//
//   C[m][n] = sum_k A[m][k] * dequant(W)[n][k]      (fp32 accumulation)
//
// At 33-128 batch rows the GEMM is a dense contraction (455 flop per weight
// byte at M = 128): the batch rows are the MFMA's m-tiles, all of them in one
// workgroup, so each weight is decoded once per launch and multiplied against
// every batch row.  (Slicing the batch in launches of 32 rows, as the K-split
// kernel must, streams the weights once per slice.)
//
// * Work units: a unit is one super-group (256 k) of one row group (128
//   weight rows), T = row groups x super-groups of them in row-group-major
//   order.  The grid is one workgroup per CU (G <= 256), and workgroup p takes
//   the contiguous units [p T / G, (p + 1) T / G): every CU gets the same
//   share whatever N and K are (17408 rows are 136 row groups: with whole row
//   groups per workgroup only 136 of 256 CUs would work).  A workgroup's range
//   falls into pieces, one per row group it touches; a piece that covers its
//   row group's whole K is stored to C directly, the others (at most the first
//   and the last piece of a range) are written as fp32 partials, and the
//   workgroup that counts last on a row group's counter adds all its pieces in
//   piece order and writes C.  The order never depends on timing (results are
//   deterministic), no workgroup ever waits for another (nothing assumes the
//   grid is resident at once), and the last one resets the counter for the
//   next launch.  A writer's partial stores are complete (s_waitcnt vmcnt(0))
//   before its workgroup counts itself.
// * XCD-local pieces: the dispatcher hands workgroup b to XCD b % nx, and
//   range position p = (b % nx) (G / nx) + b / nx puts consecutive ranges on
//   one XCD, so the pieces of most row groups are written and read in that
//   XCD's L2: plain (write-back) stores, device-scope (sc1) loads that miss
//   only the L1.  A row group whose pieces straddle two XCDs' positions gets
//   device-scope stores too, which reach the point of coherence.  (With
//   write-through partials every reduction waited on memory: 17408 x 5120 at
//   M = 128 spent 30 us summing three pieces per row group.)  Each workgroup
//   checks its XCC id; one that finds itself on another XCD poisons its
//   results, so a broken placement shows as NaN, never as stale partials.
// * Two loader waves stream two kinds of units through two LDS rings with
//   direct-to-LDS loads (1 KB per instruction; per-lane offsets computed
//   once per piece, advanced per unit): per super-group, the 128 rows'
//   144-byte weight images (a ring of DW slots), and per half super-group h
//   the activation half-slab A[0:M] at the columns the half's MFMAs read
//   (64 h + 0..63 and 128 + 64 h + 0..63; rows 272 bytes apart: 16 bytes of
//   bank padding) (a ring of DA slots), in the order W(v), A(v, 0), A(v, 1),
//   W(v + 1), ... over the workgroup's units v, across piece boundaries.  A
//   loader ends its share of a unit with a one-dword marker load (a wave's
//   loads return in order); before reusing a slot it waits until the four
//   compute waves have counted the unit that held it as consumed.
// * Compute wave c owns weight rows 32c .. 32c + 31 of the row group and every
//   batch row, as 32 x 32 tiles of v_mfma_f32_32x32x16_f16 (per flop 1.6 times
//   the issue rate of the 16 x 16 form; on gfx950 a wave's MFMAs, decode and
//   LDS reads take turns rather than overlap, so the MFMA's own rate counts):
//   lane (n, g) holds row n's weight chunks 2g and 2g + 1 (bf_formats.h's
//   64-weight runs), so k-step i of half h uses weights 64 (2g + h) + 8i ..
//   + 7.  Per super-group the wave reads its rows' images (and releases the
//   weight slot), then per 16-k step decodes one fragment in registers (the
//   fp16 weights of bf_formats.h, bit-exact with the oracle's fp16 dequant)
//   and multiplies it against every m-tile's activation fragment.
// * Bounded waits poison the workgroup's results to NaN if a producer were
//   ever missing (bf_lds.h); a poisoned partial makes its row group's last
//   workgroup write NaN.
#include <algorithm>
#include <atomic>

#include "bf_launch.h"
#include "bf_lds.h"

namespace bf {
namespace {

// LDS: [0, 3072) flags: compute waves done with their partial stores at 4,
// poison at 8, the counting verdict of partial piece 0 / 1 at 16 / 20, the
// transpose counts of its reduction at 24 / 28 (written) and 32 / 36 (read); per
// unit v: weight marker of loader j at 64 + 8 v + 4 j, consumed count at
// 704 + 4 v; per activation unit u = 2 v + h: marker of loader j at
// 1024 + 8 u + 4 j, consumed count at 2304 + 4 u.  Then the weight ring (DW
// slots of 128 x 144 bytes), then the activation ring (DA slots of M x 272
// bytes).
constexpr int kDnFlags = 3072;
constexpr int kDnDone = 1, kDnPoison = 2, kDnVerdict = 4, kDnTrans = 6;
constexpr int kDnWReady = 16, kDnWCons = 176, kDnAReady = 256, kDnACons = 576, kDnMaxUnits = 80;
constexpr int kDnNC = 4, kDnNL = 2;      // compute and loader waves per workgroup
constexpr int kDnRows = 128;             // weight rows per row group (32 per compute wave)
constexpr int kDnWSlot = kDnRows * 144;  // bytes of one weight unit
constexpr int kDnARow = 272;             // LDS bytes of one activation row of a half-slab (256 + 16)
constexpr int kDnAQS = 17, kDnWQS = 9;   // instruction slots per loader: activation / weight unit
constexpr int kDnCounterStride = 64;     // one row-group counter per 256-byte line
constexpr unsigned kDnPoisonCount = 1u << 16;
constexpr int kCoherentDn = 16;          // sc1: device-scope stores and loads (the point of coherence)

__device__ __forceinline__ int xcc_id_dn() {
    int x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return x & 0xF;
}

// Units [first(p), first(p + 1)) belong to workgroup p.
__host__ __device__ __forceinline__ int range_first(int p, int T, int G) { return (int)((int64_t)p * T / G); }
// The workgroup whose range holds unit t: the largest p with range_first(p) <= t.
__host__ __device__ __forceinline__ int range_owner(int t, int T, int G) {
    return (int)(((int64_t)(t + 1) * G + T - 1) / T) - 1;
}

// One workgroup per CU (the rings fill the LDS), so at most two waves per SIMD.
template <int QT, int MT>
__global__ __launch_bounds__(64 * (kDnNC + kDnNL)) __attribute__((amdgpu_waves_per_eu(1, 2)))
void k_gemm_dense(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux, const uint16_t* __restrict__ A,
                  int lda, void* __restrict__ C, int ldc, int out_f16, int M, int N, int K, int T, int G, int DW,
                  int DA, float* __restrict__ ws, unsigned* __restrict__ counters, int nx) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    constexpr int NC = kDnNC, NL = kDnNL, ROWS = kDnRows;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = (int)blockIdx.x;
    const int grp = nx > 0 ? G / nx : G;               // range positions per XCD
    const int p = nx > 0 ? (b % nx) * grp + b / nx : b;
    const int nsg = K >> 8;
    const int t0 = range_first(p, T, G), t1 = range_first(p + 1, T, G);
    int* const flags = (int*)lds;
    const uint32_t lds0 = lds_addr(lds);
    const int a_slot = M * kDnARow;
    uint8_t* const w_ring = lds + kDnFlags;
    uint8_t* const a_ring = w_ring + DW * kDnWSlot;
    const int PA = M * 17, IA = (PA + 63) >> 6;       // activation pieces and instructions of a half-slab
    constexpr int PW = kDnRows * 9, IW = (PW + 63) >> 6;
    const int Mp = (M + 3) & ~3;                       // partial rows, whole quads
    const __amdgpu_buffer_rsrc_t wr =
        __builtin_amdgcn_make_buffer_rsrc(ws, (short)0, (int)((int64_t)2 * G * ROWS * Mp * 4), 0x00020000);

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
        // columns 8 c + 64 (c / 8) + 64 h of the super-group; the half-slab
        // (sg, h) adds 512 sg + 128 h bytes to every address
        const uint8_t* asrc[kDnAQS];
        bool aon[kDnAQS];
#pragma unroll
        for (int q2 = 0; q2 < kDnAQS; q2++) {
            const uint32_t P = 64u * (j + NL * q2) + lane;
            const uint32_t m = P / 17u, c = P - 17u * m;
            aon[q2] = P < (uint32_t)PA && c < 16;
            const int cc = min((int)c, 15);
            asrc[q2] = (const uint8_t*)(A + (int64_t)min((int)m, M - 1) * lda + 8 * cc + 64 * (cc >> 3));
        }
        int v = 0;                                     // units of this workgroup so far
        for (int t = t0; t < t1;) {
            const int rg = t / nsg, s0 = t - rg * nsg, s1 = min(nsg, s0 + (t1 - t));
            // weight instruction q = j + NL * slot: row n of the row group, part c of
            // its 144-byte image; super-group sg is sg * step bytes further
            const uint8_t* wsrc[kDnWQS];
            uint32_t wstep[kDnWQS];
#pragma unroll
            for (int q2 = 0; q2 < kDnWQS; q2++) {
                const uint32_t P = 64u * (j + NL * q2) + lane;
                wsrc[q2] = W;
                wstep[q2] = 0;
                if (P < (uint32_t)PW) {
                    const uint32_t n = P / 9u, c = P - 9u * n;
                    const int64_t row = min((int64_t)rg * ROWS + (int)n, (int64_t)N - 1);
                    wsrc[q2] = w_piece<QT>(W, Waux, row, 0, (int)c, K);
                    wstep[q2] = QT == QT_PLANES ? (c == 0 ? 16u : 128u) : 144u;
                }
            }
            for (int sg = s0; sg < s1; sg++, v++) {
                // the weight slot's previous unit must be consumed by every compute wave
                if (v >= DW) wait_count(&flags[kDnWCons + v - DW], NC, flags + kDnPoison);
                const uint32_t wb = lds0 + (uint32_t)(kDnFlags + (v % DW) * kDnWSlot);
#pragma unroll
                for (int q2 = 0; q2 < kDnWQS; q2++) {
                    const int q = j + NL * q2;
                    if (q >= IW) break;
                    if (wstep[q2]) dma16(wsrc[q2] + (uint32_t)sg * wstep[q2], wb + (uint32_t)(q << 10));
                }
                if (v == 0) clear_flags_and_meet();
                dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kDnWReady + 2 * v + j)), lane);
                for (int h = 0; h < 2; h++) {
                    const int u = 2 * v + h;
                    if (u >= DA) wait_count(&flags[kDnACons + u - DA], NC, flags + kDnPoison);
                    const uint32_t ab = lds0 + (uint32_t)(kDnFlags + DW * kDnWSlot + (u % DA) * a_slot);
                    const uint32_t off = 512u * (uint32_t)sg + 128u * (uint32_t)h;
#pragma unroll
                    for (int q2 = 0; q2 < kDnAQS; q2++) {
                        const int q = j + NL * q2;
                        if (q >= IA) break;
                        if (aon[q2]) dma16(asrc[q2] + off, ab + (uint32_t)(q << 10));
                    }
                    dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kDnAReady + 2 * u + j)), lane);
                }
            }
            t += s1 - s0;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---------------------------------------------------------------- compute wave
    clear_flags_and_meet();
    const int c = wave;
    if (nx > 1 && c == 0 && xcc_id_dn() != b % nx) mark_poison(flags + kDnPoison);
    // pieces of a row group all on one XCD: exchanged through its L2
    auto xcd_local = [&](int rg) {
        return nx > 0 && range_owner(rg * nsg, T, G) / grp == range_owner(rg * nsg + nsg - 1, T, G) / grp;
    };
    const Magic mg = make_magic();
    const int n = lane & 31, g = lane >> 5;
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = min(mt * 32 + n, M - 1) * kDnARow + 128 * g;   // pad rows reread M-1
    int part0 = -1, part1 = -1;                        // row groups of this workgroup's partial pieces
    int v = 0;
    for (int t = t0, piece = 0; t < t1; piece++) {
        const int rg = t / nsg, s0 = t - rg * nsg, s1 = min(nsg, s0 + (t1 - t));
        f16x acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[mt][e] = 0.f;
        for (int sg = s0; sg < s1; sg++, v++) {
            wait_flags(flags + kDnWReady + 2 * v, NL, lane, flags + kDnPoison);
            const uint8_t* wrow = w_ring + (v % DW) * kDnWSlot + (32 * c + n) * 144;
            Raw<QT> raw0, raw1;
            lds_raw<QT>(raw0, wrow, 2 * g);
            lds_raw<QT>(raw1, wrow, 2 * g + 1);
            // the weight images are in registers: release the slot
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnWCons + v])), "v"(1) : "memory");
            const auto sc0 = scales(raw0, 2 * g);
            const auto sc1 = scales(raw1, 2 * g + 1);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int u = 2 * v + h;
                wait_flags(flags + kDnAReady + 2 * u, NL, lane, flags + kDnPoison);
                const uint8_t* aunit = a_ring + (u % DA) * a_slot;
                // The k-step's activation fragments of every m-tile are read
                // together, the next k-step's before this one's MFMAs, so the LDS
                // latency is paid once per k-step, not once per MFMA (the
                // scheduling barrier keeps the scheduler from moving each read
                // next to its use).
                h8 a[2][MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) a[0][mt] = *(const h8*)(aunit + arow[mt]);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    if (i < 7) {
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) a[(i + 1) & 1][mt] = *(const h8*)(aunit + arow[mt] + 16 * (i + 1));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    const h8 b = h ? weights(mg, raw1, sc1, i) : weights(mg, raw0, sc0, i);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) acc[mt] = mfma32x32x16(a[i & 1][mt], b, acc[mt]);
                }
                // every LDS read of the half-slab has completed: count it consumed
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnACons + u])), "v"(1) : "memory");
            }
        }
        // this lane's outputs: weight row rg * 128 + 32 c + n, batch rows
        // 32 mt + 8 q + 4 g + 0..3 (registers 4q .. 4q + 3)
        const int64_t n_out = (int64_t)rg * ROWS + 32 * c + n;
        if (s0 == 0 && s1 == nsg) {
            // the row group's whole K: straight to C (32-bit offsets: the plan
            // keeps C below 2 GB)
            const bool bad = poisoned(flags + kDnPoison);
            const int es = out_f16 ? 2 : 4;
            const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, M * ldc * es, 0x00020000);
            if (n_out < N) {
                const int voff = (4 * g * ldc + (int)n_out) * es;     // row 4g of the m-tile
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int dm = mt * 32 + 8 * (e >> 2) + (e & 3);
                        if (dm + 4 * g < M) {
                            const float y = bad ? __builtin_nanf("") : acc[mt][e];
                            if (out_f16)
                                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)y), cr, voff,
                                                                      dm * ldc * es, 0);
                            else
                                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), cr, voff, dm * ldc * es, 0);
                        }
                    }
            }
        } else {
            // a partial piece (the range's first or last): slot 2p + which,
            // [row of the row group][Mp] fp32, one 16-byte store per quad of
            // batch rows (the register's part of the offset a constant)
            const int which = piece == 0 ? 0 : 1;
            if (which) part1 = rg;
            else part0 = rg;
            const int voff = (((2 * p + which) * ROWS + 32 * c + n) * Mp + 4 * g) * 4;
            const bool loc = xcd_local(rg);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const int dm = mt * 32 + 8 * q;
                    if (dm + 4 * g < Mp) {
                        const f4 x = f4{acc[mt][4 * q], acc[mt][4 * q + 1], acc[mt][4 * q + 2], acc[mt][4 * q + 3]};
                        if (loc) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), wr, voff, dm * 4, 0);
                        else __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, x), wr, voff, dm * 4, kCoherentDn);
                    }
                }
        }
        t += s1 - s0;
    }
    if (part0 < 0 && part1 < 0) return;

    // ------------------------------------------------- count the partial pieces
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnDone])), "v"(1) : "memory");
    if (c == 0) {
        wait_flags(&flags[kDnDone], 1, lane, flags + kDnPoison, NC);
        const unsigned add = poisoned(flags + kDnPoison) ? 1u + kDnPoisonCount : 1u;
        for (int which = 0; which < 2; which++) {
            const int rg = which ? part1 : part0;
            if (rg < 0) continue;
            const int pieces = range_owner(rg * nsg + nsg - 1, T, G) - range_owner(rg * nsg, T, G) + 1;
            unsigned* const cnt = counters + rg * kDnCounterStride;
            unsigned old = 0;
            if (lane == 0) old = __hip_atomic_fetch_add(cnt, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            old = __builtin_amdgcn_readfirstlane(old);
            const int last = (old & (kDnPoisonCount - 1)) == (unsigned)(pieces - 1);
            if (last && lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            // 1: last and clean, 3: last with a poisoned piece, 2: not last
            const int word = !last ? 2 : (old >= kDnPoisonCount || add > 1u) ? 3 : 1;
            if (lane == 0)
                asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kDnVerdict + which])), "v"(word) : "memory");
        }
    }
    // ------------------------------------ the last workgroup of a row group sums it
    for (int which = 0; which < 2; which++) {
        const int rg = which ? part1 : part0;
        if (rg < 0) continue;
        wait_flag(&flags[kDnVerdict + which], flags + kDnPoison);
        const int word = flags[kDnVerdict + which];
        if (word != 1 && word != 3) continue;
        const bool bad = word == 3 || poisoned(flags + kDnPoison);
        const int pf = range_owner(rg * nsg, T, G), pieces = range_owner(rg * nsg + nsg - 1, T, G) - pf + 1;
        const int64_t n0 = (int64_t)rg * ROWS;
        // Quad x = row * (Mp / 4) + batch quad: consecutive lanes read
        // consecutive 16 bytes of a partial.  The loads of up to four pieces x
        // eight of the lane's quads are issued together, so the latency is paid
        // about once per reduction (quads past nq reread the last one: no branch
        // between the loads).  The sums go through the (now idle) rings to be
        // written to C along its rows.
        constexpr int kIt = 16;                         // 128 rows x 32 batch quads / 256 lanes
        const int nq = ROWS * (Mp / 4);
        f4 sum[kIt];
#pragma unroll
        for (int it = 0; it < kIt; it++) sum[it] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i0 = 0; i0 < kIt; i0 += 8) {
            if (i0 * 256 >= nq) break;
            for (int j0 = 0; j0 < pieces; j0 += 4) {
                f4 y[4][8];
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if (j0 + jj >= pieces) break;
                    const int q = pf + j0 + jj;
                    const int slot = 2 * q + (range_first(q, T, G) >= rg * nsg ? 0 : 1);
                    const int sbase = slot * ROWS * Mp * 4;
#pragma unroll
                    for (int ii = 0; ii < 8; ii++) {
                        const int x = min(c * 64 + lane + 256 * (i0 + ii), nq - 1);
                        y[jj][ii] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(wr, sbase + 16 * x, 0,
                                                                                             kCoherentDn));
                    }
                }
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if (j0 + jj >= pieces) break;
#pragma unroll
                    for (int ii = 0; ii < 8; ii++) sum[i0 + ii] += y[jj][ii];     // pieces in order
                }
            }
        }
        // transpose: sums[row][batch row] at row stride Mp + 1 floats (odd: the
        // reads down a column spread over the banks)
        float* const tr = (float*)w_ring;
        const int ms = Mp + 1;
#pragma unroll
        for (int it = 0; it < kIt; it++) {
            const int x = c * 64 + lane + 256 * it;
            if (x < nq) {
                const int nl = x / (Mp / 4), m4 = 4 * (x - nl * (Mp / 4));
#pragma unroll
                for (int i = 0; i < 4; i++) tr[nl * ms + m4 + i] = sum[it][i];
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnTrans + which])), "v"(1) : "memory");
        wait_flags(&flags[kDnTrans + which], 1, lane, flags + kDnPoison, NC);
        // C[m][n0 + 4 y' .. + 3] for y = m * 32 + y': one 16-byte (fp32) or
        // 8-byte (fp16) store per lane where C's rows allow it
        const bool vec = ((uintptr_t)C & 15) == 0 && (ldc & 3) == 0;
        for (int y = c * 64 + lane; y < M * (ROWS / 4); y += NC * 64) {
            const int m = y / (ROWS / 4), nl = 4 * (y - m * (ROWS / 4));
            f4 v;
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = bad ? __builtin_nanf("") : tr[(nl + i) * ms + m];
            const int64_t o = (int64_t)m * ldc + n0 + nl;
            if (vec && n0 + nl + 3 < N) {
                if (out_f16) {
                    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                    *(h4*)((_Float16*)C + o) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                } else {
                    *(f4*)((float*)C + o) = v;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    if (n0 + nl + i >= N) break;
                    if (out_f16) ((_Float16*)C)[o + i] = (_Float16)v[i];
                    else ((float*)C)[o + i] = v[i];
                }
            }
        }
        // the next reduction reuses the transpose buffer: every wave's reads first
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnTrans + 2 + which])), "v"(1) : "memory");
        wait_flags(&flags[kDnTrans + 2 + which], 1, lane, flags + kDnPoison, NC);
    }
}

struct DensePlan {
    int MT, T, G, DW, DA, rgs, lds, nx;
};

// CUs of the current device (one workgroup each), 0 if unknown.
int device_cus() {
    static std::atomic<int> cache[64];                 // 0: not queried yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v < 1) v = -1;
        cache[dev].store(v, std::memory_order_relaxed);
        n = v;
    }
    return n > 0 ? n : 0;
}

size_t dense_counter_bytes(const DensePlan& p) { return (size_t)p.rgs * kDnCounterStride * 4; }
size_t dense_partial_bytes(const GemmArgs& g, const DensePlan& p) {
    return ((size_t)2 * p.G * kDnRows * ((g.M + 3) & ~3) * 4 + 255) & ~(size_t)255;
}

// Rings: two weight slots, as many activation slots as fit (up to 6).  One
// workgroup per CU, whole rounds of the XCD round robin when there are enough
// units.  The plan never depends on the workspace on offer: the ranges decide
// how partial sums are grouped, so every caller gets the same bits.
bool plan_dense(const GemmArgs& g, DensePlan& p, int cus, int nx) {
    if (g.M < 1 || g.M > 128 || g.K % 256 || g.N < 1) return false;
    if ((int64_t)g.M * g.ldc * (g.out_f16 ? 2 : 4) >= (1LL << 31)) return false;   // C by 32-bit offsets
    const int MT = std::max(2, (g.M + 31) / 32);       // 32-row m-tiles
    if ((g.M * 17 + 63) / 64 > kDnNL * kDnAQS || (kDnRows * 9 + 63) / 64 > kDnNL * kDnWQS) return false;
    const int DW = 2, a_slot = g.M * kDnARow;
    const int DA = std::min(6, (kMaxLds - kDnFlags - DW * kDnWSlot) / a_slot);
    if (DA < 2) return false;
    const int64_t rgs = (g.N + kDnRows - 1) / kDnRows, nsg = g.K / 256;
    if (rgs * nsg >= (1LL << 30)) return false;
    const int T = (int)(rgs * nsg);
    const int G0 = std::min(T, cus > 0 ? cus : 256);
    const int G = nx > 0 && G0 >= nx ? G0 / nx * nx : G0;
    if ((T + G - 1) / G > kDnMaxUnits) return false;
    if ((int64_t)2 * G * kDnRows * ((g.M + 3) & ~3) * 4 >= (1LL << 31)) return false;   // 32-bit offsets
    p = DensePlan{MT, T, G, DW, DA, (int)rgs, kDnFlags + DW * kDnWSlot + DA * a_slot, nx > 0 && G % nx == 0 ? nx : 0};
    return true;
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
    e = split_workspace(scratch, st, dense_counter_bytes(p), dense_partial_bytes(g, p), &counters, &parts);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(p.G), dim3(64 * (kDnNC + kDnNL)), p.lds, st, g.W, g.Waux, g.A, g.lda, g.C, g.ldc,
                       g.out_f16, g.M, g.N, g.K, p.T, p.G, p.DW, p.DA, parts, counters, p.nx);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_dense(const GemmArgs& g, const DensePlan& p, const Scratch* scratch, hipStream_t st) {
    if (p.MT == 2) return launch_dense<QT, 2>(g, p, scratch, st);
    if (p.MT == 3) return launch_dense<QT, 3>(g, p, scratch, st);
    return launch_dense<QT, 4>(g, p, scratch, st);
}

}  // namespace

bool dense_supports(const GemmArgs& g) {
    DensePlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return plan_dense(g, p, device_cus(), device_xcds());
}

size_t dense_scratch_bytes(const GemmArgs& g, size_t limit) {
    DensePlan p;
    if (!plan_dense(g, p, device_cus(), device_xcds())) return ~(size_t)0;
    const size_t need = dense_counter_bytes(p) + dense_partial_bytes(g, p);
    return need <= limit ? need : ~(size_t)0;
}

hipError_t gemm_dense(const GemmArgs& g, const Scratch* scratch, hipStream_t st) {
    DensePlan p;
    if (!plan_dense(g, p, device_cus(), device_xcds())) return hipErrorInvalidValue;
    if (scratch && dense_counter_bytes(p) + dense_partial_bytes(g, p) > scratch->bytes) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_dense<QT_Q4_K>(g, p, scratch, st);
        case QT_PLANES: return dispatch_dense<QT_PLANES>(g, p, scratch, st);
        default: return dispatch_dense<QT_Q4_0>(g, p, scratch, st);
    }
}

}  // namespace bf
