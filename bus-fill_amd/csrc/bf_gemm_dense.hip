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
//   and the last piece of a range) are written as fp32 partials, and a second
//   launch (k_dense_sum) adds each split row group's pieces in piece order and
//   writes C, spread over rows x batch rows.  The order never depends on
//   timing (results are deterministic) and no workgroup waits for another.
//   (Summing in the workgroup that counted last on a row group's counter left
//   that one CU reading three to seven 64 KB pieces after the others had
//   finished: 12-23 us at M = 128.)
// * Loader waves (the first waves of the workgroup, which the dispatcher
//   starts first) stream two kinds of units through two LDS rings with
//   direct-to-LDS loads (1 KB per instruction; per-lane offsets computed once
//   per piece, advanced per unit): kDnNLW waves the weights, per super-group
//   the 128 rows' 144-byte images (a ring of DW slots), and kDnNLA waves the
//   activations, per half super-group h the half-slab A[0:M] at the columns
//   the half's MFMAs read (64 h + 0..63 and 128 + 64 h + 0..63; rows 272 bytes
//   apart: 16 bytes of bank padding) (a ring of DA slots), over the
//   workgroup's units across piece boundaries.  The two streams have waves of
//   their own because a wave's loads return in issue order: an activation
//   marker behind weight loads waits for HBM (17408 x 5120 at M = 128 went
//   from 60 to 54 us; one activation wave issues too slowly, three gain
//   nothing over two).  A loader ends its share of a unit with a one-dword
//   marker load; before reusing a slot it waits until the compute waves have
//   counted the unit that held it as consumed.
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
// * Two compute waves per row block (NCW = 8, where the activation ring holds
//   at least five half-slabs): the wave of parity p takes the units v with
//   v % 2 == p, so each SIMD runs two waves working on different units and
//   one's VALU work issues while the other's MFMAs run (a single wave issues
//   them in turn: one 32x32x16 MFMA followed by eight independent VALU
//   instructions takes 64 cycles in one wave, 40 per wave with four waves on a
//   SIMD).  At the end of each piece parity 1 hands its sums to parity 0
//   through LDS, one m-tile at a time; parity 0 adds them (its own first, a
//   fixed order) and stores.
// * Bounded waits poison the workgroup's results to NaN if a producer were
//   ever missing (bf_lds.h): its C stores and partials are NaN, and so is
//   every sum a poisoned partial enters.
#include <algorithm>
#include <atomic>

#include "bf_launch.h"
#include "bf_lds.h"

namespace bf {
namespace {

// Loader waves: kDnNLW stream the weights, kDnNLA the activations.
constexpr int kDnNCU = 4;                // compute waves that consume one unit (32 rows each)
constexpr int kDnNLW = 1, kDnNLA = 2;    // loader waves of the weight and of the activation stream
constexpr int kDnNL = kDnNLW + kDnNLA;
constexpr int kDnMaxUnits = 80;          // units per workgroup
// Cache policy of the partial pieces' stores: device scope (sc1), so each
// store is written through the XCD's L2 while the kernel runs instead of
// being left dirty there for the write-back at the kernel's end (the pieces
// are read by k_dense_sum, a later launch, on any XCD).  5120 x 5120 at
// M = 64: 17.0 -> 16.0 us per GEMM; 17408 x 5120 at M = 128: 43.4-44.1 ->
// 42.1-42.8 us.
constexpr int kDnPartPolicy = 16;
// LDS flag words: poison at 2; per unit v the markers
// of the weight loaders at kDnWReady + kDnNLW v + j and the consumed count at
// kDnWCons + v; per activation half-slab u = 2 v + h the markers of the
// activation loaders at kDnAReady + kDnNLA u + j and the consumed count at
// kDnACons + u.  Then the weight ring (DW slots of 128 x 144 bytes), then the
// activation ring (DA slots of M x 272 bytes).
constexpr int kDnPoison = 2;
constexpr int kDnWReady = 16, kDnWCons = kDnWReady + kDnNLW * kDnMaxUnits, kDnAReady = kDnWCons + kDnMaxUnits,
              kDnACons = kDnAReady + 2 * kDnNLA * kDnMaxUnits;
// two compute waves per row block (NCW = 8): the words of their piece-end
// hand-over, and the LDS it goes through (one m-tile of one parity's sums)
constexpr int kDnCombW = kDnACons + 2 * kDnMaxUnits, kDnCombR = kDnCombW + kDnNCU;
constexpr int kDnFlags = ((kDnCombR + kDnNCU) * 4 + 255) & ~255;   // bytes
constexpr int kDnComb = kDnNCU * 64 * 16 * 4;
constexpr int kDnRows = 128;             // weight rows per row group (32 per compute wave)
constexpr int kDnWSlot = kDnRows * 144;  // bytes of one weight unit
constexpr int kDnARow = 272;             // LDS bytes of one activation row of a half-slab (256 + 16)
constexpr int kDnAI = 34, kDnWI = 18;    // 1 KB instructions of a half-slab (M = 128) / of a weight unit
constexpr int kDnAQS = (kDnAI + kDnNLA - 1) / kDnNLA, kDnWQS = (kDnWI + kDnNLW - 1) / kDnNLW;   // per loader

// Units [first(p), first(p + 1)) belong to workgroup p.
__host__ __device__ __forceinline__ int range_first(int p, int T, int G) { return (int)((int64_t)p * T / G); }
// The workgroup whose range holds unit t: the largest p with range_first(p) <= t.
__host__ __device__ __forceinline__ int range_owner(int t, int T, int G) {
    return (int)(((int64_t)(t + 1) * G + T - 1) / T) - 1;
}

// One GEMM's share of a launch: workgroup p of its G.
template <int QT, int MT, int NCW>
__device__ __forceinline__ void dense_body(int p, uint8_t* lds, const uint8_t* __restrict__ W,
                                           const uint8_t* __restrict__ Waux, const uint16_t* __restrict__ A, int lda,
                                           void* __restrict__ C, int ldc, int out_f16, int M, int N, int K, int T,
                                           int G, int DW, int DA, float* __restrict__ ws) {
    constexpr int NC = NCW, NL = kDnNL, ROWS = kDnRows;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsg = K >> 8;
    const int t0 = range_first(p, T, G), t1 = range_first(p + 1, T, G);
    int* const flags = (int*)lds;
    const uint32_t lds0 = lds_addr(lds);
    const int a_slot = M * kDnARow;
    uint8_t* const w_ring = lds + kDnFlags;
    uint8_t* const a_ring = w_ring + DW * kDnWSlot;
    const int PA = M * 17, IA = (PA + 63) >> 6;       // activation pieces and instructions of a half-slab
    constexpr int PW = kDnRows * 9, IW = (PW + 63) >> 6;
    const int Mp = (M + 3) & ~3;                       // batch rows of a partial slot

    auto clear_flags_and_meet = [&]() {
        for (int w = (int)threadIdx.x; w < kDnFlags / 4; w += 64 * (NC + NL)) flags[w] = 0;
        barrier_lds();
    };

    if (wave < NL) {
        // ------------------------------------------------------------ loader waves
        // The weight stream (HBM) and the activation stream (L2) have loader waves
        // of their own: a wave's loads return in issue order, so an activation
        // marker queued behind weight loads would wait for HBM.
        __builtin_amdgcn_s_setprio(3);
        const int j = wave;
        bool met = false;
        auto meet = [&]() {
            if (!met) clear_flags_and_meet();
            met = true;
        };
        if (j < kDnNLW) {
            int v = 0;                                 // units of this workgroup so far
            for (int t = t0; t < t1;) {
                const int rg = t / nsg, s0 = t - rg * nsg, s1 = min(nsg, s0 + (t1 - t));
                // weight instruction q = j + NLW * slot: row n of the row group, part c
                // of its 144-byte image; super-group sg is sg * step bytes further
                const uint8_t* wsrc[kDnWQS];
                uint32_t wstep[kDnWQS];
#pragma unroll
                for (int q2 = 0; q2 < kDnWQS; q2++) {
                    const uint32_t P = 64u * (j + kDnNLW * q2) + lane;
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
                    // the slot's previous unit must be consumed by every compute wave
                    if (v >= DW) wait_count(&flags[kDnWCons + v - DW], kDnNCU, flags + kDnPoison);
                    const uint32_t wb = lds0 + (uint32_t)(kDnFlags + (v % DW) * kDnWSlot);
#pragma unroll
                    for (int q2 = 0; q2 < kDnWQS; q2++) {
                        const int q = j + kDnNLW * q2;
                        if (q >= IW) break;
                        if (wstep[q2]) dma16(wsrc[q2] + (uint32_t)sg * wstep[q2], wb + (uint32_t)(q << 10));
                    }
                    meet();
                    dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kDnWReady + kDnNLW * v + j)), lane);
                }
                t += s1 - s0;
            }
        } else {
            // activation instruction q = ja + NLA * slot covers pieces 64 q + lane of
            // a half-slab: row m, 16-byte part c (part 16 is the row's bank
            // padding), columns 8 c + 64 (c / 8) + 64 h of the super-group; the
            // half-slab (sg, h) adds 512 sg + 128 h bytes to every address
            const int ja = j - kDnNLW;
            const uint8_t* asrc[kDnAQS];
            bool aon[kDnAQS];
#pragma unroll
            for (int q2 = 0; q2 < kDnAQS; q2++) {
                const uint32_t P = 64u * (ja + kDnNLA * q2) + lane;
                const uint32_t m = P / 17u, c = P - 17u * m;
                aon[q2] = P < (uint32_t)PA && c < 16;
                const int cc = min((int)c, 15);
                asrc[q2] = (const uint8_t*)(A + (int64_t)min((int)m, M - 1) * lda + 8 * cc + 64 * (cc >> 3));
            }
            for (int t = t0, u = 0; t < t1; t++) {
                const int sg = t % nsg;
                for (int h = 0; h < 2; h++, u++) {
                    if (u >= DA) wait_count(&flags[kDnACons + u - DA], kDnNCU, flags + kDnPoison);
                    const uint32_t ab = lds0 + (uint32_t)(kDnFlags + DW * kDnWSlot + (u % DA) * a_slot);
                    const uint32_t off = 512u * (uint32_t)sg + 128u * (uint32_t)h;
#pragma unroll
                    for (int q2 = 0; q2 < kDnAQS; q2++) {
                        const int q = ja + kDnNLA * q2;
                        if (q >= IA) break;
                        if (aon[q2]) dma16(asrc[q2] + off, ab + (uint32_t)(q << 10));
                    }
                    meet();
                    dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kDnAReady + kDnNLA * u + ja)), lane);
                }
            }
        }
        meet();                                        // (every range holds a unit: met already)
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        return;
    }

    // ---------------------------------------------------------------- compute wave
    clear_flags_and_meet();
    // compute wave: row block c (rows 32 c .. 32 c + 31 of the row group) and,
    // with NCW = 8, parity par: the waves of parity p take the units v with
    // v % 2 == p, so two waves of different units share each SIMD
    const int cw = wave - NL, c = cw & (kDnNCU - 1), par = NCW == 8 ? cw / kDnNCU : 0;
    uint8_t* const comb = a_ring + DA * a_slot;
    int chunk = 0;                                     // piece-end hand-overs so far
    const Magic mg = make_magic();
    const int n = lane & 31, g = lane >> 5;
    int arow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) arow[mt] = min(mt * 32 + n, M - 1) * kDnARow + 128 * g;   // pad rows reread M-1
    int v = 0;
    for (int t = t0, piece = 0; t < t1; piece++) {
        const int rg = t / nsg, s0 = t - rg * nsg, s1 = min(nsg, s0 + (t1 - t));
        f16x acc[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[mt][e] = 0.f;
        for (int sg = s0; sg < s1; sg++, v++) {
            if (NCW == 8 && (v & 1) != par) continue;
            wait_flags(flags + kDnWReady + kDnNLW * v, kDnNLW, lane, flags + kDnPoison);
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
                wait_flags(flags + kDnAReady + kDnNLA * u, kDnNLA, lane, flags + kDnPoison);
                const uint8_t* aunit = a_ring + (u % DA) * a_slot;
                // The k-step's activation fragments of every m-tile are read
                // together, and the next k-step's fragments and weights are read
                // and decoded in the same scheduling region as this k-step's
                // MFMAs (one region per k-step: the barrier keeps each read away
                // from its use), so the LDS latency is paid once per k-step and
                // the scheduler can place the decode between the MFMAs
                // (17408 x 5120 at M = 128: 44.6-46.5 -> 42.8-44.7 us).
                h8 a[2][MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) a[0][mt] = *(const h8*)(aunit + arow[mt]);
                h8 bw[2];
                bw[0] = h ? weights(mg, raw1, sc1, 0) : weights(mg, raw0, sc0, 0);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    __builtin_amdgcn_sched_barrier(0);
                    if (i < 7) {
#pragma unroll
                        for (int mt = 0; mt < MT; mt++) a[(i + 1) & 1][mt] = *(const h8*)(aunit + arow[mt] + 16 * (i + 1));
                        bw[(i + 1) & 1] = h ? weights(mg, raw1, sc1, i + 1) : weights(mg, raw0, sc0, i + 1);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) acc[mt] = mfma32x32x16(a[i & 1][mt], bw[i & 1], acc[mt]);
                }
                // every LDS read of the half-slab has completed: count it consumed
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (lane == 0) asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kDnACons + u])), "v"(1) : "memory");
            }
        }
        if constexpr (NCW == 8) {
            // the two parities' sums of the piece: parity 1 hands its m-tiles
            // over through LDS one at a time, parity 0 adds them (its own
            // first: a fixed order) and stores
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                chunk++;
                float* const cb = (float*)(comb + c * 4096) + lane * 16;
                if (par == 1) {
                    if (chunk > 1) wait_flags(flags + kDnCombR + c, 1, lane, flags + kDnPoison, chunk - 1);
#pragma unroll
                    for (int e = 0; e < 16; e += 4)
                        *(f4*)(cb + e) = f4{acc[mt][e], acc[mt][e + 1], acc[mt][e + 2], acc[mt][e + 3]};
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    if (lane == 0)
                        asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kDnCombW + c])), "v"(chunk) : "memory");
                } else {
                    wait_flags(flags + kDnCombW + c, 1, lane, flags + kDnPoison, chunk);
#pragma unroll
                    for (int e = 0; e < 16; e += 4) {
                        const f4 q = *(const f4*)(cb + e);
                        acc[mt][e] += q[0];
                        acc[mt][e + 1] += q[1];
                        acc[mt][e + 2] += q[2];
                        acc[mt][e + 3] += q[3];
                    }
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    if (lane == 0)
                        asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kDnCombR + c])), "v"(chunk) : "memory");
                }
            }
            if (par == 1) {
                t += s1 - s0;
                continue;
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
            // a partial piece (the range's first or last): slot 2 p + which,
            // [batch row][row of the row group] fp32, summed by k_dense_sum
            const bool bad = poisoned(flags + kDnPoison);
            const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
                ws + (size_t)(2 * p + (piece == 0 ? 0 : 1)) * Mp * ROWS, (short)0, Mp * ROWS * 4, 0x00020000);
            const int voff = (4 * g * ROWS + 32 * c + n) * 4;   // batch row 4g of the m-tile
            if (M >= 32 * MT) {
                // every m-tile full: no per-element exec masks
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int dm = mt * 32 + 8 * (e >> 2) + (e & 3);
                        const float y = bad ? __builtin_nanf("") : acc[mt][e];
                        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), pr, voff, dm * ROWS * 4,
                                                              kDnPartPolicy);
                    }
            } else {
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int dm = mt * 32 + 8 * (e >> 2) + (e & 3);
                        if (dm + 4 * g < M) {
                            const float y = bad ? __builtin_nanf("") : acc[mt][e];
                            __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, y), pr, voff, dm * ROWS * 4,
                                                                  kDnPartPolicy);
                        }
                    }
            }
        }
        t += s1 - s0;
    }
}

// One workgroup per CU (the rings fill the LDS): 4 + 3 waves (NCW = 4) or
// 8 + 3 (NCW = 8, at most three per SIMD).
template <int QT, int MT, int NCW>
__global__ __launch_bounds__(64 * (NCW + kDnNL)) __attribute__((amdgpu_waves_per_eu(NCW == 8 ? 3 : 1, NCW == 8 ? 3 : 2)))
void k_gemm_dense(const uint8_t* __restrict__ W, const uint8_t* __restrict__ Waux, const uint16_t* __restrict__ A,
                  int lda, void* __restrict__ C, int ldc, int out_f16, int M, int N, int K, int T, int G, int DW,
                  int DA, float* __restrict__ ws) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    dense_body<QT, MT, NCW>((int)blockIdx.x, lds, W, Waux, A, lda, C, ldc, out_f16, M, N, K, T, G, DW, DA, ws);
}

// Several independent GEMMs of one batch size in one launch, their grids back
// to back: each GEMM keeps the ranges, pieces and partial slots a launch of
// its own would have (so the same bits), and one k_dense_sum_batched launch
// adds the split row groups of all of them.
constexpr int kDnMaxJobs = 8;
struct DenseJob {
    const uint8_t* W;
    const uint8_t* Waux;
    const uint16_t* A;
    void* C;
    float* ws;                           // this GEMM's partial slots
    int lda, ldc, N, K, T, G, grid0, rg0;  // rg0: the GEMM's first row group in the sum launch
};
struct DenseJobs {
    DenseJob job[kDnMaxJobs];
    int n, M, out_f16, DW, DA;
};

template <int QT, int MT, int NCW>
__global__ __launch_bounds__(64 * (NCW + kDnNL)) __attribute__((amdgpu_waves_per_eu(NCW == 8 ? 3 : 1, NCW == 8 ? 3 : 2)))
void k_gemm_dense_batched(const DenseJobs jobs) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    // the last job whose grid starts at or before this workgroup (uniform
    // selects over the kernel arguments: no dynamic indexing)
    DenseJob j = jobs.job[0];
#pragma unroll
    for (int i = 1; i < kDnMaxJobs; i++)
        if (i < jobs.n && (int)blockIdx.x >= jobs.job[i].grid0) j = jobs.job[i];
    dense_body<QT, MT, NCW>((int)blockIdx.x - j.grid0, lds, j.W, j.Waux, j.A, j.lda, j.C, j.ldc, jobs.out_f16, jobs.M, j.N,
                       j.K, j.T, j.G, jobs.DW, jobs.DA, j.ws);
}

// C for the row groups split between workgroups: the sum of their pieces in
// piece order (the workgroup order), so the bits never depend on timing.
// Block (rg, y): batch rows 8 y .. 8 y + 7, thread x: row quad x % 32 of
// batch row 8 y + x / 32.  Row groups held whole by one workgroup were
// written by it.
__device__ __forceinline__ void dense_sum_body(int rg, const float* __restrict__ ws, void* __restrict__ C, int ldc,
                                               int out_f16, int M, int N, int T, int G, int nsg) {
    constexpr int ROWS = kDnRows;
    const int m = 8 * (int)blockIdx.y + ((int)threadIdx.x >> 5);
    const int pf = range_owner(rg * nsg, T, G), pl = range_owner(rg * nsg + nsg - 1, T, G);
    if (pf == pl || m >= M) return;
    const int Mp = (M + 3) & ~3, nl = 4 * ((int)threadIdx.x & 31);
    f4 s = f4{0.f, 0.f, 0.f, 0.f};
    // up to eight pieces' loads in flight before the first add (pieces in order)
    for (int q0 = pf; q0 <= pl; q0 += 8) {
        f4 x[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int q = q0 + k;
            const int slot = 2 * q + (range_first(q, T, G) >= rg * nsg ? 0 : 1);
            x[k] = q <= pl ? *(const f4*)(ws + ((size_t)slot * Mp + m) * ROWS + nl) : f4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int k = 0; k < 8; k++)
            if (q0 + k <= pl) s += x[k];
    }
    const int64_t n0 = (int64_t)rg * ROWS + nl, o = (int64_t)m * ldc + n0;
    if (((uintptr_t)C & 15) == 0 && (ldc & 3) == 0 && n0 + 3 < N) {
        if (out_f16) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            *(h4*)((_Float16*)C + o) = h4{(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
        } else {
            *(f4*)((float*)C + o) = s;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (n0 + i >= N) break;
            if (out_f16) ((_Float16*)C)[o + i] = (_Float16)s[i];
            else ((float*)C)[o + i] = s[i];
        }
    }
}

__global__ __launch_bounds__(256) void k_dense_sum(const float* __restrict__ ws, void* __restrict__ C, int ldc,
                                                   int out_f16, int M, int N, int T, int G, int nsg) {
    dense_sum_body((int)blockIdx.x, ws, C, ldc, out_f16, M, N, T, G, nsg);
}

__global__ __launch_bounds__(256) void k_dense_sum_batched(const DenseJobs jobs) {
    DenseJob j = jobs.job[0];
#pragma unroll
    for (int i = 1; i < kDnMaxJobs; i++)
        if (i < jobs.n && (int)blockIdx.x >= jobs.job[i].rg0) j = jobs.job[i];
    dense_sum_body((int)blockIdx.x - j.rg0, j.ws, j.C, j.ldc, jobs.out_f16, jobs.M, j.N, j.T, j.G, j.K / 256);
}

struct DensePlan {
    int MT, T, G, DW, DA, rgs, lds, nc;                // nc: compute waves (4 or 8)
    bool split;                                        // some row group is split between workgroups
};

size_t dense_partial_bytes(const GemmArgs& g, const DensePlan& p) {
    return ((size_t)2 * p.G * kDnRows * ((g.M + 3) & ~3) * 4 + 255) & ~(size_t)255;
}

// Rings: two weight slots, as many activation slots as fit (up to 6).  One
// workgroup per CU.  The plan never depends on the workspace on offer: the
// ranges decide how partial sums are grouped, so every caller gets the same
// bits.
bool plan_dense(const GemmArgs& g, DensePlan& p, int cus) {
    if (g.M < 1 || g.M > 128 || g.K % 256 || g.N < 1) return false;
    if ((int64_t)g.M * g.ldc * (g.out_f16 ? 2 : 4) >= (1LL << 31)) return false;   // C by 32-bit offsets
    const int MT = (g.M + 31) / 32;                    // 32-row m-tiles
    if ((g.M * 17 + 63) / 64 > kDnNLA * kDnAQS || (kDnRows * 9 + 63) / 64 > kDnNLW * kDnWQS) return false;
    // Eight compute waves (two per SIMD, on alternate units) where the
    // activation ring holds at least five half-slabs beside the hand-over
    // area (M <= 79); otherwise four, one per SIMD.  5120 x 17408 at
    // M = 24 / 32 / 64: 23.3-23.6 / 23.2 / 28.7-29.3 -> 21.7-21.9 / 22.1 /
    // 28.0-28.5 us, the 27B-class layer at M = 32 in one batched call
    // 88.0-91.8 -> 82.4-83.8 us; with four half-slabs (M = 96) eight waves were
    // 1-2.5 % slower, with three (M = 128) 6 %.
    const int DW = 2, a_slot = g.M * kDnARow;
    const int DA8 = std::min(6, (kMaxLds - kDnFlags - DW * kDnWSlot - kDnComb) / a_slot);
    const int nc = DA8 >= 5 ? 8 : 4;
    const int DA = nc == 8 ? DA8 : std::min(6, (kMaxLds - kDnFlags - DW * kDnWSlot) / a_slot);
    if (DA < 2) return false;
    const int64_t rgs = (g.N + kDnRows - 1) / kDnRows, nsg = g.K / 256;
    if (rgs * nsg >= (1LL << 30)) return false;
    const int T = (int)(rgs * nsg);
    const int G = std::min(T, cus > 0 ? cus : 256);
    if ((T + G - 1) / G > kDnMaxUnits) return false;
    bool split = false;
    for (int rg = 0; rg < (int)rgs && !split; rg++)
        split = range_owner(rg * (int)nsg, T, G) != range_owner(rg * (int)nsg + (int)nsg - 1, T, G);
    p = DensePlan{MT, T, G, DW, DA, (int)rgs, kDnFlags + DW * kDnWSlot + DA * a_slot + (nc == 8 ? kDnComb : 0), nc,
                  split};
    return true;
}

template <int QT, int MT, int NCW>
hipError_t launch_dense(const GemmArgs& g, const DensePlan& p, const Scratch* scratch, hipStream_t st) {
    auto k = k_gemm_dense<QT, MT, NCW>;
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
    e = split_workspace(scratch, st, 0, dense_partial_bytes(g, p), &counters, &parts);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k, dim3(p.G), dim3(64 * (NCW + kDnNL)), p.lds, st, g.W, g.Waux, g.A, g.lda, g.C, g.ldc,
                       g.out_f16, g.M, g.N, g.K, p.T, p.G, p.DW, p.DA, parts);
    e = hipGetLastError();
    if (e != hipSuccess || !p.split) return e;
    hipLaunchKernelGGL(k_dense_sum, dim3(p.rgs, (g.M + 7) / 8), dim3(256), 0, st, (const float*)parts, g.C, g.ldc,
                       g.out_f16, g.M, g.N, p.T, p.G, g.K / 256);
    return hipGetLastError();
}

// Up to kDnMaxJobs GEMMs of one format, one batch size and one output type:
// one launch of their grids back to back, one sum launch.
template <int QT, int MT, int NCW>
hipError_t launch_dense_batched(const GemmArgs* gs, const DensePlan* ps, int n, const Scratch* scratch,
                                hipStream_t st) {
    auto k = k_gemm_dense_batched<QT, MT, NCW>;
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
    // one workspace: every GEMM's partial slots at its own 256-byte offset
    size_t ptot = 0;
    for (int i = 0; i < n; i++) ptot += dense_partial_bytes(gs[i], ps[i]);
    unsigned* counters = nullptr;
    float* parts = nullptr;
    e = split_workspace(scratch, st, 0, ptot, &counters, &parts);
    if (e != hipSuccess) return e;
    DenseJobs jobs = {};
    jobs.n = n;
    jobs.M = gs[0].M;
    jobs.out_f16 = gs[0].out_f16;
    jobs.DW = ps[0].DW;
    jobs.DA = ps[0].DA;
    int grid = 0, lds = 0, rgs = 0;
    bool split = false;
    size_t po = 0;
    for (int i = 0; i < n; i++) {
        const GemmArgs& g = gs[i];
        const DensePlan& p = ps[i];
        jobs.job[i] = DenseJob{g.W, g.Waux, g.A, g.C, (float*)((uint8_t*)parts + po), g.lda, g.ldc, g.N, g.K,
                               p.T, p.G, grid, rgs};
        po += dense_partial_bytes(g, p);
        grid += p.G;
        rgs += p.rgs;
        lds = std::max(lds, p.lds);
        split = split || p.split;
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(64 * (NCW + kDnNL)), lds, st, jobs);
    e = hipGetLastError();
    if (e != hipSuccess || !split) return e;
    hipLaunchKernelGGL(k_dense_sum_batched, dim3(rgs, (jobs.M + 7) / 8), dim3(256), 0, st, jobs);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_dense_batched(const GemmArgs* gs, const DensePlan* ps, int n, const Scratch* scratch,
                                  hipStream_t st) {
    if (ps[0].nc == 8) {
        // (the plan gives eight compute waves only where five half-slabs fit: M <= 79)
        if (ps[0].MT == 1) return launch_dense_batched<QT, 1, 8>(gs, ps, n, scratch, st);
        if (ps[0].MT == 2) return launch_dense_batched<QT, 2, 8>(gs, ps, n, scratch, st);
        if (ps[0].MT == 3) return launch_dense_batched<QT, 3, 8>(gs, ps, n, scratch, st);
        return hipErrorInvalidValue;
    }
    if (ps[0].MT == 1) return launch_dense_batched<QT, 1, 4>(gs, ps, n, scratch, st);
    if (ps[0].MT == 2) return launch_dense_batched<QT, 2, 4>(gs, ps, n, scratch, st);
    if (ps[0].MT == 3) return launch_dense_batched<QT, 3, 4>(gs, ps, n, scratch, st);
    return launch_dense_batched<QT, 4, 4>(gs, ps, n, scratch, st);
}

template <int QT>
hipError_t dispatch_dense(const GemmArgs& g, const DensePlan& p, const Scratch* scratch, hipStream_t st) {
    if (p.nc == 8) {
        // (the plan gives eight compute waves only where five half-slabs fit: M <= 79)
        if (p.MT == 1) return launch_dense<QT, 1, 8>(g, p, scratch, st);
        if (p.MT == 2) return launch_dense<QT, 2, 8>(g, p, scratch, st);
        if (p.MT == 3) return launch_dense<QT, 3, 8>(g, p, scratch, st);
        return hipErrorInvalidValue;
    }
    if (p.MT == 1) return launch_dense<QT, 1, 4>(g, p, scratch, st);
    if (p.MT == 2) return launch_dense<QT, 2, 4>(g, p, scratch, st);
    if (p.MT == 3) return launch_dense<QT, 3, 4>(g, p, scratch, st);
    return launch_dense<QT, 4, 4>(g, p, scratch, st);
}

}  // namespace

bool dense_supports(const GemmArgs& g) {
    DensePlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return plan_dense(g, p, device_cus());
}

size_t dense_scratch_bytes(const GemmArgs& g) {
    DensePlan p;
    if (!plan_dense(g, p, device_cus())) return 0;
    return dense_partial_bytes(g, p);
}

WsNeed dense_ws_need(const GemmArgs& g) {
    WsNeed w;
    w.p = dense_scratch_bytes(g);
    return w;
}

// The largest workspace one launch of gemm_dense_batched takes (the GEMMs in
// launches of up to kDnMaxJobs, each launch's partials side by side).
size_t dense_batched_scratch_bytes(const GemmArgs* gs, int n) {
    size_t worst = 0;
    for (int i0 = 0; i0 < n; i0 += kDnMaxJobs) {
        size_t tot = 0;
        for (int i = i0; i < std::min(n, i0 + kDnMaxJobs); i++) {
            DensePlan p;
            if (plan_dense(gs[i], p, device_cus())) tot += dense_partial_bytes(gs[i], p);
        }
        worst = std::max(worst, tot);
    }
    return worst;
}

WsNeed dense_batched_ws_need(const GemmArgs* gs, int n) {
    WsNeed w;
    w.p = dense_batched_scratch_bytes(gs, n);
    return w;
}

bool dense_batched_supports(const GemmArgs* gs, int n) {
    if (n < 1) return false;
    for (int i = 0; i < n; i++) {
        DensePlan p;
        if (gs[i].qtype != gs[0].qtype || gs[i].out_f16 != gs[0].out_f16 || gs[i].M != gs[0].M) return false;
        if (gs[i].qtype == QT_PLANES && ((uintptr_t)gs[i].Waux & 15)) return false;
        if (!plan_dense(gs[i], p, device_cus())) return false;
    }
    return true;
}

hipError_t gemm_dense_batched(const GemmArgs* gs, int n, const Scratch* scratch, hipStream_t st) {
    if (!dense_batched_supports(gs, n)) return hipErrorInvalidValue;
    if (scratch && dense_batched_scratch_bytes(gs, n) > scratch->bytes) return hipErrorInvalidValue;
    for (int i0 = 0; i0 < n; i0 += kDnMaxJobs) {
        const int m = std::min(kDnMaxJobs, n - i0);
        DensePlan ps[kDnMaxJobs];
        for (int i = 0; i < m; i++) plan_dense(gs[i0 + i], ps[i], device_cus());
        hipError_t e;
        switch (gs[0].qtype) {
            case QT_Q4_K: e = dispatch_dense_batched<QT_Q4_K>(gs + i0, ps, m, scratch, st); break;
            case QT_PLANES: e = dispatch_dense_batched<QT_PLANES>(gs + i0, ps, m, scratch, st); break;
            default: e = dispatch_dense_batched<QT_Q4_0>(gs + i0, ps, m, scratch, st); break;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t gemm_dense(const GemmArgs& g, const Scratch* scratch, hipStream_t st) {
    DensePlan p;
    if (!plan_dense(g, p, device_cus())) return hipErrorInvalidValue;
    if (scratch && dense_partial_bytes(g, p) > scratch->bytes) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_dense<QT_Q4_K>(g, p, scratch, st);
        case QT_PLANES: return dispatch_dense<QT_PLANES>(g, p, scratch, st);
        default: return dispatch_dense<QT_Q4_0>(g, p, scratch, st);
    }
}

}  // namespace bf
