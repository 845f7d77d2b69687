// LDS-staged MFMA GEMM for small batches (the decode shapes, M <= 16 when the
// activations fit in LDS).
//
//   C[m][n] = sum_k A[m][k] * dequant(W)[n][k]      (fp32 accumulation)
//
// Replaces the hot loop of the reference kernel (kernels/busfill_v1a.cu:41-104:
// one thread block per group of weight rows, weights read once from HBM,
// dequantised in registers, fp32 accumulation) with a layout built for CDNA4.
//
// * One workgroup per CU-sized slice of rows: `nsub` sub-tiles of R = 16/G
//   consecutive rows (N = 5120, G = 4: 256 workgroups of 20 rows, one per CU).
// * K segments on the MFMA's idle rows: with a batch of M <= 16/G rows per
//   segment, the 16x16x32 MFMA's 16 columns hold R weight rows times G
//   K-segments (column n = G*row + g) and its 16 rows hold 16/G batch rows
//   times the same G segments (row m = G*m' + g).  Only the entries with equal
//   segments are used; they are summed across the G lanes (DPP).  A work unit
//   ("step") is always 16 (row, super-group) pairs = 2304 bytes, whatever G is.
// * Loader waves (the first kNL waves: they start first) move every weight
//   byte HBM -> LDS with direct-to-LDS loads (global_load_lds_dwordx4: one
//   64-lane instruction moves 1 KB without touching VGPRs), as runs of G*144
//   contiguous bytes per row; loader j owns steps j, j + 4, ...  A one-dword
//   load of the workgroup's first weight line, issued before any address is
//   computed, starts the first translation early.  Loaders never wait: after
//   the last load of each step the loader issues a one-dword "marker" load of a
//   nonzero word into that step's flag.  A wave's loads return in issue order,
//   so a visible marker means the step has landed.  Loaders run at the highest
//   issue priority (s_setprio) and use a precomputed address pattern, so the
//   compute waves' VALU work never delays the next load.  The first step's
//   loads are issued before the workgroup's only barrier (the flags are
//   cleared before it).
// * Compute waves (kNC per workgroup) load the activations A[0:M][0:K] the same
//   way at the start (each raises a flag once its own loads are complete), then
//   spin on the markers (ds_read + s_sleep) and take steps from a shared LDS
//   counter (the order in which steps land).  Each step is decoded from LDS
//   into MFMA operands in one of three forms:
//     - fp16 weights (Q4_0 formats): RN_fp16((q - 8) d), the reference
//       kernel's weights, 8 MFMAs per m-tile;
//     - factored Q4_K: d * sum a (sc q) - dmin * sum_j m_j S_j with the exact
//       integers sc*q as operands and the min term as one more MFMA against a
//       table of activation block sums S_j;
//     - sub-block rows (Q4_K, batch 1): the codes enter the MFMA unscaled as
//       fp16 subnormals and MFMA row 4*kappa + g takes only lane group kappa's
//       activations, so each row is one sub-block's sum; the lane scales its
//       two sub-blocks in fp32.  Fewest VALU operations per weight.
//   The folded partial sums of each step are parked in LDS; a per-sub-tile
//   counter (ds_add_rtn) tells the wave that finishes a sub-tile's last step
//   to add the sub-tile's partials in step order (a fixed order: results are
//   deterministic) and store them.
//
// Weight layout in LDS: the workgroup's steps in order, 2304 bytes each; inside
// a step, the 144-byte super-group image of column n = 0..15 at n*144 (Q4_K and
// Q4_0 copy their 144 bytes verbatim; the planes layout stores the 16 bytes of
// the eight block scales followed by the 128 code bytes).  Lane (r, kg) reads
// column r at a 36-dword stride: the 16 lanes of a k-group fall on 16 distinct
// 4-bank groups.
#include <atomic>

#include "bf_launch.h"
#include "bf_lds.h"

namespace bf {
namespace {

// LDS layout (bytes): [0, 2048) flags: activation flag of compute wave c at 4c,
// the compute waves' next-step counter at 60, step markers at 64 + 4e,
// finished-step counters of sub-tile t at 1024 + 4t; [2048, 2048 + a_bytes)
// activations, row m at m * a_rs; then the W steps of the
// workgroup in order (2304 bytes each); then one parked partial per step; then
// (Q4_K) the activation block sums, 32 bytes per batch row and super-group.
constexpr int kFlagBytes = 2048;
constexpr int kMaxSteps = (1024 - 64) / 4;
constexpr int kZeroBytes = 128;                   // [1920, 2048): stays zero (sub-block rows form)
constexpr int kMaxSub = (kFlagBytes - kZeroBytes - 1024) / 4;
constexpr int kStepCounter = 15;                  // flags[15]: next step to take

template <int QT, int G, int MT, int NC, int NL, bool BD>
__global__ __launch_bounds__(64 * (NC + NL))
void k_gemm_lds(const uint8_t* __restrict__ W, const uint16_t* __restrict__ A, int lda, int M, int N, int K,
                int nsub, int a_rs, int a_bytes, const uint8_t* __restrict__ Waux, void* __restrict__ C, int ldc,
                int out_f16) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    static_assert(NC <= kStepCounter, "activation flags sit below the step counter");
    constexpr int R = 16 / G;                          // weight rows (and batch rows) per segment
    static_assert(!BD || (QT == QT_Q4_K && G == 4), "sub-block rows: Q4_K with four K segments");
    // floats of one parked partial: batch rows x weight rows (BD: one batch row per m-tile)
    constexpr int SLOT = BD ? MT * R : MT * R * R;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsg = K >> 8, nsteps = nsg / G;
    const int S = nsub * nsteps;                       // steps of the workgroup
    const int tile0 = blockIdx.x * nsub;
    int* const flags = (int*)lds;
    uint8_t* const a_lds = lds + kFlagBytes;
    uint8_t* const w_lds = a_lds + a_bytes;
    float* const parts = (float*)(w_lds + S * kStep);
    const uint32_t lds0 = lds_addr(lds);

    // Every wave clears 128 bytes of the flags, then meets the others at the
    // one barrier of the kernel.  Loads that write no flag (weights,
    // activations) are issued before it; every marker after it.
    auto clear_flags_and_meet = [&]() {
        static_assert((NC + NL) * 128 == kFlagBytes, "each wave clears 32 flags");
        if (lane < 32) flags[32 * wave + lane] = 0;
        barrier_lds();
    };

    if (wave < NL) {
        // ------------------------------------------------------------ loader wave
        // Issues its loads in order and never waits for them: a marker load after
        // each step tells the compute waves that the step has landed.  Runs at
        // the highest issue priority so that the compute waves' VALU work never
        // delays the next load.
        //
        // Four steps (9,216 bytes) form a group of 9 instructions whose per-lane
        // address pattern repeats from group to group: instruction b of a group
        // covers pieces 64b + lane, i.e. step d_b = (64b + lane) / 144 of the
        // group and a fixed piece (column n, part c) of that step.  Loader j loads
        // step j of every group (steps j, j + 4, ...): instructions
        // b = 9j/4 .. (9j+8)/4 with only the lanes of its step enabled; the
        // instructions that straddle two steps are issued by both of their
        // loaders with complementary lanes.  Each step then has one loader, which
        // issues the step's marker after the step's last load.
        __builtin_amdgcn_s_setprio(3);
        static_assert(NL == 4, "one step of each group per loader");
        const int j = wave;
        // touch the workgroup's first weight line before computing any address, so
        // that its translation and DRAM page are under way early (the value is
        // unused; its register stays reserved until the final wait)
        uint32_t warm;
        asm volatile("global_load_dword %0, %1, off"
                     : "=v"(warm) : "v"(w_piece<QT>(W, Waux, (int64_t)tile0 * R, 0, 1, K)) : "memory");
        const int pmax = S * 144 - 1;
        const uint32_t m0 = lds0 + (uint32_t)(kFlagBytes + a_bytes);
        const int b_lo = (9 * j) / 4, b_hi = (9 * j + 8) / 4;   // this loader's instructions in a group
        uint32_t pat[3];
#pragma unroll
        for (int q = 0; q < 3; q++) {
            const int b = b_lo + q;
            // P < 576: P / 144 and r9 / 9 by 24-bit multiplies (exact over that range)
            const uint32_t P = 64u * b + lane, d = __umul24(P, 7282u) >> 20, r9 = P - 144u * d;
            const uint32_t nn = __umul24(r9, 7282u) >> 16, c = r9 - 9u * nn;
            pat[q] = step_piece_offset<QT>(nn / G, nn % G, c, K) | ((uint32_t)d << 29);
        }
        const bool clamp = (int64_t)(tile0 + nsub) * R > N;   // last workgroup: rows past N reread row N-1
        int te = 0, se = j;                            // step e = te * nsteps + se
        while (se >= nsteps) { se -= nsteps; te++; }
        for (int g4 = 0, e = j; e < S; g4++, e += 4) {
            const StepBase<QT> base = step_base<QT>((int64_t)(tile0 + te) * R, G * se, K);
#pragma unroll
            for (int q = 0; q < 3; q++) {
                const int b = b_lo + q;
                if (b > b_hi) break;
                const int i = 9 * g4 + b;
                const int P = 64 * i + lane;
                const uint32_t pb = pat[q];
                const uint8_t* src;
                if (!clamp) {
                    src = piece_addr<QT>(W, Waux, base, pb & 0x1FFFFFFFu);
                } else {
                    const int Pc = min(P, pmax);
                    const int q9 = Pc - 144 * (Pc / 144), nn = q9 / 9, c = q9 - 9 * nn;
                    const int64_t row = min((int64_t)(tile0 + te) * R + nn / G, (int64_t)N - 1);
                    src = w_piece<QT>(W, Waux, row, G * se + nn % G, c, K);
                }
                if ((pb >> 29) == (uint32_t)j && P <= pmax) dma16(src, m0 + (uint32_t)(i << 10));
            }
            if (g4 == 0) clear_flags_and_meet();
            dma_marker(g_marker_src + lane, lds0 + 64 + 4 * e, lane);
            se += 4;
            while (se >= nsteps) { se -= nsteps; te++; }
        }
        if (j >= S) clear_flags_and_meet();
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("" :: "v"(warm));
        return;
    }
    const int cw = wave - NL;                          // compute wave index

    // ---------------------------------------------------------------- compute wave
    // Activations first: row m of A is nIr 1 KB instructions at m * a_rs (lanes
    // past the row's 33 * nsg pieces are masked); compute wave c issues
    // instructions c, c + NC, ..., counted from a per-workgroup offset so that
    // the workgroups, which all read the same activations, do not all ask for the
    // same lines at once.
    {
        const int nIr = (nsg * 33 + 63) >> 6, nA = M * nIr;
        const int rot = (int)((blockIdx.x * 7u) % (unsigned)nA);
        for (int i0 = cw; i0 < nA; i0 += NC) {
            const int i = i0 + rot < nA ? i0 + rot : i0 + rot - nA;
            const int m = i / nIr, jj = i - m * nIr;
            const int P = 64 * jj + lane;
            const int sg = min(P / 33, nsg - 1), c = min(P - 33 * (P / 33), 31);
            if (P < nsg * 33)
                dma16(A + (int64_t)m * lda + 256 * sg + 8 * c, lds0 + (uint32_t)(kFlagBytes + m * a_rs + 1024 * jj));
        }
    }
    clear_flags_and_meet();
    signal_own_loads(&flags[cw], lane);

    // Steps are taken from a shared counter in step order, which is roughly the
    // order in which they land.  Each step's G-folded partial sums go to the
    // step's own slot; the wave that finishes the last step of a sub-tile adds
    // the sub-tile's slots in step order (a fixed order: results do not depend
    // on timing) and stores them.
    wait_flags(flags, NC, lane);

    // Q4_K runs in the factored form sum_k a_k w_k = d * sum_k a_k (sc q_k)
    // - dmin * sum_j m_j S_j over the sub-blocks j of a super-block, where
    // S_j = sum_{k in j} a_k.  The block sums are tabulated once: entry
    // (m, sg, kg) covers sub-blocks 2kg, 2kg+1 of super-group sg of batch row m:
    //   MFMA form: fp16 {hi_0, hi_1, lo_0, lo_1} with S / 32 = hi + lo / 2048 (hi
    //     is S / 32 rounded to fp16, lo the rounded remainder: S to about 2^-22);
    //   sub-block rows form (BD): fp32 {S_0, S_1}, and the entry's 128 bytes of
    //     activations are reordered in place, each run of eight to
    //     a0 a2 a1 a3 a4 a6 a5 a7, the order in which that form decodes codes.
    const uint8_t* const tab = (const uint8_t*)(parts + S * SLOT);
    if constexpr (BD) {
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
        for (int u = cw * 64 + lane; u < M * nsg * 4; u += NC * 64) {
            const int kq = u & 3, rest = u >> 2;
            const int m = rest / nsg, sg = rest - m * nsg;
            uint8_t* src = a_lds + m * a_rs + sg * kASg + 128 * kq;
            float sum[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float acc = 0.f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    u4 v = *(const u4*)(src + 64 * h + 16 * q);
                    acc = __builtin_amdgcn_fdot2(as_h2(v.x), one, acc, false);
                    acc = __builtin_amdgcn_fdot2(as_h2(v.y), one, acc, false);
                    acc = __builtin_amdgcn_fdot2(as_h2(v.z), one, acc, false);
                    acc = __builtin_amdgcn_fdot2(as_h2(v.w), one, acc, false);
                    const u4 o = {perm_b32(v.y, v.x, 0x05040100u), perm_b32(v.y, v.x, 0x07060302u),
                                  perm_b32(v.w, v.z, 0x05040100u), perm_b32(v.w, v.z, 0x07060302u)};
                    *(u4*)(src + 64 * h + 16 * q) = o;
                }
                sum[h] = acc;
            }
            float* dst = (float*)(tab + 8 * u);
            dst[0] = sum[0];
            dst[1] = sum[1];
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[cw])), "v"(2) : "memory");
        wait_flags(flags, NC, lane, 2);
    } else if constexpr (QT == QT_Q4_K) {
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
        for (int u = cw * 64 + lane; u < M * nsg * 4; u += NC * 64) {
            const int kq = u & 3, rest = u >> 2;
            const int m = rest / nsg, sg = rest - m * nsg;
            const uint8_t* src = a_lds + m * a_rs + sg * kASg + 128 * kq;
            uint32_t hi[2], lo[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float sum = 0.f;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const u4 v = *(const u4*)(src + 64 * h + 16 * q);
                    sum = __builtin_amdgcn_fdot2(as_h2(v.x), one, sum, false);
                    sum = __builtin_amdgcn_fdot2(as_h2(v.y), one, sum, false);
                    sum = __builtin_amdgcn_fdot2(as_h2(v.z), one, sum, false);
                    sum = __builtin_amdgcn_fdot2(as_h2(v.w), one, sum, false);
                }
                const float mean = sum * 0.03125f;
                const _Float16 mh = (_Float16)mean;
                const _Float16 ml = (_Float16)((mean - (float)mh) * 2048.0f);
                hi[h] = __builtin_bit_cast(uint16_t, mh);
                lo[h] = __builtin_bit_cast(uint16_t, ml);
            }
            uint32_t* dst = (uint32_t*)(tab + 8 * u);
            dst[0] = hi[0] | (hi[1] << 16);
            dst[1] = lo[0] | (lo[1] << 16);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[cw])), "v"(2) : "memory");
        wait_flags(flags, NC, lane, 2);
    }

    const Magic mg = make_magic();
    const int r = lane & 15, kg = lane >> 4;
    const int g = r % G, rowl = r / G;
    const uint8_t* arow[MT];
    const uint8_t* trow[MT];                           // this lane's block-sum entries (Q4_K)
    // sub-block rows form: MFMA row r = 4 kappa + g takes the activations of
    // segment g from the k slots of lane group kappa only (zeros elsewhere), so
    // that row holds the partial sums of one sub-block per column
    const bool bd_on = (r >> 2) == kg;
    const uint8_t* const zero16 = lds + kFlagBytes - kZeroBytes;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = BD ? min(mt, M - 1) : min(mt * R + r / G, M - 1);   // padding rows reread row M-1
        arow[mt] = (!BD || bd_on) ? a_lds + m * a_rs + g * kASg + 128 * kg : zero16;
        trow[mt] = tab + ((m * nsg + g) * 4 + kg) * 8;
    }

    for (;;) {
        // take the next step (steps land roughly in order; a free wave takes the next one)
        int e = 0;
        if (lane == 0)
            asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                         : "=v"(e) : "v"(lds_addr(&flags[kStepCounter])), "v"(1) : "memory");
        e = __builtin_amdgcn_readfirstlane(e);
        if (e >= S) break;
        const int t_in = e / nsteps, s_in = e - t_in * nsteps;
        wait_flag(&flags[16 + e]);
        Raw<QT> raw;
        lds_raw<QT>(raw, w_lds + e * kStep + r * 144, kg);
        const int aoff = G * s_in * kASg;
        f4 acc[MT], accm[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[mt] = accm[mt] = f4{0.f, 0.f, 0.f, 0.f};
        float d = 1.f, dmin = 0.f;
        if constexpr (BD) {
            // codes as fp16 subnormals: low nibble q -> q * 2^-24, high nibble
            // (masked in place) -> 16 q * 2^-24; exact products in the MFMA
            const BdScl sb = scales_bd(raw, kg);
            f4 alo[MT], ahi[MT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++) alo[mt] = ahi[mt] = f4{0.f, 0.f, 0.f, 0.f};
            const int astep = bd_on ? aoff : 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                h8 blo, bhi;
                codes_subnormal(raw, t, blo, bhi);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    alo[mt] = mfma16x16x32(*(const h8*)(arow[mt] + astep + 16 * t), blo, alo[mt]);
                    ahi[mt] = mfma16x16x32(*(const h8*)(arow[mt] + astep + 16 * (t + 4)), bhi, ahi[mt]);
                }
            }
            float* slot = parts + e * SLOT;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                // this lane's column n = 4 rowl + g and its sub-blocks 2kg, 2kg+1: row 4kg + g
                float plo = alo[mt][0], phi = ahi[mt][0];
#pragma unroll
                for (int gg = 1; gg < 4; gg++)
                    if (g == gg) {
                        plo = alo[mt][gg];
                        phi = ahi[mt][gg];
                    }
                const float* ts = (const float*)(trow[mt] + G * s_in * 32);
                float y = sb.d20 * __builtin_fmaf(sb.c_lo16, plo, sb.c_hi * phi) -
                          sb.dmin * __builtin_fmaf(sb.m_lo, ts[0], sb.m_hi * ts[1]);
                // sum the four lane groups (sub-block pairs), then the four segments
                y = sum_lane_xor16(y);
                y = sum_lane_xor32(y);
                y += dpp_xor(y, 1);
                y += dpp_xor(y, 2);
                if (g == 0 && kg == 0) slot[mt * R + rowl] = y;
            }
        } else if constexpr (QT == QT_Q4_K) {
            const SclK sk = scales_int(raw, kg);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h8 b = weights_int(mg, raw, sk, i);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    acc[mt] = mfma16x16x32(*(const h8*)(arow[mt] + aoff + 16 * i), b, acc[mt]);
            }
            // sum_j m_j S_j: the mins {32m, m/64} of sub-blocks 2kg, 2kg+1 meet the
            // block sums {hi, lo} of the same sub-blocks (k slots 8kg .. 8kg+3)
            const h8 bm = __builtin_bit_cast(h8, u4{sk.min_hi, sk.min_lo, 0u, 0u});
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const uint32_t* t = (const uint32_t*)(trow[mt] + G * s_in * 32);
                const h8 am = __builtin_bit_cast(h8, u4{t[0], t[1], 0u, 0u});
                accm[mt] = mfma16x16x32(am, bm, accm[mt]);
            }
            d = sk.d;
            dmin = sk.dmin;
        } else {
            const auto sc = scales(raw, kg);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h8 b = weights(mg, raw, sc, i);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    acc[mt] = mfma16x16x32(*(const h8*)(arow[mt] + aoff + 16 * i), b, acc[mt]);
            }
        }
        if constexpr (!BD) {
            // fold the G segments (lanes r = G*rowl + g) and park the partial sums
            float* slot = parts + e * SLOT;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
#pragma unroll
                for (int jj = 0; jj < 4 / G; jj++) {
                    // register G*jj + g holds batch row (4kg)/G + jj of segment g
                    float y = acc[mt][G * jj];
#pragma unroll
                    for (int gg = 1; gg < G; gg++)
                        if (g == gg) y = acc[mt][G * jj + gg];
                    if constexpr (QT == QT_Q4_K) {
                        // this lane's column is one (row, super-group): apply its d and dmin
                        float ym = accm[mt][G * jj];
#pragma unroll
                        for (int gg = 1; gg < G; gg++)
                            if (g == gg) ym = accm[mt][G * jj + gg];
                        y = __builtin_fmaf(d, y, -(dmin * ym));
                    }
                    if constexpr (G >= 2) y += dpp_xor(y, 1);
                    if constexpr (G >= 4) y += dpp_xor(y, 2);
                    if (g == 0) slot[(mt * R + (4 * kg) / G + jj) * R + rowl] = y;
                }
            }
        }
        // count the finished step; the last of the sub-tile reduces and stores it
        int old = 0;
        if (lane == 0)
            asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                         : "=v"(old) : "v"(lds_addr(&flags[256 + t_in])), "v"(1) : "memory");
        if (__builtin_amdgcn_readfirstlane(old) == nsteps - 1) {
            const int64_t row0 = (int64_t)(tile0 + t_in) * R;
            for (int v = lane; v < SLOT; v += 64) {
                const float* pp = parts + t_in * nsteps * SLOT + v;
                float sum = 0.f;
                for (int s2 = 0; s2 < nsteps; s2++) sum += pp[s2 * SLOT];
                const int m = v / R, rl = v - m * R;   // m = mt * R + m_loc
                const int64_t row = row0 + rl;
                if (m < M && row < N) {
                    if (out_f16) ((_Float16*)C)[(int64_t)m * ldc + row] = (_Float16)sum;
                    else ((float*)C)[(int64_t)m * ldc + row] = sum;
                }
            }
        }
    }
}

// LDS row stride for activations: whole kilobytes for the 528-byte super-group
// images of one row, plus 16*G bytes, so that the rows m' of one k-group sit on
// distinct bank groups (stride = 16*G mod 256 bytes).
inline int a_row_stride(int nsg, int G) {
    return (nsg * kASg + 1023) / 1024 * 1024 + 16 * G;
}

constexpr int kNC = 12, kNL = 4;      // compute and loader waves per workgroup

struct LdsPlan {
    int G, MT, nsub, grid, a_rs, a_bytes, lds;
    bool BD;                           // sub-block rows form (Q4_K, one batch row per m-tile)
};

// Sub-tiles per workgroup: about one workgroup per CU when the LDS holds all of
// its steps, otherwise the fewest rounds of 256 workgroups that fit.
bool plan_lds(const GemmArgs& g, int G, int MT, LdsPlan& p, bool BD = false) {
    const int nsg = g.K / 256;
    if (nsg % G) return false;
    const int nsteps = nsg / G, R = 16 / G;
    if (BD ? (g.qtype != QT_Q4_K || G != 4 || g.M > MT) : g.M > MT * R) return false;
    p.BD = BD;
    const int T = (g.N + R - 1) / R;
    p.G = G;
    p.MT = MT;
    p.a_rs = a_row_stride(nsg, G);
    if ((int64_t)g.M * p.a_rs > kMaxLds) return false;
    p.a_bytes = (int)(((int64_t)g.M * p.a_rs + 15) / 16 * 16);
    for (int rounds = 1; rounds <= 64; rounds++) {
        const int nsub = (T + 256 * rounds - 1) / (256 * rounds);
        const int S = nsub * nsteps;
        if (S > kMaxSteps || nsub > kMaxSub) continue;
        const int64_t tab = g.qtype == QT_Q4_K ? (int64_t)g.M * nsg * 32 : 0;   // block sums
        const int64_t slot = BD ? MT * R : MT * R * R;
        const int64_t lds = kFlagBytes + (int64_t)p.a_bytes + (int64_t)S * kStep + (int64_t)S * slot * 4 + tab;
        if (lds > kMaxLds) {
            if (nsub == 1) return false;
            continue;
        }
        p.nsub = nsub;
        p.grid = (T + nsub - 1) / nsub;
        p.lds = (int)lds;
        return true;
    }
    return false;
}

template <int QT, int G, int MT, bool BD = false>
hipError_t launch_lds(const GemmArgs& g, const LdsPlan& p, hipStream_t st) {
    auto k = k_gemm_lds<QT, G, MT, kNC, kNL, BD>;
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
    hipLaunchKernelGGL(k, dim3(p.grid), dim3(64 * (kNC + kNL)), p.lds, st, g.W, g.A, g.lda, g.M, g.N, g.K, p.nsub,
                       p.a_rs, p.a_bytes, g.Waux, g.C, g.ldc, g.out_f16);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_lds(const GemmArgs& g, const LdsPlan& p, hipStream_t st) {
    if constexpr (QT == QT_Q4_K) {
        if (p.BD) return launch_lds<QT, 4, 1, true>(g, p, st);
    }
    if (p.G == 4 && p.MT == 1) return launch_lds<QT, 4, 1>(g, p, st);
    if (p.G == 4 && p.MT == 2) return launch_lds<QT, 4, 2>(g, p, st);
    if (p.G == 2 && p.MT == 1) return launch_lds<QT, 2, 1>(g, p, st);
    return launch_lds<QT, 1, 1>(g, p, st);
}

bool choose_lds(const GemmArgs& g, LdsPlan& p) {
    // sub-block rows at batch 1 only: from two rows on, its MFMA count doubles
    // and the factored MFMA form is faster
    if (g.qtype == QT_Q4_K && g.M == 1 && plan_lds(g, 4, 1, p, true)) return true;
    if (g.M <= 4 && plan_lds(g, 4, 1, p)) return true;
    if (g.M <= 8 && plan_lds(g, 4, 2, p)) return true;
    if (g.M <= 8 && plan_lds(g, 2, 1, p)) return true;
    if (g.M <= 16 && plan_lds(g, 1, 1, p)) return true;
    return false;
}

}  // namespace

bool lds_supports(const GemmArgs& g) {
    LdsPlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return choose_lds(g, p);
}

hipError_t gemm_lds(const GemmArgs& g, hipStream_t st) {
    LdsPlan p;
    if (!choose_lds(g, p)) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_lds<QT_Q4_K>(g, p, st);
        case QT_PLANES: return dispatch_lds<QT_PLANES>(g, p, st);
        default: return dispatch_lds<QT_Q4_0>(g, p, st);
    }
}

}  // namespace bf
