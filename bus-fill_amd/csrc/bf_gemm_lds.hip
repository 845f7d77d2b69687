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
// * Activations: at batch 2-16 the loaders also load A[0:M][0:K], segment by
//   segment (a segment = the G super-groups of one step for all M rows), each
//   segment just before the first step that needs it, with one marker per
//   loader and segment; a step waits for its segment's four markers, so the
//   compute starts on the first segment instead of after all of A (80 KB at
//   M = 8).  At batch 1 (10 KB) the compute waves load A themselves at the
//   start and each raises a flag once its own loads are complete.
// * Compute waves (kNC per workgroup) spin on the markers (ds_read + s_sleep)
//   and take steps in the order in which they land: from a shared LDS counter,
//   or at batch 1 wave c takes steps c, c + kNC, ... and reads a step's marker
//   and data in one round trip.  Each step is decoded from LDS into MFMA
//   operands in one of three forms:
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
//   deterministic) and store them.  At batch 1 each lane parks its own
//   unreduced value (the cross-lane sums run once per sub-tile instead of
//   once per step), the count is a plain ds_add, and the wave that took the
//   sub-tile's last step waits for the count once its own steps are done.
//
// Weight layout in LDS: the workgroup's steps in order, 2304 bytes each; inside
// a step, the 144-byte super-group image of column n = 0..15 at n*144 (Q4_K and
// Q4_0 copy their 144 bytes verbatim; the planes layout stores the 16 bytes of
// the eight block scales followed by the 128 code bytes).  Lane (r, kg) reads
// column r at a 36-dword stride: the 16 lanes of a k-group fall on 16 distinct
// 4-bank groups.
#include <algorithm>
#include <atomic>

#include "bf_launch.h"
#include "bf_lds.h"
#include "bf_lds_plan.h"

namespace bf {
namespace {


// One GEMM's share of a launch: workgroup `bid` of its grid.  RG: steps in
// windows of `win` segments and na activation slots (plans whose activations do
// not all fit); otherwise sub-tile-major with all of A resident.  AC: the
// compute waves load all of A before the barrier (small A).  SW (batch 1 or
// AC): A[m][k] = SiLU(A[m][k]) * A[m][K + k], formed as the compute waves load
// it (the fused gate|up projection's output in, the down projection out).
// DEP (with BD or AC): A is the output of dep_n other workgroups of the same
// launch (the dependency words at dep, laid out as kDepWords describes); the
// compute waves meet the loaders first (so the weight stream starts at once),
// wait for the release flag, then load A with device-scope loads.  dep_users
// workgroups wait; the last of them past its wait clears the words.  CO: C is
// stored with device-scope stores (written through to the point of coherence:
// the output is such a dependency's A).  AF (with BD or AC): A is fp32 rows
// (lda in floats), rounded to fp16 as the compute waves load them.  EA (plans
// whose steps all have a slot of their own, no step ring): each loader issues
// the first group's step before the rest of its setup.
template <int QT, int G, int MT, int NC, int NL, bool BD, bool RG, bool AC, bool SW = false, bool DEP = false,
          bool CO = false, bool AF = false, bool EA = false>
__device__ __forceinline__ void lds_body(int bid, uint8_t* lds, const uint8_t* __restrict__ W,
                                         const uint16_t* __restrict__ A, int lda, int M, int N, int K, int nsub,
                                         int nslot, int na, int win, const uint8_t* __restrict__ Waux,
                                         void* __restrict__ C, int ldc, int out_f16, unsigned* dep = nullptr,
                                         unsigned dep_n = 0, unsigned dep_users = 0) {
    static_assert(!DEP || BD || AC, "a dependency needs A loaded by the compute waves");
    static_assert(!AF || ((BD || AC) && !SW && !DEP), "fp32 activations: loaded by the compute waves");
    constexpr int R = 16 / G;                          // weight rows (and batch rows) per segment
    static_assert(!BD || G == 4, "sub-block rows: four K segments");
    // floats of one parked partial: batch rows x weight rows (BD: one batch row per m-tile)
    constexpr int SLOT = BD ? MT * 64 : MT * R * R;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nsg = K >> 8, nsteps = nsg / G;
    const int S = nsub * nsteps;                       // steps of the workgroup
    const int tile0 = bid * nsub;
    // Step order: windows of Wn segments; in window w every sub-tile in turn
    // takes the window's segments in order (Wn = nsteps: sub-tile-major; the
    // last window may hold fewer, Wl).  na < nsteps: activation ring.
    static_assert(!(BD && RG), "batch 1 keeps all of A");
    const int Wn = RG ? win : nsteps;
    const int EW = nsub * Wn, nfull = nsteps / Wn, Wl = nsteps - nfull * Wn, E_full = nfull * EW;
    const bool a_ring = RG && na < nsteps;
    // e / d as (e * inv) >> 16: exact for e < 240, d <= 240
    const uint32_t inv_EW = (65536u + EW - 1u) / (uint32_t)EW, inv_W = (65536u + Wn - 1u) / (uint32_t)Wn;
    const uint32_t inv_Wl = Wl ? (65536u + Wl - 1u) / (uint32_t)Wl : 0u;
    const uint32_t inv_na = (65536u + na - 1u) / (uint32_t)na;
    const uint32_t inv_nslot = (65536u + nslot - 1u) / (uint32_t)nslot;
    // step e -> (sub-tile t, segment s)
    auto step_ts = [&](int e, int& t, int& sg) {
        if (!RG) {
            t = (int)(((uint32_t)e * inv_W) >> 16);
            sg = e - t * nsteps;
        } else if (e < E_full) {
            const int w = (int)(((uint32_t)e * inv_EW) >> 16), e1 = e - w * EW;
            t = (int)(((uint32_t)e1 * inv_W) >> 16);
            sg = w * Wn + e1 - t * Wn;
        } else {
            const int e1 = e - E_full;
            t = (int)(((uint32_t)e1 * inv_Wl) >> 16);
            sg = nfull * Wn + e1 - t * Wl;
        }
    };
    const int seg_bytes = M * G * 528, a_bytes = na * seg_bytes;
    // activation segment s -> its byte offset (slot s mod na of the ring)
    auto seg_off = [&](int sg) {
        if (!RG) return sg * seg_bytes;
        return (sg - (int)(((uint32_t)sg * inv_na) >> 16) * na) * seg_bytes;
    };
    int* const flags = (int*)lds;
    uint8_t* const a_lds = lds + kFlagBytes;
    uint8_t* const w_lds = a_lds + a_bytes;            // ring of nslot steps (nslot = S: no reuse)
    float* const parts = (float*)(w_lds + nslot * kStep);
    const uint32_t lds0 = lds_addr(lds);

    // Every wave clears 256 bytes of the flags, then meets the others at the
    // one barrier of the kernel.  The loaders issue their first group's data
    // loads before it and every marker after it.
    auto clear_flags_and_meet = [&]() {
        static_assert((NC + NL) * 256 == kFlagBytes, "each wave clears 64 flags");
        flags[64 * wave + lane] = 0;
        barrier_lds();
    };
    // DEP: the first compute wave polls its release flag (device scope), then
    // releases the other compute waves through an LDS flag.  A wait that gives
    // up poisons.
    auto wait_dep = [&]() {
        if (wave == NL) {
            wait_device_count(dep + kDepLine0 + 64 * (bid % kDepLines), 1u, lane, flags + kPoison);
            // an earlier launch's consumer gave up: this launch's results are NaN
            unsigned sticky = 0;
            if (lane == 0) sticky = __hip_atomic_load(dep + kDepPoison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((unsigned)__builtin_amdgcn_readfirstlane(sticky) != 0u) mark_poison(flags + kPoison);
            if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kDepFlag])), "v"(1) : "memory");
        } else {
            wait_flag(&flags[kDepFlag], flags + kPoison);
        }
    };
    // DEP: A through a buffer resource, read with device-scope loads (the
    // producers' stores were written through to the point of coherence)
    const __amdgpu_buffer_rsrc_t a_rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)A, (short)0, DEP ? (int)(((int64_t)(M - 1) * lda + 2 * K) * 2) : 0,
                                          0x00020000);
    auto swiglu_dep = [&](int64_t elem) {
        const int off = (int)(elem * 2);
        return swiglu8v(__builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off, 0, kDeviceScope)),
                        __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, off + 2 * K, 0,
                                                                                      kDeviceScope)));
    };
    // one result: C[m][row] (CO: a device-scope store)
    auto store_c = [&](int64_t m, int64_t row, float v) {
        const int64_t idx = m * ldc + row;
        if constexpr (CO) {
            const __amdgpu_buffer_rsrc_t cr = __builtin_amdgcn_make_buffer_rsrc(C, (short)0, 0x7FFFFFFF, 0x00020000);
            if (out_f16)
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (_Float16)v), cr, (int)(idx * 2), 0,
                                                      kDeviceScope);
            else
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), cr, (int)(idx * 4), 0,
                                                      kDeviceScope);
        } else {
            if (out_f16) ((_Float16*)C)[idx] = (_Float16)v;
            else ((float*)C)[idx] = v;
        }
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
        // EA: the first group's step goes out before anything else is computed
        // (the setup below is a few hundred cycles of instruction issue that
        // would delay the start of the stream), from the same address pattern
        // as the loop, which then skips it; not in the last workgroup (rows
        // past N) nor in step-ring plans (kernels of their own: the added code
        // measured slower there even where it did not run)
        bool early = false;
        if constexpr (EA) {
            early = (int64_t)(tile0 + nsub) * R <= N && j < S;
            if (early) {
                int te0 = 0, se0 = j;
                if (RG) step_ts(j, te0, se0);
                else
                    while (se0 >= nsteps) { se0 -= nsteps; te0++; }
                const StepBase<QT> base0 = step_base<QT>((int64_t)(tile0 + te0) * R, G * se0, K);
                const uint32_t m00 = lds0 + (uint32_t)(kFlagBytes + a_bytes);
                const int b0 = (9 * j) / 4, b1 = (9 * j + 8) / 4;
#pragma unroll
                for (int q = 0; q < 3; q++) {
                    const int b = b0 + q;
                    if (b > b1) break;
                    const uint32_t P = 64u * b + lane, d = __umul24(P, 7282u) >> 20, r9 = P - 144u * d;
                    const uint32_t nn = __umul24(r9, 7282u) >> 16, c = r9 - 9u * nn;
                    if (d == (uint32_t)j && (int)P < S * 144)
                        dma16(piece_addr<QT>(W, Waux, base0, step_piece_offset<QT>(nn / G, nn % G, c, K)),
                              m00 + (uint32_t)(b << 10));
                }
            }
        }
        // touch the workgroup's first weight line before computing any address, so
        // that its translation and DRAM page are under way early (the value is
        // unused; its register stays reserved until the final wait)
        uint32_t warm;
        asm volatile("global_load_dword %0, %1, off"
                     : "=v"(warm) : "v"(w_piece<QT>(W, Waux, (int64_t)tile0 * R, 0, 1, K)) : "memory");
        const int pmax = S * 144 - 1;
        const uint32_t m0 = lds0 + (uint32_t)(kFlagBytes + a_bytes);
        // groups in the ring: nslot is a multiple of 4 when the ring wraps, and
        // nslot = S (every group at its own place) when it does not
        const int G4R = (nslot + 3) >> 2;
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
        // Activations: segment s is M*G*33 16-byte pieces (piece P: batch row
        // P / (33 G), super-group g, part c; part 32 of each super-group is bank
        // padding and is not loaded), IA 1 KB instructions of which loader j issues
        // j, j + 4, ...  A piece's address advances 512 G bytes per segment.
        const int PA = M * G * 33, IA = (PA + 63) >> 6;
        const uint8_t* asrc[kASlots];
        bool aon[kASlots];
#pragma unroll
        for (int q = 0; q < kASlots; q++) {
            const uint32_t P = 64u * (j + 4 * q) + lane;     // P < 1600 (M * G <= 32)
            const uint32_t m = G == 4 ? __umul24(P, 993u) >> 17 : G == 2 ? __umul24(P, 993u) >> 16
                                                                       : __umul24(P, 1986u) >> 16;
            const uint32_t rem = P - 33u * G * m, gg = __umul24(rem, 1986u) >> 16, c = rem - 33u * gg;
            aon[q] = P < (uint32_t)PA && c < 32;
            asrc[q] = (const uint8_t*)(A + (int64_t)min((int)m, M - 1) * lda + 256 * gg + 8 * min((int)c, 31));
        }
        // RG: the next activation segment to load, its window and place in it
        // (its first step, sub-tile 0, is sw * EW + so); otherwise the step
        // e = te * nsteps + se
        int s_next = 0, sw = 0, so = 0;
        int te = 0, se = j;
        if (!RG)
            while (se >= nsteps) { se -= nsteps; te++; }
        for (int g4 = 0, e = j; 4 * g4 < S; g4++, e += 4) {
            // this loader's step of the group and its marker, then the activation
            // segments first needed by the group's steps (RG: scanned; otherwise
            // those of the first sub-tile, e < nsteps) and their markers, so that
            // no step marker waits for activation loads (batch 1, small A: the
            // compute waves load A)
            int s_lo = 4 * g4, s_hi = BD || AC ? 0 : min(4 * g4 + 4, nsteps);
            if (RG) {
                s_lo = s_next;
                while (s_next < nsteps && sw * EW + so <= 4 * g4 + 3) {
                    s_next++;
                    if (++so == Wn) { so = 0; sw++; }
                }
                s_hi = s_next;
                step_ts(e, te, se);
            }
            if (e < S && !(EA && g4 == 0 && early)) {
                // the slot's previous step must be consumed (its marker set to 2
                // by the compute wave that read it) before it is overwritten
                if (e >= nslot) wait_flag_value(&flags[kStepMark + e - nslot], 2, flags + kPoison);
                const uint32_t gbase = m0 + (uint32_t)((g4 % G4R) * 4 * kStep);
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
                    if ((pb >> 29) == (uint32_t)j && P <= pmax) dma16(src, gbase + (uint32_t)(b << 10));
                }
            }
            if (g4 == 0) clear_flags_and_meet();
            if (e < S) dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kStepMark + e)), lane);
            for (int s2 = s_lo; s2 < s_hi; s2++) {
                // the segment's slot must be released by all nsub steps of its
                // previous segment
                if (RG && s2 >= na) wait_flag_value(&flags[kSegCount + s2 - na], nsub, flags + kPoison);
                const uint32_t dst = lds0 + (uint32_t)(kFlagBytes + seg_off(s2));
#pragma unroll
                for (int q = 0; q < kASlots; q++) {
                    const int qa = j + 4 * q;
                    if (qa >= IA) break;
                    if (aon[q]) dma16(asrc[q] + (uint32_t)(512 * G * s2), dst + (uint32_t)(qa << 10));
                }
            }
            for (int s2 = s_lo; s2 < s_hi; s2++)
                dma_marker(g_marker_src + lane, lds0 + (uint32_t)(4 * (kAMark + 4 * s2 + j)), lane);
            if (!RG) {
                se += 4;
                while (se >= nsteps) { se -= nsteps; te++; }
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        asm volatile("" :: "v"(warm));
        if constexpr (DEP) {
            // off the compute waves' path: once this workgroup is past its
            // wait, count it; the last of the dep_users waiting workgroups
            // takes the counts and the release flags back to zero for the next
            // launch
            if (wave == 0) {
                wait_flag(&flags[kDepFlag], flags + kPoison);
                // this workgroup's wait gave up (or found the word set): keep
                // every later launch on the workspace from trusting its flags
                if (poisoned(flags + kPoison) && lane == 0)
                    __hip_atomic_store(dep + kDepPoison, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                unsigned old = 0;
                if (lane == 0) old = __hip_atomic_fetch_add(dep + 64, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if ((unsigned)__builtin_amdgcn_readfirstlane(old) == dep_users - 1u) {
                    if (lane < kDepLines) __hip_atomic_store(dep + kDepLine0 + 64 * lane, 0u, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT);
                    if (lane == 0) {
                        __hip_atomic_fetch_sub(dep, dep_n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_fetch_sub(dep + 64, dep_users, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
        return;
    }

    // ---------------------------------------------------------------- compute wave
    // Steps are taken in step order, which is roughly the order in which they
    // land.  Each step's partial sums go to the step's own slot; the slots of a
    // sub-tile are added in step order (a fixed order: results do not depend on
    // timing) and stored.

    // Q4_K runs in the factored form sum_k a_k w_k = d * sum_k a_k (sc q_k)
    // - dmin * sum_j m_j S_j over the sub-blocks j of a super-block, where
    // S_j = sum_{k in j} a_k.  The block sums are tabulated per segment by the
    // wave that takes the segment's first step (the others wait for its flag;
    // at batch 1 all waves tabulate everything before the first step): entry
    // (m, sg, kg) covers sub-blocks 2kg, 2kg+1 of super-group sg of batch
    // row m:
    //   MFMA form: fp16 {hi_0, hi_1, lo_0, lo_1} with S / 32 = hi + lo / 2048 (hi
    //     is S / 32 rounded to fp16, lo the rounded remainder: S to about 2^-22);
    //   sub-block rows form (BD): fp32 {S_0, S_1}, and the entry's 128 bytes of
    //     activations are reordered in place, each run of eight to
    //     a0 a2 a1 a3 a4 a6 a5 a7, the order in which that form decodes codes.
    if constexpr (BD) {
        // batch 1: the compute waves load A (row 0: 33 nsg pieces, contiguous in
        // LDS) before the barrier, c, c + NC, ... of its 1 KB instructions from a
        // per-workgroup offset (the workgroups all read the same lines), and
        // raise a flag once their own loads are complete
        const int cw = wave - NL, nA = (nsg * 33 + 63) >> 6;
        const int rot = (int)(((unsigned)bid * 7u) % (unsigned)nA);
        if constexpr (DEP) {
            clear_flags_and_meet();
            wait_dep();
        }
        for (int i0 = cw; i0 < nA; i0 += NC) {
            const int i = i0 + rot < nA ? i0 + rot : i0 + rot - nA;
            const int P = 64 * i + lane;
            const int sg = min(P / 33, nsg - 1), c = min(P - 33 * (P / 33), 31);
            if constexpr (SW && DEP) {
                if (P < nsg * 33) *(u4*)(lds + kFlagBytes + 1024 * i + 16 * lane) = swiglu_dep(256 * sg + 8 * c);
            } else if constexpr (SW) {
                if (P < nsg * 33)
                    *(u4*)(lds + kFlagBytes + 1024 * i + 16 * lane) = swiglu8(A + 256 * sg + 8 * c, A + K + 256 * sg + 8 * c);
            } else if constexpr (AF) {
                if (P < nsg * 33)
                    *(u4*)(lds + kFlagBytes + 1024 * i + 16 * lane) =
                        f32x8_to_f16((const float*)(const void*)A + 256 * sg + 8 * c);
            } else {
                if (P < nsg * 33) dma16(A + 256 * sg + 8 * c, lds0 + (uint32_t)(kFlagBytes + 1024 * i));
            }
        }
        if constexpr (!DEP) clear_flags_and_meet();
        signal_own_loads(&flags[cw], lane);
        wait_flags(flags, NC, lane, flags + kPoison);
    } else if constexpr (AC) {
        // small A, all of it resident: the compute waves load it (instruction
        // f = s * IA + i: piece 64 i + lane of segment s; wave c issues c, c + NC,
        // ...) so that the loaders stream weights only, then wait for all of it
        const int cw = wave - NL;
        const int PA = M * G * 33, IA = (PA + 63) >> 6;
        if constexpr (DEP) {
            clear_flags_and_meet();
            wait_dep();
        }
        for (int f = cw; f < nsteps * IA; f += NC) {
            const int sg = f / IA, i = f - sg * IA;
            const uint32_t P = 64u * i + lane;
            const uint32_t m = P / (33u * G), rem = P - 33u * G * m, gg = rem / 33u, c = rem - 33u * gg;
            const int64_t elem = (int64_t)min((int)m, M - 1) * lda + 256 * (G * sg + gg) + 8 * min((int)c, 31);
            const uint16_t* src = A + elem;
            if constexpr (SW && DEP) {
                if (P < (uint32_t)PA && c < 32)
                    *(u4*)(lds + kFlagBytes + sg * seg_bytes + (i << 10) + 16 * lane) = swiglu_dep(elem);
            } else if constexpr (SW) {
                if (P < (uint32_t)PA && c < 32)
                    *(u4*)(lds + kFlagBytes + sg * seg_bytes + (i << 10) + 16 * lane) = swiglu8(src, src + K);
            } else if constexpr (AF) {
                if (P < (uint32_t)PA && c < 32)
                    *(u4*)(lds + kFlagBytes + sg * seg_bytes + (i << 10) + 16 * lane) =
                        f32x8_to_f16((const float*)(const void*)A + elem);
            } else {
                if (P < (uint32_t)PA && c < 32) dma16(src, lds0 + (uint32_t)(kFlagBytes + sg * seg_bytes + (i << 10)));
            }
        }
        if constexpr (!DEP) clear_flags_and_meet();
        signal_own_loads(&flags[cw], lane);
        wait_flags(flags, NC, lane, flags + kPoison);
    } else {
        clear_flags_and_meet();
    }
    uint8_t* const tab = (uint8_t*)(parts + S * SLOT);
    // entries u0, u0 + ustep, ... < u_end of the list ordered (segment, row m,
    // super-group gg of the segment, k-group kq); a segment has M * G * 4
    auto build_table = [&](int u0, int u_end, int ustep) {
        const h2 one = {(_Float16)1.0f, (_Float16)1.0f};
        for (int u = u0; u < u_end; u += ustep) {
            const int kq = u & 3, rest = u >> 2, s_seg = rest / (M * G), mg4 = rest - s_seg * (M * G);
            const int m = mg4 / G, gg = mg4 - m * G;
            uint8_t* src = a_lds + seg_off(s_seg) + (m * G + gg) * 528 + 128 * kq;
            u4 v[8];
#pragma unroll
            for (int q = 0; q < 8; q++) v[q] = *(const u4*)(src + 16 * q);
            float sum[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                float acc = 0.f;
#pragma unroll
                for (int q = 4 * h; q < 4 * h + 4; q++) {
                    acc = __builtin_amdgcn_fdot2(as_h2(v[q].x), one, acc, false);
                    acc = __builtin_amdgcn_fdot2(as_h2(v[q].y), one, acc, false);
                    acc = __builtin_amdgcn_fdot2(as_h2(v[q].z), one, acc, false);
                    acc = __builtin_amdgcn_fdot2(as_h2(v[q].w), one, acc, false);
                }
                sum[h] = acc;
            }
            if constexpr (BD) {
                // 16-byte slot j of the entry = the operand of codes word pair t = j % 4
                // (low nibbles for j < 4, high for j >= 4), in the decode order
                // 0 2 1 3 4 6 5 7 of its eight code positions
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    u4 o;
                    if constexpr (QT == QT_PLANES) {
                        // code byte b of the run holds weights 2b (low) and 2b+1 (high)
                        const int t = j & 3;
                        const uint32_t sel = j < 4 ? 0x05040100u : 0x07060302u;
                        const u4 x = v[2 * t], y = v[2 * t + 1];
                        o = u4{perm_b32(x.z, x.x, sel), perm_b32(x.w, x.y, sel), perm_b32(y.z, y.x, sel),
                               perm_b32(y.w, y.y, sel)};
                    } else {
                        // Q4_K: runs in order (sub-block 2kg low, 2kg+1 high nibbles);
                        // Q4_0: block 2kg's code bytes hold weights b and 16+b, block
                        // 2kg+1's 32+b and 48+b: runs 0 1 4 5 | 2 3 6 7
                        constexpr int kRun0[8] = {0, 1, 4, 5, 2, 3, 6, 7};
                        const u4 x = v[QT == QT_Q4_K ? j : kRun0[j]];
                        o = u4{perm_b32(x.y, x.x, 0x05040100u), perm_b32(x.y, x.x, 0x07060302u),
                               perm_b32(x.w, x.z, 0x05040100u), perm_b32(x.w, x.z, 0x07060302u)};
                    }
                    *(u4*)(src + 16 * j) = o;
                }
            }
            uint32_t* dst = (uint32_t*)(tab + ((m * nsg + G * s_seg + gg) * 4 + kq) * 8);
            if constexpr (BD) {
                dst[0] = __builtin_bit_cast(uint32_t, sum[0]);
                dst[1] = __builtin_bit_cast(uint32_t, sum[1]);
            } else {
                uint32_t hi[2], lo[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const float mean = sum[h] * 0.03125f;
                    const _Float16 mh = (_Float16)mean;
                    const _Float16 ml = (_Float16)((mean - (float)mh) * 2048.0f);
                    hi[h] = __builtin_bit_cast(uint16_t, mh);
                    lo[h] = __builtin_bit_cast(uint16_t, ml);
                }
                dst[0] = hi[0] | (hi[1] << 16);
                dst[1] = lo[0] | (lo[1] << 16);
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };

    if constexpr (BD) {
        // batch 1: all of A (10 KB at K = 5120) at once, tabulated before the first step
        build_table((wave - NL) * 64 + lane, nsteps * M * G * 4, NC * 64);
        if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[wave - NL])), "v"(2) : "memory");
        wait_flags(flags, NC, lane, flags + kPoison, 2);
    }

    const Magic mg = make_magic();
    const int r = lane & 15, kg = lane >> 4;
    const int g = r % G, rowl = r / G;
    int arow[MT];                                      // this lane's A fragment within a segment
    const uint8_t* trow[MT];                           // this lane's block-sum entries (Q4_K)
    // sub-block rows form: MFMA row r = 4 kappa + g takes the activations of
    // segment g from the k slots of lane group kappa only (zeros elsewhere), so
    // that row holds the partial sums of one sub-block per column
    const bool bd_on = (r >> 2) == kg;
    // sub-block rows form: the activation operands stay zero in the lanes off
    // the block diagonal; only the 16 lanes on it read them (exec-masked)
    h8 abd[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < 8; t++) abd[mt][t] = h8{};
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = BD ? min(mt, M - 1) : min(mt * R + r / G, M - 1);   // padding rows reread row M-1
        arow[mt] = (m * G + g) * 528 + 128 * kg;
        trow[mt] = tab + ((m * nsg + g) * 4 + kg) * 8;
    }

    // Steps in the order in which they land: batch 1 (sub-block rows form):
    // compute wave c takes steps c, c + NC, ...; otherwise a free wave takes the
    // next step from the shared counter.
    int e_static = wave - NL;
    for (;;) {
        int e = 0;
        if constexpr (BD) {
            e = e_static;
            e_static += NC;
        } else {
            if (lane == 0)
                asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                             : "=v"(e) : "v"(lds_addr(&flags[kStepCounter])), "v"(1) : "memory");
            e = __builtin_amdgcn_readfirstlane(e);
        }
        if (e >= S) break;
        int t_in = 0, s_in = 0;
        step_ts(e, t_in, s_in);
        if constexpr (!BD) {
            // the segment's block sums: tabulated by the wave of its first step
            // once the segment has landed
            // The step's flags in one LDS round trip (lanes 0-3 its segment's
            // activation markers, lane 4 its own marker, lane 5 for Q4_K the
            // segment's block-sum flag), or one after the other: Q4_K with two
            // m-tiles or the rings measured faster with three round trips.
            constexpr bool kMerged = !(QT == QT_Q4_K && (MT == 2 || RG));
            if (!AC && (!kMerged || (QT == QT_Q4_K && t_in == 0))) wait_flags(flags + kAMark + 4 * s_in, NL, lane, flags + kPoison);
            if (QT == QT_Q4_K && t_in == 0) {
                build_table(s_in * M * G * 4 + lane, (s_in + 1) * M * G * 4, 64);
                if (lane == 0)
                    asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kTabFlag + s_in])), "v"(1) : "memory");
            }
            if (kMerged) {
                const int* f = lane < NL ? flags + kAMark + 4 * s_in + lane
                                         : lane == NL ? flags + kStepMark + e : flags + kTabFlag + s_in;
                wait_lanes(f, (lane <= NL && (!AC || lane == NL)) || (QT == QT_Q4_K && lane == NL + 1), flags + kPoison);
            } else {
                if (t_in != 0) wait_flag(&flags[kTabFlag + s_in], flags + kPoison);
                wait_flag(&flags[kStepMark + e], flags + kPoison);
            }
        }
        Raw<QT> raw;
        const uint8_t* const aseg = a_lds + seg_off(s_in);
        if constexpr (BD) {
            // the step's marker with the step's weight and activation reads right
            // behind it: a wave's LDS reads complete in order, so a nonzero marker
            // means the reads behind it saw the landed step (one round trip).  Only
            // the first poll carries the data reads: a wave that finds the step not
            // landed polls the marker alone and reads the step once it is set (each
            // poll's data reads would take LDS bandwidth from the loaders' stream)
            const uint8_t* const wstep = w_lds + (e - (int)(((uint32_t)e * inv_nslot) >> 16) * nslot) * kStep + r * 144;
            auto read_step = [&]() __attribute__((always_inline)) {
                lds_raw<QT>(raw, wstep, kg);
                if (bd_on) {
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
#pragma unroll
                        for (int t = 0; t < 8; t++) abd[mt][t] = *(const h8*)(aseg + arow[mt] + 16 * t);
                }
            };
            bool first = true;
            for (int it = 0;; it++) {
                int mark;
                asm volatile("ds_read_b32 %0, %1" : "=v"(mark) : "v"(lds_addr(&flags[kStepMark + e])) : "memory");
                if (it == 0) read_step();
                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(mark) :: "memory");
                if (__builtin_amdgcn_readfirstlane(mark) != 0) {
                    first = it == 0;
                    break;
                }
                if (it >= kWaitBound) {
                    mark_poison(flags + kPoison);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            if (!first) {
                read_step();
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            }
            // the step's slot is free again (its reads have completed)
            if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kStepMark + e])), "v"(2) : "memory");
        } else {
            lds_raw<QT>(raw, w_lds + (e - (int)(((uint32_t)e * inv_nslot) >> 16) * nslot) * kStep + r * 144, kg);
            // a wave's LDS operations complete in order: the slot is free once this
            // write is visible
            if (lane == 0) asm volatile("ds_write_b32 %0, %1" :: "v"(lds_addr(&flags[kStepMark + e])), "v"(2) : "memory");
        }
        f4 acc[MT], accm[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[mt] = accm[mt] = f4{0.f, 0.f, 0.f, 0.f};
        float d = 1.f, dmin = 0.f;
        if constexpr (BD) {
            // codes as fp16 subnormals: low nibble q -> q * 2^-24, high nibble
            // (masked in place) -> 16 q * 2^-24; exact products in the MFMA.
            // Accumulators: Q4_K {sub-block 2kg, sub-block 2kg+1} over t = 0..3;
            // Q4_0 formats {block 2kg low, high nibbles} over t = 0, 1 and
            // {block 2kg+1 low, high} over t = 2, 3 (each block has one scale)
            constexpr bool K4 = QT == QT_Q4_K;
            constexpr int NA = K4 ? 2 : 4;
            uint32_t wq[8];
            bd_code_words(raw, wq);
            f4 ab[MT][NA];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int ia = 0; ia < NA; ia++) ab[mt][ia] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; t++) {
                h8 blo, bhi;
                codes_subnormal(wq, t, blo, bhi);
                const int ia = K4 ? 0 : 2 * (t >> 1);
#pragma unroll
                for (int mt = 0; mt < MT; mt++) {
                    ab[mt][ia] = mfma16x16x32(abd[mt][t], blo, ab[mt][ia]);
                    ab[mt][ia + 1] = mfma16x16x32(abd[mt][t + 4], bhi, ab[mt][ia + 1]);
                }
            }
            float* slot = parts + e * SLOT;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                // this lane's column n = 4 rowl + g and its two blocks: MFMA row 4kg + g
                float p[NA];
#pragma unroll
                for (int ia = 0; ia < NA; ia++) {
                    p[ia] = ab[mt][ia][0];
#pragma unroll
                    for (int gg = 1; gg < 4; gg++)
                        if (g == gg) p[ia] = ab[mt][ia][gg];
                }
                const float* ts = (const float*)(trow[mt] + G * s_in * 32);
                float y;
                if constexpr (K4) {
                    const BdScl sb = scales_bd(raw, kg);
                    y = sb.d20 * __builtin_fmaf(sb.c_lo16, p[0], sb.c_hi * p[1]) -
                        sb.dmin * __builtin_fmaf(sb.m_lo, ts[0], sb.m_hi * ts[1]);
                } else {
                    // sum a (q - 8) d = d (2^20 (16 p_lo + p_hi) - 8 S) per block
                    float da20, db20;
                    bd_block_scales(raw, da20, db20);
                    // (8 d S = 2^-17 d20 S)
                    y = __builtin_fmaf(da20, __builtin_fmaf(16.0f, p[0], p[1]), db20 * __builtin_fmaf(16.0f, p[2], p[3])) -
                        0x1p-17f * __builtin_fmaf(da20, ts[0], db20 * ts[1]);
                }
                // parked per lane: the lane groups and segments are summed once per
                // sub-tile, after its steps
                slot[mt * 64 + lane] = y;
            }
        } else if constexpr (QT == QT_Q4_K) {
            const SclK sk = scales_int(raw, kg);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const h8 b = weights_int(mg, raw, sk, i);
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    acc[mt] = mfma16x16x32(*(const h8*)(aseg + arow[mt] + 16 * i), b, acc[mt]);
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
                    acc[mt] = mfma16x16x32(*(const h8*)(aseg + arow[mt] + 16 * i), b, acc[mt]);
            }
        }
        if constexpr (!BD) {
            // the step's activation reads are issued (a wave's LDS operations
            // complete in order): count it against its segment's slot
            if (a_ring && lane == 0)
                asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kSegCount + s_in])), "v"(1) : "memory");
            // fold the G segments (lanes r = G*rowl + g) and park the partial sums
            // (slots in sub-tile-major order whatever the step order)
            float* slot = parts + (t_in * nsteps + s_in) * SLOT;
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
        if constexpr (BD) {
            // count the finished step (no return value: the wave that took the
            // sub-tile's last step waits for the count after its own steps)
            if (lane == 0)
                asm volatile("ds_add_u32 %0, %1" :: "v"(lds_addr(&flags[kSubCount + t_in])), "v"(1) : "memory");
            continue;
        }
        // count the finished step; the last of the sub-tile reduces and stores it
        int old = 0;
        if (lane == 0)
            asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)"
                         : "=v"(old) : "v"(lds_addr(&flags[kSubCount + t_in])), "v"(1) : "memory");
        if (__builtin_amdgcn_readfirstlane(old) == nsteps - 1) {
            const int64_t row0 = (int64_t)(tile0 + t_in) * R;
            const bool bad = poisoned(flags + kPoison);
            for (int v = lane; v < SLOT; v += 64) {
                const float* pp = parts + t_in * nsteps * SLOT + v;
                float sum = 0.f;
                for (int s2 = 0; s2 < nsteps; s2++) sum += pp[s2 * SLOT];
                if (bad) sum = __builtin_nanf("");
                const int m = v / R, rl = v - m * R;   // m = mt * R + m_loc
                const int64_t row = row0 + rl;
                if (m < M && row < N) store_c(m, row, sum);
            }
        }
    }
    if constexpr (BD) {
        // the sub-tiles whose last step this wave took: once all their steps are
        // parked, each lane adds its parked values in step order, then the lane
        // groups (sub-block pairs) and the four segments are summed
        for (int t_in = 0; t_in < nsub; t_in++) {
            if ((t_in * nsteps + nsteps - 1) % NC != wave - NL) continue;
            wait_count(&flags[kSubCount + t_in], nsteps, flags + kPoison);
            const bool bad = poisoned(flags + kPoison);
            const int64_t row = (int64_t)(tile0 + t_in) * R + rowl;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                const float* pp = parts + t_in * nsteps * SLOT + mt * 64 + lane;
                float y = 0.f;
                for (int s2 = 0; s2 < nsteps; s2++) y += pp[s2 * SLOT];
                y = sum_lane_xor16(y);
                y = sum_lane_xor32(y);
                y += dpp_xor(y, 1);
                y += dpp_xor(y, 2);
                if (bad) y = __builtin_nanf("");
                if (g == 0 && kg == 0 && mt < M && row < N) store_c(mt, row, y);
            }
        }
    }
}

// The single-GEMM kernel's arguments fit in 14 dwords, all of which arrive in
// SGPRs at wave launch (kernel-argument preloading: 16 user SGPRs less the
// argument segment's address), so no argument is fetched with a scalar load.
// One that were would hold up the workgroup's barrier: the wait for the
// flags' LDS writes before it (lgkmcnt) also counts scalar loads, and at that
// moment a scalar load queues behind the weight stream the loaders have just
// started, so the loaders' second group of steps and every step marker would
// wait for it.  mo = M | out_f16 << 8 | nsub << 16 | win << 24, sl = nslot |
// na << 16 (lds_packed_args).
template <int QT, int G, int MT, int NC, int NL, bool BD, bool RG, bool AC = false, bool SW = false, bool AF = false,
          bool EA = false>
__global__ __launch_bounds__(64 * (NC + NL))
void k_gemm_lds(const uint8_t* __restrict__ W, const uint16_t* __restrict__ A, const uint8_t* __restrict__ Waux,
                void* __restrict__ C, int lda, int ldc, int N, int K, uint32_t mo, uint32_t sl) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    lds_body<QT, G, MT, NC, NL, BD, RG, AC, SW, false, false, AF, EA>((int)blockIdx.x, lds, W, A, lda, (int)(mo & 0xFFu), N, K,
                                                (int)((mo >> 16) & 0xFFu), (int)(sl & 0xFFFFu), (int)(sl >> 16),
                                                (int)(mo >> 24), Waux, C, ldc, (int)((mo >> 8) & 1u));
}

// Several independent GEMMs of one kernel shape in one launch (their grids
// back to back): a workgroup finds its GEMM by its id, and workgroups of a
// later GEMM start as those of an earlier one retire, so one GEMM's compute
// tail overlaps the next one's weight stream.
constexpr int kLdsMaxJobs = 8;
struct LdsJob {
    const uint8_t* W;
    const uint8_t* Waux;
    const uint16_t* A;
    void* C;
    int lda, ldc, M, N, K, nsub, nslot, na, win, grid0;
};
struct LdsJobs {
    LdsJob job[kLdsMaxJobs];
    int n, out_f16;
};

template <int QT, int G, int MT, int NC, int NL, bool BD, bool RG>
__global__ __launch_bounds__(64 * (NC + NL))
void k_gemm_lds_batched(const LdsJobs jobs) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    LdsJob j = jobs.job[0];
#pragma unroll
    for (int i = 1; i < kLdsMaxJobs; i++)
        if (i < jobs.n && (int)blockIdx.x >= jobs.job[i].grid0) j = jobs.job[i];
    lds_body<QT, G, MT, NC, NL, BD, RG, false>((int)blockIdx.x - j.grid0, lds, j.W, j.A, j.lda, j.M, j.N, j.K, j.nsub, j.nslot,
                                    j.na, j.win, j.Waux, j.C, j.ldc, jobs.out_f16);
}

constexpr int kNC = 12, kNL = 4;      // compute and loader waves per workgroup

LdsShape lds_shape(const GemmArgs& g) { return LdsShape{g.M, g.N, g.K, g.qtype == QT_Q4_K}; }

// The kernel's packed arguments (k_gemm_lds); false if a field does not fit
// (no plan makes such a field: M <= 16, nsub <= 128, win <= 96, nslot <= 240,
// na <= 96).
bool lds_packed_args(const GemmArgs& g, const LdsPlan& p, uint32_t& mo, uint32_t& sl) {
    if (g.M < 0 || g.M > 255 || p.nsub < 0 || p.nsub > 255 || p.win < 0 || p.win > 255 || p.nslot < 0 ||
        p.nslot > 0xFFFF || p.na < 0 || p.na > 0xFFFF)
        return false;
    mo = (uint32_t)g.M | (uint32_t)(g.out_f16 ? 1 : 0) << 8 | (uint32_t)p.nsub << 16 | (uint32_t)p.win << 24;
    sl = (uint32_t)p.nslot | (uint32_t)p.na << 16;
    return true;
}

template <int QT, int G, int MT, bool BD = false, bool RG = false, bool AC = false, bool SW = false, bool AF = false,
          bool EA = false>
hipError_t launch_lds(const GemmArgs& g, const LdsPlan& p, hipStream_t st) {
    auto k = k_gemm_lds<QT, G, MT, kNC, kNL, BD, RG, AC, SW, AF, EA>;
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
    uint32_t mo = 0, sl = 0;
    if (!lds_packed_args(g, p, mo, sl)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k, dim3(p.grid), dim3(64 * (kNC + kNL)), p.lds, st, g.W, g.A, g.Waux, g.C, g.lda, g.ldc, g.N,
                       g.K, mo, sl);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_lds(const GemmArgs& g, const LdsPlan& p, hipStream_t st) {
    // Q4_K, every step in a slot of its own (no step ring): the loaders' first
    // group early (the Q4_0 formats measured slower with it: 5120^2 at M = 1 /
    // 8 planes 6.23 / 7.95 -> 6.41 / 8.05-8.48 us, Q4_0 blocks at M = 8 7.84 ->
    // 8.16 us)
    const bool ea = QT == QT_Q4_K && p.nslot >= p.nsub * (g.K / (256 * p.G));
    if (g.a_f32) {
        if (p.BD) return ea ? launch_lds<QT, 4, 1, true, false, false, false, true, true>(g, p, st)
                            : launch_lds<QT, 4, 1, true, false, false, false, true>(g, p, st);
        if (p.AC) return ea ? launch_lds<QT, 4, 1, false, false, true, false, true, true>(g, p, st)
                            : launch_lds<QT, 4, 1, false, false, true, false, true>(g, p, st);
        return hipErrorInvalidValue;
    }
    if (p.BD) return ea ? launch_lds<QT, 4, 1, true, false, false, false, false, true>(g, p, st)
                        : launch_lds<QT, 4, 1, true>(g, p, st);
    if (p.RG) {
        if (p.G == 4 && p.MT == 1) return launch_lds<QT, 4, 1, false, true>(g, p, st);
        if (p.G == 4 && p.MT == 2) return launch_lds<QT, 4, 2, false, true>(g, p, st);
        if (p.G == 2 && p.MT == 1) return launch_lds<QT, 2, 1, false, true>(g, p, st);
        return hipErrorInvalidValue;                    // no ring kernel of this shape
    }
    if (p.AC) return ea ? launch_lds<QT, 4, 1, false, false, true, false, false, true>(g, p, st)
                        : launch_lds<QT, 4, 1, false, false, true>(g, p, st);
    if (p.G == 4 && p.MT == 1) return ea ? launch_lds<QT, 4, 1, false, false, false, false, false, true>(g, p, st)
                                         : launch_lds<QT, 4, 1>(g, p, st);
    if (p.G == 4 && p.MT == 2) return ea ? launch_lds<QT, 4, 2, false, false, false, false, false, true>(g, p, st)
                                         : launch_lds<QT, 4, 2>(g, p, st);
    if (p.G == 2 && p.MT == 1) return launch_lds<QT, 2, 1>(g, p, st);
    return launch_lds<QT, 1, 1>(g, p, st);
}

template <int QT, int G, int MT, bool BD, bool RG>
hipError_t launch_lds_batched(const GemmArgs* gs, const LdsPlan* ps, int n, hipStream_t st) {
    auto k = k_gemm_lds_batched<QT, G, MT, kNC, kNL, BD, RG>;
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
    LdsJobs jobs = {};
    jobs.n = n;
    jobs.out_f16 = gs[0].out_f16;
    int grid = 0, lds = 0;
    for (int i = 0; i < n; i++) {
        const GemmArgs& g = gs[i];
        jobs.job[i] = LdsJob{g.W, g.Waux, g.A, g.C, g.lda, g.ldc, g.M, g.N, g.K, ps[i].nsub, ps[i].nslot,
                             ps[i].na, ps[i].win, grid};
        grid += ps[i].grid;
        lds = std::max(lds, ps[i].lds);
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(64 * (kNC + kNL)), lds, st, jobs);
    return hipGetLastError();
}

// The kernel shapes that have a batched launch: batch 1 (sub-block rows) and
// G = 4 with one or two m-tiles (batch 2-8).
bool lds_batchable(const LdsPlan& p) { return p.G == 4 && (p.BD || p.MT <= 2); }

template <int QT>
hipError_t dispatch_lds_batched(const GemmArgs* gs, const LdsPlan* ps, int n, hipStream_t st) {
    if (ps[0].BD) return launch_lds_batched<QT, 4, 1, true, false>(gs, ps, n, st);
    // one job with the rings: all take the ring kernel (which runs the others'
    // plans, win = na = all segments, in the plain order)
    bool rg = false;
    for (int i = 0; i < n; i++) rg = rg || ps[i].RG;
    if (rg) {
        if (ps[0].MT == 1) return launch_lds_batched<QT, 4, 1, false, true>(gs, ps, n, st);
        return launch_lds_batched<QT, 4, 2, false, true>(gs, ps, n, st);
    }
    if (ps[0].MT == 1) return launch_lds_batched<QT, 4, 1, false, false>(gs, ps, n, st);
    return launch_lds_batched<QT, 4, 2, false, false>(gs, ps, n, st);
}

// The SwiGLU feed-forward block in one launch: the gate and up projections
// (jobs 0 and 1, fp16 outputs into the two halves of one gate|up buffer) and
// the down projection (job 2) over SiLU(gate) * up, formed as its compute
// waves load it.  Workgroups [0, g01) run the gate and up GEMMs with
// device-scope stores and count themselves in cnt[0] once those have landed;
// the last raises the release flags.  The down projection's workgroups start
// their weight stream at once and wait for a release flag before they load
// the activations.  Workgroups are dispatched
// in id order, so every producer has started before any consumer waits, and
// producers never wait on consumers: the launch cannot deadlock, whatever the
// number of CUs.  The last down workgroup past its wait takes both counts back
// (cnt[64] counts those workgroups), so the next launch that uses the
// workspace finds them at zero.
template <int QT, bool BD>
__global__ __launch_bounds__(64 * (kNC + kNL))
void k_ffn_lds(const LdsJobs jobs, unsigned* cnt) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
    constexpr bool AC = !BD;
    const int b = (int)blockIdx.x;
    const int g01 = jobs.job[2].grid0;
    if (b < g01) {
        LdsJob j = jobs.job[0];
        if (b >= jobs.job[1].grid0) j = jobs.job[1];
        lds_body<QT, 4, 1, kNC, kNL, BD, false, AC, false, false, true>(b - j.grid0, lds, j.W, j.A, j.lda, j.M, j.N,
                                                                         j.K, j.nsub, j.nslot, j.na, j.win, j.Waux,
                                                                         j.C, j.ldc, 1);
        // every wave's device-scope stores have reached the point of coherence
        // before the workgroup counts itself; the last producer raises the
        // release flags
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x < 64) {
            unsigned old = 0;
            if (threadIdx.x == 0) old = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((unsigned)__builtin_amdgcn_readfirstlane(old) == (unsigned)g01 - 1u && threadIdx.x < kDepLines)
                __hip_atomic_store(cnt + kDepLine0 + 64 * threadIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    const LdsJob j = jobs.job[2];
    lds_body<QT, 4, 1, kNC, kNL, BD, false, AC, true, true>(b - g01, lds, j.W, j.A, j.lda, j.M, j.N, j.K, j.nsub,
                                                            j.nslot, j.na, j.win, j.Waux, j.C, j.ldc, jobs.out_f16,
                                                            cnt, (unsigned)g01, gridDim.x - (unsigned)g01);
}

// Plans of the three GEMMs when the one-launch block serves them: batch 1
// (sub-block rows form everywhere) or batch 2 (G = 4, one m-tile, all of A
// resident, loaded by the compute waves).
bool ffn_plans(const GemmArgs* gs, LdsPlan* ps) {
    const int M = gs[2].M;
    if (M > 2) return false;
    for (int i = 0; i < 3; i++) {
        if (gs[i].M != M || gs[i].qtype != gs[2].qtype) return false;
        if (gs[i].qtype == QT_PLANES && ((uintptr_t)gs[i].Waux & 15)) return false;
        if (!choose_lds(lds_shape(gs[i]), ps[i])) return false;
        const LdsPlan& p = ps[i];
        if (M == 1 ? !p.BD : (p.BD || p.RG || p.G != 4 || p.MT != 1 || p.na != gs[i].K / 1024)) return false;
    }
    return true;
}

template <int QT, bool BD>
hipError_t launch_ffn(const GemmArgs* gs, const LdsPlan* ps, unsigned* cnt, hipStream_t st) {
    auto k = k_ffn_lds<QT, BD>;
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
    LdsJobs jobs = {};
    jobs.n = 3;
    jobs.out_f16 = gs[2].out_f16;
    int grid = 0, lds = 0;
    for (int i = 0; i < 3; i++) {
        const GemmArgs& g = gs[i];
        jobs.job[i] = LdsJob{g.W, g.Waux, g.A, g.C, g.lda, g.ldc, g.M, g.N, g.K, ps[i].nsub, ps[i].nslot,
                             ps[i].na, ps[i].win, grid};
        grid += ps[i].grid;
        lds = std::max(lds, ps[i].lds);
    }
    hipLaunchKernelGGL(k, dim3(grid), dim3(64 * (kNC + kNL)), lds, st, jobs, cnt);
    return hipGetLastError();
}

template <int QT>
hipError_t dispatch_ffn(const GemmArgs* gs, const LdsPlan* ps, unsigned* cnt, hipStream_t st) {
    if (ps[0].BD) return launch_ffn<QT, true>(gs, ps, cnt, st);
    return launch_ffn<QT, false>(gs, ps, cnt, st);
}

}  // namespace

bool ffn_lds_supports(const GemmArgs* gs) {
    LdsPlan ps[3];
    return ffn_plans(gs, ps);
}

hipError_t ffn_lds(const GemmArgs* gs, hipStream_t st) {
    LdsPlan ps[3];
    if (!ffn_plans(gs, ps)) return hipErrorInvalidValue;
    // the dependency words at the start of the stream's workspace (left at
    // zero by every launch that uses them)
    unsigned* cnt = nullptr;
    float* unused = nullptr;
    hipError_t e = split_workspace(nullptr, st, kDepWords * 4, 0, &cnt, &unused);
    if (e != hipSuccess) return e;
    switch (gs[0].qtype) {
        case QT_Q4_K: return dispatch_ffn<QT_Q4_K>(gs, ps, cnt, st);
        case QT_PLANES: return dispatch_ffn<QT_PLANES>(gs, ps, cnt, st);
        default: return dispatch_ffn<QT_Q4_0>(gs, ps, cnt, st);
    }
}

bool lds_batched_supports(const GemmArgs* gs, int n) {
    if (n < 1) return false;
    LdsPlan p0;
    for (int i = 0; i < n; i++) {
        LdsPlan p;
        if (gs[i].qtype != gs[0].qtype || gs[i].out_f16 != gs[0].out_f16) return false;
        if (gs[i].qtype == QT_PLANES && ((uintptr_t)gs[i].Waux & 15)) return false;
        if (!choose_lds(lds_shape(gs[i]), p) || !lds_batchable(p)) return false;
        if (i == 0) p0 = p;
        else if (p.G != p0.G || p.MT != p0.MT || p.BD != p0.BD) return false;
    }
    return true;
}

hipError_t gemm_lds_batched(const GemmArgs* gs, int n, hipStream_t st) {
    if (!lds_batched_supports(gs, n)) return hipErrorInvalidValue;
    for (int i0 = 0; i0 < n; i0 += kLdsMaxJobs) {
        const int m = std::min(kLdsMaxJobs, n - i0);
        LdsPlan ps[kLdsMaxJobs];
        for (int i = 0; i < m; i++) choose_lds(lds_shape(gs[i0 + i]), ps[i]);
        hipError_t e;
        switch (gs[0].qtype) {
            case QT_Q4_K: e = dispatch_lds_batched<QT_Q4_K>(gs + i0, ps, m, st); break;
            case QT_PLANES: e = dispatch_lds_batched<QT_PLANES>(gs + i0, ps, m, st); break;
            default: e = dispatch_lds_batched<QT_Q4_0>(gs + i0, ps, m, st); break;
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// The fused SiLU-times-up GEMM (A = the gate|up output, K columns each): the
// batch-1 kernel or the one whose compute waves load all of A (the only ones
// that read A through the compute waves, where it can be transformed).
bool lds_swiglu_plan(const GemmArgs& g, LdsPlan& p) {
    if (g.M > 2 || !choose_lds(lds_shape(g), p)) return false;
    return p.BD || (!p.RG && p.G == 4 && p.MT == 1 && p.na == g.K / 1024);
}

bool lds_swiglu_supports(const GemmArgs& g) {
    LdsPlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return lds_swiglu_plan(g, p);
}

template <int QT>
hipError_t dispatch_lds_swiglu(const GemmArgs& g, const LdsPlan& p, hipStream_t st) {
    if (p.BD) return launch_lds<QT, 4, 1, true, false, false, true>(g, p, st);
    return launch_lds<QT, 4, 1, false, false, true, true>(g, p, st);
}

hipError_t gemm_lds_swiglu(const GemmArgs& g, hipStream_t st) {
    LdsPlan p;
    if (!lds_swiglu_plan(g, p)) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_lds_swiglu<QT_Q4_K>(g, p, st);
        case QT_PLANES: return dispatch_lds_swiglu<QT_PLANES>(g, p, st);
        default: return dispatch_lds_swiglu<QT_Q4_0>(g, p, st);
    }
}

bool lds_supports(const GemmArgs& g) {
    LdsPlan p;
    if (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15)) return false;
    return choose_lds(lds_shape(g), p);
}

bool lds_f32_supports(const GemmArgs& g) {
    LdsPlan p;
    if (((uintptr_t)g.A & 15) || (g.lda & 3) || (g.qtype == QT_PLANES && ((uintptr_t)g.Waux & 15))) return false;
    return choose_lds(lds_shape(g), p) && (p.BD || p.AC);
}

hipError_t gemm_lds(const GemmArgs& g, hipStream_t st) {
    LdsPlan p;
    if (!choose_lds(lds_shape(g), p)) return hipErrorInvalidValue;
    switch (g.qtype) {
        case QT_Q4_K: return dispatch_lds<QT_Q4_K>(g, p, st);
        case QT_PLANES: return dispatch_lds<QT_PLANES>(g, p, st);
        default: return dispatch_lds<QT_Q4_0>(g, p, st);
    }
}

}  // namespace bf
