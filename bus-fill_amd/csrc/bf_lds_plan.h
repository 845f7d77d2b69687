// Plan of the LDS-staged GEMM (bf_gemm_lds.hip): the LDS layout constants,
// how many sub-tiles a workgroup takes, and the step and activation rings.
// Plain C++ without HIP: the kernel file includes it, and so does the CPU check
// of every plan (tests/lds_plan_check.cpp), which runs a model of the loader
// and compute waves' protocol on the plans this code makes.
#pragma once

#include <algorithm>
#include <cstdint>

namespace bf {

inline constexpr int kStep = 16 * 144;          // bytes of one step
inline constexpr int kMaxLds = 160 * 1024;      // LDS per workgroup on gfx950

// LDS layout: [0, 4096) flags (ints): the compute waves' next-step counter at
// 15; activation markers of loader j for segment s at 16 + 4s + j; block-sum
// table flag of segment s at 400 + s; step markers at 512 + e; finished-step
// counters of sub-tile t at 768 + t; steps done with activation segment s at
// 896 + s (activation ring only).  Then the
// activations, segment-major: segment s (super-groups G s .. G s + G - 1) at
// s * seg_bytes, its batch row m at m * G * 528, super-group g at g * 528;
// then the W steps of the workgroup in order (2304 bytes each); then one
// parked partial per step; then (Q4_K) the activation block sums, 32 bytes per
// batch row and super-group.  When the steps do not all fit, the W steps
// region is a ring of nslot step slots (whole groups of four steps); when the
// activations do not all fit either (batch 3-8 at K = 17408), they are a ring
// of na segment slots and the steps run in windows of `win` segments (in each
// window every sub-tile in turn takes the window's segments), so that each
// segment is released after its nsub steps.
inline constexpr int kFlagBytes = 4096;
inline constexpr int kAMark = 16, kMaxSeg = 96;
inline constexpr int kTabFlag = 400;
inline constexpr int kStepMark = 512, kMaxSteps = 240;
inline constexpr int kSubCount = 768, kMaxSub = 128;
inline constexpr int kSegCount = 896;                    // steps done with activation segment s, at 896 + s
inline constexpr int kStepCounter = 15;                  // flags[15]: next step to take
inline constexpr int kPoison = 13;                       // flags[13]: a bounded wait gave up (results become NaN)
inline constexpr int kDepFlag = 14;                      // flags[14]: the activations' producers are done (one launch, two phases)
inline constexpr int kASlots = 6;                        // activation instructions per loader and segment
inline constexpr int kMinRing = 16;                      // fewest steps in a ring of reused step slots
inline constexpr int kRingAhead = 16;                    // steps of lead that keep the weight stream going
inline constexpr int kAcMaxBytes = 20480;                // A per workgroup that the compute waves load (AC)

// A GEMM as the planner sees it.
struct LdsShape {
    int M, N, K;
    bool q4k;                          // Q4_K (block-sum table in the MFMA form)
};

struct LdsPlan {
    int G, MT, nsub, nslot, na, win, grid, lds;
    bool RG;                           // window order and activation ring (win or na < steps per sub-tile)
    bool AC;                           // the compute waves load all of A up front (loaders: weights only)
    bool BD;                           // sub-block rows form (Q4_K, one batch row per m-tile)
};

// Steps in windows of wn segments (each sub-tile in turn takes the window's
// segments) with na activation slots: the fewest steps by which the loaders can
// run ahead of the compute waves, or 0 unless every slot is released by a step
// of an earlier group of four -- the slot of segment s is released by the last
// step of segment s - na, and segment s is loaded in the group of its first
// step, after that group's steps.  (A release in a later group would deadlock;
// one in the same group would not, each loader issuing its step before it
// waits, but leaves the loaders no lead.)
inline int ring_ahead(int nsteps, int nsub, int wn, int na) {
    const int ew = nsub * wn;
    auto first = [&](int sg) { return (sg / wn) * ew + sg % wn; };
    auto last = [&](int sg) {
        const int w = sg / wn, width = std::min(wn, nsteps - w * wn);
        return w * ew + (nsub - 1) * width + sg % wn;
    };
    int ahead = 1 << 30;
    for (int sg = na; sg < nsteps; sg++) {
        if (last(sg - na) / 4 >= first(sg) / 4) return 0;
        ahead = std::min(ahead, first(sg) - last(sg - na));
    }
    return ahead;
}

// Sub-tiles per workgroup: about one workgroup per CU when the LDS holds all of
// its steps, otherwise the fewest rounds of 256 workgroups that fit.  With one
// round only, the weight steps may be a ring of reused slots, and (MFMA form,
// aring) the activation segments too, the steps then run in windows.
inline bool plan_lds(const LdsShape& g, int G, int MT, LdsPlan& p, bool BD = false, bool aring = false) {
    const int nsg = g.K / 256;
    if (nsg % G) return false;
    const int nsteps = nsg / G, R = 16 / G;
    if (BD ? (G != 4 || g.M > MT) : g.M > MT * R) return false;
    p.BD = BD;
    const int T = (g.N + R - 1) / R;
    p.G = G;
    p.MT = MT;
    // activation segments of G super-groups x M rows (528-byte super-group images:
    // the 16 lanes of a k-group read 16 distinct bank groups for G = 1, 2, 4)
    if (nsteps > kMaxSeg || g.M * G > 32) return false;
    const int64_t seg = (int64_t)g.M * G * 528;
    for (int rounds = 1; rounds <= 64; rounds++) {
        const int nsub = (T + 256 * rounds - 1) / (256 * rounds);
        const int S = nsub * nsteps;
        if (S > kMaxSteps || nsub > kMaxSub) continue;
        const int64_t tab = g.q4k || BD ? (int64_t)g.M * nsg * 32 : 0;   // block sums
        const int64_t slot = BD ? MT * 64 : MT * R * R;
        const int64_t base = kFlagBytes + (int64_t)S * slot * 4 + tab;
        // step slots left beside na activation segments (whole groups of four)
        auto ring = [&](int na) {
            const int64_t f = base + na * seg;
            return f < kMaxLds ? (int)((kMaxLds - f) / kStep) & ~3 : 0;
        };
        int na = nsteps, nslot = S, win = nsteps;
        if (base + nsteps * seg + (int64_t)S * kStep > kMaxLds) {
            // a second round of workgroups costs more than a ring saves
            nslot = rounds == 1 ? ring(nsteps) : 0;
            if (nslot < kMinRing && rounds == 1 && aring && !BD) {
                // both rings, steps in windows of wn segments (whole rows of
                // 576 wn bytes per step run: wn = 4 when it keeps the loaders far
                // enough ahead, else the farthest)
                int best = 0;
                for (int wn : {4, 2, 1}) {
                    if (wn > nsteps) continue;
                    for (int a = wn + 1; a < nsteps; a++) {
                        const int rs = std::min(ring(a), S);
                        if (rs < kMinRing && rs < S) continue;
                        const int ahead = ring_ahead(nsteps, nsub, wn, a);
                        if (ahead <= 0) continue;
                        const int score = std::min(rs, ahead);
                        if (score > best) {
                            best = score;
                            na = a;
                            nslot = rs;
                            win = wn;
                        }
                    }
                    if (best >= kRingAhead) break;
                }
                if (best == 0) nslot = 0;
            }
            if (nslot < kMinRing && nslot < S) {
                if (nsub == 1) return false;
                na = win = nsteps;
                continue;
            }
        }
        p.nsub = nsub;
        p.nslot = nslot;
        p.na = na;
        p.win = win;
        p.RG = na < nsteps || win < nsteps;
        // small A (batch 2 at K = 5120): loaded by the compute waves before the
        // barrier, as at batch 1, so that the loaders' weight stream starts alone
        // (measured faster there; from about 40 KB on, slower)
        p.AC = !BD && !p.RG && G == 4 && MT == 1 && (int64_t)g.M * g.K * 2 <= kAcMaxBytes;
        p.grid = (T + nsub - 1) / nsub;
        p.lds = (int)(base + na * seg + (int64_t)nslot * kStep);
        return true;
    }
    return false;
}

// The kernel shape and plan for a GEMM, or false when the LDS-staged kernel
// does not serve it.
inline bool choose_lds(const LdsShape& g, LdsPlan& p) {
    // sub-block rows at batch 1 only: from two rows on, its MFMA count doubles
    // and the factored MFMA form is faster
    if (g.M == 1 && plan_lds(g, 4, 1, p, true)) return true;
    if (g.M <= 4 && plan_lds(g, 4, 1, p, false, true)) return true;
    if (g.M <= 8 && plan_lds(g, 4, 2, p, false, true)) return true;
    if (g.M <= 8 && plan_lds(g, 2, 1, p, false, true)) return true;
    if (g.M <= 16 && plan_lds(g, 1, 1, p)) return true;
    return false;
}

}  // namespace bf
