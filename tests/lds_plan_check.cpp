// CPU check of the LDS-staged GEMM's plans (bus-fill_amd/csrc/bf_lds_plan.h):
// for every plan choose_lds() makes over a grid of shapes, the LDS layout and
// flag indices stay in bounds, and a model of the kernel's loader and compute
// waves (bf_gemm_lds.hip) finishes under many schedules without a deadlock,
// without reusing a weight-step or activation slot before its readers are
// done, and with every (sub-tile, segment) partial parked exactly once.
//
// The model follows the kernel's protocol action by action:
//   loader j, group g4 (steps 4 g4 .. 4 g4 + 3; it owns step 4 g4 + j): its
//     step (ring: wait until step e - nslot is released), the barrier after
//     group 0, the step's marker, then the activation segments whose first
//     step lies in the group (ring: wait until segment s - na has been counted
//     by all nsub of its steps) and their markers;
//   compute wave: after the barrier, take the next step (batch 1: steps
//     c, c + 12, ...), tabulate a segment's block sums on its first step (Q4_K,
//     MFMA form), wait for the step's markers (and block sums), read and
//     release the step, compute, count the step against its segment (ring) and
//     sub-tile; the last of a sub-tile reduces it (batch 1: the wave that took
//     the sub-tile's last step, after its own steps).
//   AC plans (small A): the compute waves load all of A before the barrier and
//     wait for it (no dependence on the loaders), the loaders stream weights only.
// Bounded waits: every wait of the kernel gives up after a bound, marks the
// workgroup poisoned (an LDS word every store of a result reads first) and
// goes on.  Runs with a planted missing producer (a step marker, one loader's
// activation marker, a batch-1 step count that never comes) check that the
// protocol still ends, that a wait gave up, and that every sub-tile whose
// partials were computed from data that had not landed (or were overwritten)
// is stored while the poison word is set, i.e. as NaN.  In runs without a
// missing producer no wait may give up.
// Exit status 0 and a summary line on success; the first violation otherwise.
// With --self-test it instead runs the model on plans with planted mistakes
// (activation rings whose slots wait for steps of later groups, a step ring
// that is not whole groups of four, stores that ignore the poison word) and
// succeeds only if every one is caught.
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "bf_lds_plan.h"

using namespace bf;

namespace {

constexpr int kNC = 12, kNL = 4;

[[noreturn]] void fail(const char* what, const LdsShape& g, const LdsPlan& p, int a = -1, int b = -1) {
    char buf[512];
    std::snprintf(buf, sizeof buf, "%s (%d, %d) M=%d N=%d K=%d q4k=%d: G=%d MT=%d BD=%d nsub=%d nslot=%d na=%d win=%d lds=%d",
                  what, a, b, g.M, g.N, g.K, (int)g.q4k, p.G, p.MT, (int)p.BD, p.nsub, p.nslot, p.na, p.win, p.lds);
    throw std::runtime_error(buf);
}

struct Rng {
    uint64_t s;
    uint32_t next() {
        s ^= s << 13;
        s ^= s >> 7;
        s ^= s << 17;
        return (uint32_t)(s >> 11);
    }
};

// The kernel's step order: step e -> (sub-tile t, segment s), windows of Wn
// segments; computed both with divisions and with the kernel's 16-bit
// reciprocal multiplies.
struct Order {
    int nsteps, nsub, Wn, EW, nfull, Wl, E_full;
    Order(const LdsPlan& p, int nsteps_) : nsteps(nsteps_), nsub(p.nsub) {
        Wn = p.RG ? p.win : nsteps;
        EW = nsub * Wn;
        nfull = nsteps / Wn;
        Wl = nsteps - nfull * Wn;
        E_full = nfull * EW;
    }
    static int rdiv(int e, int d) { return (int)(((uint32_t)e * ((65536u + d - 1u) / (uint32_t)d)) >> 16); }
    void ts(int e, int& t, int& s) const {
        if (e < E_full) {
            const int w = e / EW, e1 = e - w * EW;
            t = e1 / Wn;
            s = w * Wn + e1 - t * Wn;
        } else {
            const int e1 = e - E_full;
            t = e1 / Wl;
            s = nfull * Wn + e1 - t * Wl;
        }
    }
    void ts_recip(int e, int& t, int& s) const {
        if (e < E_full) {
            const int w = rdiv(e, EW), e1 = e - w * EW;
            t = rdiv(e1, Wn);
            s = w * Wn + e1 - t * Wn;
        } else {
            const int e1 = e - E_full;
            t = rdiv(e1, Wl);
            s = nfull * Wn + e1 - t * Wl;
        }
    }
};

// A producer that never delivers (planted by a run): the marker of step
// `step`, loader 0's marker of activation segment `seg`, the count of step
// `count` (batch 1).  `bound`: blocked polls before a wait gives up (0: never).
struct Drop {
    int step = -1, seg = -1, count = -1;
    int bound = 0;
    bool ignore_poison = false;        // planted mistake: stores that do not read the poison word
};

struct Model {
    const LdsShape& g;
    const LdsPlan& p;
    int nsteps, S, G4R;
    bool a_ring;
    Order ord;
    Drop drop;
    bool poison = false;
    int giveups = 0, poisoned_out = 0;
    std::vector<char> taint, taint_seg, reduced;
    // LDS state
    bool cleared = false;
    int at_barrier = 0;
    std::vector<char> amark;          // [s][j]
    std::vector<int> stepmark;        // 0 / 1 (landed) / 2 (released)
    std::vector<int> segcount, subcount;
    std::vector<char> tabflag, parked;
    std::vector<int> wslot, aslot;    // the step / segment a slot holds (-1: none)
    int counter = 0;

    struct Loader {
        int j, g4 = 0, phase = 0, s_lo = 0, s_hi = 0, s2 = 0, s_next = 0, sw = 0, so = 0, spins = 0;
        bool done = false, at_bar = false;
    };
    struct Wave {
        int c, e = -1, t = 0, s = 0, phase = 0, k = 0, red = 0, spins = 0;
        bool done = false, at_bar = false;
    };
    std::vector<Loader> L;
    std::vector<Wave> W;

    Model(const LdsShape& g_, const LdsPlan& p_, int nsteps_, Drop d = Drop())
        : g(g_), p(p_), nsteps(nsteps_), S(p_.nsub * nsteps_), G4R((p_.nslot + 3) >> 2),
          a_ring(p_.RG && p_.na < nsteps_), ord(p_, nsteps_), drop(d) {
        taint.assign(S, 0);
        taint_seg.assign(nsteps, 0);
        reduced.assign(p.nsub, 0);
        amark.assign(nsteps * kNL, 0);
        stepmark.assign(S, 0);
        segcount.assign(nsteps, 0);
        subcount.assign(p.nsub, 0);
        tabflag.assign(nsteps, 0);
        parked.assign(S, 0);
        wslot.assign(std::max(p.nslot, 4 * G4R), -1);
        aslot.assign(p.na, -1);
        for (int j = 0; j < kNL; j++) L.push_back(Loader{j});
        for (int c = 0; c < kNC; c++) W.push_back(Wave{c});
        if (p.AC) {
            if (p.na != nsteps || p.RG || p.BD) fail("AC plan without all of A resident", g, p);
            for (int sg = 0; sg < nsteps; sg++) {
                aslot[sg] = sg;
                for (int j = 0; j < kNL; j++) amark[sg * kNL + j] = 1;
            }
        }
    }
    int wslot_of(int e) const { return ((e >> 2) % G4R) * 4 + (e & 3); }

    // a blocked poll of a bounded wait: true while the wait goes on, false once
    // it gives up (the poison word is set before the wave moves on)
    bool still_waiting(int& spins) {
        if (drop.bound == 0 || ++spins < drop.bound) return true;
        spins = 0;
        poison = true;
        giveups++;
        return false;
    }
    // a slot or order check: data read after a wait gave up (or overwritten after
    // one) is garbage, which the poison word covers; otherwise a protocol bug
    void violation(const char* what, int a = -1, int b = -1, int e = -1) {
        if (!poison) fail(what, g, p, a, b);
        if (e >= 0) taint[e] = 1;
    }

    // one action of loader l; false if it is blocked
    bool step_loader(Loader& l) {
        const int e = 4 * l.g4 + l.j;
        switch (l.phase) {
            case 0: {                                          // segments first needed in this group
                if (p.RG) {
                    l.s_lo = l.s_next;
                    while (l.s_next < nsteps && l.sw * ord.EW + l.so <= 4 * l.g4 + 3) {
                        l.s_next++;
                        if (++l.so == ord.Wn) { l.so = 0; l.sw++; }
                    }
                    l.s_hi = l.s_next;
                } else {
                    l.s_lo = 4 * l.g4;
                    l.s_hi = p.BD || p.AC ? l.s_lo : std::min(4 * l.g4 + 4, nsteps);
                }
                l.s2 = l.s_lo;
                l.phase = 2;
                return true;
            }
            case 1: {                                          // load segment s2
                if (l.s2 >= l.s_hi) { l.phase = 4; return true; }
                const int s2 = l.s2;
                if (a_ring && s2 >= p.na) {
                    if (!cleared) fail("loader waits before the barrier", g, p, s2);
                    if (segcount[s2 - p.na] != p.nsub && still_waiting(l.spins)) return false;
                }
                l.spins = 0;
                const int k = s2 % p.na;
                if (aslot[k] >= 0 && aslot[k] != s2 && segcount[aslot[k]] != p.nsub)
                    violation("activation slot reused early", s2, aslot[k]);
                aslot[k] = s2;
                l.s2++;
                return true;
            }
            case 2: {                                          // this loader's step
                if (e < S) {
                    if (e >= p.nslot) {
                        if (!cleared) fail("loader waits before the barrier", g, p, e);
                        if (stepmark[e - p.nslot] != 2 && still_waiting(l.spins)) return false;
                    }
                    l.spins = 0;
                    const int k = wslot_of(e);
                    if (k >= (int)wslot.size() || (k >= p.nslot && p.nslot != S)) fail("step slot out of range", g, p, e, k);
                    if (wslot[k] >= 0 && stepmark[wslot[k]] != 2) violation("step slot reused early", e, wslot[k]);
                    wslot[k] = e;
                }
                l.phase = 3;
                return true;
            }
            case 3: {                                          // the barrier after group 0, the step's marker
                if (l.g4 == 0) {
                    if (!l.at_bar) { l.at_bar = true; at_barrier++; }
                    if (!cleared) return false;
                }
                if (e < S && e != drop.step) stepmark[e] = 1;
                l.phase = 1;
                return true;
            }
            case 4: {                                          // the segments' markers
                for (int s2 = l.s_lo; s2 < l.s_hi; s2++)
                    if (!(s2 == drop.seg && l.j == 0)) amark[s2 * kNL + l.j] = 1;
                l.g4++;
                l.phase = 0;
                if (4 * l.g4 >= S) l.done = true;
                return true;
            }
        }
        return false;
    }

    bool seg_landed(int s) const {
        for (int j = 0; j < kNL; j++)
            if (!amark[s * kNL + j]) return false;
        return true;
    }

    // sub-tile t is reduced and stored (after the wave read the poison word)
    void check_reduce(int t) {
        bool tainted = false;
        for (int s2 = 0; s2 < nsteps; s2++) {
            if (!parked[t * nsteps + s2]) violation("sub-tile reduced before all its partials", t, s2);
            tainted = tainted || !parked[t * nsteps + s2] || taint[t * nsteps + s2];
        }
        const bool nan = poison && !drop.ignore_poison;
        if (tainted && !nan) fail("sub-tile stored from data that had not landed, without the poison word", g, p, t);
        if (reduced[t]) fail("sub-tile stored twice", g, p, t);
        reduced[t] = 1;
        poisoned_out += nan;
    }

    bool step_wave(Wave& w) {
        switch (w.phase) {
            case 0:                                            // the barrier
                if (!w.at_bar) { w.at_bar = true; at_barrier++; }
                if (!cleared) return false;
                w.phase = 1;
                return true;
            case 1: {                                          // take a step
                w.e = p.BD ? w.c + kNC * w.k++ : counter++;
                if (w.e >= S) { w.phase = p.BD ? 5 : 6; w.red = 0; return true; }
                ord.ts(w.e, w.t, w.s);
                int t2, s2;
                ord.ts_recip(w.e, t2, s2);
                if (t2 != w.t || s2 != w.s) fail("reciprocal step order differs", g, p, w.e);
                w.phase = 2;
                return true;
            }
            case 2:                                            // block sums by the segment's first step
                if (!p.BD && g.q4k && w.t == 0) {
                    if (!seg_landed(w.s)) {
                        if (still_waiting(w.spins)) return false;
                        taint_seg[w.s] = 1;                    // tabulated from activations that had not landed
                    }
                    w.spins = 0;
                    if (aslot[w.s % p.na] != w.s) {
                        violation("block sums of a segment not in its slot", w.s);
                        taint_seg[w.s] = 1;
                    }
                    tabflag[w.s] = 1;
                }
                w.phase = 3;
                return true;
            case 3: {                                          // markers, read, release
                const bool ready = (p.BD || seg_landed(w.s)) && (p.BD || !g.q4k || tabflag[w.s]) && stepmark[w.e] != 0;
                if (!ready) {
                    if (still_waiting(w.spins)) return false;
                    taint[w.e] = 1;                            // read before its data landed
                }
                w.spins = 0;
                if (wslot[wslot_of(w.e)] != w.e) violation("step read from a slot holding another step", w.e, -1, w.e);
                if (!p.BD && aslot[w.s % p.na] != w.s)
                    violation("activations read from a slot holding another segment", w.s, -1, w.e);
                stepmark[w.e] = 2;
                w.phase = 4;
                return true;
            }
            case 4: {                                          // compute, count, park
                if (!p.BD && aslot[w.s % p.na] != w.s) violation("activation slot changed under a step", w.s, -1, w.e);
                if (a_ring) segcount[w.s]++;
                const int idx = w.t * nsteps + w.s;
                if (parked[idx]) fail("partial parked twice", g, p, w.t, w.s);
                parked[idx] = 1;
                if (taint_seg[w.s]) taint[idx] = 1;
                if (w.e == drop.count) {                       // a count that never comes (batch 1)
                    w.phase = 1;
                    return true;
                }
                if (++subcount[w.t] == nsteps && !p.BD) check_reduce(w.t);
                w.phase = 1;
                return true;
            }
            case 5: {                                          // batch 1: the sub-tiles whose last step this wave took
                while (w.red < p.nsub && (w.red * nsteps + nsteps - 1) % kNC != w.c) w.red++;
                if (w.red >= p.nsub) { w.phase = 6; return true; }
                if (subcount[w.red] != nsteps) {
                    if (still_waiting(w.spins)) return false;
                    taint[w.red * nsteps] = 1;                 // reduced without every count
                }
                w.spins = 0;
                check_reduce(w.red);
                w.red++;
                return true;
            }
            case 6:
                w.done = true;
                return true;
        }
        return false;
    }

    // runs to the end under one schedule (mode 0 random, 1 loaders first, 2 compute first)
    void run(uint64_t seed, int mode) {
        Rng r{seed * 0x9E3779B97F4A7C15ull + 1};
        std::vector<int> alive;
        for (int i = 0; i < kNL + kNC; i++) alive.push_back(i);
        int stall = 0;
        while (!alive.empty()) {
            if (!cleared && at_barrier == kNL + kNC) cleared = true;
            int pick;
            if (mode == 0 || r.next() % 5 == 0) {
                pick = (int)(r.next() % alive.size());
            } else {
                // prefer the first alive agent of the favoured kind
                pick = -1;
                for (int q = 0; q < (int)alive.size(); q++) {
                    const bool loader = alive[q] < kNL;
                    if ((mode == 1) == loader && r.next() % 2) { pick = q; break; }
                }
                if (pick < 0) pick = (int)(r.next() % alive.size());
            }
            const int a = alive[pick];
            bool moved, done;
            if (a < kNL) {
                moved = step_loader(L[a]);
                done = L[a].done;
            } else {
                moved = step_wave(W[a - kNL]);
                done = W[a - kNL].done;
            }
            if (done) alive.erase(alive.begin() + pick);
            stall = moved ? 0 : stall + 1;
            if (stall > 200 * (kNL + kNC)) {
                // confirm on a copy: no agent can move
                bool any = false;
                for (int q : alive) {
                    Model m2 = *this;
                    any = q < kNL ? m2.step_loader(m2.L[q]) : m2.step_wave(m2.W[q - kNL]);
                    if (any) break;
                }
                if (!any) fail("deadlock", g, p, (int)alive.size(), counter);
                stall = 0;
            }
        }
        for (int i = 0; i < S; i++)
            if (!parked[i]) fail("step never computed", g, p, i);
        for (int t = 0; t < p.nsub; t++)
            if (!reduced[t]) fail("sub-tile never stored", g, p, t);
        const bool planted = drop.step >= 0 || drop.seg >= 0 || drop.count >= 0;
        if (!planted && giveups) fail("a wait gave up without a missing producer", g, p, giveups);
        if (planted && (!giveups || !poison || !poisoned_out)) fail("missing producer not seen as poison", g, p, giveups);
    }
};

// Runs with a planted missing producer under three schedules; throws on the first violation.
void run_drops(const LdsShape& g, const LdsPlan& p, int nsteps, uint64_t seed, bool ignore_poison = false) {
    const int S = p.nsub * nsteps;
    std::vector<Drop> drops;
    Drop d;
    d.bound = 60;
    d.ignore_poison = ignore_poison;
    d.step = S / 2;
    drops.push_back(d);
    d.step = -1;
    if (!p.BD && !p.AC) {
        d.seg = nsteps / 2;
        drops.push_back(d);
        d.seg = -1;
    }
    if (p.BD) {
        d.count = S - 1;
        drops.push_back(d);
    }
    for (const Drop& dr : drops)
        for (int mode = 0; mode < 3; mode++) {
            Model m(g, p, nsteps, dr);
            m.run(seed + 31u * mode, mode);
        }
}

void check_bounds(const LdsShape& g, const LdsPlan& p) {
    const int nsg = g.K / 256, nsteps = nsg / p.G, R = 16 / p.G, S = p.nsub * nsteps;
    const int64_t seg = (int64_t)g.M * p.G * 528;
    const int64_t slot = p.BD ? p.MT * 64 : p.MT * R * R;
    const int64_t tab = g.q4k || p.BD ? (int64_t)g.M * nsg * 32 : 0;
    const int64_t lds = kFlagBytes + p.na * seg + (int64_t)p.nslot * kStep + S * slot * 4 + tab;
    if (lds != p.lds || lds > kMaxLds) fail("LDS layout", g, p, (int)lds);
    if (nsteps > kMaxSeg || kAMark + 4 * nsteps > kTabFlag || kTabFlag + nsteps > kStepMark) fail("segment flags", g, p);
    if (S > kMaxSteps || kStepMark + S > kSubCount) fail("step flags", g, p, S);
    if (p.nsub > kMaxSub || kSubCount + p.nsub > kSegCount || kSegCount + nsteps > kFlagBytes / 4) fail("counters", g, p);
    if (p.nslot != S && (p.nslot % 4 || p.nslot < kMinRing || p.nslot > S)) fail("step ring size", g, p, p.nslot);
    if (p.RG != (p.na < nsteps || p.win < nsteps) || (p.BD && p.RG)) fail("ring flag", g, p);
    if (p.na < nsteps && ring_ahead(nsteps, p.nsub, p.win, p.na) <= 0) fail("activation ring lead", g, p);
    if (g.M > (p.BD ? p.MT : p.MT * R) || g.M * p.G > 32) fail("batch rows", g, p);
    const int T = (g.N + R - 1) / R;
    if (p.grid * p.nsub < T || (p.grid - 1) * p.nsub >= T) fail("grid", g, p, p.grid);
}

}  // namespace

// Plans with planted mistakes: each must be reported.
int self_test() {
    int caught = 0, planted = 0;
    auto expect_failure = [&](const char* name, const LdsShape& g, LdsPlan p) {
        planted++;
        const int nsteps = g.K / 256 / p.G;
        try {
            for (int mode = 0; mode < 3; mode++) {
                Model m(g, p, nsteps);
                m.run(7u + mode, mode);
            }
            std::printf("not caught: %s\n", name);
        } catch (const std::exception& e) {
            caught++;
            std::printf("caught %s: %s\n", name, e.what());
        }
    };
    const LdsShape g{8, 5120, 17408, true};
    LdsPlan p{};
    if (!choose_lds(g, p) || !p.RG) {
        std::printf("no ring plan for the self-test shape\n");
        return 1;
    }
    LdsPlan a = p;                     // windows of two with one slot: a segment's slot waits for the
    a.win = 2;                         // previous segment's last step, in a later group of four
    a.na = 1;
    expect_failure("activation ring of one slot, windows of two", g, a);
    LdsPlan b = p;                     // windows of four with three slots: the window's fourth segment
    b.win = 4;                         // waits for its first, whose last step is in a later group
    b.na = 3;
    expect_failure("activation ring smaller than a window", g, b);
    const LdsShape g2{1, 17408, 5120, true};
    LdsPlan c{};
    if (!choose_lds(g2, c) || c.nslot == c.nsub * (g2.K / 256 / c.G)) {
        std::printf("no step-ring plan for the self-test shape\n");
        return 1;
    }
    c.nslot = 18;                      // not whole groups of four: slots beyond the ring or reused early
    expect_failure("step ring of 18 slots", g2, c);
    // stores that do not read the poison word, after a wait gave up on a missing producer
    auto expect_drop_failure = [&](const char* name, const LdsShape& gg) {
        planted++;
        LdsPlan pp{};
        if (!choose_lds(gg, pp)) {
            std::printf("no plan for %s\n", name);
            return;
        }
        try {
            run_drops(gg, pp, gg.K / 256 / pp.G, 11u, true);
            std::printf("not caught: %s\n", name);
        } catch (const std::exception& e) {
            caught++;
            std::printf("caught %s: %s\n", name, e.what());
        }
    };
    expect_drop_failure("batch 1 stores that ignore the poison word", LdsShape{1, 5120, 5120, true});
    expect_drop_failure("batch 8 stores that ignore the poison word", LdsShape{8, 5120, 17408, true});
    std::printf("%d of %d planted mistakes caught\n", caught, planted);
    return caught == planted ? 0 : 1;
}

int main(int argc, char** argv) {
    if (argc > 1 && std::strcmp(argv[1], "--self-test") == 0) return self_test();
    const int Ns[] = {1, 77, 512, 600, 1024, 3072, 4096, 5120, 7168, 13824, 17408, 27648};
    const int Ks[] = {256, 1024, 2048, 3072, 4096, 5120, 8192, 13824, 17408, 24576, 27648};
    int plans = 0, rings = 0, aring = 0, ac = 0, runs = 0, drop_plans = 0;
    for (int q = 0; q < 2; q++)
        for (int M = 1; M <= 16; M++)
            for (int N : Ns)
                for (int K : Ks) {
                    const LdsShape g{M, N, K, q == 1};
                    LdsPlan p{};
                    if (!choose_lds(g, p)) continue;
                    plans++;
                    try {
                        check_bounds(g, p);
                    const int nsteps = K / 256 / p.G;
                    const bool ring = p.nslot < p.nsub * nsteps;
                    rings += ring;
                    aring += p.RG;
                    ac += p.AC;
                    // the model runs each shape's first workgroup: every workgroup runs
                    // the same protocol on its own rows
                    const int seeds = ring || p.RG ? 3 : 1;
                        for (int sd = 0; sd < seeds; sd++)
                            for (int mode = 0; mode < 3; mode++) {
                                Model m(g, p, nsteps);
                                m.run((uint64_t)(sd * 7 + mode) * 1000003u + (uint64_t)(M * 131 + N) * 17u + K, mode);
                                runs++;
                            }
                        // every fifth plan: bounded waits against a missing producer
                        if (plans % 5 == 0) {
                            run_drops(g, p, nsteps, (uint64_t)(M * 131 + N) * 17u + K);
                            drop_plans++;
                        }
                    } catch (const std::exception& e) {
                        std::printf("FAIL %s\n", e.what());
                        return 1;
                    }
                }
    std::printf("ok: %d plans (%d with a step ring, %d with windows / activation ring), %d model runs, %d AC, "
                "%d with missing producers\n", plans, rings, aring, runs, ac, drop_plans);
    return 0;
}
