"""The K-split kernel's counter-free exchange (bus-fill_amd/csrc/bf_gemm_split.hip)
modelled on the CPU, for every plan its planner makes over a grid of shapes:

* roles: with the dispatcher handing workgroups to the 8 XCDs round robin from
  any starting XCD, each workgroup's (row group, split) taken from the XCD it
  runs on and its round covers every (row group, split) exactly once, and all
  splits of a row group sit on one XCD (one L2);
* slots: the words the splits store (tile-first waves: rows of their tiles,
  whole batch-row quads) are exactly the words the row group's last split
  reads and frees, and that split writes every C element of its row group
  once;
* the workspace invariant: over a sequence of launches of different shapes
  (single and batched, each GEMM's slots at its own 256-byte offset) every
  slot read holds a written partial, and the region is all free again after
  each launch, so no launch can read a stale partial of an earlier one.

Plans with planted mistakes (a reader that rounds the batch rows down, a
planner whose XCD count differs from the dispatcher's) must each be caught.
The index arithmetic restates the kernel's (split_body: roles, the partial
stores of the tile's first wave, the last split's reads)."""
import numpy as np
import pytest

NC, NX = 12, 8                    # compute waves per workgroup, XCDs
MAX_UNITS = (1024 - 64) // 16     # kSpMaxUnits
MAX_PIECES = 64 * 4 * 12          # kSpMaxPieces
MAX_LDS = 160 * 1024
MAX_S = 56


def lds_bytes(M, nt, nsgS, MT):
    unit = (M * 33 + nt * 144) * 16
    parks = max(NC - nt, 0) * MT * 1024
    return 2048 + nsgS * unit + parks


def plan(M, N, K, nx=NX):
    """plan_split: (S, nt, nsgS, MT, grid, rgs) or None."""
    if M > 32 or K % 256:
        return None
    nsg, T = K // 256, (N + 15) // 16
    MT = 1 if M <= 16 else 2
    best, p = None, None
    for S in range(1, min(nsg, MAX_S) + 1):
        if nsg % S:
            continue
        nsgS = nsg // S
        if nsgS > MAX_UNITS:
            continue
        for rounds in range(1, 17):
            nt = (T * S + 256 * rounds - 1) // (256 * rounds)
            if nt > NC or M * 33 + nt * 144 > MAX_PIECES or lds_bytes(M, nt, nsgS, MT) > MAX_LDS:
                continue
            rgs = (T + nt - 1) // nt
            sx = nx if S > 1 and nx > 0 else 0
            grid = ((rgs + sx - 1) // sx * sx if sx else rgs) * S
            per_wg = nt * nsgS * 2304 + M * nsgS * 512 + (3.0 * nt * 16 * M * 4 if S > 1 else 0.0)
            est = ((grid + 255) // 256) * per_wg
            if best is None or est < best:
                best, p = est, (S, nt, nsgS, MT, grid, rgs)
            break
    return p


def roles(grid, S, nt, N, start, nx_plan=NX, nx_hw=NX):
    """(rg, s) of every workgroup that works, for a dispatcher starting at XCD `start`."""
    out = []
    for b in range(grid):
        x = (b + start) % nx_hw % nx_plan
        jx = b // nx_plan
        q = jx // S
        rg, s = x + nx_plan * q, jx - q * S
        if rg * nt * 16 < N:
            out.append((rg, s, (b + start) % nx_hw))
    return out


def written(rg, s, nt, MT, M, N):
    """Slot words (s, n, m4) the split stores: its tiles' rows, whole quads below Mp."""
    Mp = (M + 3) & ~3
    t, r, kg, mt = np.meshgrid(np.arange(nt), np.arange(16), np.arange(4), np.arange(MT), indexing="ij")
    n = (rg * nt + t) * 16 + r
    m4 = mt * 16 + 4 * kg
    ok = (m4 < Mp) & (n < N)
    return {(s, int(a), int(b)) for a, b in zip(n[ok], m4[ok])}


def read_by_last(rg, S, nt, M, N, mp_round=lambda M: (M + 3) & ~3):
    """Slot words the last split reads (and frees), and the C elements it writes."""
    Mp = mp_round(M)
    rows = nt * 16
    nq = rows * (Mp // 4)
    n0 = rg * rows
    reads, cs = set(), []
    for c in range(NC):
        for b in range(c * 64, nq, NC * 64):
            v = b + np.arange(64)
            nl = v // (Mp // 4)
            m4 = 4 * (v - nl * (Mp // 4))
            ok = (v < nq) & (n0 + nl < N)
            for a, m in zip(nl[ok], m4[ok]):
                for s in range(S):
                    reads.add((s, int(n0 + a), int(m)))
                for i in range(4):
                    if m + i < M:
                        cs.append((int(m + i), int(n0 + a)))
    return reads, cs


SHAPES = [(M, N, K) for M in (9, 16, 17, 31, 32) for N in (200, 1000, 5120) for K in (2048, 5120)] + \
    [(32, 7168, 5120), (13, 17408, 5120), (16, 5120, 17408), (20, 3000, 4096)]


def exchange_plans():
    out = []
    for M, N, K in SHAPES:
        p = plan(M, N, K)
        if p and p[0] > 1:
            out.append((M, N, K) + p)
    return out


def check_plan(M, N, K, S, nt, nsgS, MT, grid, rgs, mp_round=lambda M: (M + 3) & ~3, nx_plan=NX):
    """Raise AssertionError on the first broken invariant."""
    for start in range(NX):
        got = roles(grid, S, nt, N, start, nx_plan=nx_plan)
        pairs = sorted((rg, s) for rg, s, _ in got)
        assert pairs == [(rg, s) for rg in range(rgs) for s in range(S)], ("roles", start)
        for rg, s, xcd in got:
            assert xcd == rg % NX, ("row group off its XCD", rg, s, xcd)
    cover = []
    for rg in range(rgs):
        w = set()
        for s in range(S):
            w |= written(rg, s, nt, MT, M, N)
        r, cs = read_by_last(rg, S, nt, M, N, mp_round)
        assert r == w, ("slots written != slots read", rg, len(w), len(r))
        cover += cs
    assert len(cover) == len(set(cover)) == M * N, ("C coverage", len(cover), len(set(cover)), M * N)


def test_planner_makes_exchange_plans():
    plans = exchange_plans()
    assert len(plans) >= 20, plans
    assert len({p[3] for p in plans}) >= 3, plans     # several split counts


@pytest.mark.parametrize("p", exchange_plans(), ids=lambda p: f"M{p[0]}-N{p[1]}-K{p[2]}-S{p[3]}-nt{p[4]}")
def test_exchange_plan(p):
    check_plan(*p)


def test_workspace_stays_free_across_launches():
    """A sequence of single and batched launches over one slot region: every
    read sees a written partial and every launch leaves the region free."""
    FREE = -1
    plans = exchange_plans()
    rng = np.random.default_rng(5)
    size = 0
    for _ in range(24):
        k = int(rng.integers(1, 4))
        jobs = [plans[int(i)] for i in rng.choice(len(plans), k)]
        need, offs = 0, []
        for M, N, K, S, nt, nsgS, MT, grid, rgs in jobs:
            offs.append(need)
            need += (S * N * ((M + 3) & ~3) * 4 + 255) // 256 * 256
        if need > size:                     # the workspace grows: a new region, all free
            size = need
            region = np.full(size // 4, FREE, np.int64)
        assert (region == FREE).all()
        stamp = int(rng.integers(1, 1 << 30))
        for (M, N, K, S, nt, nsgS, MT, grid, rgs), o in zip(jobs, offs):
            Mp = (M + 3) & ~3
            word = lambda s, n, m4: o // 4 + (s * N + n) * Mp + m4
            for rg in range(rgs):
                for s in range(S):
                    for (ss, n, m4) in written(rg, s, nt, MT, M, N):
                        region[word(ss, n, m4):word(ss, n, m4) + 4] = stamp
            for rg in range(rgs):
                r, _ = read_by_last(rg, S, nt, M, N)
                for (ss, n, m4) in r:
                    w = word(ss, n, m4)
                    assert (region[w:w + 4] == stamp).all(), "the last split would read a free or stale slot"
                    region[w:w + 4] = FREE
        assert (region == FREE).all(), "a launch left a slot written"


def test_planted_mistakes_are_caught():
    p = next(q for q in exchange_plans() if q[0] % 4)            # M not a multiple of 4
    with pytest.raises(AssertionError):
        check_plan(*p, mp_round=lambda M: M & ~3)                 # reader drops the last quad
    with pytest.raises(AssertionError):
        check_plan(*p, nx_plan=4)                                 # roles laid out for 4 XCDs on 8
