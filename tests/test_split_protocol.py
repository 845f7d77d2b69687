"""The K-split kernel's exchange (bus-fill_amd/csrc/bf_gemm_split.hip)
modelled on the CPU, for every plan its planner makes over a grid of shapes.

* Roles: with the dispatcher handing workgroups to the 8 XCDs round robin from
  any starting XCD, each workgroup's (row group, split) taken from the XCD it
  runs on and its round covers every (row group, split) exactly once, all
  splits of a row group sit on one XCD (one L2), every workgroup sees the same
  placement offset, and the last split of a row group is its last-dispatched
  workgroup (the reader waits only for workgroups that started before it).
  Exchange plans fill whole XCD rounds (no padding workgroups).
* Slots: the words the splits store (tile-first waves: rows of their tiles,
  whole batch-row quads) are exactly the words the row group's last split
  reads and frees, and it writes every C element of its row group once.
* The workspace invariant: over a sequence of launches of different shapes,
  placed round robin from any starting XCD, under random interleavings of
  the workgroups' steps, every C element is correct and the region (slots and
  tags) is all free again after each launch.
* Broken placements -- a duplicated split, a missing split, a missing last
  split, an XCD that gets no workgroup, a dispatcher that skips one XCD once
  (every later workgroup shifted by one), single workgroups moved to another
  XCD, random placements -- under random interleavings (late duplicates
  included): every C element ends correct or NaN, never stale or wrong; the
  call's output holds NaN and the workspace's poison word is set; every later
  launch on the workspace writes NaN.  A moved workgroup keeps its split, so
  it takes another row group's role of the same split: a row group then misses
  that split (its reader gives up) or, for the last split, has a second reader
  (caught by the reader's tag swap, or by its poll of slots the first reader
  freed).  Not caught: every one of a row group's splits moved onto the same
  other row group, the duplicates running only after that row group's first
  reader has finished; the test below checks that moving all but one of them
  is caught.

Planted mistakes (a reader that rounds the batch rows down, roles laid out
for 4 XCDs on 8, a give-up that writes NaN over its own row group only, a
reader that skips the tag check) must each be caught.  The index arithmetic
and the steps restate the kernel's (split_body: roles, the reader's tag swap
at its start, the partial stores of the tile's first wave, the last split's
reads, the give-up, which writes NaN over all of C)."""
import numpy as np
import pytest

NC, NX = 12, 8                    # compute waves per workgroup, XCDs
MAX_UNITS = (1024 - 64) // 16     # kSpMaxUnits
MAX_PIECES = 64 * 4 * 12          # kSpMaxPieces
MAX_LDS = 160 * 1024
MAX_S = 56
CUS = 256


def lds_bytes(M, nt, nsgS, MT):
    unit = (M * 33 + nt * 144) * 16
    parks = max(NC - nt, 0) * MT * 1024
    return 2048 + nsgS * unit + parks


def plan(M, N, K, nx=NX):
    """plan_split: (S, nt, nsgS, MT, grid, rgs) or None."""
    if M > 32 or K % 256 or N >= 1 << 24 or K // 256 > 0xFFF:
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


def in_kernel_exchange(p):
    """split_second_launch is false: the splits exchange in the kernel."""
    S, nt, nsgS, MT, grid, rgs = p
    return S > 1 and grid < 2 * CUS and rgs % NX == 0


def round_robin(start, nx=NX):
    return lambda b: (b + start) % nx


def roles(grid, S, nt, N, xcd_of, nx_plan=NX):
    """(b, rg, s, place) of every workgroup that works (the kernel's role and
    placement offset from the XCD it runs on)."""
    out = []
    for b in range(grid):
        x = xcd_of(b) % nx_plan
        jx = b // nx_plan
        q = jx // S
        rg, s = x + nx_plan * q, jx - q * S
        if rg * nt * 16 < N:
            out.append((b, rg, s, (x - b % nx_plan) % nx_plan))
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
    """Quads (n, m4) the row group's last split reads (all S slots of each)
    and frees, and the C elements (m, n) it writes, as its compute waves'
    loop visits them."""
    Mp = mp_round(M)
    rows = nt * 16
    nq = rows * (Mp // 4)
    n0 = rg * rows
    quads, cs = [], []
    for c in range(NC):
        for b in range(c * 64, nq, NC * 64):
            v = b + np.arange(64)
            nl = v // (Mp // 4)
            m4 = 4 * (v - nl * (Mp // 4))
            ok = (v < nq) & (n0 + nl < N)
            for a, m in zip(nl[ok], m4[ok]):
                quads.append((int(n0 + a), int(m)))
                cs += [(int(m + i), int(n0 + a)) for i in range(4) if m + i < M]
    return quads, cs


SHAPES = [(M, N, K) for M in (9, 16, 17, 31, 32) for N in (200, 1000, 5120) for K in (2048, 5120)] + \
    [(32, 7168, 5120), (13, 17408, 5120), (16, 5120, 17408), (20, 3000, 4096), (24, 4096, 4096), (12, 8192, 4096),
     (32, 1024, 8192), (20, 2560, 2560)]


def exchange_plans():
    out = []
    for M, N, K in SHAPES:
        p = plan(M, N, K)
        if p and in_kernel_exchange(p):
            out.append((M, N, K) + p)
    return out


def check_plan(M, N, K, S, nt, nsgS, MT, grid, rgs, mp_round=lambda M: (M + 3) & ~3, nx_plan=NX):
    """Raise AssertionError on the first broken invariant."""
    assert grid == rgs * S, ("padding workgroups", grid, rgs, S)
    for start in range(NX):
        got = roles(grid, S, nt, N, round_robin(start), nx_plan=nx_plan)
        pairs = sorted((rg, s) for _, rg, s, _ in got)
        assert pairs == [(rg, s) for rg in range(rgs) for s in range(S)], ("roles", start)
        assert len({pl for *_, pl in got}) == 1, ("placement offsets differ", start)
        last = {}
        for b, rg, s, _ in got:
            assert round_robin(start)(b) == rg % NX, ("row group off its XCD", rg, s)
            last[rg] = max(last.get(rg, (-1, -1)), (b, s))
        assert all(s == S - 1 for _, s in last.values()), "the reader is not its row group's last workgroup"
    cover = []
    for rg in range(rgs):
        w = set()
        for s in range(S):
            w |= written(rg, s, nt, MT, M, N)
        quads, cs = read_by_last(rg, S, nt, M, N, mp_round)
        r = {(ss, n, m4) for n, m4 in quads for ss in range(S)}
        assert r == w, ("slots written != slots read", rg, len(w), len(r))
        cover += cs
    assert len(cover) == len(set(cover)) == M * N, ("C coverage", len(cover), len(set(cover)), M * N)


def test_planner_makes_exchange_plans():
    plans = exchange_plans()
    assert len(plans) >= 16, plans
    assert len({p[3] for p in plans}) >= 3, plans     # several split counts


@pytest.mark.parametrize("p", exchange_plans(), ids=lambda p: f"M{p[0]}-N{p[1]}-K{p[2]}-S{p[3]}-nt{p[4]}")
def test_exchange_plan(p):
    check_plan(*p)


# ------------------------------------------------------------------ the protocol, step by step
FREE = None


class Workspace:
    """The slot region (slots and the readers' tags; absent = free) and its poison word."""

    def __init__(self):
        self.slots, self.tags, self.poisoned = {}, {}, False

    def free(self):
        return not self.slots and not self.tags


def run_launch(ws, job, launch_id, xcd_of, rng, give_up_all=True, check_tags=True):
    """One launch of one GEMM through the exchange, its workgroups' steps
    interleaved at random (a reader's poll is taken only when its slots are
    all there, or when nothing else can run: then it gives up).  Returns C, a
    dict (m, n) -> "ok" | "nan" | "stale" | "wrong"."""
    M, N, K, S, nt, nsgS, MT, grid, rgs = job
    C = {(m, n): "stale" for m in range(M) for n in range(N)}
    sticky = ws.poisoned

    def give_up(rg):
        for e in (list(C) if give_up_all else
                  [e for e in C if rg * nt * 16 <= e[1] < (rg + 1) * nt * 16]):
            C[e] = "nan"
        ws.poisoned = True

    def writer(b, rg, s, place):
        yield
        for w in written(rg, s, nt, MT, M, N):                  # the partial stores
            ws.slots[w] = launch_id

    def reader(b, rg, s, place):
        old = ws.tags.get(rg, FREE)                             # the tag swap at the start
        ws.tags[rg] = "taken"
        yield
        for w in written(rg, s, nt, MT, M, N):                  # its own partial stores
            ws.slots[w] = launch_id
        yield
        quads, cs = read_by_last(rg, S, nt, M, N)
        late = False
        while any(ws.slots.get((ss, n, m4)) is FREE for n, m4 in quads for ss in range(S)):
            yield "wait"                                        # the bounded poll
            if state["stuck"]:
                late = True
                break
        vals = [ws.slots.get((ss, n, m4)) for n, m4 in quads for ss in range(S)]
        yield
        if not late and check_tags and (old is not FREE or sticky):   # own swap, poison word
            late = True
        if not check_tags and sticky:
            late = True
        for n, m4 in quads:                                     # write C, free the slots
            for ss in range(S):
                ws.slots.pop((ss, n, m4), None)
        fresh = all(v == launch_id for v in vals)
        for e in cs:
            C[e] = "nan" if late else ("ok" if fresh else "wrong")
        ws.tags.pop(rg, None)                                   # the last wave frees the tag
        if late:
            give_up(rg)

    present = roles(grid, S, nt, N, xcd_of)
    gens = [(writer if s < S - 1 else reader)(b, rg, s, place) for b, rg, s, place in present]
    # workgroups start in dispatch order (a random prefix of them may be
    # running); a waiting reader wakes when another step made progress, and
    # gives up only when nothing else can run
    state = {"stuck": False}
    active, waiting = [], []
    pending = list(gens)
    while pending or active or waiting:
        while pending and (not active or rng.random() < 0.3):
            active.append(pending.pop(0))
        if not active:
            state["stuck"] = True
            active, waiting = waiting, []
        g = active.pop(int(rng.integers(len(active))))
        try:
            r = next(g)
        except StopIteration:
            r = "done"
        if r == "wait" and not state["stuck"]:
            waiting.append(g)
            continue
        if r != "done":
            active.append(g)
        if r != "wait":
            state["stuck"] = False
            active.extend(waiting)
            waiting.clear()
    return C


def broken_placements(job, rng):
    """xcd_of functions that are not round robin, with a name."""
    M, N, K, S, nt, nsgS, MT, grid, rgs = job
    rr = round_robin(0)
    out = []
    # a duplicated split (and so a missing one): workgroup 0 on workgroup 1's XCD
    out.append(("duplicate", lambda b: rr(1) if b == 0 else rr(b)))
    # the last split of row group 0 missing: its workgroup lands on the XCD of the next one
    last = next(b for b, rg, s, _ in roles(grid, S, nt, N, rr) if rg == 0 and s == S - 1)
    out.append(("missing last split", lambda b, last=last: rr(last + 1) if b == last else rr(b)))
    # an XCD that gets no workgroup (the dispatcher round robin over 7 of 8)
    out.append(("XCD 3 skipped", lambda b: [0, 1, 2, 4, 5, 6, 7][b % 7]))
    # the dispatcher skips one XCD once inside a round of NX workgroups: every
    # workgroup from k on one XCD further (a skip between rounds only changes
    # the placement offset: a valid placement)
    k = int(rng.integers(0, grid // NX)) * NX + int(rng.integers(1, NX))
    out.append(("one skip", lambda b, k=k: rr(b + 1) if b >= k else rr(b)))
    # single workgroups moved to another XCD
    for b0, d in zip(rng.integers(0, grid, size=3), rng.integers(1, NX, size=3)):
        out.append((f"moved {int(b0)}+{int(d)}",
                    lambda b, b0=int(b0), d=int(d): rr(b + d) if b == b0 else rr(b)))
    perm = [int(x) for x in rng.integers(0, NX, size=grid)]
    out.append(("random", lambda b, perm=perm: perm[b]))
    return out


def small_jobs(count=2):
    """The smallest exchange plans (step-by-step simulation), several split
    counts among them."""
    plans = sorted(exchange_plans(), key=lambda p: p[0] * p[1])
    out = []
    for p in plans:
        if len(out) < count and (p[3], p[4]) not in {(q[3], q[4]) for q in out}:
            out.append(p)
    return out


def test_round_robin_launches_leave_workspace_free():
    """A sequence of launches with round-robin placements from every
    starting XCD under random interleavings: every C element correct, the
    region free after each launch, the poison word never set."""
    rng = np.random.default_rng(5)
    ws = Workspace()
    jobs = small_jobs()
    assert len(jobs) == 2, jobs
    for i in range(30):
        job = jobs[int(rng.integers(len(jobs)))]
        C = run_launch(ws, job, i, round_robin(int(rng.integers(NX))), rng)
        assert all(v == "ok" for v in C.values())
        assert ws.free() and not ws.poisoned


def test_skip_between_rounds_is_a_valid_placement():
    """A dispatcher that skips an XCD between two rounds of NX workgroups
    shifts the placement offset of the later rounds only: every role is still
    taken once on its XCD, and the result is correct."""
    rng = np.random.default_rng(23)
    ws = Workspace()
    for job in small_jobs():
        grid = job[7]
        for k in (NX, grid // 2 // NX * NX, grid - NX):
            C = run_launch(ws, job, k, lambda b, k=k: (b + 1) % NX if b >= k else b % NX, rng)
            assert all(v == "ok" for v in C.values()), k
            assert ws.free() and not ws.poisoned


def test_broken_placements_show_as_nan():
    """Each broken placement under several random interleavings: every C
    element correct or NaN (never stale or wrong), NaN somewhere, the poison
    word set; the next launch, with a round-robin placement, is NaN
    everywhere."""
    rng = np.random.default_rng(11)
    seen = set()
    for job in small_jobs():
        for name, xcd_of in broken_placements(job, rng):
            for rep in range(3):
                ws = Workspace()
                C = run_launch(ws, job, 1, xcd_of, rng)
                assert all(v in ("ok", "nan") for v in C.values()), (name, job[:3], rep)
                assert any(v == "nan" for v in C.values()), (name, job[:3], rep)
                assert ws.poisoned, name
                C2 = run_launch(ws, job, 2, round_robin(0), rng)
                assert all(v == "nan" for v in C2.values()), name
            seen.add(name)
    assert {"duplicate", "missing last split", "XCD 3 skipped", "one skip", "random"} <= seen
    assert sum(n.startswith("moved") for n in seen) >= 3


def test_all_but_one_split_moved_is_caught():
    """Row group 0's splits but one moved onto row group 1's XCD (their
    duplicates late or early): the row group left without that split gives up,
    the output holds NaN and the workspace is poisoned."""
    rng = np.random.default_rng(17)
    for job in small_jobs():
        M, N, K, S, nt, nsgS, MT, grid, rgs = job
        rr = round_robin(0)
        for keep in (0, S // 2, S - 1):
            moved = {b for b, rg, s, _ in roles(grid, S, nt, N, rr) if rg == 0 and s != keep}
            xcd_of = lambda b, moved=moved: rr(b + 1) if b in moved else rr(b)
            for rep in range(2):
                ws = Workspace()
                C = run_launch(ws, job, 1, xcd_of, rng)
                assert all(v in ("ok", "nan") for v in C.values()), (keep, rep)
                assert any(v == "nan" for v in C.values()) and ws.poisoned, (keep, rep)


def test_planted_mistakes_are_caught():
    p = next(q for q in exchange_plans() if q[0] % 4)            # M not a multiple of 4
    with pytest.raises(AssertionError):
        check_plan(*p, mp_round=lambda M: M & ~3)                 # reader drops the last quad
    with pytest.raises(AssertionError):
        check_plan(*p, nx_plan=4)                                 # roles laid out for 4 XCDs on 8
    rng = np.random.default_rng(3)
    caught = {"own row group": False, "no tag check": False}
    for job in small_jobs():
        for name, xcd_of in broken_placements(job, rng):
            for rep in range(3):
                C = run_launch(Workspace(), job, 1, xcd_of, rng, give_up_all=False)
                caught["own row group"] |= any(v not in ("ok", "nan") for v in C.values())
                C = run_launch(Workspace(), job, 1, xcd_of, rng, check_tags=False)
                caught["no tag check"] |= any(v not in ("ok", "nan") for v in C.values())
    assert all(caught.values()), caught
