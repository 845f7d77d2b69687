"""The workspace contract of the exchanging kernels (K-split and dense).

* Caller-owned workspace (bf_gemm_ws, bf_gemm_batched_ws, bf_busfill_q4_ws):
  the same bits as the calls on the library's workspace, with the size the
  size queries report; a workspace one byte too small is refused before
  anything is enqueued (C untouched).
* The library's workspace for a stream is never freed while a graph captured
  from the stream may use it: a graph holding a small K-split call, captured
  before a larger call grows the stream's workspace, replays correctly
  afterwards (against the oracle, several replays with eager work between).
* A call that would need to allocate while its stream is capturing enqueues
  nothing and returns BF_ERR_UNSUPPORTED (bf_gemm_batched included, which
  plans all its launches first).
* Host threads that share one stream while another grows its workspace get
  the bits of the single-threaded calls, also when both issue calls of two
  launches (dense GEMMs and their second-launch sums, the ggml hook's
  staging and GEMM) that share the stream's workspace.
All calls go through the C-ABI."""
import threading

import numpy as np
import pytest
import torch

import busfill as bf
import oracle as O

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    a = np.ascontiguousarray(a)
    return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)


def case(qt, N, K, M, seed, dev):
    w = O.gen_weights(qt, N, K, seed=seed)
    A = O.gen_act(M, K, seed=seed + 1)
    return w, to_dev(w.W, dev), (to_dev(w.W_aux, dev) if w.W_aux is not None else None), A, to_dev(A, dev)


def bits(C):
    a = C.cpu().numpy()
    return a.view(np.uint32 if a.dtype == np.float32 else np.uint16)


def workspace(nbytes, dev):
    """A 256-byte aligned device buffer of nbytes (None for 0)."""
    if nbytes == 0:
        return None
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=dev)
    off = (-buf.data_ptr()) % 256
    return buf, buf.data_ptr() + off


def new_stream():
    """A stream no earlier call has used (torch's streams come from a pool)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    h = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(h)) == 0
    return torch.cuda.ExternalStream(h.value)


@pytest.mark.parametrize("qt,N,K,M", [(O.Q4_K, 5120, 5120, 16), (O.Q4_K, 5120, 5120, 32), (O.Q4_0, 7168, 5120, 24),
                                      (O.Q4_K, 17408, 5120, 32), (O.Q4_K, 5120, 17408, 64),
                                      (O.Q4_0_PLANES, 5120, 5120, 128), (O.Q4_K, 5120, 5120, 200),
                                      (O.Q4_K, 5120, 5120, 1), (O.Q4_K, 5120, 5120, 8)])
def test_gemm_ws_matches_gemm(dev, qt, N, K, M):
    w, W, aux, A, Ad = case(qt, N, K, M, 40 + M, dev)
    need = bf.gemm_workspace_bytes(qt, M, N, K)
    if M > 8:
        assert need > 0, (qt, N, K, M)
    else:
        assert need == 0                      # the LDS-staged kernel exchanges nothing
    C0 = torch.full((M, N), float("nan"), device=dev)
    C1 = torch.full((M, N), float("nan"), device=dev)
    bf.gemm(qt, W, aux, Ad, C0, M, N, K)
    ws = workspace(need, dev)
    bf.gemm_ws(qt, W, aux, Ad, C1, M, N, K, ws[1] if ws else None, need)
    torch.cuda.synchronize()
    assert np.isfinite(C0.cpu().numpy()).all()
    assert (bits(C0) == bits(C1)).all(), (qt, N, K, M)
    if need:
        # one byte short: refused, nothing enqueued
        C2 = torch.full((M, N), 7.0, device=dev)
        with pytest.raises(bf.BusfillInvalid, match="workspace"):
            bf.gemm_ws(qt, W, aux, Ad, C2, M, N, K, ws[1], need - 1)
        torch.cuda.synchronize()
        assert (C2.cpu().numpy() == 7.0).all()


def test_gemm_ws_against_oracle_and_reuse(dev):
    """Two shapes in a row through one workspace (the larger first): both
    within the gate against the oracle."""
    shapes = [(O.Q4_K, 5120, 17408, 32), (O.Q4_0, 2048, 5120, 20)]
    need = max(bf.gemm_workspace_bytes(qt, M, N, K) for qt, N, K, M in shapes)
    ws = workspace(need, dev)
    for i, (qt, N, K, M) in enumerate(shapes):
        w, W, aux, A, Ad = case(qt, N, K, M, 60 + i, dev)
        C = torch.full((M, N), float("nan"), device=dev)
        bf.gemm_ws(qt, W, aux, Ad, C, M, N, K, ws[1], need)
        torch.cuda.synchronize()
        ok, mae, rfe, nf = O.gate(C.cpu().numpy().astype(np.float64), O.gemm_f64(w, A))
        assert ok, (qt, N, K, M, mae, rfe, nf)


def test_busfill_q4_ws_matches_busfill_q4(dev):
    """The reference-compatible entry at the reference's own Bsz = 32 (the
    K-split kernel) with a caller-owned workspace."""
    Bsz, N, K = 32, 5120, 5120
    w, W, aux, A, Ad = case(O.Q4_0_PLANES, N, K, Bsz, 70, dev)
    need = bf.gemm_workspace_bytes(O.Q4_0_PLANES, Bsz, N, K)
    assert need > 0
    ws = workspace(need, dev)
    C0 = torch.full((Bsz, N), float("nan"), device=dev)
    C1 = torch.full((Bsz, N), float("nan"), device=dev)
    bf.busfill_q4(Ad, W, aux, C0, Bsz, K, N)
    bf.busfill_q4_ws(Ad, W, aux, C1, Bsz, K, N, ws[1], need)
    torch.cuda.synchronize()
    assert (bits(C0) == bits(C1)).all()


@pytest.mark.parametrize("M", [1, 32, 128])
def test_gemm_batched_ws_matches_batched(dev, M):
    """A 27B-class decoder layer's five linears (at M = 32: two on the K-split
    kernel, three on the dense kernel) through one caller-owned workspace."""
    layer = [(7168, 5120), (5120, 5120), (17408, 5120), (17408, 5120), (5120, 17408)]
    keep, gem0, gem1 = [], [], []
    for i, (N, K) in enumerate(layer):
        w, W, aux, A, Ad = case(O.Q4_K, N, K, M, 80 + i, dev)
        C0 = torch.full((M, N), float("nan"), device=dev)
        C1 = torch.full((M, N), float("nan"), device=dev)
        keep += [W, Ad, C0, C1]
        gem0.append((W, None, Ad, C0, M, N, K))
        gem1.append((W, None, Ad, C1, M, N, K))
    need = bf.gemm_batched_workspace_bytes(O.Q4_K, gem1)
    assert (need > 0) == (M > 8)
    ws = workspace(need, dev)
    bf.gemm_batched(O.Q4_K, gem0)
    bf.gemm_batched_ws(O.Q4_K, gem1, ws[1] if ws else None, need)
    torch.cuda.synchronize()
    for (_, _, _, C0, *_), (_, _, _, C1, *_) in zip(gem0, gem1):
        assert np.isfinite(C0.cpu().numpy()).all()
        assert (bits(C0) == bits(C1)).all()
    if need:
        C = gem1[0][3]
        C.fill_(7.0)
        with pytest.raises(bf.BusfillInvalid, match="workspace"):
            bf.gemm_batched_ws(O.Q4_K, gem1, ws[1], need - 1)
        torch.cuda.synchronize()
        assert (C.cpu().numpy() == 7.0).all()


def test_graph_survives_workspace_growth(dev):
    """A graph captured with a small K-split call, the stream's workspace
    then grown by a larger call: every replay of the graph (with eager work
    and synchronizations between) matches the oracle and the eager result."""
    s = new_stream()
    N, K, M = 5120, 5120, 16
    w, W, aux, A, Ad = case(O.Q4_K, N, K, M, 90, dev)
    ref = O.gemm_f64(w, A)
    C = torch.full((M, N), float("nan"), device=dev)
    with torch.cuda.stream(s):
        bf.gemm(O.Q4_K, W, aux, Ad, C, M, N, K, stream=s)        # creates the stream's workspace
        s.synchronize()
        eager = C.cpu().numpy().copy()
        g = torch.cuda.CUDAGraph()
        C.fill_(float("nan"))
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            bf.gemm(O.Q4_K, W, aux, Ad, C, M, N, K, stream=s)
        # a larger call on the stream: more partials and slots than the first
        w2, W2, aux2, A2, Ad2 = case(O.Q4_K, 17408, 5120, 32, 91, dev)
        C2 = torch.full((32, 17408), float("nan"), device=dev)
        bf.gemm(O.Q4_K, W2, aux2, Ad2, C2, 32, 17408, 5120, stream=s)
        big = torch.empty(64 << 20, dtype=torch.uint8, device=dev).fill_(0xFF)   # memory traffic between
        s.synchronize()
        for r in range(4):
            C.fill_(float("nan"))
            s.synchronize()
            g.replay()
            s.synchronize()
            out = C.cpu().numpy()
            assert (out.view(np.uint32) == eager.view(np.uint32)).all(), r
            ok, mae, rfe, nf = O.gate(out.astype(np.float64), ref)
            assert ok, (r, mae, rfe, nf)
            big.add_(1)
            bf.gemm(O.Q4_K, W2, aux2, Ad2, C2, 32, 17408, 5120, stream=s)
    torch.cuda.synchronize()
    ok, mae, rfe, nf = O.gate(C2.cpu().numpy().astype(np.float64), O.gemm_f64(w2, A2))
    assert ok, (mae, rfe, nf)


def test_capture_without_workspace_enqueues_nothing(dev):
    """On a new stream, a K-split call and a batched call (whose first group
    needs no workspace, its second does) under capture: BF_ERR_UNSUPPORTED
    and nothing of the call in the graph; the same calls uncaptured then
    succeed."""
    s = new_stream()
    N, K = 5120, 5120
    _, W, aux, _, Ad32 = case(O.Q4_K, N, K, 32, 95, dev)
    _, W1, aux1, _, Ad1 = case(O.Q4_K, N, K, 1, 96, dev)
    C = torch.full((32, N), 7.0, device=dev)
    C1 = torch.full((1, N), 7.0, device=dev)
    gemms = [(W1, None, Ad1, C1, 1, N, K), (W1, None, Ad1, C1, 1, N, K), (W, None, Ad32, C, 32, N, K)]
    with torch.cuda.stream(s):
        for call in (lambda: bf.gemm(O.Q4_K, W, aux, Ad32, C, 32, N, K, stream=s),
                     lambda: bf.gemm_batched(O.Q4_K, gemms, stream=s)):
            g = torch.cuda.CUDAGraph()
            mark = torch.zeros(1, device=dev)
            with pytest.raises(bf.BusfillError, match="capture"):
                with torch.cuda.graph(g, stream=s):
                    mark.add_(1)                 # the graph is not empty
                    call()
            s.synchronize()
            assert (C.cpu().numpy() == 7.0).all() and (C1.cpu().numpy() == 7.0).all()
        bf.gemm_batched(O.Q4_K, gemms, stream=s)
        s.synchronize()
    assert np.isfinite(C.cpu().numpy()).all() and np.isfinite(C1.cpu().numpy()).all()


def test_threads_share_a_stream_while_it_grows(dev):
    """Two host threads issue calls on one stream; one of them grows the
    stream's workspace part way through.  Every output equals the
    single-threaded call's bits."""
    s = new_stream()
    N, K = 5120, 5120
    _, W, aux, _, Ad = case(O.Q4_K, N, K, 16, 97, dev)
    _, W2, aux2, _, Ad2 = case(O.Q4_K, 17408, 5120, 32, 98, dev)
    ref = torch.full((16, N), float("nan"), device=dev)
    ref2 = torch.full((32, 17408), float("nan"), device=dev)
    bf.gemm(O.Q4_K, W, aux, Ad, ref, 16, N, K)
    bf.gemm(O.Q4_K, W2, aux2, Ad2, ref2, 32, 17408, 5120)
    torch.cuda.synchronize()
    outs_a = [torch.full((16, N), float("nan"), device=dev) for _ in range(40)]
    outs_b = [torch.full((32, 17408), float("nan"), device=dev) for _ in range(4)]
    errors = []

    def run(fn):
        try:
            fn()
        except Exception as e:          # noqa: BLE001 -- reported by the main thread
            errors.append(e)

    def a():
        for C in outs_a:
            bf.gemm(O.Q4_K, W, aux, Ad, C, 16, N, K, stream=s)

    def b():
        for C in outs_b:
            bf.gemm(O.Q4_K, W2, aux2, Ad2, C, 32, 17408, 5120, stream=s)

    ts = [threading.Thread(target=run, args=(f,)) for f in (a, b)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    s.synchronize()
    assert not errors, errors
    for C in outs_a:
        assert (bits(C) == bits(ref)).all()
    for C in outs_b:
        assert (bits(C) == bits(ref2)).all()


def test_threads_interleave_two_launch_calls_on_one_stream(dev):
    """Two host threads issue calls of two launches each on one stream: dense
    GEMMs (the kernel, then the second-launch sum of its partial pieces) and
    ggml mul_mat calls with fp32 activations (a staging launch, then the
    GEMM), with different operands per thread.  The launches of one call stay
    together on the stream, so no thread's partials or staged activations are
    overwritten by the other's between its two launches: every output equals
    the single-threaded call's bits."""
    s = new_stream()
    N, K, M, MG = 5120, 5120, 64, 4
    ops = []
    for t in range(2):
        _, W, aux, _, Ad = case(O.Q4_K, N, K, M, 200 + 10 * t, dev)
        x = torch.from_numpy(np.random.default_rng(300 + t).standard_normal((MG, K)).astype(np.float32)).to(dev)
        ops.append((W, Ad, x))

    def gemm_call(t, C):
        W, Ad, _ = ops[t]
        bf.gemm(O.Q4_K, W, None, Ad, C, M, N, K, stream=s)

    def ggml_call(t, D):
        W, _, x = ops[t]
        bf.ggml_mul_mat(bf.ggml_view(W, bf.GGML_Q4_K), bf.ggml_view(x, bf.GGML_F32), bf.ggml_view(D), stream=s)

    refs = []
    for t in range(2):
        C = torch.full((M, N), float("nan"), device=dev)
        D = torch.full((MG, N), float("nan"), device=dev)
        gemm_call(t, C)
        ggml_call(t, D)
        s.synchronize()
        assert np.isfinite(C.cpu().numpy()).all() and np.isfinite(D.cpu().numpy()).all()
        refs.append((bits(C), bits(D)))
    assert not (refs[0][0] == refs[1][0]).all() and not (refs[0][1] == refs[1][1]).all()
    outs = [[(torch.full((M, N), float("nan"), device=dev), torch.full((MG, N), float("nan"), device=dev))
             for _ in range(24)] for _ in range(2)]
    errors = []

    def run(t):
        try:
            for C, D in outs[t]:
                gemm_call(t, C)
                ggml_call(t, D)
        except Exception as e:          # noqa: BLE001 -- reported by the main thread
            errors.append(e)

    ts = [threading.Thread(target=run, args=(t,)) for t in range(2)]
    for th in ts:
        th.start()
    for th in ts:
        th.join()
    s.synchronize()
    assert not errors, errors
    for t in range(2):
        for C, D in outs[t]:
            assert (bits(C) == refs[t][0]).all()
            assert (bits(D) == refs[t][1]).all()
