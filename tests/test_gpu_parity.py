"""GPU parity of libbusfill against the CPU oracle (run on an MI355X).

Bar: bit-exact for the fp16 dequant.  For the GEMM, every value finite, and
  * max |C - ref| <= 0.6 (the repo gate, kernels/q4k_batched.py:102) and
    relative Frobenius error <= 1e-3, where ref is the fp64 dequantize-then-
    matmul of the reference check (kernels/busfill_v1a.cu:159-167) over the
    oracle's unrounded weights -- applied when the output has >= 64 elements
    (on one or two outputs the relative error of fp16 weights alone can exceed
    1e-3);
  * an elementwise forward-error bound for the kernel's weight form, which any
    wrong index, scale or dropped term exceeds by orders of magnitude:
      fp16 weights (the reference kernel's form, kernels/busfill_v1a.cu:85-86):
        |C - ref16| <= 1e-4 * (|A| . |W16|^T) + 1e-6, ref16 the fp64 matmul
        over the bit-exact fp16 dequant W16;
      factored Q4_K (d * sum a (sc q) - dmin * sum m S, unrounded weights):
        |C - ref| <= 1e-4 * (|A| . (|d sc q| + |dmin m|)^T) + 1e-6, the bound
        for the difference of the two terms, whose sizes the oracle gives as
        the dequant with dmin = 0 and with d = 0.
All calls go through the C-ABI (busfill.* are thin ctypes wrappers).
"""
import numpy as np
import pytest
import torch

import busfill as bf
import oracle as O

pytestmark = pytest.mark.gpu

QTS = [O.Q4_0_PLANES, O.Q4_0, O.Q4_K]
QT_NAME = {O.Q4_0_PLANES: "planes", O.Q4_0: "q4_0", O.Q4_K: "q4_k"}


def to_dev(a, dev):
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return torch.from_numpy(a).to(dev)


def upload(w, dev):
    return to_dev(w.W, dev), (to_dev(w.W_aux, dev) if w.W_aux is not None else None)


def gpu_gemm(w, A, dev, algo=bf.ALGO_AUTO, otype=bf.OUT_F32, dw=None):
    M = A.shape[0]
    Wd, auxd = dw if dw is not None else upload(w, dev)
    Ad = to_dev(A, dev)
    C = torch.full((M, w.N), float("nan"), device=dev,
                   dtype=torch.float32 if otype == bf.OUT_F32 else torch.float16)
    bf.gemm(w.qtype, Wd, auxd, Ad, C, M, w.N, w.K, otype=otype, algo=algo)
    torch.cuda.synchronize()
    return C.float().cpu().numpy().astype(np.float64)


def gpu_dequant(w, dev):
    Wd, auxd = upload(w, dev)
    out = torch.empty((w.N, w.K), dtype=torch.int16, device=dev)
    bf.dequant_f16(w.qtype, Wd, auxd, out, w.N, w.K)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16)


def assert_gate(C, ref, what):
    ok, mae, rfe, nf = O.gate(C, ref)
    assert ok, f"{what}: max_abs={mae:.4g} rel_frob={rfe:.3g} nonfinite={nf}"
    return mae, rfe


def q4k_term_sizes(w):
    """|d sc q| + |dmin m| per weight of a Q4_K matrix, from the oracle's
    unrounded dequant of two copies: dmin zeroed (d sc q) and d zeroed (-dmin m)."""
    blk = w.W.reshape(-1, 144)
    wd, wm = blk.copy(), blk.copy()
    wd[:, 2:4] = 0
    wm[:, 0:2] = 0
    t1 = O.dequant_f32(O.QWeights(O.Q4_K, w.N, w.K, wd.reshape(w.W.shape)))
    t2 = O.dequant_f32(O.QWeights(O.Q4_K, w.N, w.K, wm.reshape(w.W.shape)))
    return np.abs(t1) + np.abs(t2)


class Ref:
    """Oracle references for weights w and activations A (rows sliceable).

    check(form=...): "f16" for fp16-weight kernels, "f32" for the forms that
    scale exact codes in fp32 (factored Q4_K, and the batch-1 sub-block rows
    form of every format); None accepts either (automatic kernel choice)."""

    def __init__(self, w, A):
        self.exact = O.gemm_f64(w, A)
        self.f16w = O.gemm_f64(w, A, round_w=True)
        Aabs = np.abs(A.view(np.float16).astype(np.float32))
        W16 = np.abs(O.dequant_f16(w).view(np.float16).astype(np.float32))
        self.bounds = {"f16": (self.f16w, 1e-4 * (Aabs @ W16.T).astype(np.float64) + 1e-6)}
        if w.qtype == O.Q4_K:
            self.bounds["f32"] = (self.exact, 1e-4 * (Aabs @ q4k_term_sizes(w).T).astype(np.float64) + 1e-6)
        else:
            # (q - 8) d is exact in fp32: the unrounded weights' magnitudes
            W32 = np.abs(O.dequant_f32(w))
            self.bounds["f32"] = (self.exact, 1e-4 * (Aabs @ W32.T).astype(np.float64) + 1e-6)

    def check(self, C, what, rows=None, form=None):
        sl = slice(None) if rows is None else slice(0, rows)
        assert np.isfinite(C).all(), f"{what}: non-finite output"
        forms = [form] if form is not None else list(self.bounds)
        excess = {}
        for f in forms:
            if f not in self.bounds:
                continue
            ref, bound = self.bounds[f]
            excess[f] = float((np.abs(C - ref[sl]) / bound[sl]).max()) if C.size else 0.0
        assert excess, f"{what}: no bound for form {form}"
        assert min(excess.values()) <= 1.0, f"{what}: beyond the forward-error bound, worst excess {excess}"
        if C.size >= 64:
            assert_gate(C, self.exact[sl], what)


def check_gemm(C, w, A, what):
    Ref(w, A).check(C, what)


# ------------------------------------------------------------------ dequant
@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("N,K", [(64, 256), (37, 5120), (16, 17408)])
def test_dequant_bitexact(dev, qt, N, K):
    w = O.gen_weights(qt, N, K, seed=N * 7 + K)
    assert (gpu_dequant(w, dev) == O.dequant_f16(w)).all()


def test_dequant_bitexact_every_finite_scale(dev):
    scales = np.arange(65536, dtype=np.uint16)
    scales = scales[(scales & 0x7C00) != 0x7C00]
    K = 512
    N = scales.size // (K // 32)
    j = np.arange(16, dtype=np.uint8)
    Wq = np.tile((j | ((15 - j) << 4)).astype(np.uint8), (N, K // 32))
    w = O.QWeights(O.Q4_0_PLANES, N, K, Wq, scales.reshape(N, K // 32).copy())
    assert (gpu_dequant(w, dev) == O.dequant_f16(w)).all()
    b = O.planes_to_blocks(w)
    assert (gpu_dequant(b, dev) == O.dequant_f16(b)).all()


def test_dequant_q4k_extreme_scales(dev):
    # d and dmin over many binades (incl. subnormal and negative), all 6-bit codes
    rng = np.random.default_rng(5)
    w = O.gen_weights(O.Q4_K, 64, 4096, seed=77)
    blk = w.W.reshape(-1, 144)
    finite = np.arange(65536, dtype=np.uint16)
    finite = finite[((finite & 0x7C00) != 0x7C00) & ((finite & 0x7FFF) < 0x5000)]   # |x| < 32
    hd = rng.choice(finite, blk.shape[0]).astype(np.uint16)
    hm = rng.choice(finite, blk.shape[0]).astype(np.uint16)
    blk[:, 0:2] = hd.view(np.uint8).reshape(-1, 2)
    blk[:, 2:4] = hm.view(np.uint8).reshape(-1, 2)
    assert (gpu_dequant(w, dev) == O.dequant_f16(w)).all()


# ------------------------------------------------------------------ GEMM parity
M_LIST = [1, 2, 3, 4, 8, 15, 16, 17, 31, 32, 33, 64, 128]


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("K", [5120, 17408])
def test_gemm_parity_batch_sweep(dev, qt, K):
    N = 200                                   # not a multiple of 16: masked tail tile
    w = O.gen_weights(qt, N, K, seed=K + qt)
    dw = upload(w, dev)
    A_all = O.gen_act(max(M_LIST), K, seed=K * 3 + qt)
    ref = Ref(w, A_all)
    for M in M_LIST:
        for algo in (bf.ALGO_AUTO, bf.ALGO_MFMA):
            C = gpu_gemm(w, A_all[:M], dev, algo=algo, dw=dw)
            ref.check(C, f"{QT_NAME[qt]} K={K} M={M} algo={algo}", rows=M,
                      form=None if algo == bf.ALGO_AUTO else "f16")


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("M", [1, 8, 32])
def test_gemm_full_size_5120(dev, qt, M):
    w = O.gen_weights(qt, 5120, 5120, seed=1000 + qt)
    A = O.gen_act(M, 5120, seed=2000 + M)
    check_gemm(gpu_gemm(w, A, dev), w, A, f"{QT_NAME[qt]} 5120^2 M={M}")


@pytest.mark.parametrize("N,K", [(7168, 5120), (17408, 5120), (5120, 17408)])
def test_gemm_layer_shapes_q4k(dev, N, K):
    w = O.gen_weights(O.Q4_K, N, K, seed=N + K)
    A = O.gen_act(4, K, seed=N)
    check_gemm(gpu_gemm(w, A, dev), w, A, f"q4_k {N}x{K} M=4")


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
def test_gemm_simple_path_matches(dev, qt):
    w = O.gen_weights(qt, 48, 1024, seed=31)
    A = O.gen_act(5, 1024, seed=32)
    check_gemm(gpu_gemm(w, A, dev, algo=bf.ALGO_SIMPLE), w, A, "simple")


@pytest.mark.parametrize("qt,K", [(O.Q4_0_PLANES, 32 * 5), (O.Q4_0, 32 * 37), (O.Q4_K, 256 * 3)])
def test_gemm_odd_shapes(dev, qt, K):
    # K not a multiple of 256 (Q4_0 formats) and tiny / ragged N, M
    for N, M in [(1, 1), (17, 3), (100, 9)]:
        w = O.gen_weights(qt, N, K, seed=N + K)
        A = O.gen_act(M, K, seed=M + K)
        check_gemm(gpu_gemm(w, A, dev), w, A, f"{QT_NAME[qt]} N={N} K={K} M={M}")


def test_gemm_large_m_is_sliced(dev):
    w = O.gen_weights(O.Q4_K, 64, 1024, seed=41)
    A = O.gen_act(300, 1024, seed=42)
    check_gemm(gpu_gemm(w, A, dev), w, A, "M=300")


# ------------------------------------------------------------------ interface behaviour
def test_reference_entry_beyond_32_rows(dev):
    """bf_busfill_q4 keeps busfill_q4's arguments; rows >= 32 are computed (the
    reference dropped them, kernels/busfill_v1a.cu:55-56,98-99)."""
    N, K, B = 512, 5120, 40
    w = O.gen_weights(O.Q4_0_PLANES, N, K, seed=51)
    A = O.gen_act(B, K, seed=52)
    Wq, Ws = upload(w, dev)
    Ad = to_dev(A, dev)
    C = torch.full((B, N), float("nan"), device=dev)
    bf.busfill_q4(Ad, Wq, Ws, C, B, K, N)
    torch.cuda.synchronize()
    check_gemm(C.cpu().numpy().astype(np.float64), w, A, "busfill_q4 B=40")


def test_strided_operands_and_untouched_rows(dev):
    N, K, M = 96, 2048, 5
    lda, ldc = K + 24, N + 40
    w = O.gen_weights(O.Q4_K, N, K, seed=61)
    A = O.gen_act(M, K, seed=62)
    Apad = np.zeros((M, lda), np.uint16)
    Apad[:, :K] = A
    Wd, _ = upload(w, dev)
    Ad = to_dev(Apad, dev)
    C = torch.full((M + 2, ldc), 12345.0, device=dev)
    bf.gemm(O.Q4_K, Wd, None, Ad, C, M, N, K, lda=lda, ldc=ldc)
    torch.cuda.synchronize()
    Ch = C.cpu().numpy()
    check_gemm(Ch[:M, :N].astype(np.float64), w, A, "strided")
    assert (Ch[:M, N:] == 12345.0).all() and (Ch[M:] == 12345.0).all()


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
def test_output_f16(dev, qt):
    w = O.gen_weights(qt, 256, 5120, seed=71)
    A = O.gen_act(16, 5120, seed=72)
    dw = upload(w, dev)
    C16 = gpu_gemm(w, A, dev, otype=bf.OUT_F16, dw=dw)
    C32 = gpu_gemm(w, A, dev, otype=bf.OUT_F32, dw=dw)
    assert_gate(C16, O.gemm_f64(w, A), "f16 out")
    assert (C32.astype(np.float32).astype(np.float16).astype(np.float64) == C16).all()


def test_nan_injection_fails_the_gate(dev):
    w = O.gen_weights(O.Q4_K, 128, 1024, seed=81)
    A = O.gen_act(4, 1024, seed=82)
    A[1, 7] = 0x7E00                       # fp16 NaN
    C = gpu_gemm(w, A, dev)
    ref = O.gemm_f64(w, O.gen_act(4, 1024, seed=82))
    assert not np.isfinite(C[1]).any()
    assert np.isfinite(C[[0, 2, 3]]).all()
    assert not O.gate(C, ref)[0]
    assert O.gate(C[[0, 2, 3]], ref[[0, 2, 3]])[0]


def test_one_hot_probe_of_output_scatter(dev):
    """frag_probe-style known answers: one nonzero weight and one nonzero
    activation must land on exactly one output element."""
    N, K, M = 48, 512, 128
    Ws = np.full((N, K // 32), np.float16(1.0).view(np.uint16), np.uint16)
    for (m, n, k) in [(0, 0, 0), (5, 15, 7), (17, 16, 8), (127, 33, 31), (64, 47, 32), (9, 3, 255), (33, 20, 333)]:
        Wq = np.full((N, K // 2), 0x88, np.uint8)                # every weight 0
        byte = Wq[n, k // 2]
        Wq[n, k // 2] = (byte & 0xF0) | 0x9 if k % 2 == 0 else (byte & 0x0F) | 0x90   # weight 1 at (n, k)
        A = np.zeros((M, K), np.uint16)
        A[m, k] = np.float16(2.0).view(np.uint16)
        w = O.QWeights(O.Q4_0_PLANES, N, K, Wq, Ws)
        for algo in (bf.ALGO_AUTO, bf.ALGO_MFMA, bf.ALGO_SIMPLE):
            C = gpu_gemm(w, A, dev, algo=algo)
            expect = np.zeros((M, N))
            expect[m, n] = 2.0
            assert (C == expect).all(), (m, n, k, algo)


@pytest.mark.parametrize("qt", [O.Q4_0, O.Q4_K], ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("N,K", [(1, 256), (77, 2048), (200, 5120), (5120, 5120), (600, 17408)])
def test_slab_batch_parity(dev, qt, N, K):
    """The slab-streamed kernel (weights + activation slabs through an LDS ring):
    one or two row tiles per workgroup, ragged N, ring wrap-around (K = 17408 has
    68 steps over 5 slots), every batch size it serves."""
    w = O.gen_weights(qt, N, K, seed=K * 7 + N + qt)
    dw = upload(w, dev)
    A = O.gen_act(32, K, seed=K + 13)
    ref = Ref(w, A)
    for M in (1, 5, 9, 16, 17, 31, 32):
        C = gpu_gemm(w, A[:M], dev, algo=bf.ALGO_SLAB, dw=dw)
        ref.check(C, f"slab {QT_NAME[qt]} N={N} K={K} M={M}", rows=M, form="f16")
        assert (gpu_gemm(w, A[:M], dev, algo=bf.ALGO_SLAB, dw=dw) == C).all()
    with pytest.raises(bf.BusfillError):                  # M > 32 is not served
        gpu_gemm(w, O.gen_act(33, K, seed=1), dev, algo=bf.ALGO_SLAB, dw=dw)


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("N,K", [(1, 256), (77, 2048), (200, 5120), (5120, 5120), (600, 17408), (7168, 5120)])
def test_split_batch_parity(dev, qt, N, K):
    """The K-split kernel: splits combined through the per-stream workspace
    (last split adds them in split order), ragged N (clamped weight rows), every
    batch size it serves, identical results on repeated runs."""
    w = O.gen_weights(qt, N, K, seed=K * 11 + N + qt)
    dw = upload(w, dev)
    A = O.gen_act(32, K, seed=K + 17)
    ref = Ref(w, A)
    for M in (1, 5, 9, 16, 17, 31, 32):
        C = gpu_gemm(w, A[:M], dev, algo=bf.ALGO_SPLIT, dw=dw)
        ref.check(C, f"split {QT_NAME[qt]} N={N} K={K} M={M}", rows=M, form="f16")
        assert (gpu_gemm(w, A[:M], dev, algo=bf.ALGO_SPLIT, dw=dw) == C).all()
    with pytest.raises(bf.BusfillError):                  # M > 32 is not served
        gpu_gemm(w, O.gen_act(33, K, seed=1), dev, algo=bf.ALGO_SPLIT, dw=dw)


def test_split_exchange_on_every_stream(dev):
    """The K-split kernel's XCD-local exchange on streams whose hardware queues
    start the workgroup round robin on different XCDs (the null stream and
    several created streams): finite, identical bits on every stream, and
    single and batched launches agree on each (a workgroup takes its row group
    from the XCD it runs on, whatever the starting XCD)."""
    N, K, M = 5120, 5120, 32
    w = O.gen_weights(O.Q4_K, N, K, seed=41)
    dw = upload(w, dev)
    A = O.gen_act(M, K, seed=42)
    Ad = to_dev(A, dev)
    ref = None
    streams = [None] + [torch.cuda.Stream() for _ in range(5)]
    torch.cuda.synchronize()
    for i, s in enumerate(streams):
        C = torch.full((M, N), float("nan"), device=dev)
        C2 = torch.full((M, N), float("nan"), device=dev)
        st = s.cuda_stream if s is not None else 0
        bf.gemm(O.Q4_K, dw[0], None, Ad, C, M, N, K, algo=bf.ALGO_SPLIT, stream=st)
        d = (bf.GemmDesc * 2)(bf.GemmDesc(dw[0].data_ptr(), None, Ad.data_ptr(), K, C2.data_ptr(), N, M, N // 2, K),
                              bf.GemmDesc(dw[0].data_ptr() + (N // 2) * (K // 256) * 144, None, Ad.data_ptr(), K,
                                          C2.data_ptr() + (N // 2) * 4, N, M, N // 2, K))
        assert bf.lib().bf_gemm_batched(O.Q4_K, bf.OUT_F32, 2, d, st) == 0
        torch.cuda.synchronize()
        got = C.cpu().numpy().astype(np.float64)
        assert np.isfinite(got).all(), f"stream {i}"
        if ref is None:
            ref = got
            Ref(w, A).check(got, "split on the null stream", form="f16")
        assert (got == ref).all(), f"stream {i}"
        assert np.isfinite(C2.cpu().numpy()).all(), f"batched, stream {i}"


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("N,K", [(1, 256), (77, 2048), (200, 5120), (5120, 5120), (600, 17408), (7168, 5120)])
def test_dense_batch_parity(dev, qt, N, K):
    """The dense kernel (all batch rows of a launch per workgroup, the weights
    streamed once): ragged N (clamped weight rows), batches of 1-128 rows (one
    to four 32-row m-tiles, padded rows), row groups split between workgroups
    and summed by the second launch, fp16 weights, identical results on
    repeated runs."""
    w = O.gen_weights(qt, N, K, seed=K * 13 + N + qt)
    dw = upload(w, dev)
    A = O.gen_act(128, K, seed=K + 19)
    ref = Ref(w, A)
    # (79 / 80: the last batch with two compute waves per SIMD and the first with one)
    for M in (1, 9, 17, 32, 33, 48, 64, 65, 79, 80, 96, 100, 128):
        C = gpu_gemm(w, A[:M], dev, algo=bf.ALGO_DENSE, dw=dw)
        ref.check(C, f"dense {QT_NAME[qt]} N={N} K={K} M={M}", rows=M, form="f16")
        assert (gpu_gemm(w, A[:M], dev, algo=bf.ALGO_DENSE, dw=dw) == C).all()
    # more than 128 rows: launches of 128 rows and the rest
    A2 = O.gen_act(130, K, seed=K + 23)
    Ref(w, A2).check(gpu_gemm(w, A2, dev, algo=bf.ALGO_DENSE, dw=dw), f"dense {QT_NAME[qt]} N={N} K={K} M=130",
                     form="f16")


def test_split_workspace_reuse_across_shapes(dev):
    """Launches of different shapes back to back on one stream share its
    workspace: the per-row-group counters must be back at zero after every
    launch, or a later launch would finish with the wrong split."""
    cases = [(5120, 5120, 32), (200, 5120, 9), (7168, 5120, 17), (5120, 5120, 32), (600, 17408, 32)]
    prepared = []
    for i, (N, K, M) in enumerate(cases):
        w = O.gen_weights(O.Q4_K, N, K, seed=300 + i)
        A = O.gen_act(M, K, seed=400 + i)
        prepared.append((w, upload(w, dev), A, Ref(w, A)))
    outs = []
    for rep in range(3):
        for (w, dw, A, _) in prepared:
            Ad = to_dev(A, dev)
            Cd = torch.full((A.shape[0], w.N), float("nan"), device=dev)
            bf.gemm(w.qtype, dw[0], dw[1], Ad, Cd, A.shape[0], w.N, w.K, algo=bf.ALGO_SPLIT)
            outs.append(Cd)
    torch.cuda.synchronize()
    for rep in range(3):
        for i, (w, _, A, ref) in enumerate(prepared):
            C = outs[rep * len(prepared) + i].cpu().numpy().astype(np.float64)
            ref.check(C, f"split reuse rep={rep} case={i}", form="f16")
            assert (C == outs[i].cpu().numpy()).all()


def test_one_hot_probe_lds_segments(dev):
    """Known answers for the K-segment mapping of the LDS-staged kernel: one
    weight (n, k) and one activation (m, k) set, everything else zero, for k in
    every segment and sub-block and m across the batch rows of each segment."""
    N, K, M = 24, 2048, 8
    Ws = np.full((N, K // 32), np.float16(1.0).view(np.uint16), np.uint16)
    cases = [(0, 0, 0), (7, 23, 2047), (3, 5, 256), (4, 6, 511), (1, 17, 1024 + 33), (6, 8, 1536 + 255),
             (2, 3, 768 + 64), (5, 12, 300)]
    for (m, n, k) in cases:
        Wq = np.full((N, K // 2), 0x88, np.uint8)
        byte = Wq[n, k // 2]
        Wq[n, k // 2] = (byte & 0xF0) | 0x9 if k % 2 == 0 else (byte & 0x0F) | 0x90
        w = O.QWeights(O.Q4_0_PLANES, N, K, Wq, Ws)
        for Mb in (1, 4, 8):
            if m >= Mb:
                continue
            A = np.zeros((Mb, K), np.uint16)
            A[m, k] = np.float16(-3.0).view(np.uint16)
            expect = np.zeros((Mb, N))
            expect[m, n] = -3.0
            for ww in (w, O.planes_to_blocks(w)):
                C = gpu_gemm(ww, A, dev, algo=bf.ALGO_LDS)
                assert (C == expect).all(), (m, n, k, Mb, ww.qtype)


def test_one_hot_probe_lds_q4k_factored(dev):
    """Known answers for the factored Q4_K form of the LDS-staged kernel: with a
    single activation a at (m, k), row m of C is a times column k of the
    unrounded weights (every sub-block's scale and min, through the block-sum
    table) and every other row is exactly zero."""
    N, K = 24, 2048
    w = O.gen_weights(O.Q4_K, N, K, seed=404)
    dw = upload(w, dev)
    W32 = O.dequant_f32(w).astype(np.float64)
    mag = q4k_term_sizes(w).astype(np.float64)
    for (m, k) in [(0, 0), (7, 2047), (3, 256 + 31), (4, 511), (1, 1024 + 32), (6, 1536 + 200), (2, 64), (5, 95)]:
        for Mb in (1, 4, 8):
            if m >= Mb:
                continue
            a = -3.0
            A = np.zeros((Mb, K), np.uint16)
            A[m, k] = np.float16(a).view(np.uint16)
            C = gpu_gemm(w, A, dev, algo=bf.ALGO_LDS, dw=dw)
            others = np.delete(C, m, axis=0)
            assert (others == 0).all(), (m, k, Mb)
            err = np.abs(C[m] - a * W32[:, k])
            assert (err <= 1e-4 * abs(a) * mag[:, k] + 1e-6).all(), (m, k, Mb, float(err.max()))


def test_formats_agree_bitwise_and_runs_are_deterministic(dev):
    """Planes and llama.cpp blocks holding the same weights: bit-identical at
    batch 8 and 32 (same fp16 weights in the same MFMA k slots).  At batch 1
    the sub-block rows form feeds the codes in each layout's own nibble order,
    so the fp32 sums are grouped differently: both stay within the exact-weight
    bound and agree to a few ulps of the sums' magnitude."""
    w = O.gen_weights(O.Q4_0_PLANES, 1024, 5120, seed=91)
    b = O.planes_to_blocks(w)
    for M in (1, 8, 32):
        A = O.gen_act(M, 5120, seed=92)
        Cp = gpu_gemm(w, A, dev)
        Cb = gpu_gemm(b, A, dev)
        if M == 1:
            ref = Ref(w, A)
            ref.check(Cp, "planes M=1", form="f32")
            ref.check(Cb, "blocks M=1", form="f32")
            _, bound = ref.bounds["f32"]
            assert (np.abs(Cp - Cb) <= 0.01 * bound).all()
        else:
            assert (Cp == Cb).all()
        assert (gpu_gemm(w, A, dev) == Cp).all()
        assert (gpu_gemm(b, A, dev) == Cb).all()


BATCH_SHAPES = [(1792, 5120), (1280, 5120), (600, 17408), (77, 2048), (5120, 5120)]


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("Ms,otype", [((32,) * 5, bf.OUT_F32), ((16,) * 5, bf.OUT_F32), ((32,) * 5, bf.OUT_F16),
                                      ((1,) * 5, bf.OUT_F32), ((1,) * 5, bf.OUT_F16), ((2,) * 5, bf.OUT_F32),
                                      ((8,) * 5, bf.OUT_F32), ((32, 32, 1, 32, 9), bf.OUT_F32)],
                         ids=["m32", "m16", "m32-f16", "m1", "m1-f16", "m2", "m8", "mixed"])
def test_batched_matches_single_launches(dev, qt, Ms, otype):
    """bf_gemm_batched: GEMMs of different shapes in one call give bit-identical
    results to one bf_gemm each (one launch when all of them take the same
    LDS-staged kernel shape or all are K-split GEMMs, one launch per GEMM
    otherwise), and the per-stream workspace stays consistent when single and
    batched calls alternate."""
    ws = [O.gen_weights(qt, N, K, seed=N + K + 13 * qt + i) for i, (N, K) in enumerate(BATCH_SHAPES)]
    dws = [upload(w, dev) for w in ws]
    As = [O.gen_act(M, w.K, seed=w.K + 7 * i) for i, (M, w) in enumerate(zip(Ms, ws))]
    dAs = [to_dev(A, dev) for A in As]
    dt = torch.float32 if otype == bf.OUT_F32 else torch.float16
    for rep in range(2):
        singles = [gpu_gemm(w, A, dev, otype=otype, dw=dw) for w, A, dw in zip(ws, As, dws)]
        Cs = [torch.full((M, w.N), float("nan"), device=dev, dtype=dt) for M, w in zip(Ms, ws)]
        bf.gemm_batched(qt, [(dw[0], dw[1], dA, C, M, w.N, w.K) for dw, dA, C, M, w in zip(dws, dAs, Cs, Ms, ws)],
                        otype=otype)
        torch.cuda.synchronize()
        for i, (C, ref) in enumerate(zip(Cs, singles)):
            got = C.float().cpu().numpy().astype(np.float64)
            assert (got == ref).all(), (rep, i, BATCH_SHAPES[i], Ms[i])
            if rep == 0:
                # and each batched output against the oracle itself
                if otype == bf.OUT_F32:
                    Ref(ws[i], As[i]).check(got, f"batched {QT_NAME[qt]} {BATCH_SHAPES[i]} M={Ms[i]}")
                else:
                    assert_gate(got, O.gemm_f64(ws[i], As[i]), f"batched f16 {QT_NAME[qt]} {BATCH_SHAPES[i]}")


def test_batched_matches_single_launches_large_matrices(dev):
    """bf_gemm sums a K-split GEMM whose grid takes more than one workgroup per
    CU in a second launch (k_split_sum) and sends 9-32 rows on matrices of
    3 * 2^24 weights or more to the dense kernel; bf_gemm_batched's one launch
    sums splits in-kernel.  Same split order, so the same bits; a GEMM that
    bf_gemm gives the dense kernel goes to the batch's dense launch."""
    for shapes in ([(17408, 5120, 16), (7168, 5120, 16)], [(7168, 5120, 32), (1792, 5120, 32)],
                   [(5120, 17408, 32), (1792, 5120, 32)]):
        ws = [O.gen_weights(O.Q4_K, N, K, seed=N + K + M) for N, K, M in shapes]
        dws = [upload(w, dev) for w in ws]
        As = [O.gen_act(M, K, seed=K + M + i) for i, (N, K, M) in enumerate(shapes)]
        singles = [gpu_gemm(w, A, dev, dw=dw) for w, A, dw in zip(ws, As, dws)]
        Cs = [torch.full((M, N), float("nan"), device=dev) for N, K, M in shapes]
        bf.gemm_batched(O.Q4_K, [(dw[0], dw[1], to_dev(A, dev), C, M, N, K)
                                 for dw, A, C, (N, K, M) in zip(dws, As, Cs, shapes)])
        torch.cuda.synchronize()
        for i, (C, ref) in enumerate(zip(Cs, singles)):
            got = C.cpu().numpy().astype(np.float64)
            assert (got == ref).all(), shapes[i]
            Ref(ws[i], As[i]).check(got, f"batched q4_k {shapes[i]}")


@pytest.mark.parametrize("M,shapes", [
    (32, [(7168, 5120), (5120, 5120), (17408, 5120), (17408, 5120), (5120, 17408)]),   # a 27B-class layer
    (64, [(200, 5120), (5120, 2048), (77, 2048), (1792, 5120)]),
    (128, [(5120, 5120), (300, 1024)]),
    (9, [(17408, 5120), (5120, 17408), (1000, 2048)]),
], ids=["layer-m32", "m64", "m128", "m9"])
def test_batched_groups_by_kernel(dev, M, shapes):
    """bf_gemm_batched groups the GEMMs by the kernel bf_gemm gives each: the
    K-split ones share a launch, the dense ones share a launch (each with the
    ranges of a launch of its own) and one sum launch.  Bit-identical to one
    bf_gemm per GEMM, twice in a row (the workspace reused), and the smaller
    outputs against the oracle."""
    ws = [O.gen_weights(O.Q4_K, N, K, seed=N + 3 * K + M) for N, K in shapes]
    dws = [upload(w, dev) for w in ws]
    As = [O.gen_act(M, K, seed=K + M + i) for i, (N, K) in enumerate(shapes)]
    dAs = [to_dev(A, dev) for A in As]
    for rep in range(2):
        singles = [gpu_gemm(w, A, dev, dw=dw) for w, A, dw in zip(ws, As, dws)]
        Cs = [torch.full((M, N), float("nan"), device=dev) for N, K in shapes]
        bf.gemm_batched(O.Q4_K, [(dw[0], dw[1], dA, C, M, N, K) for dw, dA, C, (N, K) in zip(dws, dAs, Cs, shapes)])
        torch.cuda.synchronize()
        for i, (C, ref) in enumerate(zip(Cs, singles)):
            got = C.cpu().numpy().astype(np.float64)
            assert np.isfinite(got).all(), (rep, shapes[i])
            assert (got == ref).all(), (rep, shapes[i], M)
            if rep == 0 and shapes[i][0] * shapes[i][1] <= 5120 * 5120:
                Ref(ws[i], As[i]).check(got, f"batched q4_k {shapes[i]} M={M}")


def test_batched_mixed_batch_sizes(dev):
    """One bf_gemm_batched call holding GEMMs of several batch sizes: each
    kernel's group is split by batch size (dense at 32 and 64 rows, the
    LDS-staged kernel at 1 row, the K-split kernel at 16 rows), and every
    output is bit-identical to its own bf_gemm call."""
    descs = [(17408, 5120, 32), (5120, 17408, 32), (17408, 5120, 64), (5120, 17408, 64),
             (5120, 5120, 1), (7168, 5120, 1), (5120, 5120, 16), (7168, 5120, 16), (2048, 1024, 3)]
    ws = [O.gen_weights(O.Q4_K, N, K, seed=N + K + M) for N, K, M in descs]
    dws = [upload(w, dev) for w in ws]
    As = [O.gen_act(M, K, seed=7 * i + M) for i, (N, K, M) in enumerate(descs)]
    dAs = [to_dev(A, dev) for A in As]
    singles = [gpu_gemm(w, A, dev, dw=dw) for w, A, dw in zip(ws, As, dws)]
    Cs = [torch.full((M, N), float("nan"), device=dev) for N, K, M in descs]
    bf.gemm_batched(O.Q4_K, [(dw[0], dw[1], dA, C, M, N, K) for dw, dA, C, (N, K, M) in zip(dws, dAs, Cs, descs)])
    torch.cuda.synchronize()
    for C, ref, d in zip(Cs, singles, descs):
        got = C.cpu().numpy().astype(np.float64)
        assert np.isfinite(got).all(), d
        assert (got == ref).all(), d


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
def test_full_size_exact_properties(dev, qt):
    """Size-independent checks at the benchmark shape: scaling A by 2 is exact
    in fp16 and fp32, so C(2A) == 2 C(A) bit for bit; permuting batch rows
    permutes output rows bit for bit."""
    w = O.gen_weights(qt, 5120, 5120, seed=101)
    dw = upload(w, dev)
    A = O.gen_act(32, 5120, seed=102)
    C = gpu_gemm(w, A, dev, dw=dw)
    A2 = (A.view(np.float16) * np.float16(2)).view(np.uint16)
    assert (gpu_gemm(w, A2, dev, dw=dw) == 2 * C).all()
    perm = np.random.default_rng(3).permutation(32)
    assert (gpu_gemm(w, A[perm], dev, dw=dw) == C[perm]).all()
    assert np.isfinite(C).all()


@pytest.mark.parametrize("K", [256, 1792, 2048, 5120, 7168, 17408])
@pytest.mark.parametrize("N", [1, 3, 200])
def test_dot2_small_batch_parity(dev, K, N):
    """The row-streaming v_dot2 kernel (Q4_K, M <= 2): super-block groups of
    seven per load, ragged tails, every N."""
    w = O.gen_weights(O.Q4_K, N, K, seed=K * 3 + N)
    dw = upload(w, dev)
    A = O.gen_act(2, K, seed=K + 5)
    ref = Ref(w, A)
    for M in (1, 2):
        if M * K * 2 > 48 * 1024:          # staged activations beyond the kernel's LDS budget
            with pytest.raises(bf.BusfillError):
                gpu_gemm(w, A[:M], dev, algo=bf.ALGO_DOT2, dw=dw)
            continue
        C = gpu_gemm(w, A[:M], dev, algo=bf.ALGO_DOT2, dw=dw)
        ref.check(C, f"dot2 N={N} K={K} M={M}", rows=M, form="f16")
        assert (gpu_gemm(w, A[:M], dev, algo=bf.ALGO_DOT2, dw=dw) == C).all()


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("K", [256, 1024, 5120, 7168, 17408])
@pytest.mark.parametrize("N", [1, 3, 200, 1000])
def test_lds_small_batch_parity(dev, qt, K, N):
    """The LDS-staged kernel: K segments on the MFMA rows (G = 4, 2, 1), steps
    split across waves and sub-tiles, ragged N, every batch size it serves."""
    w = O.gen_weights(qt, N, K, seed=K * 5 + N + qt)
    dw = upload(w, dev)
    A = O.gen_act(16, K, seed=K + 9)
    ref = Ref(w, A)
    for M in (1, 2, 3, 4, 5, 8, 9, 16):
        must = (M <= 4 and M * K <= 4 * 5120) or (M <= 8 and K <= 5120)
        try:
            C = gpu_gemm(w, A[:M], dev, algo=bf.ALGO_LDS, dw=dw)
        except bf.BusfillError as e:
            assert not must, f"LDS path refused N={N} K={K} M={M}: {e}"
            continue
        ref.check(C, f"lds {QT_NAME[qt]} N={N} K={K} M={M}", rows=M,
                  form="f32" if qt == O.Q4_K or M == 1 else "f16")
        assert (gpu_gemm(w, A[:M], dev, algo=bf.ALGO_LDS, dw=dw) == C).all()


def test_gguf_tensors_feed_the_gemm(dev, tmp_path):
    """Weights written to a GGUF file, read back and uploaded by the library's
    reader, give the oracle's GEMM results (the blocks need no repack)."""
    from test_gguf import GGML, write_gguf
    wk = O.gen_weights(O.Q4_K, 256, 5120, seed=77)
    w0 = O.gen_weights(O.Q4_0, 100, 2048, seed=78)
    path = tmp_path / "model.gguf"
    write_gguf(path, [(b"general.architecture", 8, b"llama")],
               [(b"blk.0.ffn_down.weight", GGML["q4_k"][0], [5120, 256], wk.W.tobytes()),
                (b"blk.0.attn_k.weight", GGML["q4_0"][0], [2048, 100], w0.W.tobytes())], alignment=64)
    with bf.Gguf(path) as g:
        for name, w in (("blk.0.ffn_down.weight", wk), ("blk.0.attn_k.weight", w0)):
            t = g.find(name)
            assert t.qtype == w.qtype and (t.dims[0], t.dims[1]) == (w.K, w.N)
            Wd = torch.empty(t.nbytes, dtype=torch.uint8, device=dev)
            g.upload(t, Wd)
            for M in (1, 8, 32):
                A = O.gen_act(M, w.K, seed=M + w.K)
                C = gpu_gemm(w, A, dev, dw=(Wd, None))
                Ref(w, A).check(C, f"gguf {name} M={M}")


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408), (600, 17408), (4096, 13824)])
def test_lds_step_ring_parity(dev, qt, N, K):
    """Shapes whose steps do not all fit in LDS next to the activations (85
    steps of 2,304 bytes per workgroup at 5120 x 17408): the steps cycle through
    a ring of slots, each reloaded once the compute wave that read it has
    released it, instead of a second round of workgroups; from batch 3-5 on at
    K = 17408 the activation segments do not fit either and cycle through a
    ring of their own, the steps then taken segment by segment."""
    w = O.gen_weights(qt, N, K, seed=N + K + qt)
    dw = upload(w, dev)
    A = O.gen_act(8, K, seed=K + 3)
    ref = Ref(w, A)
    for M in range(1, 9):
        C = gpu_gemm(w, A[:M], dev, algo=bf.ALGO_LDS, dw=dw)
        # batch 1 takes the sub-block rows form (fp32 scaling) when K is a multiple of 1024
        bd = M == 1 and (K // 256) % 4 == 0
        ref.check(C, f"ring {QT_NAME[qt]} N={N} K={K} M={M}", rows=M, form="f32" if qt == O.Q4_K or bd else "f16")
        assert (gpu_gemm(w, A[:M], dev, algo=bf.ALGO_LDS, dw=dw) == C).all()


def random_case(seed):
    """A seeded shape: format, batch rows, rows and K (multiples of 256, often
    large enough that the LDS-staged kernel needs its step and activation rings;
    every sixth case batch 2, where small activations are loaded by the compute
    waves)."""
    rng = np.random.default_rng(1000 + seed)
    qt = QTS[seed % 3]
    K = int(rng.choice([256 * int(rng.integers(1, 40)), 13824, 17408, 24576, 27648]))
    N = int(rng.integers(1, 2600))
    M = int(rng.integers(1, 17)) if seed % 4 else int(rng.integers(17, 41))
    if seed % 6 == 5:
        M = 2
    return qt, M, N, K


@pytest.mark.parametrize("seed", range(48), ids=lambda s: f"case{s}")
def test_random_shapes_every_kernel(dev, seed):
    """Seeded random shapes through every kernel that takes them (automatic
    choice, LDS-staged, K-split), each within the oracle's bounds and
    reproducible bit for bit."""
    qt, M, N, K = random_case(seed)
    w = O.gen_weights(qt, N, K, seed=seed)
    dw = upload(w, dev)
    A = O.gen_act(M, K, seed=seed + 77)
    ref = Ref(w, A)
    ran = 0
    for algo in (bf.ALGO_AUTO, bf.ALGO_LDS, bf.ALGO_SPLIT):
        try:
            C = gpu_gemm(w, A, dev, algo=algo, dw=dw)
        except bf.BusfillError:
            assert algo != bf.ALGO_AUTO
            continue
        ran += 1
        ref.check(C, f"{QT_NAME[qt]} M={M} N={N} K={K} algo={algo}")
        assert (gpu_gemm(w, A, dev, algo=algo, dw=dw) == C).all()
    assert ran >= 1


def gen_gate_up(M, K, seed):
    """gate|up rows (fp16 bits [M][2K]): gate ~ N(0, 2^2) with a few extreme
    values, up ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    g = (rng.normal(size=(M, K)) * 2).astype(np.float16)
    g[:, :4] = np.array([0, 30, -30, -65504], np.float16)
    u = rng.normal(size=(M, K)).astype(np.float16)
    return np.concatenate([g, u], axis=1).view(np.uint16)


@pytest.mark.parametrize("K", [1024, 5120, 17408])
def test_swiglu_f16_matches_oracle(dev, K):
    """The elementwise SiLU(g) * u against the oracle's fp32 restatement: at
    most one fp16 ulp apart (the device exp and numpy's may round differently)."""
    M = 3
    gu = gen_gate_up(M, K, seed=K)
    out = torch.empty((M, K), dtype=torch.int16, device=dev)
    bf.swiglu_f16(to_dev(gu, dev), out, M, K)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.float16).astype(np.float64)
    ref = O.swiglu_f16(gu, K).view(np.float16).astype(np.float64)
    assert np.isfinite(got).all()
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert (np.abs(got - ref) <= ulp).all()


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("N,K", [(5120, 17408), (1000, 5120), (300, 2048)])
def test_gemm_swiglu_equals_swiglu_then_gemm(dev, qt, N, K):
    """bf_gemm_swiglu (SiLU * up formed while the activations are loaded) is
    bit-identical to bf_swiglu_f16 followed by bf_gemm, at batch 1 (sub-block
    rows form) and 2 (activations loaded by the compute waves), and within the
    oracle's bounds for the activations it used."""
    w = O.gen_weights(qt, N, K, seed=N + K + qt)
    dw = upload(w, dev)
    for M in (1, 2):
        gu = gen_gate_up(M, K, seed=M + N)
        gud = to_dev(gu, dev)
        C = torch.full((M, N), float("nan"), device=dev)
        bf.gemm_swiglu(qt, dw[0], dw[1], gud, C, M, N, K)
        a = torch.empty((M, K), dtype=torch.int16, device=dev)
        bf.swiglu_f16(gud, a, M, K)
        torch.cuda.synchronize()
        A = a.cpu().numpy().view(np.uint16)
        C2 = gpu_gemm(w, A, dev, dw=dw)
        got = C.cpu().numpy().astype(np.float64)
        assert (got == C2).all(), (QT_NAME[qt], N, K, M)
        Ref(w, A).check(got, f"swiglu {QT_NAME[qt]} N={N} K={K} M={M}")


def test_gemm_swiglu_refuses_shapes_it_does_not_fuse(dev):
    w = O.gen_weights(O.Q4_K, 256, 1024, seed=3)
    dw = upload(w, dev)
    gud = to_dev(gen_gate_up(3, 1024, seed=3), dev)
    C = torch.empty((3, 256), device=dev)
    with pytest.raises(bf.BusfillError) as err:
        bf.gemm_swiglu(O.Q4_K, dw[0], None, gud, C, 3, 256, 1024)
    assert err.value.status == bf.ERR_UNSUPPORTED


# ---------------------------------------------------------------- integer-dot path
def gpu_quantize_q8(A, dev):
    M, K = A.shape
    Ad = to_dev(A, dev)
    Aq = torch.full((bf.q8_bytes(M, K),), 0xAB, dtype=torch.uint8, device=dev)
    bf.quantize_q8(Ad, Aq, M, K)
    torch.cuda.synchronize()
    return Aq


def q8_special_rows(K):
    """Rows with an all-zero block, a d = 1 block of ties (x.5 values), and tiny values."""
    rows = np.zeros((3, K), np.float16)
    rows[1, :32] = np.array([127, -127, 0.5, -0.5, 1.5, 2.5, -2.5, 126.5] * 4, np.float16)
    rows[2, :] = np.float16(6e-8) * np.arange(K).astype(np.float16) % 7
    return rows.view(np.uint16)


@pytest.mark.parametrize("M,K", [(1, 64), (5, 4096), (16, 5120)])
def test_quantize_q8_bitexact(dev, M, K):
    A = O.gen_act(M, K, 31 + M)
    A[: min(M, 3)] = q8_special_rows(K)[: min(M, 3)]
    Aq = gpu_quantize_q8(A, dev).cpu().numpy()
    assert (Aq == O.q8_pack(*O.quantize_q8(A))).all()


@pytest.mark.parametrize("qt", QTS)
@pytest.mark.parametrize("M,N,K", [(1, 40, 1024), (2, 300, 1536), (3, 64, 5120), (5, 129, 2048),
                                   (8, 512, 1024), (11, 200, 768), (16, 256, 2560)])
def test_gemm_q8_parity(dev, qt, M, N, K):
    """Integer-dot GEMM against the oracle's restatement: the integer dots are
    exact, the fp32 scale terms and sums within (K/32 + 32) * 2^-24 of the sum
    of the terms' magnitudes; and within half a quantization step of the fp16
    activation GEMM (sum_k |W| d/2)."""
    w = O.gen_weights(qt, N, K, 100 + M)
    A = O.gen_act(M, K, 200 + N)
    Aq = gpu_quantize_q8(A, dev)
    Wd, auxd = upload(w, dev)
    C = torch.full((M, N), float("nan"), device=dev)
    bf.gemm_q8(qt, Wd, auxd, Aq, C, M, N, K)
    torch.cuda.synchronize()
    Cg = C.cpu().numpy().astype(np.float64)
    q, d, s = O.quantize_q8(A)
    ref, mag = O.gemm_q8(w, q, d, s)
    assert np.isfinite(Cg).all()
    tol = (K / 32 + 32) * 2.0 ** -24 * mag + 1e-30
    assert (np.abs(Cg - ref) <= tol).all(), f"worst excess {float((np.abs(Cg - ref) / tol).max())}"
    half_step = d.astype(np.float64).repeat(32, axis=1) / 2
    bound = half_step @ np.abs(O.dequant_f32(w).astype(np.float64)).T
    assert (np.abs(Cg - O.gemm_f64(w, A)) <= bound * (1 + 1e-4) + tol).all()


@pytest.mark.parametrize("qt", QTS)
@pytest.mark.parametrize("N", [5120, 9001, 12300, 17408])
def test_gemm_q8_mfma_row_tiles(dev, qt, N):
    """The MFMA form of the integer-dot GEMM (batch 3-16), one workgroup per CU
    over ceil(N / CUs) rows as 2-5 tiles of 16, the last overlapping the one
    before it (ragged N: the last workgroup holds one row), against the
    oracle's integer restatement at M = 3, 8 and 16."""
    K = 1024
    w = O.gen_weights(qt, N, K, 300 + N)
    Wd, auxd = upload(w, dev)
    for M in (3, 8, 16):
        A = O.gen_act(M, K, 400 + M)
        Aq = gpu_quantize_q8(A, dev)
        C = torch.full((M, N), float("nan"), device=dev)
        bf.gemm_q8(qt, Wd, auxd, Aq, C, M, N, K)
        torch.cuda.synchronize()
        Cg = C.cpu().numpy().astype(np.float64)
        q, d, s = O.quantize_q8(A)
        ref, mag = O.gemm_q8(w, q, d, s)
        assert np.isfinite(Cg).all(), (QT_NAME[qt], N, M)
        tol = (K / 32 + 32) * 2.0 ** -24 * mag + 1e-30
        assert (np.abs(Cg - ref) <= tol).all(), (QT_NAME[qt], N, M, float((np.abs(Cg - ref) / tol).max()))


def rows_of(w, idx):
    """The weight rows idx of w as a matrix of their own (every output row
    depends on its weight row only)."""
    W = w.W.reshape(w.N, -1)[idx]
    aux = None if w.W_aux is None else w.W_aux.reshape(w.N, -1)[idx]
    return O.QWeights(w.qtype, len(idx), w.K, np.ascontiguousarray(W), aux)


@pytest.mark.parametrize("N,Ks", [(5120, (17408,)), (12300, (8192, 30208)), (16384, (32768,)), (17408, (30208,))])
def test_gemm_q8_large_k(dev, N, Ks):
    """The integer-dot GEMM at K = 17408-32768, checked on 96 rows against the
    oracle's integer restatement at M = 3, 8 and 16: the down projection's
    K = 17408; a larger K after a smaller one on the same kernel instance
    (12300 rows: four 16-row tiles, 67 KB then 156 KB of LDS, so the LDS limit
    must not stay at the first call's size); and shapes whose block-scale
    table does not fit next to the tiles' sums in 160 KB (four and five tiles
    at K >= 30208 or 32768), which take the v_dot4 form instead of failing."""
    rng = np.random.default_rng(N)
    idx = np.unique(np.concatenate([[0, N - 1], rng.choice(N, 94, replace=False)]))
    for K in Ks:
        w = O.gen_weights(O.Q4_K, N, K, 500 + K)
        ws = rows_of(w, idx)
        Wd, auxd = upload(w, dev)
        for M in (3, 8, 16):
            A = O.gen_act(M, K, 600 + M)
            Aq = gpu_quantize_q8(A, dev)
            C = torch.full((M, N), float("nan"), device=dev)
            bf.gemm_q8(O.Q4_K, Wd, auxd, Aq, C, M, N, K)
            torch.cuda.synchronize()
            Cg = C.cpu().numpy().astype(np.float64)
            assert np.isfinite(Cg).all(), (N, K, M)
            q, d, s = O.quantize_q8(A)
            ref, mag = O.gemm_q8(ws, q, d, s)
            tol = (K / 32 + 32) * 2.0 ** -24 * mag + 1e-30
            err = np.abs(Cg[:, idx] - ref)
            assert (err <= tol).all(), (N, K, M, float((err / tol).max()))


def test_gemm_q8_full_size_strided_f16_and_deterministic(dev):
    """Q4_K 5120 x 5120 at batch 16 into an fp16 output with ldc > N: rows
    beyond M and columns beyond N untouched, values within the oracle's bound
    plus one fp16 rounding, two runs bit-identical."""
    M, N, K = 16, 5120, 5120
    w = O.gen_weights(O.Q4_K, N, K, 77)
    A = O.gen_act(M, K, 78)
    Aq = gpu_quantize_q8(A, dev)
    Wd, auxd = upload(w, dev)
    ldc = N + 8
    outs = []
    for _ in range(2):
        C = torch.full((M + 1, ldc), 7.0, device=dev, dtype=torch.float16)
        bf.gemm_q8(O.Q4_K, Wd, auxd, Aq, C, M, N, K, ldc=ldc, otype=bf.OUT_F16)
        torch.cuda.synchronize()
        outs.append(C.cpu().numpy())
    assert (outs[0].view(np.uint16) == outs[1].view(np.uint16)).all()
    C = outs[0]
    assert (C[M] == 7).all() and (C[:M, N:] == 7).all()
    q, d, s = O.quantize_q8(A)
    ref, mag = O.gemm_q8(w, q, d, s)
    tol = (K / 32 + 32) * 2.0 ** -24 * mag + np.abs(ref) * 2.0 ** -11 + 6e-8
    assert (np.abs(C[:M, :N].astype(np.float64) - ref) <= tol).all()


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408)])
def test_sweep_shapes_full_size_large_batches(dev, N, K):
    """The batch sweep's two 50 MB shapes at full size against the oracle at
    M = 16, 32, 64 and 128 (the K-split plans at N = 17408 and K = 17408, and the
    large-batch path), through the automatic choice."""
    w = O.gen_weights(O.Q4_K, N, K, seed=N * 3 + K)
    dw = upload(w, dev)
    A = O.gen_act(128, K, seed=K + 128)
    ref = Ref(w, A)
    for M in (16, 32, 64, 128):
        C = gpu_gemm(w, A[:M], dev, dw=dw)
        ref.check(C, f"q4_k {N}x{K} M={M}", rows=M)
