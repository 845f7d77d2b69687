"""GPU parity of the ggml mul_mat hook (bf_ggml_mul_mat / _ws) on an MI355X.

Bar:
  * the fp32 -> fp16 staging of src1 is bit-exact with the oracle's rounding
    (round to nearest even, overflow to infinity), read out through identity
    weights (each output is one activation times 1.0 plus zeros);
  * every dst slice is bit for bit bf_gemm on that slice's fp16 activations
    and its (broadcast) src0 matrix -- bf_gemm itself is pinned against the
    oracle in test_gpu_parity -- and the first and last slice of each case
    also pass the repo gate against the oracle's fp64 dequantize-then-matmul.
Cases: Q4_0 / Q4_K weights x F32 / F16 activations, batch 1 to 130, src0
broadcast over src1's outer dimensions, src1 contiguous, permuted, strided
along K and with padded or misaligned rows, dst with padded rows.
"""
import numpy as np
import pytest
import torch

import busfill as bf
import oracle as O

pytestmark = pytest.mark.gpu

OQT = {bf.GGML_Q4_0: O.Q4_0, bf.GGML_Q4_K: O.Q4_K}
BQT = {bf.GGML_Q4_0: bf.Q4_0, bf.GGML_Q4_K: bf.Q4_K}


def src1_view(x, layout, dev):
    """x [ne3][ne2][M][K] (float32 or float16, host) on the device in one of
    the layouts; returns the logical [ne3][ne2][M][K] view."""
    t = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    if layout == "contig":
        return t
    if layout == "permuted":            # rows of one slice ne2 rows apart
        return t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    if layout == "kstride":             # consecutive k a whole column apart (nb[0] != element size)
        return t.transpose(-1, -2).contiguous().transpose(-1, -2)
    pad = {"padded": 8, "odd": 1}[layout]
    base = torch.zeros(t.shape[:-1] + (t.shape[-1] + pad,), dtype=t.dtype, device=dev)
    base[..., :t.shape[-1]] = t
    return base[..., :t.shape[-1]]


def run_case(dev, t0, t1, N, M, K, ne2, ne3, r2, r3, layout, dst_pad=0, use_ws=False, seed=0):
    n2, n3 = ne2 // r2, ne3 // r3
    ws = [[O.gen_weights(OQT[t0], N, K, seed=seed + 100 * i3 + i2) for i2 in range(n2)] for i3 in range(n3)]
    Wd = torch.from_numpy(np.stack([np.stack([w.W for w in row]) for row in ws])).to(dev)
    rng = np.random.default_rng(seed + 7)
    x = rng.standard_normal((ne3, ne2, M, K)).astype(np.float32)
    if t1 == bf.GGML_F16:
        x = x.astype(np.float16)
    s1 = src1_view(x, layout, dev)
    dbase = torch.full((ne3, ne2, M, N + dst_pad), float("nan"), device=dev)
    d = dbase[..., :N]
    args = (bf.ggml_view(Wd, t0), bf.ggml_view(s1, t1), bf.ggml_view(d))
    if use_ws:
        nbytes = bf.ggml_mul_mat_workspace_bytes(*args)
        wsb = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=dev)
        bf.ggml_mul_mat_ws(*args, wsb, nbytes)
    else:
        bf.ggml_mul_mat(*args)
    torch.cuda.synchronize()
    out = d.cpu().numpy()
    assert np.isfinite(out).all(), "non-finite dst"
    # per slice: bf_gemm on the slice's fp16 activations, bit for bit
    A16 = O.f32_to_f16_bits(x.astype(np.float32)) if t1 == bf.GGML_F32 else x.view(np.uint16)
    for i3 in range(ne3):
        for i2 in range(ne2):
            w = ws[i3 // r3][i2 // r2]
            Ad = torch.from_numpy(np.ascontiguousarray(A16[i3, i2]).view(np.int16)).to(dev)
            C = torch.full((M, N), float("nan"), device=dev)
            bf.gemm(BQT[t0], Wd[i3 // r3, i2 // r2], None, Ad, C, M, N, K)
            torch.cuda.synchronize()
            ref = C.cpu().numpy()
            assert np.array_equal(out[i3, i2], ref), f"slice ({i2}, {i3}) differs from bf_gemm"
            if (i3, i2) in ((0, 0), (ne3 - 1, ne2 - 1)):
                ok, mae, rfe, nf = O.gate(out[i3, i2].astype(np.float64), O.gemm_f64(w, A16[i3, i2]))
                assert ok, f"slice ({i2}, {i3}): max_abs={mae:.4g} rel_frob={rfe:.3g}"
    assert torch.isnan(dbase[..., N:]).all(), "padding of dst rows written"
    return out


Q0, QK, F32, F16 = bf.GGML_Q4_0, bf.GGML_Q4_K, bf.GGML_F32, bf.GGML_F16
CASES = [
    # t0, t1, N, M, K, ne2, ne3, r2, r3, src1 layout
    (QK, F32, 64, 1, 256, 1, 1, 1, 1, "contig"),
    (Q0, F32, 64, 1, 256, 1, 1, 1, 1, "contig"),
    (QK, F16, 160, 7, 512, 1, 1, 1, 1, "contig"),       # fp16 rows read in place
    (Q0, F16, 160, 7, 512, 1, 1, 1, 1, "contig"),
    (QK, F32, 96, 33, 256, 3, 1, 1, 1, "contig"),
    (Q0, F32, 96, 16, 512, 2, 2, 2, 1, "permuted"),
    (QK, F16, 64, 9, 256, 4, 3, 2, 3, "permuted"),      # fp16 rows ne2 rows apart: in place
    (QK, F32, 128, 130, 256, 1, 1, 1, 1, "contig"),     # above 128 rows (sliced)
    (Q0, F32, 64, 5, 256, 2, 1, 1, 1, "kstride"),
    (QK, F16, 64, 3, 512, 1, 2, 1, 2, "kstride"),
    (Q0, F16, 200, 64, 256, 1, 1, 1, 1, "padded"),      # fp16, row stride K + 8: in place
    (Q0, F16, 64, 4, 256, 1, 1, 1, 1, "odd"),           # fp16, row stride K + 1: staged
    (QK, F32, 5120, 1, 5120, 1, 1, 1, 1, "contig"),     # a decode step of a 27B-class layer
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(str(v) for v in c))
def test_ggml_mul_mat_matches_bf_gemm_and_oracle(dev, case):
    run_case(dev, *case, seed=CASES.index(case))


@pytest.mark.parametrize("case", [CASES[4], CASES[6], CASES[10]], ids=lambda c: "-".join(str(v) for v in c))
def test_ggml_mul_mat_ws_same_bits(dev, case):
    a = run_case(dev, *case, seed=11)
    b = run_case(dev, *case, use_ws=True, seed=11)
    assert np.array_equal(a, b)


def test_ggml_dst_padded_rows(dev):
    run_case(dev, QK, F32, 64, 32, 256, 2, 1, 2, 1, "contig", dst_pad=5)


def test_ggml_staging_grows_and_shrinks(dev):
    """The stream's staging buffer grows on a larger call and keeps serving
    smaller ones."""
    for M in (2, 70, 3):
        run_case(dev, QK, F32, 64, M, 512, 1, 1, 1, 1, "contig", seed=M)


def identity_q4_0(K):
    """Q4_0 blocks of the K x K identity: d = 1.0, code 9 on the diagonal and 8
    elsewhere ((q - 8) d is 1 or 0)."""
    qs = np.full((K, K // 32, 16), 0x88, np.uint8)
    for n in range(K):
        b, j = divmod(n, 32)
        qs[n, b, j % 16] = (0x89 if j < 16 else 0x98)
    blk = np.empty((K, K // 32, 18), np.uint8)
    blk[..., 0:2] = np.array([0x00, 0x3C], np.uint8)    # fp16 1.0, little-endian
    blk[..., 2:] = qs
    return blk.reshape(K, K // 32 * 18)


def test_ggml_staging_rounding_bit_exact(dev):
    """src1 values chosen around fp16's rounding points (halfway cases, the
    subnormal range, the largest finite value) read back through identity
    weights: each output is exactly the staged fp16 value."""
    K, M = 256, 64
    rng = np.random.default_rng(3)
    ulp = np.float32(2.0 ** -10)
    vals = [1 + ulp / 2, 1 + 3 * ulp / 2, -(1 + ulp / 2), 2049.0, 2051.0, 65504.0, 65519.0, -65519.0,
            2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1e-30, 0.1, 1 / 3]
    x = (rng.standard_normal((M, K)) * 10.0 ** rng.integers(-8, 5, (M, K))).astype(np.float32)
    x = np.clip(x, -65000, 65000)
    x.reshape(-1)[:len(vals)] = np.array(vals, np.float32)
    # overflow to infinity, one per row (its other outputs are inf x 0 = NaN)
    over = {M - 2: (7, 65520.0), M - 1: (19, -1e6)}
    for m, (k, v) in over.items():
        x[m] = 0.0
        x[m, k] = v
    W = torch.from_numpy(identity_q4_0(K)).to(dev)
    s1 = torch.from_numpy(x).to(dev)
    d = torch.full((M, K), float("nan"), device=dev)
    bf.ggml_mul_mat(bf.ggml_view(W, Q0), bf.ggml_view(s1), bf.ggml_view(d))
    torch.cuda.synchronize()
    got = d.cpu().numpy()
    want = O.f16_bits_to_f32(O.f32_to_f16_bits(x))
    rows = [m for m in range(M) if m not in over]
    assert np.array_equal(got[rows], want[rows])
    for m, (k, v) in over.items():
        assert got[m, k] == np.float32(np.inf if v > 0 else -np.inf)


@pytest.mark.parametrize("own_ws", [True, False], ids=["caller_ws", "library_ws"])
def test_ggml_call_replays_in_a_graph(dev, own_ws):
    """The hook captured in a HIP graph (F32 src1 staged, then a K-split GEMM
    that uses the workspace): after one uncaptured call of the shape, every
    replay -- src1 rewritten and other work on the stream between -- gives
    the bits of the uncaptured call on the same src1."""
    N = K = 5120
    M = 16
    w = O.gen_weights(O.Q4_K, N, K, seed=41)
    Wd = torch.from_numpy(w.W).to(dev)
    x = torch.randn((M, K), device=dev)
    d = torch.full((M, N), float("nan"), device=dev)
    args = (bf.ggml_view(Wd, QK), bf.ggml_view(x), bf.ggml_view(d))
    nbytes = bf.ggml_mul_mat_workspace_bytes(*args)
    assert nbytes > M * K * 2                            # staging and the K-split's slots
    wsb = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream()

    def call():
        if own_ws:
            bf.ggml_mul_mat_ws(*args, wsb, nbytes, stream=s)
        else:
            bf.ggml_mul_mat(*args, stream=s)

    with torch.cuda.stream(s):
        call()
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            call()
        big = torch.zeros(16 << 20, dtype=torch.uint8, device=dev)
        for r in range(4):
            x.copy_(torch.randn((M, K), device=dev) * (r + 1))
            big.add_(1)
            d.fill_(float("nan"))
            s.synchronize()
            g.replay()
            s.synchronize()
            got = d.clone()
            d.fill_(float("nan"))
            call()
            s.synchronize()
            assert torch.isfinite(got).all() and torch.equal(got, d), r
    torch.cuda.synchronize()


def test_ggml_capture_on_a_new_stream_enqueues_nothing(dev):
    """bf_ggml_mul_mat on a stream with no staging buffer yet, under capture:
    BF_ERR_UNSUPPORTED and dst untouched; the same call uncaptured then works."""
    w = O.gen_weights(O.Q4_K, 256, 512, seed=43)
    Wd = torch.from_numpy(w.W).to(dev)
    x = torch.randn((3, 512), device=dev)
    d = torch.full((3, 256), 7.0, device=dev)
    args = (bf.ggml_view(Wd, QK), bf.ggml_view(x), bf.ggml_view(d))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        mark = torch.zeros(1, device=dev)
        with pytest.raises(bf.BusfillError, match="capture"):
            with torch.cuda.graph(g, stream=s):
                mark.add_(1)
                bf.ggml_mul_mat(*args, stream=s)
        s.synchronize()
        assert (d.cpu().numpy() == 7.0).all()
        bf.ggml_mul_mat(*args, stream=s)
        s.synchronize()
    assert np.isfinite(d.cpu().numpy()).all()


def halfway_row(K, seed):
    """fp32 activations with every seventh value on an fp16 rounding midpoint
    (ties to even decide it) and the rest random."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(K).astype(np.float32)
    h = x.astype(np.float16)
    up = np.nextafter(h, np.float16(np.inf))
    mid = ((h.astype(np.float64) + up.astype(np.float64)) / 2).astype(np.float32)   # exact in fp32
    x[::7] = mid[::7]
    return x


@pytest.mark.parametrize("t0", [QK, Q0], ids=["q4_k", "q4_0"])
@pytest.mark.parametrize("M,N,K,pad", [(1, 5120, 5120, 0), (1, 17408, 5120, 0), (1, 5120, 17408, 0),
                                       (2, 5120, 5120, 0), (2, 5120, 5120, 8), (2, 17408, 5120, 0)])
def test_ggml_f32_decode_row_fused(dev, t0, M, N, K, pad):
    """One or two fp32 activation rows (decode steps) on the LDS kernel's forms
    that load all of A through the compute waves: no workspace and no staging
    launch (the kernel rounds the rows as it loads them; rows pad floats
    apart beyond K), and bf_gemm's bits on the rows rounded by the oracle,
    rounding midpoints included."""
    w = O.gen_weights(OQT[t0], N, K, seed=N + K + t0)
    Wd = torch.from_numpy(w.W).to(dev)
    x = np.stack([halfway_row(K, N + t0 + 7 * m) for m in range(M)])
    base = torch.zeros((M, K + pad), device=dev)
    base[:, :K] = torch.from_numpy(x).to(dev)
    s1 = base[:, :K]
    d = torch.full((M, N), float("nan"), device=dev)
    args = (bf.ggml_view(Wd, t0), bf.ggml_view(s1), bf.ggml_view(d))
    assert bf.ggml_mul_mat_workspace_bytes(*args) == 0
    bf.ggml_mul_mat(*args)
    A16 = O.f32_to_f16_bits(x)
    C = torch.full((M, N), float("nan"), device=dev)
    bf.gemm(BQT[t0], Wd, None, torch.from_numpy(A16.view(np.int16)).to(dev), C, M, N, K)
    torch.cuda.synchronize()
    got, ref = d.cpu().numpy(), C.cpu().numpy()
    assert np.isfinite(got).all() and np.array_equal(got, ref)
    ok, mae, rfe, nf = O.gate(got.astype(np.float64), O.gemm_f64(w, A16))
    assert ok, (mae, rfe, nf)


def test_ggml_f32_decode_row_captures_on_a_new_stream(dev):
    """The fused decode-row call needs no buffer, so it captures into a graph
    on a stream that has run nothing; every replay gives the eager bits."""
    N = K = 5120
    w = O.gen_weights(O.Q4_K, N, K, seed=51)
    Wd = torch.from_numpy(w.W).to(dev)
    x = torch.from_numpy(halfway_row(K, 52)).reshape(1, K).to(dev)
    d = torch.full((1, N), float("nan"), device=dev)
    args = (bf.ggml_view(Wd, QK), bf.ggml_view(x), bf.ggml_view(d))
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            bf.ggml_mul_mat(*args, stream=s)
        for r in range(3):
            x.mul_(-1.5)
            d.fill_(float("nan"))
            s.synchronize()
            g.replay()
            s.synchronize()
            got = d.clone()
            d.fill_(float("nan"))
            bf.ggml_mul_mat(*args, stream=s)
            s.synchronize()
            assert torch.isfinite(got).all() and torch.equal(got, d), r
    torch.cuda.synchronize()
