"""GPU parity of bf_ffn_swiglu, the SwiGLU feed-forward block (gate and up
projections, SiLU(gate) * up, down projection), against the calls it replaces
and against the oracle (run on an MI355X).

Bar: C and the gate|up intermediate bit-identical to bf_gemm (gate, fp16 out),
bf_gemm (up, fp16 out), bf_swiglu_f16, bf_gemm (down) on the same inputs --
those calls are themselves pinned to the oracle by test_gpu_parity.py -- and C
within the repo gate (max |err| <= 0.6, relative Frobenius error <= 1e-3) of the
oracle's chain: fp64 dequantize-then-matmul for gate and up, rounded to fp16,
the oracle's SiLU(g) * u, fp64 dequantize-then-matmul for down.
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


# Q4_K scales ten times smaller than the single-GEMM workloads': with d, dmin ~
# U[0.001, 0.01] the weights have a mean near 1, the gate and up projections
# reach |x| ~ 100 and SiLU(g) * u overflows fp16 (identically in every path).
FFN_SCALES = {O.Q4_K: (1e-4, 1e-3)}


class Block:
    """One feed-forward block's weights (gate, up [F][K], down [N][F]) on the device."""

    def __init__(self, qt, K, F, N, seed, dev):
        self.qt, self.K, self.F, self.N = qt, K, F, N
        sr = FFN_SCALES.get(qt)
        self.w = [O.gen_weights(qt, F, K, seed=seed, scale_range=sr),
                  O.gen_weights(qt, F, K, seed=seed + 1, scale_range=sr),
                  O.gen_weights(qt, N, F, seed=seed + 2, scale_range=sr)]
        self.d = [upload(w, dev) for w in self.w]

    def fused(self, A, dev, otype=bf.OUT_F32, stream=None, form=bf.FFN_ONE_LAUNCH):
        """bf_ffn_swiglu_ex in one form: (C, gate_up) as device tensors."""
        M = A.shape[0]
        gu = torch.full((M, 2 * self.F), -1, dtype=torch.int16, device=dev)
        C = torch.full((M, self.N), float("nan"), device=dev,
                       dtype=torch.float32 if otype == bf.OUT_F32 else torch.float16)
        bf.ffn_swiglu(self.qt, self.d[0], self.d[1], self.d[2], A, gu, C, M, self.K, self.F, self.N,
                      otype=otype, form=form, stream=stream)
        return C, gu

    def calls(self, A, dev, otype=bf.OUT_F32):
        """The four calls the block replaces: (C, gate_up, h)."""
        M = A.shape[0]
        gu = torch.full((M, 2 * self.F), -1, dtype=torch.int16, device=dev)
        bf.gemm(self.qt, self.d[0][0], self.d[0][1], A, gu, M, self.F, self.K, ldc=2 * self.F, otype=bf.OUT_F16)
        bf.gemm(self.qt, self.d[1][0], self.d[1][1], A, gu[:, self.F:], M, self.F, self.K, ldc=2 * self.F,
                otype=bf.OUT_F16)
        h = torch.empty((M, self.F), dtype=torch.int16, device=dev)
        bf.swiglu_f16(gu, h, M, self.F)
        C = torch.full((M, self.N), float("nan"), device=dev,
                       dtype=torch.float32 if otype == bf.OUT_F32 else torch.float16)
        bf.gemm(self.qt, self.d[2][0], self.d[2][1], h, C, M, self.N, self.F, otype=otype)
        return C, gu, h


def bits(t):
    return t.view(torch.int32 if t.dtype == torch.float32 else torch.int16).cpu().numpy()


@pytest.mark.parametrize("qt", QTS, ids=lambda q: QT_NAME[q])
@pytest.mark.parametrize("K,F,N", [(5120, 17408, 5120), (2048, 4096, 1024), (1024, 2048, 3000)])
def test_ffn_forms_equal_the_calls(dev, qt, K, F, N):
    """Batch 1 and 2: the one-launch, two-launch, calls and automatic forms
    give C bit for bit as the four calls make it (fp32 and fp16 output), and
    gate|up as they make it (SiLU(g) * u in the gate half for the calls form)."""
    blk = Block(qt, K, F, N, seed=K + F + N + qt, dev=dev)
    for M in (1, 2):
        A = to_dev(O.gen_act(M, K, seed=M + qt), dev)
        for otype in (bf.OUT_F32, bf.OUT_F16):
            C2, gu2, h2 = blk.calls(A, dev, otype)
            for form in (bf.FFN_ONE_LAUNCH, bf.FFN_TWO_LAUNCHES, bf.FFN_CALLS, bf.FFN_AUTO):
                C, gu = blk.fused(A, dev, otype, form=form)
                torch.cuda.synchronize()
                what = f"{QT_NAME[qt]} K={K} F={F} N={N} M={M} otype={otype} form={form}"
                assert torch.isfinite(C.float()).all(), what
                if form == bf.FFN_CALLS:
                    assert (bits(gu[:, :F]) == bits(h2)).all(), "gate half: " + what
                    assert (bits(gu[:, F:]) == bits(gu2[:, F:])).all(), "up half: " + what
                else:
                    assert (bits(gu) == bits(gu2)).all(), "gate|up: " + what
                assert (bits(C) == bits(C2)).all(), "C: " + what


@pytest.mark.parametrize("qt", [O.Q4_K, O.Q4_0], ids=lambda q: QT_NAME[q])
def test_ffn_against_the_oracle_chain(dev, qt):
    """C against the oracle's own chain (fp64 dequantize-then-matmul, fp16
    intermediate, oracle SiLU * up), batch 1, 2 and 5 (three launches)."""
    K, F, N = 2048, 3072, 1536
    blk = Block(qt, K, F, N, seed=7 + qt, dev=dev)
    for M in (1, 2, 5):
        A = O.gen_act(M, K, seed=100 + M)
        C, _ = blk.fused(to_dev(A, dev), dev, form=bf.FFN_ONE_LAUNCH if M <= 2 else bf.FFN_AUTO)
        torch.cuda.synchronize()
        g = O.gemm_f64(blk.w[0], A).astype(np.float16)
        u = O.gemm_f64(blk.w[1], A).astype(np.float16)
        h = O.swiglu_f16(np.concatenate([g, u], axis=1).view(np.uint16), F)
        ref = O.gemm_f64(blk.w[2], h)
        ok, mae, rfe, nf = O.gate(C.cpu().numpy().astype(np.float64), ref)
        assert ok, f"{QT_NAME[qt]} M={M}: max_abs={mae:.4g} rel_frob={rfe:.3g} nonfinite={nf}"


@pytest.mark.parametrize("M", [3, 8, 16, 32])
def test_ffn_other_batches_run_as_calls(dev, M):
    """Batches the one-launch block does not serve: the same C as the calls,
    and gate_up holds SiLU(g) * u in the gate half and the up projection."""
    K, F, N = 2048, 4096, 1024
    blk = Block(O.Q4_K, K, F, N, seed=M, dev=dev)
    A = to_dev(O.gen_act(M, K, seed=M), dev)
    for form in (bf.FFN_ONE_LAUNCH, bf.FFN_TWO_LAUNCHES):
        with pytest.raises(bf.BusfillError) as err:
            blk.fused(A, dev, form=form)
        assert err.value.status == bf.ERR_UNSUPPORTED
    C, gu = blk.fused(A, dev, form=bf.FFN_AUTO)
    C2, gu2, h = blk.calls(A, dev)
    torch.cuda.synchronize()
    assert (bits(C) == bits(C2)).all()
    assert (bits(gu[:, :F]) == bits(h)).all()
    assert (bits(gu[:, F:]) == bits(gu2[:, F:])).all()


def test_ffn_repeated_and_interleaved_launches(dev):
    """Back-to-back one-launch blocks on one stream, with K-split GEMMs (which
    share the stream's workspace counters) between them: every block finds its
    counters at zero and gives the same bits."""
    K, F, N = 5120, 17408, 5120
    blk = Block(O.Q4_K, K, F, N, seed=11, dev=dev)
    ws = O.gen_weights(O.Q4_K, 5120, 5120, seed=12)
    wsd = upload(ws, dev)
    A1 = to_dev(O.gen_act(1, K, seed=1), dev)
    A16 = to_dev(O.gen_act(16, 5120, seed=2), dev)
    ref, _ = blk.fused(A1, dev)
    torch.cuda.synchronize()
    ref = bits(ref)
    outs = []
    for i in range(4):
        C16 = torch.empty((16, 5120), device=dev)
        bf.gemm(O.Q4_K, wsd[0], None, A16, C16, 16, 5120, 5120, algo=bf.ALGO_SPLIT)
        C, _ = blk.fused(A1, dev)
        outs.append(C)
    torch.cuda.synchronize()
    for i, C in enumerate(outs):
        assert (bits(C) == ref).all(), f"launch {i}"


def test_ffn_graph_replays(dev):
    """The one-launch block captured in a HIP graph (after one uncaptured call
    on the capture stream, which sets up its workspace) and replayed several
    times with eager work between the replays: every replay gives the eager
    result."""
    K, F, N = 2048, 4096, 1024
    blk = Block(O.Q4_K, K, F, N, seed=21, dev=dev)
    s = torch.cuda.Stream()
    A = to_dev(O.gen_act(2, K, seed=3), dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        Ce, _ = blk.fused(A, dev, stream=s)
        gu = torch.full((2, 2 * F), -1, dtype=torch.int16, device=dev)
        C = torch.full((2, N), float("nan"), device=dev)
    s.synchronize()
    eager = bits(Ce)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        bf.ffn_swiglu(O.Q4_K, blk.d[0], blk.d[1], blk.d[2], A, gu, C, 2, K, F, N, stream=s)
    for i in range(3):
        C.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert (bits(C) == eager).all(), f"replay {i}"
        # eager work between replays
        Cx, _ = blk.fused(A, dev)
        torch.cuda.synchronize()
        assert (bits(Cx) == eager).all()
