"""Committed golden fixtures (tests/golden/golden.npz, made by
tests/golden/make_golden.py): the oracle must reproduce them exactly, and the
GPU kernels must match them (bit-exact dequant, gated GEMM)."""
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


def cases():
    z = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("/")[0] for k in z.files})
    out = []
    for n in names:
        qt, N, K, M, seed = (int(x) for x in z[f"{n}/meta"])
        aux = z[f"{n}/W_aux"] if f"{n}/W_aux" in z.files else None
        out.append((n, O.QWeights(qt, N, K, z[f"{n}/W"], aux), z[f"{n}/A"],
                    z[f"{n}/deq_f16"], z[f"{n}/C_f64"], seed))
    return out


@pytest.mark.parametrize("case", cases(), ids=lambda c: c[0])
def test_oracle_reproduces_golden(case):
    name, w, A, deq, C, seed = case
    regen = O.gen_weights(w.qtype, w.N, w.K, seed=seed)
    assert (regen.W == w.W).all()
    assert (O.gen_act(A.shape[0], w.K, seed=seed + 100) == A).all()
    assert (O.dequant_f16(w) == deq).all()
    assert np.array_equal(O.gemm_f64(w, A), C)


@pytest.mark.gpu
@pytest.mark.parametrize("case", cases(), ids=lambda c: c[0])
def test_gpu_matches_golden(dev, case):
    import torch
    import busfill as bf
    name, w, A, deq, C, seed = case

    def to_dev(a):
        a = np.ascontiguousarray(a)
        return torch.from_numpy(a.view(np.int16) if a.dtype == np.uint16 else a).to(dev)

    Wd = to_dev(w.W)
    aux = to_dev(w.W_aux) if w.W_aux is not None else None
    out = torch.empty((w.N, w.K), dtype=torch.int16, device=dev)
    bf.dequant_f16(w.qtype, Wd, aux, out, w.N, w.K)
    Cd = torch.empty((A.shape[0], w.N), dtype=torch.float32, device=dev)
    bf.gemm(w.qtype, Wd, aux, to_dev(A), Cd, A.shape[0], w.N, w.K)
    torch.cuda.synchronize()
    assert (out.cpu().numpy().view(np.uint16) == deq).all()
    ok, mae, rfe, nf = O.gate(Cd.cpu().numpy(), C)
    assert ok, (mae, rfe, nf)
