"""bf_gemm_noalloc: the same results as bf_gemm, bit for bit, with the K-split
kernel's counters and partials and the dense kernel's partials in the
library's static per-GPU scratch array instead of a workspace allocated per
stream.  Two calls in a row, the second
on a smaller input (the array keeps the first call's contents); calls
alternating with bf_gemm on one stream; batches above 32 rows (several K-split
launches in one call); and a shape that needs more scratch than the array
holds, which is refused before anything is enqueued."""
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
    W = to_dev(w.W, dev)
    aux = to_dev(w.W_aux, dev) if w.W_aux is not None else None
    A = to_dev(O.gen_act(M, K, seed=seed + 1), dev)
    return W, aux, A


def both(qt, W, aux, A, M, N, K, dev, otype=bf.OUT_F32):
    dt = torch.float32 if otype == bf.OUT_F32 else torch.float16
    C0 = torch.full((M, N), float("nan"), device=dev, dtype=dt)
    C1 = torch.full((M, N), float("nan"), device=dev, dtype=dt)
    bf.gemm(qt, W, aux, A, C0, M, N, K, otype=otype)
    bf.gemm_noalloc(qt, W, aux, A, C1, M, N, K, otype=otype)
    torch.cuda.synchronize()
    a, b = C0.cpu().numpy(), C1.cpu().numpy()
    assert np.isfinite(a).all()
    assert (a.view(np.uint32 if otype == bf.OUT_F32 else np.uint16) ==
            b.view(np.uint32 if otype == bf.OUT_F32 else np.uint16)).all(), (qt, M, N, K)
    return b


def test_noalloc_matches_gemm_two_calls_second_smaller(dev):
    # the K-split kernel at 32 rows (the scratch holds 4 splits x 5120 rows of partials) ...
    W, aux, A = case(O.Q4_K, 5120, 5120, 32, 11, dev)
    both(O.Q4_K, W, aux, A, 32, 5120, 5120, dev)
    # ... then a smaller one on the same array: fewer row groups, other splits
    W, aux, A = case(O.Q4_0, 1000, 5120, 17, 12, dev)
    both(O.Q4_0, W, aux, A, 17, 1000, 5120, dev)


def test_noalloc_alternating_shapes_formats_and_batches(dev):
    cases = [(O.Q4_0_PLANES, 600, 17408, 32), (O.Q4_K, 17408, 5120, 32), (O.Q4_K, 200, 5120, 9),
             (O.Q4_K, 5120, 17408, 128), (O.Q4_0, 7168, 5120, 24), (O.Q4_K, 5120, 5120, 1)]
    for i, (qt, N, K, M) in enumerate(cases):
        W, aux, A = case(qt, N, K, M, 20 + i, dev)
        both(qt, W, aux, A, M, N, K, dev)
        both(qt, W, aux, A, M, N, K, dev, otype=bf.OUT_F16)


def test_noalloc_refuses_more_scratch_than_it_holds(dev):
    # 16 batch rows with N > K run on the K-split kernel; its plan for
    # 49152 x 16384 has 16 splits (fewer leave more units per workgroup than
    # the LDS holds): 16 x 49152 x 16 fp32 partials are 48 MiB
    N, K, M = 49152, 16384, 16
    W = torch.zeros(N * K * 9 // 16, dtype=torch.uint8, device=dev)
    A = torch.zeros((M, K), dtype=torch.float16, device=dev)
    C = torch.full((M, N), 7.0, device=dev)
    with pytest.raises(bf.BusfillInvalid) as err:
        bf.gemm_noalloc(O.Q4_K, W, None, A, C, M, N, K)
    assert "scratch" in str(err.value)
    torch.cuda.synchronize()
    assert bool((C == 7.0).all())
