"""The GEMM kernels' own effective weights, read out bit for bit.

With A holding a single 1.0 per batch row (at column k_m), every output C[m][n]
is one weight W[n][k_m] times one plus exact zeros.  A kernel that computes
with fp16 weights must therefore return the oracle's fp16 dequant bit for bit
(the reference kernel's weights, kernels/busfill_v0.cu:74,78-81, and ggml's
Q4_K formula rounded to fp16), and a kernel that scales exact codes in fp32 must
return the oracle's fp32 dequant bit for bit.  This is the unique-value probe of
kernels/frag_probe.cu:34-46 turned on the weights: it pins the decode inside
every kernel, not only in the standalone bf_dequant_f16.

Scales span many binades (subnormal, negative, up to 32).  For Q4_K a share of
the blocks pairs a tiny d with a large dmin (or the reverse), where q*s - dm
needs more than 24 bits: there RN16(RN32(x)) and a single rounding of x to fp16
differ, and the test checks that its sample holds such weights, so a decode
that rounds once would fail it.
"""
import numpy as np
import pytest
import torch

import busfill as bf
import oracle as O

pytestmark = pytest.mark.gpu

QT_NAME = {O.Q4_0_PLANES: "planes", O.Q4_0: "q4_0", O.Q4_K: "q4_k"}
N, K = 256, 5120


def finite_halves(rng, n, max_exp_bits):
    """n random finite fp16 bit patterns with |x| < 2^(max_exp_bits - 15), both signs, subnormals included."""
    mag = rng.integers(1, max_exp_bits << 10, n).astype(np.uint16)
    sign = (rng.integers(0, 2, n).astype(np.uint16) << 15)
    return mag | sign


def wide_scale_weights(qt, seed):
    rng = np.random.default_rng(seed)
    if qt == O.Q4_K:
        w = O.gen_weights(O.Q4_K, N, K, seed=seed)
        blk = w.W.reshape(-1, 144)
        nb = blk.shape[0]
        blk[:, 4:] = rng.integers(0, 256, (nb, 140), dtype=np.uint8)        # every scale/min code, every nibble
        d = finite_halves(rng, nb, 20)                                      # |d|, |dmin| < 32
        dm = finite_halves(rng, nb, 20)
        # a third of the blocks: tiny d with large dmin, a third the reverse
        tiny = (rng.integers(0x0400, 0x2400, nb) | (rng.integers(0, 2, nb) << 15)).astype(np.uint16)
        big = (rng.integers(0x3C00, 0x4C00, nb) | (rng.integers(0, 2, nb) << 15)).astype(np.uint16)
        sel = rng.integers(0, 3, nb)
        d = np.where(sel == 1, tiny, np.where(sel == 2, big, d)).astype(np.uint16)
        dm = np.where(sel == 1, big, np.where(sel == 2, tiny, dm)).astype(np.uint16)
        blk[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        blk[:, 2:4] = dm.view(np.uint8).reshape(-1, 2)
        # a quarter of the blocks crafted for double rounding: d = +-(1 + 2^-10),
        # dmin = 2^-24, every sc = m = 1, so codes 3, 6 and 12 put q*d*sc exactly
        # halfway between two fp16 values and dmin*m below half an fp32 ulp
        tie = rng.integers(0, 4, nb) == 0
        blk[tie, 0:2] = (np.uint16(0x3C01) | (rng.integers(0, 2, int(tie.sum())) << 15).astype(np.uint16)
                         ).view(np.uint8).reshape(-1, 2)
        blk[tie, 2:4] = np.array([0x01, 0x00], np.uint8)
        blk[tie, 4:16] = np.frombuffer(O.q4k_pack_scales([1] * 8, [1] * 8), np.uint8)
        return w
    w = O.gen_weights(O.Q4_0_PLANES, N, K, seed=seed)
    w.W[:] = rng.integers(0, 256, w.W.shape, dtype=np.uint8)
    w.W_aux[:] = finite_halves(rng, w.W_aux.size, 26).reshape(w.W_aux.shape)   # |d| < 2048: no overflow
    return w if qt == O.Q4_0_PLANES else O.planes_to_blocks(w)


def k_columns(rng, count):
    """Columns spread over every super-group, sub-block and nibble half."""
    ks = np.concatenate([[0, K - 1, 31, 32, 255, 256], rng.choice(K, count - 6, replace=False)])
    return np.unique(ks)[:count] if np.unique(ks).size >= count else np.unique(ks)


def readout(w, dw, ks, M, algo, dev):
    """W_eff[:, ks] as computed by kernel `algo` at batch M (rows of A one-hot)."""
    cols = []
    for i0 in range(0, ks.size, M):
        chunk = ks[i0:i0 + M]
        A = np.zeros((M, K), np.uint16)
        A[np.arange(chunk.size), chunk] = np.float16(1.0).view(np.uint16)
        Ad = torch.from_numpy(A.view(np.int16)).to(dev)
        C = torch.full((M, N), float("nan"), device=dev)
        bf.gemm(w.qtype, dw[0], dw[1], Ad, C, M, N, K, algo=algo)
        torch.cuda.synchronize()
        Ch = C.cpu().numpy()
        cols.append(Ch[:chunk.size].T)
        if chunk.size < M:
            assert (Ch[chunk.size:] == 0).all(), "rows with all-zero activations must be zero"
    return np.concatenate(cols, axis=1)


def single_rounding_q4k(w, ks):
    """RN16 of the exact Q4_K value (one rounding, no fp32 step) at columns ks."""
    blk = w.W.reshape(N, K // 256, 144)
    out = np.empty((N, ks.size), np.float16)
    for j, k in enumerate(ks):
        b = blk[:, k // 256]
        e = k % 256
        c, l, hi = e // 64, e % 32, (e // 32) % 2
        sub = 2 * c + hi
        sc = np.empty(N, np.int64)
        m = np.empty(N, np.int64)
        for n in range(N):
            sc[n], m[n] = O.q4k_get_scale_min(sub, bytes(b[n, 4:16]))
        q = (b[:, 16 + 32 * c + l] >> (4 * hi)) & 0xF
        d = b[:, 0:2].copy().view(np.float16).ravel().astype(np.float64)
        dmin = b[:, 2:4].copy().view(np.float16).ravel().astype(np.float64)
        # exact in float64: q * (d sc) has <= 21 significant bits, dmin m <= 17, exponents < 2^5 apart from 2^-24
        out[:, j] = (q * (d * sc) - dmin * m).astype(np.float16)
    return out


# (algo, M, expected form) per format; "f16" = the fp16 dequant, "f32" = the unrounded fp32 dequant
KERNELS = {
    O.Q4_K: [(bf.ALGO_SPLIT, 32, "f16"), (bf.ALGO_SPLIT, 9, "f16"), (bf.ALGO_SLAB, 32, "f16"),
             (bf.ALGO_MFMA, 32, "f16"), (bf.ALGO_MFMA, 64, "f16"), (bf.ALGO_LDS, 4, "f32"), (bf.ALGO_LDS, 8, "f32"),
             (bf.ALGO_LDS, 1, "f32"), (bf.ALGO_DOT2, 2, "f32"), (bf.ALGO_SIMPLE, 32, "f32"),
             (bf.ALGO_DENSE, 64, "f16"), (bf.ALGO_DENSE, 128, "f16"), (bf.ALGO_AUTO, 96, "f16"),
             (bf.ALGO_AUTO, 32, "f16"), (bf.ALGO_AUTO, 1, "f32")],
    O.Q4_0: [(bf.ALGO_SPLIT, 32, "f16"), (bf.ALGO_SLAB, 32, "f16"), (bf.ALGO_MFMA, 32, "f16"),
             (bf.ALGO_LDS, 4, "f16"), (bf.ALGO_LDS, 8, "f16"), (bf.ALGO_LDS, 1, "f32"), (bf.ALGO_SIMPLE, 32, "f32"),
             (bf.ALGO_DENSE, 128, "f16"), (bf.ALGO_AUTO, 32, "f16"), (bf.ALGO_AUTO, 1, "f32")],
}
KERNELS[O.Q4_0_PLANES] = [k for k in KERNELS[O.Q4_0] if k[0] != bf.ALGO_SLAB]     # the slab kernel reads blocks only


@pytest.mark.parametrize("qt", [O.Q4_K, O.Q4_0, O.Q4_0_PLANES], ids=lambda q: QT_NAME[q])
def test_kernel_weights_bitwise(dev, qt):
    w = wide_scale_weights(qt, seed=900 + qt)
    Wd = torch.from_numpy(w.W).to(dev)
    auxd = torch.from_numpy(w.W_aux.view(np.int16)).to(dev) if w.W_aux is not None else None
    rng = np.random.default_rng(7)
    ks = k_columns(rng, 96)
    ref = {"f16": O.dequant_f16(w).view(np.float16)[:, ks].astype(np.float32),
           "f32": O.dequant_f32(w)[:, ks]}
    assert np.isfinite(ref["f16"]).all() and np.isfinite(ref["f32"]).all()
    if qt == O.Q4_K:
        # the sample holds weights where one rounding of the exact value differs from the dequant
        once = single_rounding_q4k(w, ks).astype(np.float32)
        assert (once != ref["f16"]).sum() >= 3
    for algo, M, form in KERNELS[qt]:
        got = readout(w, (Wd, auxd), ks, M, algo, dev)
        bad = np.nonzero(got != ref[form])              # as values: +0 and -0 are one weight
        assert bad[0].size == 0, (f"{QT_NAME[qt]} algo={algo} M={M}: {bad[0].size} weights differ from the "
                                  f"{form} dequant, first at n={bad[0][0]} k={ks[bad[1][0]]}: "
                                  f"{got[bad[0][0], bad[1][0]]!r} vs {ref[form][bad[0][0], bad[1][0]]!r}")
