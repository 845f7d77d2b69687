"""Pins the CPU oracle (no GPU needed).

The reference ships no tests, golden vectors or fixtures for this path, so the
oracle is pinned by
  * numpy's own RNE float16 conversion (an independent implementation),
    exhaustively over the fp16 inputs that matter;
  * known-answer blocks whose bytes and expected values are written out by hand
    from the published block formats (Q4_0 18-byte block, Q4_K 144-byte block,
    the reference's Q4_0 planes: kernels/busfill_v0.cu:119-123);
  * closed forms of the GEMM (all-zero weights, constant codes) and numpy's
    float64 matmul for the contraction/indexing;
  * planted mistakes that the comparisons must catch.
"""
import hashlib

import numpy as np
import pytest

import oracle as O


# ------------------------------------------------------------------ fp16
def test_f16_to_f32_all_halves():
    h = np.arange(65536, dtype=np.uint16)
    mine = O.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (mine.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(mine) & np.isnan(ref))
    assert same.all()


def _np_f16(x):
    with np.errstate(over="ignore"):
        return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def test_f32_to_f16_ties_and_neighbours():
    # every gap between consecutive finite halves: exact midpoint (a tie) and the
    # floats one ulp either side of it, for both signs
    h = np.arange(0, 0x7BFF, dtype=np.uint16)            # positive finite, excluding max
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)            # exact in fp32
    cases = [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))]
    x = np.concatenate(cases + [-c for c in cases]).astype(np.float32)
    assert (O.f32_to_f16_bits(x) == _np_f16(x)).all()


def test_f32_to_f16_random_and_specials():
    rng = np.random.default_rng(1234)
    bits = rng.integers(0, 2**32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    mine, ref = O.f32_to_f16_bits(x), _np_f16(x)
    nan = np.isnan(x)
    assert (mine[~nan] == ref[~nan]).all()
    assert ((mine[nan] & 0x7C00) == 0x7C00).all() and ((mine[nan] & 0x3FF) != 0).all()
    sp = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.996, 65520, 2**-24, 2**-25,
                   2**-25 * 1.0000001, 2**-14, 2**-14 * (1 - 2**-11)], np.float32)
    assert (O.f32_to_f16_bits(sp) == _np_f16(sp)).all()


# ------------------------------------------------------------------ Q4_0
def _all_finite_halves():
    h = np.arange(65536, dtype=np.uint16)
    return h[(h & 0x7C00) != 0x7C00]                   # 63,488 finite values


def _exhaustive_planes():
    """Every finite fp16 scale x every code, in the reference planes layout:
    one 32-element block per scale, byte j = code j (lo) | code 15-j (hi)."""
    scales = _all_finite_halves()
    K = 512
    N = scales.size // (K // 32)
    Ws = scales.reshape(N, K // 32).copy()
    j = np.arange(16, dtype=np.uint8)
    block = (j | ((15 - j) << 4)).astype(np.uint8)
    Wq = np.tile(block, (N, K // 32))
    return O.QWeights(O.Q4_0_PLANES, N, K, Wq, Ws)


def _numpy_planes_dequant(w):
    q = np.empty((w.N, w.K), np.int32)
    q[:, 0::2] = w.W & 0xF
    q[:, 1::2] = w.W >> 4
    d = np.repeat(w.W_aux.view(np.float16).astype(np.float32), 32, axis=1)
    return ((q - 8).astype(np.float32) * d).astype(np.float16).view(np.uint16)


def test_q4_0_planes_dequant_exhaustive():
    w = _exhaustive_planes()
    got = O.dequant_f16(w)
    ref = _numpy_planes_dequant(w)
    assert (got == ref).all()


def test_q4_0_blocks_dequant_exhaustive_matches_planes():
    w = _exhaustive_planes()
    b = O.planes_to_blocks(w)
    assert (O.dequant_f16(b) == O.dequant_f16(w)).all()
    back = O.blocks_to_planes(b)
    assert (back.W == w.W).all() and (back.W_aux == w.W_aux).all()


def test_q4_0_planted_scale_error_is_caught():
    # a plausible slip: scaling by d/2 in the high-nibble path only
    w = _exhaustive_planes()
    ref = _numpy_planes_dequant(w)
    q = (w.W >> 4).astype(np.int32)
    d = np.repeat(w.W_aux.view(np.float16).astype(np.float32), 16, axis=1)
    bad = ref.copy()
    bad[:, 1::2] = ((q - 8).astype(np.float32) * (d * np.float32(0.5))).astype(np.float16).view(np.uint16)
    assert (bad != O.dequant_f16(w)).any()


def test_q4_0_block_kat():
    # llama.cpp block_q4_0: fp16 d then qs[16]; elem j = qs[j] & 0xF, elem j+16 = qs[j] >> 4
    d = np.float16(0.5).view(np.uint16)
    qs = [(j | ((15 - j) << 4)) for j in range(16)]
    blk = np.array([d & 0xFF, d >> 8] + qs, np.uint8).reshape(1, 18)
    y = O.dequant_f16(O.QWeights(O.Q4_0, 1, 32, blk)).view(np.float16).astype(np.float32)[0]
    expect = [0.5 * (j - 8) for j in range(16)] + [0.5 * (7 - j) for j in range(16)]
    assert y.tolist() == expect


def test_q4_0_planes_kat():
    # reference planes: byte j -> elems 2j (low nibble) and 2j+1 (high nibble)
    Wq = np.array([[0x1F, 0x80] + [0x88] * 14], np.uint8)
    Ws = np.array([[np.float16(0.25).view(np.uint16)]], np.uint16)
    y = O.dequant_f16(O.QWeights(O.Q4_0_PLANES, 1, 32, Wq, Ws)).view(np.float16).astype(np.float32)[0]
    assert y[:4].tolist() == [0.25 * (15 - 8), 0.25 * (1 - 8), 0.25 * (0 - 8), 0.25 * (8 - 8)]
    assert (y[4:] == 0).all()


def test_q4_0_rounding_tie_kat():
    # (q-8)*d = 3*(1+2^-10) = 3 + 1.5*2^-9: a tie between 0x4201 and 0x4202 -> even 0x4202
    Wq = np.array([[0x5B] + [0x88] * 15], np.uint8)    # elem0 = 11 (q-8 = 3), elem1 = 5 (q-8 = -3)
    Ws = np.array([[0x3C01]], np.uint16)
    y = O.dequant_f16(O.QWeights(O.Q4_0_PLANES, 1, 32, Wq, Ws))[0]
    assert int(y[0]) == 0x4202 and int(y[1]) == 0xC202


def test_magic_bias_identities_exhaustive():
    """The device decode's arithmetic premise, for every byte value b:
    (b & 0x0F) | 0x6400 reads as 1024 + lo, (b & 0xF0) | 0x5400 reads as 64 + hi,
    and the planes pair {(b&0xF)|0x6400, (b<<16 & 0xF00000)|0x5400<<16} reads as
    {1024 + lo, 64 + hi}; subtracting the bias is exact in fp16."""
    b = np.arange(256, dtype=np.uint32)
    lo = ((b & 0x0F) | 0x6400).astype(np.uint16).view(np.float16)
    hi = ((b & 0xF0) | 0x5400).astype(np.uint16).view(np.float16)
    assert (lo.astype(np.float64) == 1024 + (b & 0xF)).all()
    assert (hi.astype(np.float64) == 64 + (b >> 4)).all()
    assert ((lo - np.float16(1032)).astype(np.float64) == (b & 0xF).astype(np.int64) - 8).all()
    assert ((hi - np.float16(72)).astype(np.float64) == (b >> 4).astype(np.int64) - 8).all()
    # v_perm_b32 [b,0,b,0] then v_and_or_b32 with mask 0x00F0000F, bits 0x54006400
    pair = (((b | (b << 16)) & 0x00F0000F) | 0x54006400).astype(np.uint32)
    halves = pair.view(np.uint16).reshape(-1, 2).view(np.float16).astype(np.float64)
    assert (halves[:, 0] == 1024 + (b & 0xF)).all() and (halves[:, 1] == 64 + (b >> 4)).all()


# ------------------------------------------------------------------ Q4_K
KAT_SC = [63, 0, 21, 42, 48, 33, 63, 17]
KAT_M = [5, 63, 40, 9, 63, 32, 1, 50]
# the 12 scale bytes for KAT_SC / KAT_M, derived by hand from the format:
#   bytes 0-3 : sc[i] | (sc[i+4] >> 4) << 6     bytes 4-7: m[i] | (m[i+4] >> 4) << 6
#   bytes 8-11: (sc[i+4] & 0xF) | (m[i+4] & 0xF) << 4
KAT_SCALES = bytes([0xFF, 0x80, 0xD5, 0x6A, 0xC5, 0xBF, 0x28, 0xC9, 0xF0, 0x01, 0x1F, 0x21])


def test_q4k_scale_min_kat():
    for j in range(8):
        assert O.q4k_get_scale_min(j, KAT_SCALES) == (KAT_SC[j], KAT_M[j]), j
    assert O.q4k_pack_scales(KAT_SC, KAT_M) == KAT_SCALES


def test_q4k_scale_roundtrip_exhaustive():
    rng = np.random.default_rng(7)
    for j in range(8):
        for sc in range(64):
            base_sc = rng.integers(0, 64, 8)
            base_m = rng.integers(0, 64, 8)
            for m in range(0, 64, 3):
                base_sc[j], base_m[j] = sc, m
                packed = O.q4k_pack_scales(base_sc, base_m)
                assert O.q4k_get_scale_min(j, packed) == (sc, m)
    # every byte pattern decodes to 16 six-bit values and re-encodes to itself
    for _ in range(200):
        s = rng.integers(0, 256, 12, dtype=np.uint8).tobytes()
        pairs = [O.q4k_get_scale_min(j, s) for j in range(8)]
        assert O.q4k_pack_scales([p[0] for p in pairs], [p[1] for p in pairs]) == s


def _q4k_block(d, dmin, scales, qs):
    d = np.float16(d).view(np.uint16)
    dm = np.float16(dmin).view(np.uint16)
    return np.array([d & 0xFF, d >> 8, dm & 0xFF, dm >> 8] + list(scales) + list(qs), np.uint8)


def test_q4k_element_order_kat():
    # d = 1, dmin = 0, every sc = 1, m = 0 -> y = q.  qs byte 32c+l holds
    # element 64c+l (low nibble) and element 64c+32+l (high nibble).
    scales = O.q4k_pack_scales([1] * 8, [0] * 8)
    qs = [(l % 16) | ((15 - l % 16) << 4) for c in range(4) for l in range(32)]
    blk = _q4k_block(1.0, 0.0, scales, qs).reshape(1, 144)
    y = O.dequant_f16(O.QWeights(O.Q4_K, 1, 256, blk)).view(np.float16).astype(np.float32)[0]
    for c in range(4):
        for l in range(32):
            assert y[64 * c + l] == l % 16
            assert y[64 * c + 32 + l] == 15 - l % 16


def test_q4k_value_kat():
    # d = 0.5, dmin = 0.25, sc/m from the hand-packed KAT bytes, q = l % 16:
    # y = 0.5*sc_j*q - 0.25*m_j (every value exact in fp16)
    qs = [(l % 16) | ((l % 16) << 4) for c in range(4) for l in range(32)]
    blk = _q4k_block(0.5, 0.25, KAT_SCALES, qs).reshape(1, 144)
    y = O.dequant_f16(O.QWeights(O.Q4_K, 1, 256, blk)).view(np.float16).astype(np.float64)[0]
    for e in range(256):
        j, q = e // 32, (e % 32) % 16
        assert y[e] == 0.5 * KAT_SC[j] * q - 0.25 * KAT_M[j], e


def test_q4k_rounding_kat():
    # (d*sc)*q - dmin*m with d = 1+2^-10, sc = 3, q = 1, dmin*m = 0:
    # 3 + 1.5*2^-9 is a tie -> even 0x4202; the fp32 stage is exact here.
    scales = O.q4k_pack_scales([3] * 8, [0] * 8)
    qs = [0x01] * 128
    blk = _q4k_block(np.uint16(0x3C01).view(np.float16), 0.0, scales, qs).reshape(1, 144)
    y = O.dequant_f16(O.QWeights(O.Q4_K, 1, 256, blk))[0]
    assert (y[[64 * c + l for c in range(4) for l in range(32)]] == 0x4202).all()
    assert (y[[64 * c + 32 + l for c in range(4) for l in range(32)]] == 0).all()


def test_q4k_min_sign_planted_error_is_caught():
    w = O.gen_weights(O.Q4_K, 8, 512, seed=3)
    good = O.dequant_f32(w)
    # planted: + dmin*m instead of - dmin*m
    blk = w.W.reshape(-1, 144)
    d = blk[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = blk[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    bad = good.reshape(-1, 256).copy()
    for b in range(blk.shape[0]):
        for j in range(8):
            sc, m = O.q4k_get_scale_min(j, blk[b, 4:16].tobytes())
            bad[b, 32 * j:32 * j + 32] += np.float32(2) * dmin[b] * np.float32(m)
    assert not np.array_equal(bad.reshape(good.shape), good)
    assert np.isfinite(good).all() and np.abs(good).max() < 10.0 and d.min() > 0


# ------------------------------------------------------------------ generators
def test_generators_deterministic_and_pinned():
    h = hashlib.sha256()
    for qt in (O.Q4_0_PLANES, O.Q4_0, O.Q4_K):
        w = O.gen_weights(qt, 16, 512, seed=42)
        h.update(w.W.tobytes())
        if w.W_aux is not None:
            h.update(w.W_aux.tobytes())
        w2 = O.gen_weights(qt, 16, 512, seed=42)
        assert (w2.W == w.W).all()
    h.update(O.gen_act(3, 512, seed=42).tobytes())
    assert h.hexdigest() == GEN_HASH


# sha256 of the generated bytes above; a change here means every seeded input
# of every test and benchmark changed
GEN_HASH = "92ece6d2107c9658f281ebc7cdeef079ff5354fd5962e87d0c4e7763f10ded86"


def test_generator_distributions():
    w = O.gen_weights(O.Q4_0_PLANES, 256, 5120, seed=9)
    codes = np.concatenate([w.W & 0xF, w.W >> 4]).ravel()
    counts = np.bincount(codes, minlength=16)
    assert counts.min() > 0.97 * codes.size / 16 and counts.max() < 1.03 * codes.size / 16
    d = w.W_aux.view(np.float16).astype(np.float32)
    assert d.min() >= 0.002 - 1e-6 and d.max() <= 0.02 + 1e-5
    wk = O.gen_weights(O.Q4_K, 64, 5120, seed=9).W.reshape(-1, 144)
    dd = wk[:, 0:4].copy().view(np.float16).astype(np.float32)
    assert dd.min() >= 0.001 - 1e-6 and dd.max() <= 0.01 + 1e-5
    sc = np.array([O.q4k_get_scale_min(j, wk[b, 4:16].tobytes()) for b in range(200) for j in range(8)])
    assert sc.min() == 0 and sc.max() == 63 and abs(sc.mean() - 31.5) < 2.0
    A = O.gen_act(8, 5120, seed=1).view(np.float16).astype(np.float64)
    assert abs(A.mean()) < 0.02 and abs(A.std() - 1) < 0.02


# ------------------------------------------------------------------ GEMM
@pytest.mark.parametrize("qt", [O.Q4_0_PLANES, O.Q4_0, O.Q4_K])
def test_gemm_f64_matches_numpy_contraction(qt):
    w = O.gen_weights(qt, 48, 768, seed=5)
    A = O.gen_act(5, 768, seed=6)
    C = O.gemm_f64(w, A)
    ref = A.view(np.float16).astype(np.float64) @ O.dequant_f32(w).astype(np.float64).T
    assert C.shape == (5, 48)
    np.testing.assert_allclose(C, ref, rtol=1e-12, atol=1e-12)
    # the fp16-rounded-weight variant differs only by weight rounding
    C16 = O.gemm_f64(w, A, round_w=True)
    ok, mae, rfe, _ = O.gate(C16, C)
    assert ok and rfe < 1e-3


def test_gemm_closed_forms():
    N, K, M = 8, 256, 3
    A = O.gen_act(M, K, seed=11)
    Af = A.view(np.float16).astype(np.float64)
    Ws = O.gen_weights(O.Q4_0_PLANES, N, K, seed=12).W_aux
    zero = O.QWeights(O.Q4_0_PLANES, N, K, np.full((N, K // 2), 0x88, np.uint8), Ws)
    assert (O.gemm_f64(zero, A) == 0).all()
    one = O.QWeights(O.Q4_0_PLANES, N, K, np.full((N, K // 2), 0x99, np.uint8), Ws)   # q - 8 = 1
    d = Ws.view(np.float16).astype(np.float64)                                          # [N][K/32]
    expect = np.einsum("mbk,nb->mn", Af.reshape(M, K // 32, 32), d)
    np.testing.assert_allclose(O.gemm_f64(one, A), expect, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("qt", [O.Q4_0_PLANES, O.Q4_K])
def test_cpu_baseline_matches_reference(qt):
    w = O.gen_weights(qt, 256, 1024, seed=21)
    A = O.gen_act(4, 1024, seed=22)
    C, tdq, tmm = O.cpu_dequant_matmul(w, A, threads=2)
    ok, mae, rfe, _ = O.gate(C, O.gemm_f64(w, A))
    assert ok and rfe < 1e-5 and tdq >= 0 and tmm >= 0


def test_gate_rejects_nonfinite_and_large_errors():
    ref = np.ones((4, 8))
    assert O.gate(ref.copy(), ref)[0]
    bad = ref.copy(); bad[1, 2] = np.nan
    ok, _, _, nf = O.gate(bad, ref)
    assert not ok and nf == 1
    bad = ref.copy(); bad[0, 0] += 0.7
    assert not O.gate(bad, ref)[0]
    assert not O.gate(ref * (1 + 2e-3), ref)[0]


def test_shape_rejection():
    w = O.gen_weights(O.Q4_K, 4, 256, seed=1)
    w.K = 200
    with pytest.raises(ValueError):
        O.dequant_f16(w)


def test_swiglu_closed_forms_and_float64():
    """SiLU(g) * u: SiLU(0) = 0, SiLU(g) -> g for large g and -> -0 for very
    negative g, u scales linearly; and within one fp16 ulp of the same
    formula in float64 over a sweep of every fp16 exponent."""
    def pack(g, u):
        return np.concatenate([np.asarray(g, np.float16).reshape(1, -1),
                               np.asarray(u, np.float16).reshape(1, -1)], axis=1).view(np.uint16)
    K = 6
    out = O.swiglu_f16(pack([0, 30, -30, 65504, -65504, 2.0], [1, 1, 1, 1, 1, 3.0]), K).view(np.float16)[0]
    assert out[0] == 0 and out[1] == np.float16(30) and out[3] == np.float16(65504)
    assert out[2] <= 0 and abs(float(out[2])) < 1e-10 and out[4] == 0
    assert out[5] == np.float16(3 * 2 / (1 + np.exp(-2.0)))
    # sweep: magnitudes over all fp16 binades, both signs, random u
    rng = np.random.default_rng(4)
    g = (rng.choice([-1, 1], 4096) * 2.0 ** rng.uniform(-14, 15.9, 4096)).astype(np.float16)
    u = rng.normal(size=4096).astype(np.float16)
    got = O.swiglu_f16(pack(g, u), 4096).view(np.float16)[0].astype(np.float64)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    ref = (g64 / (1 + np.exp(-g64)) * u64).astype(np.float16).astype(np.float64)
    fin = np.isfinite(ref)
    assert (got[~fin] == ref[~fin]).all()                 # products beyond fp16: the same infinity
    ulp = np.spacing(np.abs(ref[fin]).astype(np.float16)).astype(np.float64)
    assert (np.abs(got[fin] - ref[fin]) <= ulp).all()


# ---------------------------------------------------------------- q8 activations
def _f16(vals):
    return np.asarray(vals, np.float16).view(np.uint16)


def test_quantize_q8_closed_forms():
    """d = 1 blocks (amax = 127): q is the input rounded half away from zero --
    2.5 -> 3 and -2.5 -> -3 (round-to-even would give 2), the largest fp16
    below 0.5 -> 0 (a float32 |y| + 0.5 would round up to 1) -- and the
    all-zero block gives q = d = s = 0."""
    below_half = float(np.nextafter(np.float16(0.5), np.float16(0)))
    vals = [127, -127, 0.5, -0.5, 1.5, 2.5, -2.5, below_half, -below_half, 126.5, -126.5, 3, -3, 0, 64.25, -0.75]
    vals += [0.0] * (32 - len(vals))
    expect = [127, -127, 1, -1, 2, 3, -3, 0, 0, 127, -127, 3, -3, 0, 64, -1] + [0] * 16
    A = np.stack([_f16(vals), _f16(np.zeros(32))])
    q, d, s = O.quantize_q8(A)
    assert d[0, 0] == np.float32(1.0) and d[1, 0] == 0
    assert q[0].tolist() == expect
    assert s[0, 0] == sum(expect) and s[1, 0] == 0 and not q[1].any()


def test_quantize_q8_invariants():
    """Random blocks: the largest magnitude maps to +-127, every |x - d q| <=
    d/2 (up to the fp32 quotient's rounding), |q| <= 127 and s = sum q."""
    A = O.gen_act(7, 4096, 11)
    A[3, 64:96] = _f16(np.linspace(-1e-3, 2e-3, 32))       # a small-scale block
    q, d, s = O.quantize_q8(A)
    x = A.view(np.float16).astype(np.float64).reshape(7, 128, 32)
    qb = q.astype(np.int64).reshape(7, 128, 32)
    imax = np.abs(x).argmax(-1)
    assert (np.abs(np.take_along_axis(qb, imax[..., None], -1)) == 127).all()
    err = np.abs(x - d[..., None].astype(np.float64) * qb)
    assert (err <= d[..., None] * (0.5 + 1e-5)).all()
    assert np.abs(qb).max() <= 127 and (s == qb.sum(-1)).all()
    # pack / unpack round trip
    q2, d2, s2 = O.q8_unpack(O.q8_pack(q, d, s), 7, 4096)
    assert (q2 == q).all() and (d2 == d).all() and (s2 == s).all()


@pytest.mark.parametrize("qt", [O.Q4_0_PLANES, O.Q4_0, O.Q4_K])
def test_gemm_q8_equals_dequant_route(qt):
    """The integer-dot restatement (codes, scale*dot - offset*s) equals the
    float64 matmul of the quantized activations d*q with the C oracle's fp32
    dequant (a different route to the same number), and differs from the fp16
    activation GEMM by at most sum_k |W[n][k]| * d_blk(k) / 2."""
    M, N, K = 3, 24, 512
    w = O.gen_weights(qt, N, K, 5)
    A = O.gen_act(M, K, 6)
    q, d, s = O.quantize_q8(A)
    C, mag = O.gemm_q8(w, q, d, s)
    Wf = O.dequant_f32(w).astype(np.float64)
    xq = (d.astype(np.float64).repeat(32, axis=1)) * q.astype(np.float64)
    ref = xq @ Wf.T
    assert np.abs(C - ref).max() <= 1e-12 * mag.max()
    half_step = d.astype(np.float64).repeat(32, axis=1) / 2
    bound = half_step @ np.abs(Wf).T
    assert (np.abs(C - O.gemm_f64(w, A)) <= bound * (1 + 1e-5) + 1e-12).all()


def test_gemm_q8_brute_force_tiny():
    """One output by explicit loops over the byte layout of Q4_0 (block d,
    code = nibble - 8) against gemm_q8."""
    K = 64
    w = O.gen_weights(O.Q4_0, 1, K, 9)
    A = O.gen_act(1, K, 10)
    q, d, s = O.quantize_q8(A)
    blk = w.W.reshape(K // 32, 18)
    total = 0.0
    for b in range(K // 32):
        db = float(np.frombuffer(blk[b, :2].tobytes(), np.float16)[0])
        for i in range(16):
            lo, hi = int(blk[b, 2 + i]) & 15, int(blk[b, 2 + i]) >> 4
            total += float(d[0, b]) * db * ((lo - 8) * int(q[0, 32 * b + i]) + (hi - 8) * int(q[0, 32 * b + 16 + i]))
    C, _ = O.gemm_q8(w, q, d, s)
    assert abs(C[0, 0] - total) <= 1e-12 * max(1.0, abs(total))
