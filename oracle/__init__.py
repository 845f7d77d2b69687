"""CPU oracle for the batched int4-block-weight x fp16-activation GEMM.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py, and there only as the checker (or, for the CPU
baseline, as the host-side thing being timed).  The product path under
``bus-fill_amd/`` never imports it.

Thin numpy/ctypes front end over ``liboracle.so`` (plain C, ``oracle.c``); each
C function cites the reference file:line it restates (see ``oracle.h``).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

Q4_0 = 0          # llama.cpp block_q4_0, 18 B / 32 weights
Q4_0_PLANES = 1   # reference planes Wq[N][K/2] u8 + Ws[N][K/32] fp16
Q4_K = 2          # llama.cpp block_q4_K, 144 B / 256 weights

# value distributions of the benchmark workloads
Q4_0_SCALE_RANGE = (0.002, 0.02)
Q4_K_SCALE_RANGE = (0.001, 0.01)

_lib = None


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", _HERE, "liboracle.so"],
                       check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, i, u64, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_float
        L.or_f32_to_f16.argtypes = [f]; L.or_f32_to_f16.restype = ctypes.c_uint16
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]; L.or_f16_to_f32.restype = f
        L.or_f32_to_f16_array.argtypes = [vp, vp, ctypes.c_size_t]
        L.or_f16_to_f32_array.argtypes = [vp, vp, ctypes.c_size_t]
        L.or_rand.argtypes = [u64, u64, u64]; L.or_rand.restype = u64
        L.or_unif_f16.argtypes = [u64, f, f]; L.or_unif_f16.restype = ctypes.c_uint16
        L.or_gen_q4_0_planes.argtypes = [u64, i, i, f, f, vp, vp]
        L.or_gen_q4_0_blocks.argtypes = [u64, i, i, f, f, vp]
        L.or_gen_q4_k.argtypes = [u64, i, i, f, f, vp]
        L.or_gen_act.argtypes = [u64, i, i, vp]
        L.or_q4k_get_scale_min.argtypes = [i, vp, vp, vp]
        L.or_q4k_pack_scales.argtypes = [vp, vp, vp]
        L.or_q4_0_planes_to_blocks.argtypes = [vp, vp, i, i, vp]
        L.or_q4_0_blocks_to_planes.argtypes = [vp, i, i, vp, vp]
        for name in ("or_dequant_f16", "or_dequant_f32"):
            getattr(L, name).argtypes = [i, vp, vp, i, i, vp]
            getattr(L, name).restype = i
        for name in ("or_gemm_f64", "or_gemm_f16w_f64"):
            getattr(L, name).argtypes = [i, vp, vp, vp, i, i, i, vp, i]
            getattr(L, name).restype = i
        L.or_cpu_dequant_matmul.argtypes = [i, vp, vp, vp, i, i, i, vp, vp, i,
                                            ctypes.POINTER(ctypes.c_double),
                                            ctypes.POINTER(ctypes.c_double)]
        L.or_cpu_dequant_matmul.restype = i
        L.or_max_threads.restype = i
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _check(rc, what):
    if rc != 0:
        raise ValueError(f"oracle {what} rejected its arguments (rc={rc})")


# ---------------------------------------------------------------- fp16
def f32_to_f16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().or_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().or_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


# ---------------------------------------------------------------- weights
class QWeights:
    """One quantized matrix W[N][K] in one of the three formats (host bytes)."""

    def __init__(self, qtype: int, N: int, K: int, W: np.ndarray, W_aux: np.ndarray | None = None):
        self.qtype, self.N, self.K, self.W, self.W_aux = qtype, N, K, W, W_aux

    @property
    def nbytes(self) -> int:
        return self.W.nbytes + (0 if self.W_aux is None else self.W_aux.nbytes)


def weight_bytes(qtype: int, N: int, K: int) -> int:
    """Bytes of one N x K matrix (4.5 bits per weight for all three formats)."""
    return N * K * 9 // 16


def gen_weights(qtype: int, N: int, K: int, seed: int, scale_range=None) -> QWeights:
    L = lib()
    if qtype == Q4_0_PLANES:
        lo, hi = scale_range or Q4_0_SCALE_RANGE
        Wq = np.empty((N, K // 2), np.uint8)
        Ws = np.empty((N, K // 32), np.uint16)
        L.or_gen_q4_0_planes(seed, N, K, lo, hi, _p(Wq), _p(Ws))
        return QWeights(qtype, N, K, Wq, Ws)
    if qtype == Q4_0:
        lo, hi = scale_range or Q4_0_SCALE_RANGE
        B = np.empty((N, K // 32 * 18), np.uint8)
        L.or_gen_q4_0_blocks(seed, N, K, lo, hi, _p(B))
        return QWeights(qtype, N, K, B)
    if qtype == Q4_K:
        lo, hi = scale_range or Q4_K_SCALE_RANGE
        B = np.empty((N, K // 256 * 144), np.uint8)
        L.or_gen_q4_k(seed, N, K, lo, hi, _p(B))
        return QWeights(qtype, N, K, B)
    raise ValueError(f"unknown qtype {qtype}")


def gen_act(M: int, K: int, seed: int) -> np.ndarray:
    """A[M][K] ~ N(0,1) rounded to fp16 (as uint16 bits)."""
    A = np.empty((M, K), np.uint16)
    lib().or_gen_act(seed, M, K, _p(A))
    return A


def swiglu_f16(gate_up: np.ndarray, K: int) -> np.ndarray:
    """RN_fp16(SiLU(g) * u) for g = gate_up[:, :K], u = gate_up[:, K:2K] (fp16
    bits), evaluated in fp32 as g / (1 + e^-g) * u (the device evaluates the
    exponential and reciprocal to about one fp32 ulp: results may differ by one
    fp16 ulp near a rounding boundary).  No counterpart in the
    reference (its survey lists the fused SiLU-mul down projection as a next
    step); pinned by closed forms and a float64 evaluation in
    tests/test_oracle.py."""
    g = gate_up[:, :K].view(np.float16).astype(np.float32)
    u = gate_up[:, K:2 * K].view(np.float16).astype(np.float32)
    with np.errstate(over="ignore"):
        s = g / (np.float32(1) + np.exp(-g))
    return (s * u).astype(np.float16).view(np.uint16)


def planes_to_blocks(w: QWeights) -> QWeights:
    assert w.qtype == Q4_0_PLANES
    B = np.empty((w.N, w.K // 32 * 18), np.uint8)
    lib().or_q4_0_planes_to_blocks(_p(w.W), _p(w.W_aux), w.N, w.K, _p(B))
    return QWeights(Q4_0, w.N, w.K, B)


def blocks_to_planes(w: QWeights) -> QWeights:
    assert w.qtype == Q4_0
    Wq = np.empty((w.N, w.K // 2), np.uint8)
    Ws = np.empty((w.N, w.K // 32), np.uint16)
    lib().or_q4_0_blocks_to_planes(_p(w.W), w.N, w.K, _p(Wq), _p(Ws))
    return QWeights(Q4_0_PLANES, w.N, w.K, Wq, Ws)


def q4k_get_scale_min(j: int, scales: bytes):
    s = np.frombuffer(bytes(scales), np.uint8).copy()
    sc = np.zeros(1, np.uint8); m = np.zeros(1, np.uint8)
    lib().or_q4k_get_scale_min(j, _p(s), _p(sc), _p(m))
    return int(sc[0]), int(m[0])


def q4k_pack_scales(sc, m) -> bytes:
    sc = np.ascontiguousarray(sc, np.uint8); m = np.ascontiguousarray(m, np.uint8)
    out = np.zeros(12, np.uint8)
    lib().or_q4k_pack_scales(_p(sc), _p(m), _p(out))
    return out.tobytes()


# ---------------------------------------------------------------- dequant / gemm
def dequant_f16(w: QWeights) -> np.ndarray:
    """Bit-exact fp16 dequant contract, [N][K] uint16 bits."""
    out = np.empty((w.N, w.K), np.uint16)
    _check(lib().or_dequant_f16(w.qtype, _p(w.W), _p(w.W_aux), w.N, w.K, _p(out)), "dequant_f16")
    return out


def dequant_f32(w: QWeights) -> np.ndarray:
    """Unrounded fp32 dequant (the reference's refW), [N][K]."""
    out = np.empty((w.N, w.K), np.float32)
    _check(lib().or_dequant_f32(w.qtype, _p(w.W), _p(w.W_aux), w.N, w.K, _p(out)), "dequant_f32")
    return out


def gemm_f64(w: QWeights, A: np.ndarray, threads: int = 0, round_w: bool = False) -> np.ndarray:
    """C[M][N] = A . dequant(W)^T accumulated in fp64."""
    A = np.ascontiguousarray(A, np.uint16)
    M = A.shape[0]
    assert A.shape[1] == w.K
    C = np.empty((M, w.N), np.float64)
    fn = lib().or_gemm_f16w_f64 if round_w else lib().or_gemm_f64
    _check(fn(w.qtype, _p(w.W), _p(w.W_aux), _p(A), M, w.N, w.K, _p(C), threads), "gemm_f64")
    return C


def cpu_dequant_matmul(w: QWeights, A: np.ndarray, threads: int = 0, scratch=None):
    """CPU baseline: full fp32 dequant then fp32-accumulated matmul.

    Returns (C float32 [M][N], t_dequant_s, t_matmul_s)."""
    A = np.ascontiguousarray(A, np.uint16)
    M = A.shape[0]
    if scratch is None or scratch.size < w.N * w.K:
        scratch = np.empty(w.N * w.K, np.float32)
    C = np.empty((M, w.N), np.float32)
    tdq, tmm = ctypes.c_double(), ctypes.c_double()
    _check(lib().or_cpu_dequant_matmul(w.qtype, _p(w.W), _p(w.W_aux), _p(A), M, w.N, w.K,
                                       _p(scratch), _p(C), threads,
                                       ctypes.byref(tdq), ctypes.byref(tmm)), "cpu_dequant_matmul")
    return C, tdq.value, tmm.value


def max_threads() -> int:
    return int(lib().or_max_threads())


def gate(C, C_ref, max_abs: float = 0.6, rel_frob: float = 1e-3):
    """The GEMM acceptance gate: every value finite, max |C - ref| <= max_abs
    (kernels/q4k_batched.py:102) and ||C - ref||_F / ||ref||_F <= rel_frob.
    Returns (ok, max_abs_err, rel_frob_err, n_nonfinite)."""
    C = np.asarray(C, np.float64)
    C_ref = np.asarray(C_ref, np.float64)
    nonfinite = int(np.count_nonzero(~np.isfinite(C)))
    if nonfinite:
        return False, float("inf"), float("inf"), nonfinite
    diff = C - C_ref
    mae = float(np.max(np.abs(diff))) if diff.size else 0.0
    denom = float(np.linalg.norm(C_ref))
    rfe = float(np.linalg.norm(diff)) / denom if denom > 0 else float(np.linalg.norm(diff))
    return (mae <= max_abs and rfe <= rel_frob), mae, rfe, 0


# ---------------------------------------------------------------- q8 activations
# Integer-dot activation path.  No counterpart in the reference's own kernels:
# its results credit llama.cpp's quantized-GEMM path (pinned clone
# Ajay9o9/llama.cpp @ d493f84, RESULTS.md:244) with packing the activations as
# int8 per 32 values and multiplying them with one integer 4-way dot per four
# weights (RESULTS.md:72-77, 93-96).  Restated from llama.cpp's published
# quantize_q8_1 (ggml-cuda quantize.cu): amax = max|x| over the block,
# d = amax / 127, q = round(x / d) (half away from zero; 0 when amax = 0).  This
# build keeps d in fp32 (llama.cpp stores it as fp16) and the block's sum as the
# exact integer sum of q (llama.cpp keeps a float sum).  Pinned in
# tests/test_oracle.py by closed forms: d = 1 blocks whose q are the rounded
# inputs (ties away from zero), amax -> +-127, the error bound |x - d q| <= d/2,
# the all-zero block, and integer dots against brute force.


def quantize_q8(A: np.ndarray):
    """A[M][K] fp16 bits -> (q int8 [M][K], d float32 [M][K/32], s int32 [M][K/32])."""
    A = np.ascontiguousarray(A, np.uint16)
    M, K = A.shape
    assert K % 32 == 0
    x = A.view(np.float16).astype(np.float32).reshape(M, K // 32, 32)
    amax = np.abs(x).max(axis=-1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        y = (x / d[..., None]).astype(np.float64)     # fp32 quotient, then exact rounding in fp64
    q = np.where(amax[..., None] == 0, 0.0, np.sign(y) * np.floor(np.abs(y) + 0.5)).astype(np.int8)
    s = q.astype(np.int32).sum(axis=-1).astype(np.int32)
    return q.reshape(M, K), d, s


def q8_pack(q, d, s) -> np.ndarray:
    """The device buffer of bf_quantize_q8: q [M][K] int8, then d [M][K/32]
    float32, then s [M][K/32] int32, each region contiguous."""
    return np.concatenate([np.ascontiguousarray(q).view(np.uint8).ravel(),
                           np.ascontiguousarray(d, np.float32).view(np.uint8).ravel(),
                           np.ascontiguousarray(s, np.int32).view(np.uint8).ravel()])


def q8_unpack(buf: np.ndarray, M: int, K: int):
    buf = np.ascontiguousarray(buf).view(np.uint8).ravel()
    nq, nb = M * K, M * (K // 32)
    q = buf[:nq].view(np.int8).reshape(M, K)
    d = buf[nq:nq + 4 * nb].view(np.float32).reshape(M, K // 32)
    s = buf[nq + 4 * nb:nq + 8 * nb].view(np.int32).reshape(M, K // 32)
    return q, d, s


def weight_codes(w: QWeights):
    """(codes uint8 [N][K] in 0..15, scale f64 [N][K/32], offset f64 [N][K/32])
    with dequant(W)[n][k] = scale * code - offset for the block of k: Q4_0 and
    planes offset = 8 d, Q4_K scale = d sc and offset = dmin m of the
    sub-block (byte layouts as in oracle.c's dequant_row_f32)."""
    N, K = w.N, w.K
    if w.qtype == Q4_0_PLANES:
        b = w.W.reshape(N, K // 2)
        codes = np.stack([b & 15, b >> 4], axis=-1).reshape(N, K)
        dd = f16_bits_to_f32(w.W_aux.reshape(N, K // 32)).astype(np.float64)
        return codes, dd, 8 * dd
    if w.qtype == Q4_0:
        blk = w.W.reshape(N, K // 32, 18)
        qs = blk[:, :, 2:]
        codes = np.concatenate([qs & 15, qs >> 4], axis=-1).reshape(N, K)
        dd = f16_bits_to_f32(blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8))
        dd = dd.astype(np.float64)
        return codes, dd, 8 * dd
    blk = w.W.reshape(N, K // 256, 144)
    d = f16_bits_to_f32(blk[:, :, 0].astype(np.uint16) | (blk[:, :, 1].astype(np.uint16) << 8)).astype(np.float64)
    dmin = f16_bits_to_f32(blk[:, :, 2].astype(np.uint16) | (blk[:, :, 3].astype(np.uint16) << 8)).astype(np.float64)
    sb = blk[:, :, 4:16].astype(np.int32)
    sc = np.empty((N, K // 256, 8), np.int32)
    mn = np.empty((N, K // 256, 8), np.int32)
    for j in range(8):     # ggml get_scale_min_k4
        if j < 4:
            sc[:, :, j] = sb[:, :, j] & 63
            mn[:, :, j] = sb[:, :, j + 4] & 63
        else:
            sc[:, :, j] = (sb[:, :, j + 4] & 0xF) | ((sb[:, :, j - 4] >> 6) << 4)
            mn[:, :, j] = (sb[:, :, j + 4] >> 4) | ((sb[:, :, j] >> 6) << 4)
    qs = blk[:, :, 16:].reshape(N, K // 256, 4, 32)
    codes = np.stack([qs & 15, qs >> 4], axis=3).reshape(N, K)
    return codes, (d[..., None] * sc).reshape(N, K // 32), (dmin[..., None] * mn).reshape(N, K // 32)


def gemm_q8(w: QWeights, q, d, s):
    """C[M][N] of the integer-dot path in fp64, and the sum of the magnitudes of
    its terms (for a forward-error bound):
        C[m][n] = sum_b d8[m][b] * (scale[n][b] * dot_b - offset[n][b] * s[m][b]),
        dot_b = sum_{k in b} code[n][k] * q[m][k]   (exact integers)."""
    codes, scale, offset = weight_codes(w)
    M, K = q.shape
    nb = K // 32
    qb = q.astype(np.int64).reshape(M, nb, 32)
    cb = codes.astype(np.int64).reshape(w.N, nb, 32)
    dots = np.einsum("mbk,nbk->mnb", qb, cb)                        # exact int64
    d8 = d.astype(np.float64)[:, None, :]
    t1 = d8 * scale[None] * dots
    t2 = d8 * offset[None] * s.astype(np.float64)[:, None, :]
    return (t1 - t2).sum(-1), (np.abs(t1) + np.abs(t2)).sum(-1)
