"""Host-side mirror of the busfill C-ABI (``include/busfill.h``).

Loads ``bus-fill_amd/lib/libbusfill.so`` with ctypes and exposes the entry
points on device tensors.  PyTorch is used only to own device memory and to
name the HIP stream; every kernel that runs is in libbusfill.  There is no
fallback: if the library is missing, importing the loader raises.

Reference interface mirrored: the kernel symbol ``busfill_q4(A, Wq, Ws, C, Bsz,
K, N)`` of kernels/busfill_v1a.cu:41-46, launched at :154,169; here
``busfill_q4(...)`` keeps that argument order and meaning and adds the stream.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.dirname(_HERE)
# BUSFILL_LIBDIR points the loader at another build of the same library
LIB_PATH = os.path.join(os.environ.get("BUSFILL_LIBDIR") or os.path.join(PKG_DIR, "lib"), "libbusfill.so")
HEADER = os.path.join(os.path.dirname(PKG_DIR), "include", "busfill.h")

# bf_status
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 0, 1, 2, 3
# bf_qtype
Q4_0, Q4_0_PLANES, Q4_K = 0, 1, 2
# bf_otype
OUT_F32, OUT_F16 = 0, 1
# bf_ffn_form
FFN_AUTO, FFN_ONE_LAUNCH, FFN_TWO_LAUNCHES, FFN_CALLS = 0, 1, 2, 3
# bf_algo
ALGO_AUTO, ALGO_MFMA, ALGO_DOT2, ALGO_SIMPLE, ALGO_LDS, ALGO_SLAB, ALGO_SPLIT, ALGO_DENSE = 0, 1, 2, 3, 4, 5, 6, 7

EXPORTS = ("bf_busfill_q4", "bf_busfill_q4_ws", "bf_gemm", "bf_gemm_ex", "bf_gemm_noalloc", "bf_gemm_ws",
           "bf_gemm_workspace_bytes", "bf_gemm_batched", "bf_gemm_batched_ws", "bf_gemm_batched_workspace_bytes",
           "bf_dequant_f16", "bf_gemm_swiglu",
           "bf_swiglu_f16", "bf_ffn_swiglu", "bf_ffn_swiglu_ex", "bf_q8_bytes", "bf_quantize_q8", "bf_gemm_q8",
           "bf_gguf_open", "bf_gguf_close", "bf_gguf_tensor_count", "bf_gguf_tensor_at", "bf_gguf_find",
           "bf_gguf_get_u64", "bf_gguf_get_str", "bf_gguf_upload",
           "bf_ggml_mul_mat", "bf_ggml_mul_mat_workspace_bytes", "bf_ggml_mul_mat_ws",
           "bf_status_str", "bf_last_error", "bf_version")


class GemmDesc(ctypes.Structure):
    """bf_gemm_desc: one GEMM of a bf_gemm_batched call."""
    _fields_ = [("W", ctypes.c_void_p), ("W_aux", ctypes.c_void_p), ("A", ctypes.c_void_p),
                ("lda", ctypes.c_int), ("C", ctypes.c_void_p), ("ldc", ctypes.c_int),
                ("M", ctypes.c_int), ("N", ctypes.c_int), ("K", ctypes.c_int)]


class QWeights(ctypes.Structure):
    """bf_qweights: the weights of one linear (W, and the scale plane for planes)."""
    _fields_ = [("W", ctypes.c_void_p), ("W_aux", ctypes.c_void_p)]


class GgufTensor(ctypes.Structure):
    """bf_gguf_tensor: one tensor of a GGUF file."""
    _fields_ = [("name", ctypes.c_char_p), ("ggml_type", ctypes.c_uint32), ("qtype", ctypes.c_int32),
                ("n_dims", ctypes.c_uint32), ("dims", ctypes.c_uint64 * 4), ("offset", ctypes.c_uint64),
                ("nbytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]


# ggml type codes (bf_ggml_type)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q4_K = 0, 1, 2, 12


class GgmlTensor(ctypes.Structure):
    """bf_ggml_tensor: ggml's type code, device address, ne[4] and nb[4]."""
    _fields_ = [("type", ctypes.c_int32), ("data", ctypes.c_void_p), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_uint64 * 4)]


def ggml_tensor(type_: int, data, ne, nb) -> GgmlTensor:
    """A bf_ggml_tensor from ggml-order ne / nb (ne[0] innermost; missing
    outer dimensions are 1, their strides the whole tensor's span)."""
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    return GgmlTensor(type_, _ptr(data), (ctypes.c_int64 * 4)(*ne), (ctypes.c_uint64 * 4)(*nb))


def ggml_view(t, type_: int | None = None) -> GgmlTensor:
    """The ggml view of a torch tensor (shape and strides reversed into ne and
    nb).  type_ defaults to F32 / F16 from the dtype; quantized weights pass
    their type and a uint8 tensor of shape [..., rows, row bytes]."""
    import torch
    if type_ is None:
        type_ = {torch.float32: GGML_F32, torch.float16: GGML_F16}[t.dtype]
    es = t.element_size()
    shape, strides = list(t.shape)[::-1], [s * es for s in t.stride()][::-1]
    if type_ in (GGML_Q4_0, GGML_Q4_K):
        blk, bb = (32, 18) if type_ == GGML_Q4_0 else (256, 144)
        assert shape[0] % bb == 0 and strides[0] == 1, "quantized rows: whole contiguous blocks"
        shape[0], strides[0] = shape[0] // bb * blk, bb
    return ggml_tensor(type_, t, shape, strides)


class BusfillError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str):
        self.status = status
        super().__init__(f"{where}: status {status} ({detail})")


class BusfillInvalid(BusfillError, ValueError):
    pass


_lib = None


def lib() -> ctypes.CDLL:
    """Load libbusfill.so (raises FileNotFoundError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is missing: run `python bus-fill_amd/build.py` "
                                    "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        vp, i = ctypes.c_void_p, ctypes.c_int
        L.bf_busfill_q4.argtypes = [vp, vp, vp, vp, i, i, i, vp]
        L.bf_gemm.argtypes = [i, vp, vp, vp, i, vp, i, i, i, i, i, vp]
        L.bf_gemm_ex.argtypes = [i, vp, vp, vp, i, vp, i, i, i, i, i, i, vp]
        L.bf_gemm_noalloc.argtypes = [i, vp, vp, vp, i, vp, i, i, i, i, i, vp]
        sz = ctypes.c_size_t
        L.bf_busfill_q4_ws.argtypes = [vp, vp, vp, vp, i, i, i, vp, sz, vp]
        L.bf_gemm_ws.argtypes = [i, vp, vp, vp, i, vp, i, i, i, i, i, vp, sz, vp]
        L.bf_gemm_workspace_bytes.argtypes = [i, i, i, i, i]
        L.bf_gemm_workspace_bytes.restype = sz
        L.bf_dequant_f16.argtypes = [i, vp, vp, vp, i, i, vp]
        L.bf_gemm_batched.argtypes = [i, i, i, ctypes.POINTER(GemmDesc), vp]
        L.bf_gemm_batched_ws.argtypes = [i, i, i, ctypes.POINTER(GemmDesc), vp, sz, vp]
        L.bf_gemm_batched_workspace_bytes.argtypes = [i, i, i, ctypes.POINTER(GemmDesc)]
        L.bf_gemm_batched_workspace_bytes.restype = sz
        L.bf_gemm_swiglu.argtypes = [i, vp, vp, vp, i, vp, i, i, i, i, i, vp]
        L.bf_swiglu_f16.argtypes = [vp, i, vp, i, i, i, vp]
        L.bf_ffn_swiglu.argtypes = [i, QWeights, QWeights, QWeights, vp, i, vp, i, vp, i, i, i, i, i, i, vp]
        L.bf_ffn_swiglu_ex.argtypes = [i, QWeights, QWeights, QWeights, vp, i, vp, i, vp, i, i, i, i, i, i, i, vp]
        L.bf_q8_bytes.argtypes = [i, i]
        L.bf_q8_bytes.restype = ctypes.c_size_t
        L.bf_quantize_q8.argtypes = [vp, i, vp, i, i, vp]
        L.bf_gemm_q8.argtypes = [i, vp, vp, vp, vp, i, i, i, i, i, vp]
        L.bf_gguf_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp)]
        L.bf_gguf_close.argtypes = [vp]
        L.bf_gguf_close.restype = None
        L.bf_gguf_tensor_count.argtypes = [vp]
        L.bf_gguf_tensor_count.restype = ctypes.c_int64
        L.bf_gguf_tensor_at.argtypes = [vp, ctypes.c_int64, ctypes.POINTER(GgufTensor)]
        L.bf_gguf_find.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(GgufTensor)]
        L.bf_gguf_get_u64.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]
        L.bf_gguf_get_str.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.POINTER(ctypes.c_uint64)]
        L.bf_gguf_upload.argtypes = [vp, ctypes.POINTER(GgufTensor), vp, vp]
        for f in ("bf_gguf_open", "bf_gguf_tensor_at", "bf_gguf_find", "bf_gguf_get_u64", "bf_gguf_get_str",
                  "bf_gguf_upload"):
            getattr(L, f).restype = i
        for f in ("bf_busfill_q4", "bf_busfill_q4_ws", "bf_gemm", "bf_gemm_ex", "bf_gemm_noalloc", "bf_gemm_ws",
                  "bf_gemm_batched", "bf_gemm_batched_ws", "bf_dequant_f16", "bf_gemm_swiglu",
                  "bf_swiglu_f16", "bf_ffn_swiglu", "bf_ffn_swiglu_ex", "bf_quantize_q8", "bf_gemm_q8"):
            getattr(L, f).restype = i
        gp = ctypes.POINTER(GgmlTensor)
        L.bf_ggml_mul_mat.argtypes = [gp, gp, gp, vp]
        L.bf_ggml_mul_mat.restype = i
        L.bf_ggml_mul_mat_workspace_bytes.argtypes = [gp, gp, gp]
        L.bf_ggml_mul_mat_workspace_bytes.restype = sz
        L.bf_ggml_mul_mat_ws.argtypes = [gp, gp, gp, vp, sz, vp]
        L.bf_ggml_mul_mat_ws.restype = i
        L.bf_status_str.argtypes = [i]
        L.bf_status_str.restype = ctypes.c_char_p
        L.bf_last_error.restype = ctypes.c_char_p
        L.bf_version.restype = i
        _lib = L
    return _lib


def _check(status: int, where: str) -> None:
    if status != OK:
        detail = lib().bf_last_error().decode() or lib().bf_status_str(status).decode()
        cls = BusfillInvalid if status == ERR_INVALID else BusfillError
        raise cls(status, where, detail)


def _ptr(t) -> int | None:
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def gemm(qtype: int, W, W_aux, A, C, M: int, N: int, K: int, *, lda: int | None = None,
         ldc: int | None = None, otype: int = OUT_F32, algo: int = ALGO_AUTO, stream=None) -> None:
    """C[M][N] = A[M][K] . dequant(W)^T on the GPU (all arguments device tensors
    or raw device addresses; C is overwritten)."""
    st = lib().bf_gemm_ex(qtype, _ptr(W), _ptr(W_aux), _ptr(A), K if lda is None else lda,
                          _ptr(C), N if ldc is None else ldc, otype, M, N, K, algo, _stream(stream))
    _check(st, "bf_gemm_ex")


def gemm_noalloc(qtype: int, W, W_aux, A, C, M: int, N: int, K: int, *, lda: int | None = None,
                 ldc: int | None = None, otype: int = OUT_F32, stream=None) -> None:
    """bf_gemm_noalloc: bf_gemm with the K-split scratch in a per-GPU static
    array instead of a workspace allocated per stream."""
    st = lib().bf_gemm_noalloc(qtype, _ptr(W), _ptr(W_aux), _ptr(A), K if lda is None else lda,
                               _ptr(C), N if ldc is None else ldc, otype, M, N, K, _stream(stream))
    _check(st, "bf_gemm_noalloc")


def gemm_workspace_bytes(qtype: int, M: int, N: int, K: int, *, otype: int = OUT_F32) -> int:
    """Bytes of caller-owned workspace gemm_ws needs for this shape (0: none)."""
    return int(lib().bf_gemm_workspace_bytes(qtype, otype, M, N, K))


def gemm_ws(qtype: int, W, W_aux, A, C, M: int, N: int, K: int, workspace, workspace_bytes: int, *,
            lda: int | None = None, ldc: int | None = None, otype: int = OUT_F32, stream=None) -> None:
    """bf_gemm_ws: bf_gemm with a caller-owned workspace (a device tensor or
    address of workspace_bytes, 256-byte aligned; None with 0 bytes when the
    call needs none)."""
    st = lib().bf_gemm_ws(qtype, _ptr(W), _ptr(W_aux), _ptr(A), K if lda is None else lda, _ptr(C),
                          N if ldc is None else ldc, otype, M, N, K, _ptr(workspace), workspace_bytes,
                          _stream(stream))
    _check(st, "bf_gemm_ws")


def gemm_swiglu(qtype: int, W, W_aux, gate_up, C, M: int, N: int, K: int, *, ld: int | None = None,
                ldc: int | None = None, otype: int = OUT_F32, stream=None) -> None:
    """C[M][N] = (SiLU(G) * U) . dequant(W)^T with G, U = columns [0, K) and
    [K, 2K) of gate_up[M][ld] (batch 1-2; BusfillError BF_ERR_UNSUPPORTED
    otherwise)."""
    st = lib().bf_gemm_swiglu(qtype, _ptr(W), _ptr(W_aux), _ptr(gate_up), 2 * K if ld is None else ld, _ptr(C),
                              N if ldc is None else ldc, otype, M, N, K, _stream(stream))
    _check(st, "bf_gemm_swiglu")


def ffn_swiglu(qtype: int, gate, up, down, A, gate_up, C, M: int, K: int, F: int, N: int, *,
               lda: int | None = None, ldgu: int | None = None, ldc: int | None = None, otype: int = OUT_F32,
               form: int = FFN_AUTO, stream=None) -> None:
    """C[M][N] = (SiLU(A . Wg^T) * (A . Wu^T)) . Wd^T.  gate, up and down are
    (W, W_aux) pairs (W_aux None except for the planes format); gate_up is the
    caller's fp16 [M][ldgu >= 2F] intermediate; form one of FFN_*."""
    qw = [QWeights(_ptr(w), _ptr(a)) for (w, a) in (gate, up, down)]
    st = lib().bf_ffn_swiglu_ex(qtype, qw[0], qw[1], qw[2], _ptr(A), K if lda is None else lda, _ptr(gate_up),
                                2 * F if ldgu is None else ldgu, _ptr(C), N if ldc is None else ldc, otype, M, K, F, N,
                                form, _stream(stream))
    _check(st, "bf_ffn_swiglu_ex")


def swiglu_f16(gate_up, out, M: int, K: int, *, ld: int | None = None, ldo: int | None = None,
               stream=None) -> None:
    """out[M][K] (fp16 bits) = RN_fp16(SiLU(G) * U), G and U as for gemm_swiglu."""
    _check(lib().bf_swiglu_f16(_ptr(gate_up), 2 * K if ld is None else ld, _ptr(out), K if ldo is None else ldo,
                               M, K, _stream(stream)), "bf_swiglu_f16")


def q8_bytes(M: int, K: int) -> int:
    """Bytes of the int8 activation buffer for M rows of K (0 for a bad shape)."""
    return int(lib().bf_q8_bytes(M, K))


def quantize_q8(A, Aq, M: int, K: int, *, lda: int | None = None, stream=None) -> None:
    """Aq (q8_bytes(M, K) bytes) = A[M][K] fp16 quantized to int8 per 32 values."""
    _check(lib().bf_quantize_q8(_ptr(A), K if lda is None else lda, _ptr(Aq), M, K, _stream(stream)),
           "bf_quantize_q8")


def gemm_q8(qtype: int, W, W_aux, Aq, C, M: int, N: int, K: int, *, ldc: int | None = None,
            otype: int = OUT_F32, stream=None) -> None:
    """C[M][N] from quantize_q8's activations and the weights in place (M <= 16)."""
    _check(lib().bf_gemm_q8(qtype, _ptr(W), _ptr(W_aux), _ptr(Aq), _ptr(C), N if ldc is None else ldc, otype,
                            M, N, K, _stream(stream)), "bf_gemm_q8")


def _descs(gemms):
    descs = (GemmDesc * max(1, len(gemms)))()
    for d, (W, W_aux, A, C, M, N, K) in zip(descs, gemms):
        d.W, d.W_aux, d.A, d.lda, d.C, d.ldc, d.M, d.N, d.K = (_ptr(W), _ptr(W_aux), _ptr(A), K, _ptr(C), N,
                                                               M, N, K)
    return descs


def gemm_batched(qtype: int, gemms, *, otype: int = OUT_F32, stream=None) -> None:
    """Independent GEMMs in as few launches as the library can: `gemms` is a
    list of (W, W_aux, A, C, M, N, K) with device tensors or addresses (lda = K,
    ldc = N); each C is overwritten as by gemm()."""
    _check(lib().bf_gemm_batched(qtype, otype, len(gemms), _descs(gemms), _stream(stream)), "bf_gemm_batched")


def gemm_batched_workspace_bytes(qtype: int, gemms, *, otype: int = OUT_F32) -> int:
    """Bytes of caller-owned workspace gemm_batched_ws needs for these GEMMs."""
    return int(lib().bf_gemm_batched_workspace_bytes(qtype, otype, len(gemms), _descs(gemms)))


def gemm_batched_ws(qtype: int, gemms, workspace, workspace_bytes: int, *, otype: int = OUT_F32,
                    stream=None) -> None:
    """gemm_batched with a caller-owned workspace (as gemm_ws)."""
    _check(lib().bf_gemm_batched_ws(qtype, otype, len(gemms), _descs(gemms), _ptr(workspace), workspace_bytes,
                                    _stream(stream)), "bf_gemm_batched_ws")


class Gguf:
    """A GGUF file opened by the library's reader (memory-mapped).

    tensors(): every tensor's GgufTensor; find(name); get_u64 / get_str for
    metadata; upload(tensor, device_tensor_or_address) copies the bytes to the
    device unchanged (Q4_0 / Q4_K blocks are bf_gemm's layouts)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _check(lib().bf_gguf_open(os.fsencode(path), ctypes.byref(h)), "bf_gguf_open")
        self._h = h

    def close(self):
        if self._h:
            lib().bf_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensors(self):
        out = []
        for i in range(lib().bf_gguf_tensor_count(self._h)):
            t = GgufTensor()
            _check(lib().bf_gguf_tensor_at(self._h, i, ctypes.byref(t)), "bf_gguf_tensor_at")
            out.append(t)
        return out

    def find(self, name: str) -> GgufTensor:
        t = GgufTensor()
        _check(lib().bf_gguf_find(self._h, name.encode(), ctypes.byref(t)), "bf_gguf_find")
        return t

    def get_u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        _check(lib().bf_gguf_get_u64(self._h, key.encode(), ctypes.byref(v)), "bf_gguf_get_u64")
        return v.value

    def get_str(self, key: str) -> bytes:
        p, n = ctypes.c_char_p(), ctypes.c_uint64()
        _check(lib().bf_gguf_get_str(self._h, key.encode(), ctypes.byref(p), ctypes.byref(n)), "bf_gguf_get_str")
        return ctypes.string_at(p, n.value)

    def data(self, t: GgufTensor) -> bytes:
        """The tensor's bytes as mapped (a copy)."""
        return ctypes.string_at(t.data, t.nbytes) if t.nbytes else b""

    def upload(self, t: GgufTensor, dst, stream=None) -> None:
        _check(lib().bf_gguf_upload(self._h, ctypes.byref(t), _ptr(dst), _stream(stream)), "bf_gguf_upload")


def busfill_q4(A, Wq, Ws, C, Bsz: int, K: int, N: int, stream=None) -> None:
    """Reference-compatible call: Q4_0 planes, fp32 C[Bsz][N]."""
    _check(lib().bf_busfill_q4(_ptr(A), _ptr(Wq), _ptr(Ws), _ptr(C), Bsz, K, N, _stream(stream)),
           "bf_busfill_q4")


def busfill_q4_ws(A, Wq, Ws, C, Bsz: int, K: int, N: int, workspace, workspace_bytes: int, stream=None) -> None:
    """busfill_q4 with a caller-owned workspace (as gemm_ws)."""
    _check(lib().bf_busfill_q4_ws(_ptr(A), _ptr(Wq), _ptr(Ws), _ptr(C), Bsz, K, N, _ptr(workspace),
                                  workspace_bytes, _stream(stream)), "bf_busfill_q4_ws")


def dequant_f16(qtype: int, W, W_aux, out, N: int, K: int, stream=None) -> None:
    """out[N][K] (fp16 bits) = bit-exact dequant of W."""
    _check(lib().bf_dequant_f16(qtype, _ptr(W), _ptr(W_aux), _ptr(out), N, K, _stream(stream)),
           "bf_dequant_f16")


def ggml_mul_mat(src0: GgmlTensor, src1: GgmlTensor, dst: GgmlTensor, stream=None) -> None:
    """dst = ggml_mul_mat(src0, src1) (ggml's semantics; bf_ggml_tensor views)."""
    _check(lib().bf_ggml_mul_mat(ctypes.byref(src0), ctypes.byref(src1), ctypes.byref(dst), _stream(stream)),
           "bf_ggml_mul_mat")


def ggml_mul_mat_workspace_bytes(src0: GgmlTensor, src1: GgmlTensor, dst: GgmlTensor) -> int:
    return lib().bf_ggml_mul_mat_workspace_bytes(ctypes.byref(src0), ctypes.byref(src1), ctypes.byref(dst))


def ggml_mul_mat_ws(src0: GgmlTensor, src1: GgmlTensor, dst: GgmlTensor, workspace, workspace_bytes: int,
                    stream=None) -> None:
    _check(lib().bf_ggml_mul_mat_ws(ctypes.byref(src0), ctypes.byref(src1), ctypes.byref(dst), _ptr(workspace),
                                    workspace_bytes, _stream(stream)), "bf_ggml_mul_mat_ws")


def version() -> int:
    return int(lib().bf_version())


def weight_bytes(N: int, K: int) -> int:
    """Bytes streamed for one N x K matrix: 4.5 bits/weight in all three formats."""
    return N * K * 9 // 16
