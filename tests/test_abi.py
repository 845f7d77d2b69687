"""C-ABI checks that need no GPU: the library loads, exports exactly what
include/busfill.h declares, and rejects bad arguments before enqueuing work
(validation happens before any HIP call, so no device is touched)."""
import ctypes
import os
import re

import pytest

import busfill as bf

HDR = open(bf.HEADER).read()


def declared_functions():
    body = re.sub(r"/\*.*?\*/", "", HDR, flags=re.S)
    return sorted(set(re.findall(r"\b(bf_[a-z0-9_]+)\s*\(", body)))


def test_header_declares_expected_entry_points():
    assert declared_functions() == sorted(bf.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = bf.lib()
    for name in declared_functions():
        assert hasattr(L, name), name
    # and the symbols are real dynamic exports
    out = os.popen(f"nm -D --defined-only {bf.LIB_PATH}").read()
    for name in declared_functions():
        assert re.search(rf"\bT {name}\b", out), name


def test_status_strings_and_version():
    L = bf.lib()
    assert L.bf_status_str(0) == b"BF_OK"
    assert L.bf_status_str(1) == b"BF_ERR_INVALID"
    assert L.bf_status_str(2) == b"BF_ERR_UNSUPPORTED"
    assert L.bf_status_str(3) == b"BF_ERR_HIP"
    assert bf.version() >= 100


FAKE = 0x10000   # never dereferenced: every case below is rejected in validation


@pytest.mark.parametrize("kw,needle", [
    (dict(qtype=7), "qtype"),
    (dict(W=None), "W is NULL"),
    (dict(qtype=bf.Q4_0_PLANES, W_aux=None), "W_aux"),
    (dict(qtype=bf.Q4_K, W_aux=FAKE), "must be NULL"),
    (dict(K=100), "multiple of 32"),
    (dict(qtype=bf.Q4_K, K=4096 + 32), "multiple of 256"),
    (dict(M=0), "M=0"),
    (dict(N=0), "N=0"),
    (dict(lda=100), "lda"),
    (dict(ldc=10), "ldc"),
    (dict(A=None), "NULL"),
    (dict(C=None), "NULL"),
    (dict(otype=5), "otype"),
    (dict(algo=9), "algo"),
    (dict(A=FAKE + 1), "aligned"),
])
def test_gemm_rejects_invalid_arguments(kw, needle):
    args = dict(qtype=bf.Q4_0, W=FAKE, W_aux=None, A=FAKE, lda=None, C=FAKE, ldc=None,
                otype=bf.OUT_F32, M=4, N=64, K=512, algo=bf.ALGO_AUTO)
    args.update(kw)
    lda = args["lda"] if args["lda"] is not None else args["K"]
    ldc = args["ldc"] if args["ldc"] is not None else args["N"]
    st = bf.lib().bf_gemm_ex(args["qtype"], args["W"], args["W_aux"], args["A"], lda, args["C"], ldc,
                             args["otype"], args["M"], args["N"], args["K"], args["algo"], None)
    assert st == bf.ERR_INVALID
    assert needle in bf.lib().bf_last_error().decode()


def test_reference_entry_rejects_bad_shape():
    st = bf.lib().bf_busfill_q4(FAKE, FAKE, FAKE, FAKE, 1, 33, 64, None)
    assert st == bf.ERR_INVALID
    with pytest.raises(bf.BusfillInvalid):
        bf.busfill_q4(FAKE, FAKE, FAKE, FAKE, 0, 64, 64, stream=0)


def test_dequant_rejects_bad_arguments():
    assert bf.lib().bf_dequant_f16(bf.Q4_K, FAKE, None, None, 4, 256, None) == bf.ERR_INVALID
    assert bf.lib().bf_dequant_f16(bf.Q4_K, FAKE, None, FAKE, 4, 100, None) == bf.ERR_INVALID
    assert bf.lib().bf_dequant_f16(bf.Q4_0_PLANES, FAKE, None, FAKE, 4, 256, None) == bf.ERR_INVALID


def test_product_path_has_no_fallback(tmp_path, monkeypatch):
    """The loader raises when libbusfill.so is absent; nothing substitutes for it."""
    monkeypatch.setattr(bf, "LIB_PATH", str(tmp_path / "missing.so"))
    monkeypatch.setattr(bf, "_lib", None)
    with pytest.raises(FileNotFoundError):
        bf.lib()


def test_product_sources_do_not_use_the_oracle():
    pkg = os.path.dirname(bf.PKG_DIR)
    for dirpath, _, files in os.walk(os.path.join(pkg, "bus-fill_amd")):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")):
                text = open(os.path.join(dirpath, f)).read()
                assert "import oracle" not in text and "liboracle" not in text, f


def test_batched_rejects_invalid_descs_before_any_launch():
    L = bf.lib()
    d = (bf.GemmDesc * 2)()
    for x in d:
        x.W, x.W_aux, x.A, x.lda, x.C, x.ldc, x.M, x.N, x.K = FAKE, None, FAKE, 512, FAKE, 64, 32, 64, 512
    d[1].M = 0
    assert L.bf_gemm_batched(bf.Q4_0, bf.OUT_F32, 2, d, None) == bf.ERR_INVALID
    assert "M=0" in L.bf_last_error().decode()
    d[1].M, d[1].lda = 32, 100
    assert L.bf_gemm_batched(bf.Q4_0, bf.OUT_F32, 2, d, None) == bf.ERR_INVALID
    assert L.bf_gemm_batched(bf.Q4_0, bf.OUT_F32, -1, d, None) == bf.ERR_INVALID
    assert L.bf_gemm_batched(bf.Q4_0, bf.OUT_F32, 1, None, None) == bf.ERR_INVALID
    assert L.bf_gemm_batched(bf.Q4_0, bf.OUT_F32, 0, None, None) == bf.OK


def test_gemm_desc_layout_matches_header():
    # pointers at 0, 8, 16; lda at 24; C at 32 (after padding); ldc, M, N, K at 40..52
    assert ctypes.sizeof(bf.GemmDesc) == 56
    assert bf.GemmDesc.C.offset == 32 and bf.GemmDesc.K.offset == 52
    assert "bf_gemm_desc" in HDR


def test_swiglu_entries_reject_before_any_launch():
    """bf_gemm_swiglu / bf_swiglu_f16 argument checks (no GPU needed: every
    case returns before a launch)."""
    L = bf.lib()
    K, N = 1024, 256
    # batch 3: not fused
    assert L.bf_gemm_swiglu(bf.Q4_K, FAKE, None, FAKE, 2 * K, FAKE, N, bf.OUT_F32, 3, N, K, None) == bf.ERR_UNSUPPORTED
    assert "bf_swiglu_f16 then bf_gemm" in L.bf_last_error().decode()
    # ld must cover gate and up
    assert L.bf_gemm_swiglu(bf.Q4_K, FAKE, None, FAKE, K, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    # rows 16-byte aligned
    assert L.bf_gemm_swiglu(bf.Q4_K, FAKE, None, FAKE + 2, 2 * K, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_swiglu(bf.Q4_K, FAKE, None, FAKE, 2 * K + 4, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_swiglu(bf.Q4_K, None, None, FAKE, 2 * K, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_swiglu_f16(None, 2 * K, FAKE, K, 1, K, None) == bf.ERR_INVALID
    assert L.bf_swiglu_f16(FAKE, 2 * K, FAKE, K, 1, 12, None) == bf.ERR_INVALID
    assert L.bf_swiglu_f16(FAKE, K, FAKE, K, 1, K, None) == bf.ERR_INVALID
    assert L.bf_swiglu_f16(FAKE, 2 * K, FAKE + 8, K, 1, K, None) == bf.ERR_INVALID


def test_ffn_entry_rejects_before_any_launch():
    """bf_ffn_swiglu argument checks: every case returns before a launch (and
    before the workspace is looked up), so no GPU is needed."""
    L = bf.lib()
    K, F, N = 1024, 2048, 512
    w = bf.QWeights(FAKE, None)

    def call(qtype=bf.Q4_K, gate=w, up=w, down=w, A=FAKE, lda=K, gu=FAKE, ldgu=2 * F, C=FAKE, ldc=N,
             otype=bf.OUT_F32, M=1, K_=K, F_=F, N_=N):
        return L.bf_ffn_swiglu(qtype, gate, up, down, A, lda, gu, ldgu, C, ldc, otype, M, K_, F_, N_, None)

    assert call(gu=None) == bf.ERR_INVALID
    assert call(F_=12) == bf.ERR_INVALID                       # F % 8
    assert call(ldgu=2 * F - 8) == bf.ERR_INVALID              # gate and up must both fit
    assert call(gu=FAKE + 8) == bf.ERR_INVALID                 # 16-byte rows
    assert call(ldgu=2 * F + 4) == bf.ERR_INVALID
    assert call(gate=bf.QWeights(None, None)) == bf.ERR_INVALID
    assert call(up=bf.QWeights(None, None)) == bf.ERR_INVALID
    assert call(down=bf.QWeights(FAKE, FAKE)) == bf.ERR_INVALID   # W_aux only for planes
    assert call(qtype=bf.Q4_0_PLANES) == bf.ERR_INVALID          # planes without scale planes
    assert call(K_=1000) == bf.ERR_INVALID
    assert call(F_=2048 + 8, ldgu=2 * 2048 + 16) == bf.ERR_INVALID   # down's K = F: multiple of 256 for Q4_K
    assert "multiple of 256" in L.bf_last_error().decode()
    assert call(A=None) == bf.ERR_INVALID
    assert call(C=None) == bf.ERR_INVALID
    assert call(ldc=N - 1) == bf.ERR_INVALID
    assert call(M=0) == bf.ERR_INVALID
    assert call(otype=3) == bf.ERR_INVALID
    assert L.bf_ffn_swiglu_ex(bf.Q4_K, w, w, w, FAKE, K, FAKE, 2 * F, FAKE, N, bf.OUT_F32, 1, K, F, N, 4,
                              None) == bf.ERR_INVALID          # unknown form
    # forms that do not serve batch 3 refuse before anything is enqueued
    for form in (bf.FFN_ONE_LAUNCH, bf.FFN_TWO_LAUNCHES):
        assert L.bf_ffn_swiglu_ex(bf.Q4_K, w, w, w, FAKE, K, FAKE, 2 * F, FAKE, N, bf.OUT_F32, 3, K, F, N, form,
                                  None) == bf.ERR_UNSUPPORTED


def test_qweights_layout_matches_header():
    assert ctypes.sizeof(bf.QWeights) == 16 and bf.QWeights.W_aux.offset == 8
    assert "bf_qweights" in HDR


def test_q8_entries_reject_before_any_launch():
    """bf_q8_bytes / bf_quantize_q8 / bf_gemm_q8 argument checks (no GPU needed:
    every call below is rejected before a launch)."""
    L = bf.lib()
    N, K = 64, 512
    assert L.bf_q8_bytes(3, 512) == 3 * 512 + 8 * 3 * 16
    assert L.bf_q8_bytes(0, 512) == 0 and L.bf_q8_bytes(1, 48) == 0
    assert L.bf_quantize_q8(None, K, FAKE, 1, K, None) == bf.ERR_INVALID
    assert L.bf_quantize_q8(FAKE, K, FAKE, 1, 48, None) == bf.ERR_INVALID
    assert L.bf_quantize_q8(FAKE, K - 8, FAKE, 1, K, None) == bf.ERR_INVALID
    assert L.bf_quantize_q8(FAKE + 8, K, FAKE, 1, K, None) == bf.ERR_INVALID
    assert L.bf_quantize_q8(FAKE, K + 4, FAKE, 2, K, None) == bf.ERR_INVALID
    assert L.bf_quantize_q8(FAKE, K, FAKE + 4, 1, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_q8(bf.Q4_K, FAKE, None, FAKE, FAKE, N, bf.OUT_F32, 17, N, K, None) == bf.ERR_UNSUPPORTED
    assert "batch 1-16" in L.bf_last_error().decode()
    assert L.bf_gemm_q8(bf.Q4_0, FAKE, None, FAKE, FAKE, N, bf.OUT_F32, 2, N, 96, None) == bf.ERR_UNSUPPORTED
    assert L.bf_gemm_q8(bf.Q4_K, FAKE, None, None, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_q8(bf.Q4_K, FAKE, None, FAKE + 4, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_q8(bf.Q4_K, FAKE + 4, None, FAKE, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_q8(bf.Q4_K, FAKE, None, FAKE, FAKE, N - 1, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_q8(bf.Q4_0_PLANES, FAKE, None, FAKE, FAKE, N, bf.OUT_F32, 1, N, K, None) == bf.ERR_INVALID
    assert L.bf_gemm_q8(bf.Q4_K, FAKE, None, FAKE, FAKE, N, 7, 1, N, K, None) == bf.ERR_INVALID


def test_workspace_entries_validate_before_any_launch():
    """The caller-owned workspace entries reject a NULL or misaligned workspace
    (and the size queries answer 0 for invalid requests) before any HIP call."""
    L = bf.lib()
    st = L.bf_gemm_ws(bf.Q4_K, FAKE, None, FAKE, 5120, FAKE, 5120, bf.OUT_F32, 32, 5120, 5120, None, 4096, None)
    assert st == bf.ERR_INVALID and b"NULL" in L.bf_last_error()
    st = L.bf_gemm_ws(bf.Q4_K, FAKE, None, FAKE, 5120, FAKE, 5120, bf.OUT_F32, 32, 5120, 5120, FAKE + 64, 4096, None)
    assert st == bf.ERR_INVALID and b"256-byte" in L.bf_last_error()
    st = L.bf_busfill_q4_ws(FAKE, FAKE, FAKE, FAKE, 32, 5120, 5120, FAKE + 8, 1 << 20, None)
    assert st == bf.ERR_INVALID
    st = L.bf_gemm_batched_ws(bf.Q4_K, bf.OUT_F32, -1, None, None, 0, None)
    assert st == bf.ERR_INVALID and b"count" in L.bf_last_error()
    assert L.bf_gemm_batched_workspace_bytes(bf.Q4_K, bf.OUT_F32, -1, None) == 0
    assert L.bf_gemm_workspace_bytes(bf.Q4_K, bf.OUT_F32, 32, 5120, 5000) == 0      # K % 256 != 0
    assert L.bf_gemm_workspace_bytes(7, bf.OUT_F32, 32, 5120, 5120) == 0            # unknown format


def test_ggml_tensor_layout_matches_header():
    # type at 0, data at 8, ne[4] at 16, nb[4] at 48: 80 bytes
    assert ctypes.sizeof(bf.GgmlTensor) == 80
    assert bf.GgmlTensor.ne.offset == 16 and bf.GgmlTensor.nb.offset == 48
    assert "bf_ggml_tensor" in HDR
    for name, code in (("BF_GGML_F32", 0), ("BF_GGML_F16", 1), ("BF_GGML_Q4_0", 2), ("BF_GGML_Q4_K", 12)):
        assert re.search(rf"\b{name} = {code}\b", HDR), name


def _ggml_case(K=512, N=64, M=4, t0=bf.GGML_Q4_K, t1=bf.GGML_F32, ne2=(1, 1), nr=(1, 1)):
    """Valid views (fake addresses) of a Q4 src0 [r2 r3 slices][N][K], an
    src1 [ne2 x ne3][M][K] and an F32 dst."""
    blk, bb = (256, 144) if t0 == bf.GGML_Q4_K else (32, 18)
    rb = K // blk * bb
    s0 = bf.ggml_tensor(t0, FAKE, [K, N, ne2[0] // nr[0], ne2[1] // nr[1]], [bb, rb])
    es = 4 if t1 == bf.GGML_F32 else 2
    s1 = bf.ggml_tensor(t1, FAKE, [K, M, ne2[0], ne2[1]], [es, es * K])
    d = bf.ggml_tensor(bf.GGML_F32, FAKE, [N, M, ne2[0], ne2[1]], [4, 4 * N])
    return s0, s1, d


@pytest.mark.parametrize("edit,status,needle", [
    (lambda s0, s1, d: setattr(s0, "type", bf.GGML_F32), bf.ERR_UNSUPPORTED, "src0 type"),
    (lambda s0, s1, d: setattr(s1, "type", bf.GGML_Q4_0), bf.ERR_UNSUPPORTED, "src1 type"),
    (lambda s0, s1, d: setattr(d, "type", bf.GGML_F16), bf.ERR_UNSUPPORTED, "dst type"),
    (lambda s0, s1, d: s1.ne.__setitem__(0, 256), bf.ERR_INVALID, "ne[0]"),
    (lambda s0, s1, d: (s0.ne.__setitem__(2, 2), s1.ne.__setitem__(2, 3)), bf.ERR_INVALID, "multiples"),
    (lambda s0, s1, d: d.ne.__setitem__(1, 5), bf.ERR_INVALID, "dst ne"),
    (lambda s0, s1, d: s0.ne.__setitem__(1, 0), bf.ERR_INVALID, "ne[1]=0"),
    (lambda s0, s1, d: setattr(s1, "data", None), bf.ERR_INVALID, "NULL"),
    (lambda s0, s1, d: s0.nb.__setitem__(1, 2 * 288), bf.ERR_UNSUPPORTED, "contiguous blocks"),
    (lambda s0, s1, d: d.nb.__setitem__(0, 8), bf.ERR_UNSUPPORTED, "F32 rows"),
    (lambda s0, s1, d: d.nb.__setitem__(1, 4 * 63), bf.ERR_UNSUPPORTED, "F32 rows"),
    (lambda s0, s1, d: s1.nb.__setitem__(1, 4 * 512 + 2), bf.ERR_UNSUPPORTED, "element size"),
])
def test_ggml_mul_mat_rejects_before_any_launch(edit, status, needle):
    s0, s1, d = _ggml_case()
    edit(s0, s1, d)
    L = bf.lib()
    st = L.bf_ggml_mul_mat(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), None)
    assert st == status, L.bf_last_error()
    assert needle in L.bf_last_error().decode()
    assert L.bf_ggml_mul_mat_workspace_bytes(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d)) == 0


def test_ggml_mul_mat_shape_rules():
    """ggml_can_mul_mat: K must match and src1's outer dimensions be multiples
    of src0's (broadcast); Q4_K rows are whole 256-weight blocks; overlapping
    dst slices and a NULL tensor are refused."""
    L = bf.lib()
    s0, s1, d = _ggml_case(ne2=(6, 2), nr=(3, 2))
    s1.ne[3] = 3   # 3 % 1 == 0 but dst ne[3] still 2
    assert L.bf_ggml_mul_mat(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), None) == bf.ERR_INVALID
    s0, s1, d = _ggml_case(K=288, t0=bf.GGML_Q4_K)
    assert L.bf_ggml_mul_mat(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), None) == bf.ERR_INVALID
    assert b"whole blocks" in L.bf_last_error()
    s0, s1, d = _ggml_case(ne2=(2, 1))
    d.nb[2] = 4 * 64 * 3   # slices 3 rows apart, 4 rows each
    assert L.bf_ggml_mul_mat(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), None) == bf.ERR_UNSUPPORTED
    assert b"overlap" in L.bf_last_error()
    assert L.bf_ggml_mul_mat(None, ctypes.byref(s1), ctypes.byref(d), None) == bf.ERR_INVALID
    s0, s1, d = _ggml_case()
    st = L.bf_ggml_mul_mat_ws(ctypes.byref(s0), ctypes.byref(s1), ctypes.byref(d), None, 4096, None)
    assert st == bf.ERR_INVALID and b"NULL" in L.bf_last_error()
