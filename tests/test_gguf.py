"""The GGUF reader (bf_gguf_*): files written here by an independent writer
that follows the public GGUF specification (version 3, little-endian), read
back through the C ABI.  No GPU: only bf_gguf_upload touches the device and it
is exercised by the GPU parity tests."""
import ctypes
import struct

import numpy as np
import pytest

import busfill as bf
import oracle as O

# metadata value types of the specification
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
          U64: "<Q", I64: "<q", F64: "<d"}
# ggml tensor types used here: (code, block size, bytes per block)
GGML = {"f32": (0, 1, 4), "f16": (1, 1, 2), "q4_0": (2, 32, 18), "q4_k": (12, 256, 144)}


def gstr(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def gvalue(t, v) -> bytes:
    if t == STRING:
        return gstr(v)
    if t == ARRAY:
        et, items = v
        body = b"".join(gvalue(et, x) for x in items)
        return struct.pack("<IQ", et, len(items)) + body
    return struct.pack(SCALAR[t], v)


def write_gguf(path, kv, tensors, alignment=None, version=3):
    """kv: [(key, type, value)]; tensors: [(name, ggml_code, dims, data bytes)]."""
    kv = list(kv)
    align = 32 if alignment is None else alignment
    if alignment is not None:
        kv.append((b"general.alignment", U32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kv))
    head += b"".join(gstr(k) + struct.pack("<I", t) + gvalue(t, v) for k, t, v in kv)
    infos, data, offsets = b"", b"", []
    for name, code, dims, payload in tensors:
        data += b"\0" * (-len(data) % align)
        offsets.append(len(data))
        infos += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", code, offsets[-1])
        data += payload
    blob = head + infos
    blob += b"\0" * (-len(blob) % align)
    data0 = len(blob)
    with open(path, "wb") as f:
        f.write(blob + data)
    return data0, offsets


def sample_tensors():
    wk = O.gen_weights(O.Q4_K, 3, 512, seed=5)
    w0 = O.gen_weights(O.Q4_0, 5, 64, seed=6)
    f32 = np.arange(7, dtype=np.float32) * 0.5
    f16 = np.arange(6, dtype=np.float16)
    return [(b"blk.0.ffn_up.weight", GGML["q4_k"][0], [512, 3], wk.W.tobytes()),
            (b"blk.0.attn_q.weight", GGML["q4_0"][0], [64, 5], w0.W.tobytes()),
            (b"output_norm.weight", GGML["f32"][0], [7], f32.tobytes()),
            (b"token_types", GGML["f16"][0], [3, 2], f16.tobytes())]


SAMPLE_KV = [(b"general.architecture", STRING, b"llama"), (b"general.name", STRING, "café".encode()),
             (b"llama.block_count", U32, 62), (b"llama.context_length", U64, 131072),
             (b"u8", U8, 200), (b"i8", I8, 7), (b"i8neg", I8, -1), (b"u16", U16, 65535), (b"i16", I16, 1234),
             (b"i32neg", I32, -5), (b"i64", I64, 1 << 40), (b"f32", F32, 1.5), (b"f64", F64, -2.25),
             (b"flag", BOOL, True), (b"tokens", ARRAY, (STRING, [b"<s>", b"</s>", b"hello"])),
             (b"ids", ARRAY, (I32, [1, -2, 3])), (b"empty", ARRAY, (U64, []))]


@pytest.fixture
def sample(tmp_path):
    path = tmp_path / "sample.gguf"
    tensors = sample_tensors()
    data0, offsets = write_gguf(path, SAMPLE_KV, tensors, alignment=64)
    return path, tensors, data0, offsets


def test_reads_tensors_and_their_bytes(sample):
    path, tensors, data0, offsets = sample
    with bf.Gguf(path) as g:
        got = g.tensors()
        assert [t.name for t in got] == [t[0] for t in tensors]
        for t, (name, code, dims, payload), off in zip(got, tensors, offsets):
            assert t.ggml_type == code
            assert t.n_dims == len(dims)
            assert list(t.dims) == dims + [1] * (4 - len(dims))
            assert t.offset == data0 + off and t.offset % 64 == 0
            assert t.nbytes == len(payload)
            assert g.data(t) == payload
        assert [t.qtype for t in got] == [bf.Q4_K, bf.Q4_0, -1, -1]
        # find() returns the same record
        f = g.find("blk.0.attn_q.weight")
        assert (f.offset, f.nbytes, f.qtype) == (got[1].offset, got[1].nbytes, bf.Q4_0)
        with pytest.raises(bf.BusfillError):
            g.find("missing")


def test_q4_blocks_come_back_in_the_gemm_layout(sample):
    """A Q4_K tensor read from the file dequantizes (oracle) to the same values
    as the blocks that were written: the reader hands out bf_gemm's layout."""
    path, _, _, _ = sample
    wk = O.gen_weights(O.Q4_K, 3, 512, seed=5)
    with bf.Gguf(path) as g:
        t = g.find("blk.0.ffn_up.weight")
        raw = np.frombuffer(g.data(t), np.uint8).reshape(wk.W.shape)
    back = O.QWeights(O.Q4_K, 3, 512, raw.copy())
    assert (O.dequant_f16(back) == O.dequant_f16(wk)).all()


def test_metadata_values(sample):
    path, _, _, _ = sample
    with bf.Gguf(path) as g:
        assert g.get_str("general.architecture") == b"llama"
        assert g.get_str("general.name") == "café".encode()
        assert g.get_u64("llama.block_count") == 62
        assert g.get_u64("llama.context_length") == 131072
        assert g.get_u64("u8") == 200 and g.get_u64("i8") == 7 and g.get_u64("u16") == 65535
        assert g.get_u64("i16") == 1234 and g.get_u64("i64") == 1 << 40 and g.get_u64("flag") == 1
        assert g.get_u64("general.alignment") == 64
        for key in ("i8neg", "i32neg"):
            with pytest.raises(bf.BusfillError, match="negative"):
                g.get_u64(key)
        for key in ("f32", "tokens", "general.architecture"):
            with pytest.raises(bf.BusfillError):
                g.get_u64(key)
        with pytest.raises(bf.BusfillError):
            g.get_str("llama.block_count")
        with pytest.raises(bf.BusfillError):
            g.get_u64("no.such.key")


def test_default_alignment_and_version_2(tmp_path):
    path = tmp_path / "v2.gguf"
    tensors = sample_tensors()
    data0, offsets = write_gguf(path, SAMPLE_KV[:3], tensors, version=2)
    with bf.Gguf(path) as g:
        got = g.tensors()
        assert all(t.offset % 32 == 0 for t in got)
        assert [t.offset for t in got] == [data0 + o for o in offsets]
        assert g.data(got[2]) == tensors[2][3]


def open_status(path):
    h = ctypes.c_void_p()
    st = bf.lib().bf_gguf_open(str(path).encode(), ctypes.byref(h))
    if st == bf.OK:
        bf.lib().bf_gguf_close(h)
    return st


@pytest.mark.parametrize("mutate,needle", [
    (lambda b: b"GGUX" + b[4:], "magic"),
    (lambda b: b[:4] + struct.pack("<I", 1) + b[8:], "version"),
    (lambda b: b[:8] + struct.pack("<Q", 1 << 60) + b[16:], "implausible"),
])
def test_rejects_malformed_headers(tmp_path, sample, mutate, needle):
    path, _, _, _ = sample
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(mutate(path.read_bytes()))
    assert open_status(bad) == bf.ERR_INVALID
    assert needle in bf.lib().bf_last_error().decode()


def test_every_truncation_is_an_error_not_a_crash(tmp_path, sample):
    path, _, _, _ = sample
    blob = path.read_bytes()
    cut = tmp_path / "cut.gguf"
    for n in list(range(0, 600)) + list(range(600, len(blob), 97)):
        cut.write_bytes(blob[:n])
        assert open_status(cut) == bf.ERR_INVALID, n
    cut.write_bytes(blob)
    assert open_status(cut) == bf.OK


def test_random_corruption_never_crashes(tmp_path, sample):
    """Flipped bytes anywhere in the header and tensor table: open either
    succeeds with in-bounds tensors or reports an error."""
    path, _, data0, _ = sample
    blob = bytearray(path.read_bytes())
    rng = np.random.default_rng(3)
    bad = tmp_path / "flip.gguf"
    for _ in range(300):
        b = bytearray(blob)
        for pos in rng.integers(0, data0, size=3):
            b[pos] ^= int(rng.integers(1, 256))
        bad.write_bytes(bytes(b))
        h = ctypes.c_void_p()
        st = bf.lib().bf_gguf_open(str(bad).encode(), ctypes.byref(h))
        assert st in (bf.OK, bf.ERR_INVALID)
        if st == bf.OK:
            n = bf.lib().bf_gguf_tensor_count(h)
            for i in range(n):
                t = bf.GgufTensor()
                assert bf.lib().bf_gguf_tensor_at(h, i, ctypes.byref(t)) == bf.OK
                assert t.offset + t.nbytes <= len(b)
            bf.lib().bf_gguf_close(h)


def test_rejects_bad_tensor_records(tmp_path):
    w0 = O.gen_weights(O.Q4_0, 2, 64, seed=1)
    ok = [(b"w", GGML["q4_0"][0], [64, 2], w0.W.tobytes())]
    p = tmp_path / "t.gguf"
    # a row that is not whole blocks
    write_gguf(p, [], [(b"w", GGML["q4_0"][0], [48, 2], w0.W.tobytes())])
    assert open_status(p) == bf.ERR_INVALID and "whole blocks" in bf.lib().bf_last_error().decode()
    # more rows than the file holds
    write_gguf(p, [], [(b"w", GGML["q4_0"][0], [64, 1 << 40], w0.W.tobytes())])
    assert open_status(p) == bf.ERR_INVALID
    # an alignment that is not a power of two
    write_gguf(p, [], ok, alignment=48)
    assert open_status(p) == bf.ERR_INVALID and "power of two" in bf.lib().bf_last_error().decode()
    # five dimensions
    write_gguf(p, [], [(b"w", GGML["f32"][0], [1, 1, 1, 1, 1], b"\0" * 4)])
    assert open_status(p) == bf.ERR_INVALID
    write_gguf(p, [], ok)
    assert open_status(p) == bf.OK
