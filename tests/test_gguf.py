"""GGUF v3 reader (qk_gguf_*, the reference's Reader / GGUF structs,
inferencer.cu:130-176, 204-340) on files written by tests/gguf_writer.py:
every metadata value type, tokenizer arrays, the tensor table and the mapped
bytes round-trip; each malformed file is rejected with QK_ERR_FORMAT (never
a crash), including the cases the reference lets through (tensor data past
the end of the file, unaligned offsets, duplicate names).  CPU only: nothing
here touches a device."""
import ctypes
import struct

import numpy as np
import pytest

import gguf_writer as gw


def _open_status(qk, path):
    h = ctypes.c_void_p()
    st = qk.lib().qk_gguf_open(str(path).encode(), ctypes.byref(h))
    if st == qk.QK_OK:
        qk.lib().qk_gguf_close(h)
    return st, qk.lib().qk_last_error().decode()


def _basic(alignment=None):
    w = gw.GGUFWriter(alignment)
    w.add("general.architecture", gw.STRING, "llama")
    w.add("test.u8", gw.U8, 250)
    w.add("test.i8", gw.I8, -7)
    w.add("test.u16", gw.U16, 65000)
    w.add("test.i16", gw.I16, -30000)
    w.add("test.u32", gw.U32, 4000000000)
    w.add("test.i32", gw.I32, -2000000000)
    w.add("test.f32", gw.F32, 1e-5)
    w.add("test.bool", gw.BOOL, 1)
    w.add("test.u64", gw.U64, 2 ** 40 + 3)
    w.add("test.i64", gw.I64, -(2 ** 40))
    w.add("test.f64", gw.F64, 500000.0)
    w.add("test.ints", gw.ARRAY, (gw.I32, [1, 2, 3]))
    w.add("test.nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]), (gw.STRING, ["a", "bc"])]))
    w.add("tokenizer.ggml.tokens", gw.ARRAY, (gw.STRING, ["<s>", "hello", "", "été", "x" * 300]))
    w.add("tokenizer.ggml.merges", gw.ARRAY, (gw.STRING, ["h e", "l l"]))
    rng = np.random.default_rng(5)
    q4 = rng.integers(0, 256, 2 * 144, dtype=np.uint8).tobytes()
    q6 = rng.integers(0, 256, 3 * 210, dtype=np.uint8).tobytes()
    f32 = np.arange(10, dtype=np.float32).tobytes()
    f16 = np.arange(6, dtype=np.float16).tobytes()
    w.add_tensor("a.q4", [256, 2], 12, q4)
    w.add_tensor("b.q6", [256, 3], 14, q6)
    w.add_tensor("c.f32", [10], 0, f32)
    w.add_tensor("d.f16", [2, 3], 1, f16)
    w.add_tensor("e.4d", [256, 1, 1, 1], 12, q4[:144])
    return w, {"a.q4": q4, "b.q6": q6, "c.f32": f32, "d.f16": f16, "e.4d": q4[:144]}


@pytest.mark.parametrize("alignment", [None, 64, 1])
def test_round_trip(qk, tmp_path, alignment):
    w, data = _basic(alignment)
    path = tmp_path / "m.gguf"
    w.write(path)
    with qk.GGUF(path) as g:
        assert g.string("general.architecture") == "llama"
        expect = {"test.u8": 250, "test.i8": -7, "test.u16": 65000, "test.i16": -30000, "test.u32": 4000000000,
                  "test.i32": -2000000000, "test.bool": 1, "test.u64": 2 ** 40 + 3, "test.i64": -(2 ** 40),
                  "test.f64": 500000.0}
        for k, v in expect.items():
            assert g.param(k) == v, k
        assert g.param("test.f32") == float(np.float32(1e-5))
        with pytest.raises(qk.QKError):
            g.param("test.ints")                  # arrays are skipped
        with pytest.raises(qk.QKError):
            g.param("missing.key")
        assert g.tokens(0) == [b"<s>", b"hello", b"", "été".encode(), b"x" * 300]
        assert g.tokens(1) == [b"h e", b"l l"]
        tensors = g.tensors()
        assert [t.name.decode() for t in tensors] == ["a.q4", "b.q6", "c.f32", "d.f16", "e.4d"]
        a = 32 if alignment is None else alignment
        host, nbytes, align = g.data()
        assert align == a
        for t in tensors:
            name = t.name.decode()
            assert t.offset % a == 0
            assert t.bytes == len(data[name])
            assert t.host == host + t.offset
            assert g.host_bytes(name).tobytes() == data[name]
            assert t.device is None
        t = g.tensor("d.f16")
        assert (t.type, t.n_dims, list(t.dims)) == (1, 2, [2, 3, 1, 1])
        t = g.tensor("b.q6")
        assert (t.type, t.n_dims, list(t.dims)) == (14, 2, [256, 3, 1, 1])
        with pytest.raises(qk.QKError):
            g.tensor("nope")


def test_data_start_is_aligned(qk, tmp_path):
    for alignment in (32, 64, 256, 4096):
        w, _ = _basic(alignment)
        raw = w.write(tmp_path / "m.gguf")
        with qk.GGUF(tmp_path / "m.gguf") as g:
            host, nbytes, _ = g.data()
            t0 = g.tensors()[0]
            assert t0.host == host
            start = len(raw) - nbytes
            assert start % alignment == 0


def _malformed(tmp_path, raw: bytes):
    p = tmp_path / "bad.gguf"
    p.write_bytes(raw)
    return p


def test_missing_file_is_io_error(qk, tmp_path):
    st, msg = _open_status(qk, tmp_path / "absent.gguf")
    assert st == qk.QK_ERR_IO and "cannot open" in msg


@pytest.mark.parametrize("case,needle", [
    ("magic", "no GGUF header"),
    ("version", "takes version 3"),
    ("ndims0", "dimensions"),
    ("ndims5", "dimensions"),
    ("dim0", "dimensions"),
    ("type", "storage type"),
    ("quant_shape", "not a multiple of 256"),
    ("past_end", "outside the file"),
    ("offset_unaligned", "not aligned"),
    ("alignment0", "alignment"),
    ("alignment3", "alignment"),
    ("string_len", "1e8-byte limit"),
    ("array_len", "1e7-entry limit"),
    ("meta_type", "metadata type"),
    ("tokens_not_strings", "non-string entries"),
    ("duplicate", "duplicate"),
    ("no_data", "file size"),
    ("counts", "entry counts"),
])
def test_rejects_malformed(qk, tmp_path, case, needle):
    w, _ = _basic()
    kw = {}
    if case == "magic":
        w.magic = b"GGUG"
    elif case == "version":
        w.version = 2
    elif case == "ndims0":
        w.add_tensor("z", [], 0, b"")
    elif case == "ndims5":
        w.add_tensor("z", [1, 1, 1, 1, 4], 0, bytes(16))
    elif case == "dim0":
        w.add_tensor("z", [256, 0], 12, b"")
    elif case == "type":
        w.add_tensor("z", [32], 2, bytes(18))           # Q4_0: not a storage type of the reference
    elif case == "quant_shape":
        w.add_tensor("z", [128, 3], 12, bytes(144))
    elif case == "past_end":
        # offset < data size (the reference's only test) but the bytes run past the end.
        w.add_tensor("z", [256, 1], 14, bytes(210), offset=2048)
        raw = w.to_bytes()
        raw = raw[: len(raw) - 100]
        st, msg = _open_status(qk, _malformed(tmp_path, raw))
        assert st == qk.QK_ERR_FORMAT and needle in msg, msg
        return
    elif case == "offset_unaligned":
        w.add_tensor("z", [4], 0, bytes(16), offset=4096 + 8)
    elif case == "alignment0":
        w = _basic(0)[0]
    elif case == "alignment3":
        w = _basic(3)[0]
    elif case == "string_len":
        w.add_raw_meta(struct.pack("<Q", 100000001) + b"k")
    elif case == "array_len":
        w.add_raw_meta(gw.gguf_string("k") + struct.pack("<IIQ", gw.ARRAY, gw.U8, 10000001))
    elif case == "meta_type":
        w.add_raw_meta(gw.gguf_string("k") + struct.pack("<I", 13) + bytes(8))
    elif case == "tokens_not_strings":
        w.add("tokenizer.ggml.tokens", gw.ARRAY, (gw.I32, [1, 2]))
    elif case == "duplicate":
        w.add_tensor("a.q4", [256, 1], 12, bytes(144))
    elif case == "no_data":
        w.tensors = []
    elif case == "counts":
        kw = dict(n_tensors=2 ** 60)
    raw = w.to_bytes(**kw)
    st, msg = _open_status(qk, _malformed(tmp_path, raw))
    assert st == qk.QK_ERR_FORMAT, (st, msg)
    assert needle in msg, msg


def test_every_truncation_is_rejected(qk, tmp_path):
    """Every prefix of a valid file that cuts into the header or the tensor
    data is a format error."""
    w, _ = _basic()
    raw = w.to_bytes()
    with qk.GGUF(_malformed(tmp_path, raw)) as g:
        _, nbytes, _ = g.data()
        last_end = max(t.offset + t.bytes for t in g.tensors())
    data_start = len(raw) - nbytes
    for n in list(range(0, data_start + 1, 7)) + [data_start + last_end - 1]:
        st, msg = _open_status(qk, _malformed(tmp_path, raw[:n]))
        assert st == qk.QK_ERR_FORMAT, (n, st, msg)


def test_random_corruption_never_crashes(qk, tmp_path):
    """Seeded byte flips anywhere in the header: open either succeeds or
    reports a format error, and a successful open yields a consistent table."""
    w, _ = _basic()
    raw = bytearray(w.to_bytes())
    with qk.GGUF(_malformed(tmp_path, bytes(raw))) as g:
        _, nbytes, _ = g.data()
    header = len(raw) - nbytes
    rng = np.random.default_rng(17)
    outcomes = {qk.QK_OK: 0, qk.QK_ERR_FORMAT: 0}
    for _ in range(400):
        b = bytearray(raw)
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(0, header))] = int(rng.integers(0, 256))
        p = _malformed(tmp_path, bytes(b))
        st, _ = _open_status(qk, p)
        assert st in outcomes, st
        outcomes[st] += 1
        if st == qk.QK_OK:
            with qk.GGUF(p) as g:
                _, nb, _ = g.data()
                for t in g.tensors():
                    assert t.offset + t.bytes <= nb
    assert outcomes[qk.QK_ERR_FORMAT] > 0


def test_llama_tensors_by_name(qk, tmp_path, workloads):
    """A Llama model written under the reference's tensor names: every
    lookup qk_gguf_llama makes is present with its type and dims; without an
    upload qk_gguf_llama refuses (no device pointers yet)."""
    cfg = dict(dim=256, layers=2, heads=4, kv_heads=2, hidden=512, vocab=300, context=32, eps=1e-5,
               rope_theta=10000.0)
    W = workloads.llama_weights(cfg, 3)
    w = gw.llama_writer(cfg, W, workloads.tensor_shape, tokens=[f"t{i}" for i in range(cfg["vocab"])])
    path = tmp_path / "llama.gguf"
    w.write(path)
    with qk.GGUF(path) as g:
        assert g.param("llama.block_count") == 2
        assert len(g.tokens(0)) == cfg["vocab"]
        assert g.tensor("token_embd.weight").type == 14
        assert list(g.tensor("blk.1.ffn_down.weight").dims[:2]) == [512, 256]
        assert g.host_bytes("blk.0.attn_v.weight").tobytes() == W["layers"][0]["v"].tobytes()
        with pytest.raises(qk.QKError) as e:
            g.llama(32)
        assert "upload" in str(e.value)
