"""The C ABI of libqk.so without a GPU: the library loads, exports every
function include/qk.h declares (and the ctypes mirror binds exactly those),
the pure host helpers return the reference's sizes (inferencer.cu:252-259),
and argument validation answers with status codes before any device call,
mirroring FastGPU::matvec's checks (inferencer.cu:1157-1158)."""
import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qk.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return set(re.findall(r"\b(qk_[a-z0-9_]+)\s*\(", text))


def test_header_declares_the_entry_points():
    names = declared_functions()
    for must in ("qk_gemv_f32", "qk_gemv_multi_f32", "qk_gemv_batched_f32", "qk_gemv_multi_batched_f32",
                 "qk_dequant_rows", "qk_embedding", "qk_quantize_x32", "qk_gemv_i8", "qk_status_string",
                 "qk_llama_forward"):
        assert must in names


def test_library_exports_every_declared_symbol(qk):
    lib = qk.lib()
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_mirror_binds_exactly_the_header(qk):
    assert set(qk.SIGNATURES) == declared_functions()


def test_status_strings(qk):
    lib = qk.lib()
    seen = set()
    for code in range(7):
        s = lib.qk_status_string(code).decode()
        assert s and s not in seen
        seen.add(s)
    assert lib.qk_status_string(0).decode().lower().startswith("ok")
    assert lib.qk_status_string(99)


@pytest.mark.parametrize("qtype,cols,rows,want", [
    (12, 2048, 2048, 2_359_296),
    (14, 2048, 128256, 215_470_080),
    (12, 3072, 8192, 14_155_776),
    (14, 8192, 3072, 20_643_840),
])
def test_tensor_bytes_match_reference_size_rule(qk, qtype, cols, rows, want):
    lib = qk.lib()
    assert lib.qk_block_bytes(qtype) == {12: 144, 14: 210}[qtype]
    assert lib.qk_tensor_bytes(qtype, cols, rows) == want
    assert qk.tensor_bytes(qtype, cols, rows) == want


@pytest.mark.parametrize("cols,rows", [(256, 1), (2048, 128256), (3072, 5), (8192, 3)])
def test_split_tensor_bytes_pad_rows_to_16(qk, cols, rows):
    """The split Q6_K layout keeps 210 bytes per block and rounds each row
    up to a 16-byte multiple."""
    lib = qk.lib()
    want = (cols // 256 * 210 + 15) // 16 * 16 * rows
    assert lib.qk_block_bytes(114) == 210
    assert lib.qk_tensor_bytes(114, cols, rows) == want
    assert qk.tensor_bytes(114, cols, rows) == want


def test_block_bytes_rejects_other_types(qk):
    lib = qk.lib()
    assert lib.qk_block_bytes(0) == 0 and lib.qk_block_bytes(13) == 0


def _gemv(qk, qtype, w, x, y, cols, rows):
    return qk.lib().qk_gemv_f32(qtype, w, x, y, cols, rows, None)


def test_gemv_validation_without_device(qk):
    lib = qk.lib()
    # Addresses are never dereferenced: every call below fails validation.
    good, x, y = 0x10000, 0x20000, 0x30000
    assert _gemv(qk, 0, good, x, y, 2048, 16) == qk.QK_ERR_TYPE
    assert b"type" in lib.qk_last_error()
    assert _gemv(qk, 13, good, x, y, 2048, 16) == qk.QK_ERR_TYPE
    assert _gemv(qk, 12, good, x, y, 300, 16) == qk.QK_ERR_SHAPE
    assert _gemv(qk, 12, good, x, y, 2048, 0) == qk.QK_ERR_SHAPE
    assert _gemv(qk, 12, None, x, y, 2048, 16) == qk.QK_ERR_INVALID_ARG
    assert _gemv(qk, 12, good + 8, x, y, 2048, 16) == qk.QK_ERR_ALIGN
    assert _gemv(qk, 14, good, None, y, 2048, 16) == qk.QK_ERR_INVALID_ARG
    assert _gemv(qk, 14, good, x + 4, y, 2048, 16) == qk.QK_ERR_ALIGN
    assert b"qk_gemv_f32" in lib.qk_last_error()


def test_multi_validation_without_device(qk):
    lib = qk.lib()
    mats = (qk.qk_matrix * 9)()
    for m in mats:
        m.type, m.rows, m.w, m.y = 12, 16, 0x10000, 0x30000
    assert lib.qk_gemv_multi_f32(mats, 0, 0x20000, 2048, None) == qk.QK_ERR_INVALID_ARG
    assert lib.qk_gemv_multi_f32(mats, 9, 0x20000, 2048, None) == qk.QK_ERR_INVALID_ARG
    mats[1].type = 13
    assert lib.qk_gemv_multi_f32(mats, 2, 0x20000, 2048, None) == qk.QK_ERR_TYPE
    mats[1].type, mats[1].w = 14, 0x10002
    assert lib.qk_gemv_multi_f32(mats, 2, 0x20000, 2048, None) == qk.QK_ERR_ALIGN


def test_dequant_and_embedding_validation(qk):
    lib = qk.lib()
    assert lib.qk_dequant_rows(12, 0x10000, None, 2048, 0, 4, None) == qk.QK_ERR_INVALID_ARG
    assert lib.qk_dequant_rows(12, 0x10000, 0x20000, 2048, -1, 4, None) == qk.QK_ERR_INVALID_ARG
    assert lib.qk_dequant_rows(12, 0x10000, 0x20000, 2048, 0, 0, None) == qk.QK_OK   # empty range: no launch
    assert lib.qk_dequant_rows(0, 0x10000, 0x20000, 2048, 0, 4, None) == qk.QK_ERR_TYPE


def test_int8_validation(qk):
    lib = qk.lib()
    w, xq, xs, y = 0x10000, 0x20000, 0x30000, 0x40000
    assert lib.qk_gemv_i8(12, w, xq, 2048, xs, 64, y, 16, 2048, 16, 0, None) == qk.QK_OK   # no tokens
    assert lib.qk_gemv_i8(12, w, xq, 1024, xs, 64, y, 16, 2048, 16, 1, None) == qk.QK_ERR_INVALID_ARG
    assert lib.qk_gemv_i8(12, w, xq + 1, 2048, xs, 64, y, 16, 2048, 16, 1, None) == qk.QK_ERR_ALIGN
    assert lib.qk_gemv_i8(12, w, None, 2048, xs, 64, y, 16, 2048, 16, 1, None) == qk.QK_ERR_INVALID_ARG
    mats = (qk.qk_matrix * 2)()
    for m in mats:
        m.type, m.rows, m.w, m.y = 12, 16, w, y
    assert lib.qk_gemv_multi_i8(mats, 0, xq, xs, 2048, None) == qk.QK_ERR_INVALID_ARG
    assert lib.qk_gemv_multi_i8(mats, 2, None, xs, 2048, None) == qk.QK_ERR_INVALID_ARG
    assert lib.qk_gemv_multi_i8(mats, 2, xq + 8, xs, 2048, None) == qk.QK_ERR_ALIGN
    mats[1].type = 13
    assert lib.qk_gemv_multi_i8(mats, 2, xq, xs, 2048, None) == qk.QK_ERR_TYPE
    assert lib.qk_llama_set_int8(None, 1, 1) == qk.QK_ERR_INVALID_ARG


def test_rmsnorm_quantize_validation(qk):
    lib = qk.lib()
    x, w, o, xq, xs = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    f = lib.qk_rmsnorm_quantize_x32
    assert f(x, 2048, w, o, 2048, xq, 2048, xs, 64, 2048, 0, 1e-5, None) == qk.QK_OK        # no tokens
    assert f(None, 2048, w, o, 2048, xq, 2048, xs, 64, 2048, 1, 1e-5, None) == qk.QK_ERR_INVALID_ARG
    assert f(x, 2048, w, o, 2048, xq, 2048, xs, 64, 2040, 1, 1e-5, None) == qk.QK_ERR_SHAPE  # cols % 32
    assert f(x, 2048, w, o, 2048, xq, 2048, xs, 63, 2048, 1, 1e-5, None) == qk.QK_ERR_INVALID_ARG
    assert f(x + 4, 2048, w, o, 2048, xq, 2048, xs, 64, 2048, 1, 1e-5, None) == qk.QK_ERR_ALIGN
    assert f(x, 2050, w, o, 2048, xq, 2048, xs, 64, 2048, 1, 1e-5, None) == qk.QK_ERR_ALIGN
    assert f(x, 2048, w, o, 2048, xq + 2, 2048, xs, 64, 2048, 1, 1e-5, None) == qk.QK_ERR_ALIGN
    assert f(x, 2048, w, o, 2048, xq, 2050, xs, 64, 2048, 1, 1e-5, None) == qk.QK_ERR_ALIGN


def test_batched_workspace_sizes(qk):
    lib = qk.lib()
    assert lib.qk_gemv_batched_workspace_bytes(0, 64, 32) == 0
    assert lib.qk_gemv_batched_workspace_bytes(2048, 64, 0) == 0
    assert lib.qk_gemv_batched_workspace_bytes(2048, 64, 4) == 0         # below the matrix-core path
    # Packed records: 33,920 B per (32-token tile, 256 columns).
    big = lib.qk_gemv_batched_workspace_bytes(3072, 16384, 256)          # fills the chip unsplit
    assert big == 8 * 12 * 33920
    a = lib.qk_gemv_batched_workspace_bytes(8192, 3072, 32)              # split: records + partials
    assert a > 32 * 33920 and a % 256 == 0 and a == lib.qk_gemv_batched_workspace_bytes(8192, 3072, 17)
    assert lib.qk_argmax_workspace_bytes(128256) > 0


def test_ffn_validation_and_workspace(qk):
    lib = qk.lib()
    ws_bytes = lib.qk_ffn_batched_workspace_bytes
    n32 = ws_bytes(3072, 8192, 32)
    assert n32 > 0 and n32 % 256 == 0
    assert ws_bytes(3072, 8192, 0) == 0 and ws_bytes(3000, 8192, 32) == 0 and ws_bytes(3072, 8000, 32) == 0
    for k in (1, 5, 7, 8, 31, 32):                    # a size for n tokens serves every smaller call
        assert 0 < ws_bytes(3072, 8192, k) <= n32
    assert ws_bytes(3072, 8192, 5) == 2 * 5 * 8192 * 4   # below 8 tokens: gate and up outputs
    g, u, d, x, y, ws = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000

    def f(gt=12, gp=g, dt=14, xp=x, ldy=3072, n=32, wsp=ws, wsn=n32):
        return lib.qk_ffn_batched_f32(gt, gp, 12, u, dt, d, xp, 3072, y, ldy, 3072, 8192, n, 0, wsp, wsn, None)
    assert f(n=0, wsp=None, wsn=0) == qk.QK_OK          # no tokens: nothing launched
    assert f(gt=13) == qk.QK_ERR_TYPE
    assert f(dt=0) == qk.QK_ERR_TYPE
    assert f(gp=None) == qk.QK_ERR_INVALID_ARG
    assert f(gp=g + 8) == qk.QK_ERR_ALIGN
    assert f(xp=x + 4) == qk.QK_ERR_ALIGN
    assert f(ldy=3000) == qk.QK_ERR_INVALID_ARG
    assert f(wsn=n32 - 256) == qk.QK_ERR_INVALID_ARG
    assert b"qk_ffn_batched_workspace_bytes" in lib.qk_last_error()
    assert f(wsp=ws + 16) == qk.QK_ERR_ALIGN


def test_python_mirror_rejects_wrong_shapes(qk):
    t = qk.Tensor((2048, 16), qk.Q4_K, None)
    assert t.cols() == 2048 and t.rows() == 16
    with pytest.raises(qk.QKError):
        qk.matvec(t, None, None, 4096, 16)
