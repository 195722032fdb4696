"""MI355X (gfx950) Q4_K / Q6_K dequant-GEMV: Python host mirror of the C ABI.

libqk.so (built from csrc/ by the Makefile) exports the C ABI declared in
include/qk.h.  This module binds it with ctypes and mirrors the reference's
host-side interface for the path (inferencer.cu:178-186 Tensor,
1101-1180 FastGPU, 1265-1278 batch_matvec): the same names, argument meaning
and error behaviour -- a failing call raises QKError("where: message") like
cuda_check (inferencer.cu:126-128).

Device buffers are passed as raw pointers; torch tensors (or anything with
data_ptr()) are accepted for convenience, torch being only the allocator and
stream provider.  There is no CPU fallback: if libqk.so is missing, loading
raises ImportError.
"""
from __future__ import annotations

import ctypes
import pathlib
from dataclasses import dataclass
from typing import Sequence

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "libqk.so"

F32, F16, Q4_K, Q6_K = 0, 1, 12, 14
Q6_K_SPLIT = 114   # Q6_K in the split row layout of qk_q6k_split (16-byte aligned fields)
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q6_K_SPLIT: 210}
QUANT_TYPES = (Q4_K, Q6_K, Q6_K_SPLIT)
STORAGE_NAMES = {F32: "FP32", F16: "FP16", Q4_K: "Q4_K", Q6_K: "Q6_K", Q6_K_SPLIT: "Q6_K (split)"}
MAX_FUSED = 8

QK_OK = 0
QK_ERR_INVALID_ARG = 1
QK_ERR_SHAPE = 2
QK_ERR_TYPE = 3
QK_ERR_ALIGN = 4
QK_ERR_DEVICE = 5
QK_ERR_LIMIT = 6
QK_ERR_FORMAT = 7
QK_ERR_IO = 8


class QKError(RuntimeError):
    """A non-zero qk status; .status holds the code."""

    def __init__(self, where: str, status: int, detail: str):
        super().__init__(f"{where}: {detail}")
        self.status = status


class qk_matrix(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int),
                ("w", ctypes.c_void_p), ("y", ctypes.c_void_p)]


class qk_batch_token(ctypes.Structure):
    """One token of a ragged decode batch (include/qk.h)."""
    _fields_ = [("pos", ctypes.c_int32), ("seq", ctypes.c_int32), ("kv_row", ctypes.c_int64)]


class qk_llama_config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "layers", "heads", "kv_heads", "hidden", "vocab", "context")] + \
               [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class qk_llama_layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("q_type", "k_type", "v_type", "o_type", "gate_type", "up_type",
                                             "down_type")] + \
               [(n, ctypes.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "ffn_norm")]


class qk_llama_weights(ctypes.Structure):
    _fields_ = [("embd_type", ctypes.c_int), ("token_embd", ctypes.c_void_p), ("output_type", ctypes.c_int),
                ("output", ctypes.c_void_p), ("output_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(qk_llama_layer))]


class qk_llama_memory(ctypes.Structure):
    _fields_ = [("weight_copies", ctypes.c_uint64), ("kv_cache", ctypes.c_uint64), ("buffers", ctypes.c_uint64)]


class qk_gguf_tensor(ctypes.Structure):
    """One tensor-table entry of a GGUF file (include/qk.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("dims", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64),
                ("host", ctypes.c_void_p), ("device", ctypes.c_void_p)]


_i, _vp, _f = ctypes.c_int, ctypes.c_void_p, ctypes.c_float
# name -> (restype, argtypes), exactly the declarations of include/qk.h.
SIGNATURES = {
    "qk_status_string": (ctypes.c_char_p, [_i]),
    "qk_last_error": (ctypes.c_char_p, []),
    "qk_block_bytes": (_i, [_i]),
    "qk_tensor_bytes": (ctypes.c_int64, [_i, ctypes.c_int64, ctypes.c_int64]),
    "qk_gemv_f32": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp]),
    "qk_gemv_multi_f32": (_i, [ctypes.POINTER(qk_matrix), _i, _vp, _i, _vp]),
    "qk_gemv_batched_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i]),
    "qk_gemv_batched_f32": (_i, [_i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp, ctypes.c_size_t, _vp]),
    "qk_gemv_multi_batched_f32": (_i, [ctypes.POINTER(qk_matrix), _i, _vp, _i, _i, _i, _vp, ctypes.c_size_t, _vp]),
    "qk_dequant_rows": (_i, [_i, _vp, _vp, _i, _i, _i, _vp]),
    "qk_embedding": (_i, [_i, _vp, _vp, _i, _vp, _i, _i, _vp]),
    "qk_q6k_split": (_i, [_vp, _vp, _i, _i, _vp]),
    "qk_gemv_argmax_workspace_bytes": (ctypes.c_size_t, []),
    "qk_gemv_argmax_f32": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp]),
    "qk_gemv_argmax_f32_noalloc": (_i, [_i, _vp, _vp, _vp, _i, _i, _vp, _vp]),
    "qk_quantize_x32": (_i, [_vp, _i, _vp, _i, _vp, _i, _i, _i, _vp]),
    "qk_gemv_multi_i8": (_i, [ctypes.POINTER(qk_matrix), _i, _vp, _vp, _i, _vp]),
    "qk_llama_set_int8": (_i, [_vp, _i, _i]),
    "qk_rmsnorm_quantize_x32": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, ctypes.c_float, _vp]),
    "qk_gemv_i8": (_i, [_i, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "qk_gemv_batched_i8": (_i, [_i, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _vp, ctypes.c_size_t, _vp]),
    "qk_gemv_batched_i8_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i]),
    "qk_gemv_multi_batched_i8": (_i, [ctypes.POINTER(qk_matrix), _i, _vp, _i, _vp, _i, _i, _i, _vp, ctypes.c_size_t,
                                      _vp]),
    "qk_ffn_batched_i8_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i]),
    "qk_ffn_batched_i8": (_i, [_i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp,
                               ctypes.c_size_t, _vp]),
    "qk_rmsnorm_f32": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "qk_rope_kv_write": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "qk_attention_f32": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "qk_add_f32": (_i, [_vp, _vp, _i, _vp]),
    "qk_silu_mul_f32": (_i, [_vp, _vp, _i, _vp]),
    "qk_argmax_workspace_bytes": (ctypes.c_size_t, [_i]),
    "qk_argmax_f32": (_i, [_vp, _i, _vp, _vp, _vp]),
    "qk_llama_create": (_i, [ctypes.POINTER(qk_llama_config), ctypes.POINTER(qk_llama_weights), _vp,
                             ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_destroy": (_i, [_vp]),
    "qk_llama_kv_cache": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_logits": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_residual": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_matrix_calls": (_i, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
    "qk_llama_forward": (_i, [_vp, _i, _i, _i, ctypes.POINTER(ctypes.c_int)]),
    "qk_rope_kv_write_batched": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, ctypes.c_int64, _vp, _i, _i, _i, _i, _i,
                                      _vp]),
    "qk_ffn_batched_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i]),
    "qk_ffn_batched_f32": (_i, [_i, _vp, _i, _vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, ctypes.c_size_t,
                                _vp]),
    "qk_attention_batched_f32": (_i, [_vp, _vp, _vp, _vp, _i, ctypes.c_int64, _vp, _i, _i, _i, _i, _i, _vp]),
    "qk_attention_split_workspace_bytes": (ctypes.c_size_t, [_i, _i, _i, _i, _i, _i]),
    "qk_attention_split_f32": (_i, [_vp, _vp, _vp, _vp, _i, ctypes.c_int64, _vp, _i, _i, _i, _i, _i, _i, _vp,
                                    ctypes.c_size_t, _vp]),
    "qk_argmax_rows_workspace_bytes": (ctypes.c_size_t, [_i, _i]),
    "qk_argmax_rows_f32": (_i, [_vp, _i, ctypes.c_int64, _i, _vp, _vp, _vp]),
    "qk_llama_batch_create": (_i, [ctypes.POINTER(qk_llama_config), ctypes.POINTER(qk_llama_weights), _i,
                                   ctypes.c_int64, _vp, ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_batch_destroy": (_i, [_vp]),
    "qk_llama_memory_bytes": (_i, [_vp, ctypes.POINTER(qk_llama_memory)]),
    "qk_llama_batch_memory_bytes": (_i, [_vp, ctypes.POINTER(qk_llama_memory)]),
    "qk_llama_batch_kv_cache": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_batch_logits": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_batch_residual": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p)]),
    "qk_llama_batch_matrix_calls": (_i, [_vp, ctypes.POINTER(ctypes.c_uint64)]),
    "qk_llama_batch_set_int8": (_i, [_vp, _i, _i]),
    "qk_llama_set_trace": (_i, [_vp, _vp, _vp]),
    "qk_llama_batch_set_trace": (_i, [_vp, _vp, _vp]),
    "qk_llama_batch_forward": (_i, [_vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(qk_batch_token), _i, _i,
                                    ctypes.POINTER(ctypes.c_int32)]),
    "qk_llama_batch_forward_rows": (_i, [_vp, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(qk_batch_token), _i,
                                         ctypes.POINTER(ctypes.c_int32), _i, ctypes.POINTER(ctypes.c_int32)]),
    "qk_gguf_open": (_i, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)]),
    "qk_gguf_close": (_i, [_vp]),
    "qk_gguf_param": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "qk_gguf_string": (ctypes.c_char_p, [_vp, ctypes.c_char_p]),
    "qk_gguf_tensor_count": (ctypes.c_int64, [_vp]),
    "qk_gguf_tensor_at": (_i, [_vp, ctypes.c_int64, ctypes.POINTER(qk_gguf_tensor)]),
    "qk_gguf_find_tensor": (_i, [_vp, ctypes.c_char_p, ctypes.POINTER(qk_gguf_tensor)]),
    "qk_gguf_token_count": (ctypes.c_int64, [_vp, _i]),
    "qk_gguf_token": (_vp, [_vp, _i, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64)]),
    "qk_gguf_data": (_i, [_vp, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_uint64),
                          ctypes.POINTER(ctypes.c_uint64)]),
    "qk_gguf_upload": (_i, [_vp, _vp]),
    "qk_gguf_llama": (_i, [_vp, _i, ctypes.POINTER(qk_llama_config), ctypes.POINTER(qk_llama_weights),
                           ctypes.POINTER(qk_llama_layer), _i]),
}

_LIB = None


def lib() -> ctypes.CDLL:
    """The loaded libqk.so with every signature bound (raises if unbuilt)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(status: int, where: str) -> None:
    """Raise QKError for a non-zero status (the cuda_check convention)."""
    if status != QK_OK:
        detail = lib().qk_last_error().decode() or lib().qk_status_string(status).decode()
        raise QKError(where, status, detail)


def ptr(a) -> int | None:
    """Device address of a tensor-like (data_ptr()), an int, or None."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    return a.data_ptr()


def stream_handle(stream) -> int | None:
    """hipStream_t of a torch stream / raw handle; None = null stream."""
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def tensor_bytes(qtype: int, cols: int, rows: int) -> int:
    """Bytes of a quantized tensor: the size rule of inferencer.cu:252-259."""
    if qtype not in BLOCK_BYTES or cols % 256 or cols <= 0 or rows < 0:
        raise QKError("tensor_bytes", QK_ERR_SHAPE, "Invalid quantized tensor shape")
    row = cols // 256 * BLOCK_BYTES[qtype]
    if qtype == Q6_K_SPLIT:
        row = (row + 15) // 16 * 16   # split rows start 16-byte aligned
    return row * rows


@dataclass
class Tensor:
    """A quantized weight view: Tensor{dims, type, gpu} of inferencer.cu:178-186.

    dims[0] = cols (contiguous), dims[1] = rows; data is a device buffer."""
    dims: Sequence[int]
    type: int
    data: object

    def cols(self) -> int:
        return int(self.dims[0])

    def rows(self) -> int:
        return int(self.dims[1])

    @property
    def gpu(self) -> int:
        return ptr(self.data)


def matvec(t: Tensor, inp, out, expected_cols: int, expected_rows: int, stream=None) -> None:
    """FastGPU::matvec (inferencer.cu:1156-1171), FP32 mode: out = W inp."""
    if t.cols() != expected_cols or t.rows() != expected_rows or t.type not in QUANT_TYPES:
        raise QKError("matvec", QK_ERR_SHAPE, "Unexpected quantized matrix shape")
    check(lib().qk_gemv_f32(t.type, t.gpu, ptr(inp), ptr(out), expected_cols, expected_rows,
                            stream_handle(stream)), "quantized matrix launch")


def matvec_argmax(t: Tensor, inp, out, token_out, workspace, stream=None) -> None:
    """The LM head with its greedy pick (inferencer.cu:1414, 1523-1526): out = W inp and token_out[0] = the
    lowest index among the maxima of out; workspace of qk_gemv_argmax_workspace_bytes() bytes."""
    if t.type not in QUANT_TYPES:
        raise QKError("matvec_argmax", QK_ERR_SHAPE, "Unexpected quantized matrix shape")
    check(lib().qk_gemv_argmax_f32(t.type, t.gpu, ptr(inp), ptr(out), t.cols(), t.rows(), ptr(token_out),
                                   ptr(workspace), stream_handle(stream)), "LM head with greedy pick")


def multi_matvec_i8(pairs, xq, xscale, cols: int, stream=None) -> None:
    """qkv_cuda / gate_up_cuda with dp4a (inferencer.cu:753-804): one fused INT8 launch over (Tensor, out) pairs."""
    for t, _ in pairs:
        if t.cols() != cols:
            raise QKError("multi_matvec_i8", QK_ERR_SHAPE, "Unexpected quantized matrix shape")
    arr = _matrices(pairs)
    check(lib().qk_gemv_multi_i8(arr, len(pairs), ptr(xq), ptr(xscale), cols, stream_handle(stream)),
          "fused INT8 matrix launch")


def _matrices(pairs) -> ctypes.Array:
    arr = (qk_matrix * len(pairs))()
    for i, (t, out) in enumerate(pairs):
        arr[i].type, arr[i].rows, arr[i].w, arr[i].y = t.type, t.rows(), t.gpu, ptr(out)
    return arr


def multi_matvec(pairs, inp, cols: int, stream=None) -> None:
    """One fused launch of out_m = W_m inp over (Tensor, out) pairs sharing inp."""
    for t, _ in pairs:
        if t.cols() != cols:
            raise QKError("multi_matvec", QK_ERR_SHAPE, "Unexpected quantized matrix shape")
    arr = _matrices(pairs)
    check(lib().qk_gemv_multi_f32(arr, len(pairs), ptr(inp), cols, stream_handle(stream)),
          "fused quantized matrix launch")


def qkv(wq: Tensor, wk: Tensor, wv: Tensor, x, q, k, v, dim: int, kv_dim: int, stream=None) -> None:
    """qkv_cuda (inferencer.cu:753-784), FP32 mode: Q4_K q/k, Q4_K or Q6_K v."""
    if (wq.rows(), wk.rows(), wv.rows()) != (dim, kv_dim, kv_dim) or wq.type != Q4_K or wk.type != Q4_K \
            or wv.type not in QUANT_TYPES:
        raise QKError("qkv", QK_ERR_SHAPE, "Unexpected QKV quantization")
    multi_matvec([(wq, q), (wk, k), (wv, v)], x, dim, stream)


def gate_up(wgate: Tensor, wup: Tensor, x, gate, up, dim: int, hidden: int, stream=None) -> None:
    """gate_up_cuda (inferencer.cu:786-804), FP32 mode."""
    if wgate.type != Q4_K or wup.type != Q4_K or wgate.rows() != hidden or wup.rows() != hidden:
        raise QKError("gate_up", QK_ERR_SHAPE, "Unexpected feedforward quantization")
    multi_matvec([(wgate, gate), (wup, up)], x, dim, stream)


def batch_workspace_bytes(cols: int, rows: int, count: int) -> int:
    """Workspace bytes of a multi-token call (rows: total output rows)."""
    return int(lib().qk_gemv_batched_workspace_bytes(cols, rows, count))


def batch_matvec(t: Tensor, inp, out, cols: int, rows: int, count: int, workspace=None,
                 workspace_bytes: int = 0, stream=None) -> None:
    """FastRunner::batch_matvec (inferencer.cu:1265-1278) with FP32 semantics:
    out[t*rows + r] = sum_c W[r][c] inp[t*cols + c] for t < count."""
    if t.cols() != cols or t.rows() != rows or t.type not in QUANT_TYPES:
        raise QKError("batch_matvec", QK_ERR_SHAPE, "Unexpected batched matrix shape")
    check(lib().qk_gemv_batched_f32(t.type, t.gpu, ptr(inp), cols, ptr(out), rows, cols, rows, count,
                                    ptr(workspace), workspace_bytes, stream_handle(stream)),
          "batched matrix launch")


def dequant_rows(t: Tensor, out, row0: int, nrows: int, stream=None) -> None:
    """Rows row0 .. row0+nrows-1 of t as fp32 (q4_value / q6_value, inferencer.cu:454-487)."""
    if row0 < 0 or nrows < 0 or row0 + nrows > t.rows():
        raise QKError("dequant_rows", QK_ERR_INVALID_ARG, "row range outside the tensor")
    check(lib().qk_dequant_rows(t.type, t.gpu, ptr(out), t.cols(), row0, nrows, stream_handle(stream)),
          "dequant launch")


def split_q6k(t: Tensor, stream=None) -> Tensor:
    """A copy of a Q6_K tensor in the split layout (qk_q6k_split): same block
    bytes, every field 16-byte aligned."""
    import torch

    if t.type != Q6_K:
        raise QKError("split_q6k", QK_ERR_TYPE, "split_q6k takes a Q6_K tensor")
    dst = torch.empty(tensor_bytes(Q6_K_SPLIT, t.cols(), t.rows()), dtype=torch.uint8, device="cuda")
    check(lib().qk_q6k_split(t.gpu, ptr(dst), t.cols(), t.rows(), stream_handle(stream)), "Q6_K split")
    return Tensor((t.cols(), t.rows()), Q6_K_SPLIT, dst)


def embedding(t: Tensor, tokens, out, n_tokens: int, stream=None) -> None:
    """embedding_cuda / embedding_batch_cuda (inferencer.cu:806-819)."""
    check(lib().qk_embedding(t.type, t.gpu, ptr(tokens), n_tokens, ptr(out), t.cols(), t.rows(),
                             stream_handle(stream)), "embedding launch")


def quantize(x, xq, xscale, cols: int, n_tokens: int = 1, ldx: int | None = None, ldxq: int | None = None,
             ldscale: int | None = None, stream=None) -> None:
    """FastGPU::quantize / quantize_batch_cuda (inferencer.cu:1151-1155, 891-904)."""
    ldx = cols if ldx is None else ldx
    ldxq = cols if ldxq is None else ldxq
    ldscale = (cols + 31) // 32 if ldscale is None else ldscale
    check(lib().qk_quantize_x32(ptr(x), ldx, ptr(xq), ldxq, ptr(xscale), ldscale, cols, n_tokens,
                                stream_handle(stream)), "activation quantization launch")


def rmsnorm_quantize(x, weight, out, xq, xscale, cols: int, n_tokens: int = 1, eps: float = 1e-5,
                     ldx: int | None = None, ldout: int | None = None, ldxq: int | None = None,
                     ldscale: int | None = None, stream=None) -> None:
    """rmsnorm_quantize_cuda / rmsnorm_quantize_batch_cuda (inferencer.cu:839-889): RMSNorm then the
    per-32 quantization in one launch (out may be None)."""
    ldx = cols if ldx is None else ldx
    ldout = cols if ldout is None else ldout
    ldxq = cols if ldxq is None else ldxq
    ldscale = cols // 32 if ldscale is None else ldscale
    check(lib().qk_rmsnorm_quantize_x32(ptr(x), ldx, ptr(weight), ptr(out), ldout, ptr(xq), ldxq, ptr(xscale),
                                        ldscale, cols, n_tokens, eps, stream_handle(stream)),
          "fused RMSNorm quantization launch")


def matvec_i8(t: Tensor, xq, xscale, out, cols: int, rows: int, n_tokens: int = 1, ldxq: int | None = None,
              ldscale: int | None = None, ldy: int | None = None, stream=None) -> None:
    """gemv_q4_dp4a / gemv_q6_dp4a / gemv_batch_dp4a (inferencer.cu:558-569, 663-699)."""
    if t.cols() != cols or t.rows() != rows or t.type not in QUANT_TYPES:
        raise QKError("matvec_i8", QK_ERR_SHAPE, "Unexpected quantized matrix shape")
    ldxq = cols if ldxq is None else ldxq
    ldscale = cols // 32 if ldscale is None else ldscale
    ldy = rows if ldy is None else ldy
    check(lib().qk_gemv_i8(t.type, t.gpu, ptr(xq), ldxq, ptr(xscale), ldscale, ptr(out), ldy, cols, rows,
                           n_tokens, stream_handle(stream)), "INT8 matrix launch")


def _upload_weights(owner, cfg: dict, weights: dict):
    """Device copies of workloads.llama_weights-style host arrays, kept alive
    by owner._dev; returns (qk_llama_config, qk_llama_weights)."""
    import numpy as np
    import torch
    owner._dev = []

    def up(a):
        t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
        owner._dev.append(t)
        return t.data_ptr()

    layers = (qk_llama_layer * cfg["layers"])()
    for i, L in enumerate(weights["layers"]):
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            setattr(layers[i], name + "_type", L[name + "_type"])
            setattr(layers[i], name, up(L[name]))
        layers[i].attn_norm = up(L["attn_norm"])
        layers[i].ffn_norm = up(L["ffn_norm"])
    owner._layers = layers
    out = weights.get("output")
    w = qk_llama_weights(embd_type=weights["embd_type"], token_embd=up(weights["token_embd"]),
                         output_type=weights.get("output_type", 0), output=up(out) if out is not None else None,
                         output_norm=up(weights["output_norm"]), layers=layers)
    c = qk_llama_config(**{k: cfg[k] for k in ("dim", "layers", "heads", "kv_heads", "hidden", "vocab",
                                                "context")}, eps=cfg["eps"], rope_theta=cfg["rope_theta"])
    return c, w


class GGUF:
    """A GGUF v3 model file (the reference's GGUF struct, inferencer.cu:204-340)
    through qk_gguf_*: parameters, string values, tokenizer arrays, the
    tensor table, and the device copy made by upload()."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().qk_gguf_open(str(path).encode(), ctypes.byref(h)), "GGUF")
        self.handle = h
        self.path = str(path)

    def close(self):
        # At interpreter exit the module's globals may already be gone.
        if getattr(self, "handle", None) and _LIB is not None:
            _LIB.qk_gguf_close(self.handle)
        self.handle = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def param(self, key: str) -> float:
        v = ctypes.c_double()
        check(lib().qk_gguf_param(self.handle, key.encode(), ctypes.byref(v)), "GGUF parameter")
        return v.value

    def string(self, key: str):
        v = lib().qk_gguf_string(self.handle, key.encode())
        return None if v is None else v.decode("utf-8", "surrogateescape")

    def tensors(self) -> list:
        out = []
        for i in range(lib().qk_gguf_tensor_count(self.handle)):
            t = qk_gguf_tensor()
            check(lib().qk_gguf_tensor_at(self.handle, i, ctypes.byref(t)), "GGUF tensor")
            out.append(t)
        return out

    def tensor(self, name: str) -> qk_gguf_tensor:
        t = qk_gguf_tensor()
        check(lib().qk_gguf_find_tensor(self.handle, name.encode(), ctypes.byref(t)), "GGUF tensor")
        return t

    def host_bytes(self, name: str):
        """A copy of a tensor's bytes from the mapping (numpy uint8)."""
        import numpy as np
        t = self.tensor(name)
        return np.frombuffer(ctypes.string_at(t.host, t.bytes), dtype=np.uint8).copy()

    def tokens(self, which: int = 0) -> list:
        """tokenizer.ggml.tokens (0) or tokenizer.ggml.merges (1) as bytes."""
        out = []
        n = ctypes.c_int64()
        for i in range(lib().qk_gguf_token_count(self.handle, which)):
            p = lib().qk_gguf_token(self.handle, which, i, ctypes.byref(n))
            out.append(ctypes.string_at(p, n.value) if n.value else b"")
        return out

    def data(self):
        p, n, a = ctypes.c_void_p(), ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().qk_gguf_data(self.handle, ctypes.byref(p), ctypes.byref(n), ctypes.byref(a)), "GGUF data")
        return p.value, n.value, a.value

    def upload(self, stream=None) -> None:
        check(lib().qk_gguf_upload(self.handle, stream_handle(stream)), "GGUF upload")

    def llama(self, context: int):
        """(qk_llama_config, qk_llama_weights, layer array) of the uploaded model."""
        c, w = qk_llama_config(), qk_llama_weights()
        n = int(self.param("llama.block_count"))
        layers = (qk_llama_layer * max(n, 1))()
        check(lib().qk_gguf_llama(self.handle, context, ctypes.byref(c), ctypes.byref(w), layers, n), "GGUF llama")
        return c, w, layers


def _config_dict(c: qk_llama_config) -> dict:
    return {k: getattr(c, k) for k in ("dim", "layers", "heads", "kv_heads", "hidden", "vocab", "context", "eps",
                                       "rope_theta")}


class Runner:
    """FastRunner (inferencer.cu:1182-1532) over the C ABI's decode driver.

    weights is a dict of host numpy arrays (workloads.llama_weights layout);
    they are copied to device memory owned by this object.  from_gguf builds
    it from an uploaded GGUF file instead."""

    def __init__(self, cfg: dict, weights: dict, stream=None):
        self.cfg = cfg
        c, w = _upload_weights(self, cfg, weights)
        self._create(c, w, stream)

    def _create(self, c, w, stream):
        h = ctypes.c_void_p()
        check(lib().qk_llama_create(ctypes.byref(c), ctypes.byref(w), stream_handle(stream), ctypes.byref(h)),
              "FastRunner")
        self.handle = h

    @classmethod
    def from_gguf(cls, model: GGUF, context: int, stream=None) -> "Runner":
        self = cls.__new__(cls)
        c, w, self._layers = model.llama(context)
        self._model = model
        self.cfg = _config_dict(c)
        self._create(c, w, stream)
        return self

    def close(self):
        # At interpreter exit the module's globals may already be gone.
        if getattr(self, "handle", None) and _LIB is not None:
            _LIB.qk_llama_destroy(self.handle)
        self.handle = None

    __del__ = close

    def memory(self) -> dict:
        """Device bytes the handle holds (qk_llama_memory_bytes)."""
        m = qk_llama_memory()
        check(lib().qk_llama_memory_bytes(self.handle, ctypes.byref(m)), "memory")
        return {k: int(getattr(m, k)) for k, _ in m._fields_}

    def set_int8(self, q4k: bool = True, q6k: bool = True) -> None:
        """The reference's INT8 GEMV modes (use_dp4a, use_q6_dp4a; inferencer.cu:1159-1166)."""
        check(lib().qk_llama_set_int8(self.handle, int(q4k), int(q6k)), "set_int8")

    def kv_cache(self) -> tuple[int, int]:
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib().qk_llama_kv_cache(self.handle, ctypes.byref(k), ctypes.byref(v)), "kv_cache")
        return k.value, v.value

    def logits_ptr(self) -> int:
        p = ctypes.c_void_p()
        check(lib().qk_llama_logits(self.handle, ctypes.byref(p)), "logits")
        return p.value

    def residual(self):
        """The residual stream x after the last step (host copy, float32 [dim])."""
        import numpy as np
        p = ctypes.c_void_p()
        check(lib().qk_llama_residual(self.handle, ctypes.byref(p)), "residual")
        return copy_to_host(p.value, self.cfg["dim"], np.float32)

    def set_trace(self, residuals: "DeviceBuffer | None", quantized: "DeviceBuffer | None" = None) -> None:
        """Per-layer residuals [layer][dim] and INT8 inputs [layer][4][max(dim,
        hidden)] of every following step (qk_llama_set_trace); None stops."""
        self._trace = (residuals, quantized)
        check(lib().qk_llama_set_trace(self.handle, residuals.ptr if residuals else None,
                                       quantized.ptr if quantized else None), "set_trace")

    def matrix_calls(self) -> int:
        """Quantized matrix products issued since create (qk_llama_matrix_calls)."""
        n = ctypes.c_uint64()
        check(lib().qk_llama_matrix_calls(self.handle, ctypes.byref(n)), "matrix_calls")
        return n.value

    def forward(self, token: int, pos: int, need_logits: bool = True) -> int:
        nxt = ctypes.c_int(-1)
        check(lib().qk_llama_forward(self.handle, token, pos, int(need_logits), ctypes.byref(nxt)), "forward")
        return nxt.value


class BatchRunner:
    """Ragged decode batches over the C ABI's batched driver
    (qk_llama_batch_*): every token of a step belongs to its own sequence,
    whose KV rows start at desc.kv_row in caches of cache_rows rows per
    layer."""

    def __init__(self, cfg: dict, weights: dict, max_tokens: int, cache_rows: int, stream=None):
        self.cfg = cfg
        self.cache_rows = cache_rows
        c, w = _upload_weights(self, cfg, weights)
        self._create(c, w, max_tokens, cache_rows, stream)

    def _create(self, c, w, max_tokens, cache_rows, stream):
        self.max_tokens = max_tokens
        h = ctypes.c_void_p()
        check(lib().qk_llama_batch_create(ctypes.byref(c), ctypes.byref(w), max_tokens, cache_rows,
                                          stream_handle(stream), ctypes.byref(h)), "batched runner")
        self.handle = h

    @classmethod
    def from_gguf(cls, model: GGUF, context: int, max_tokens: int, cache_rows: int, stream=None) -> "BatchRunner":
        """context bounds every token's position (the RoPE table length)."""
        self = cls.__new__(cls)
        c, w, self._layers = model.llama(context)
        self._model = model
        self.cfg = _config_dict(c)
        self.cache_rows = cache_rows
        self._create(c, w, max_tokens, cache_rows, stream)
        return self

    def close(self):
        # At interpreter exit the module's globals may already be gone.
        if getattr(self, "handle", None) and _LIB is not None:
            _LIB.qk_llama_batch_destroy(self.handle)
        self.handle = None

    __del__ = close

    def kv_cache(self) -> tuple[int, int]:
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        check(lib().qk_llama_batch_kv_cache(self.handle, ctypes.byref(k), ctypes.byref(v)), "kv_cache")
        return k.value, v.value

    def memory(self) -> dict:
        """Device bytes the handle holds (qk_llama_batch_memory_bytes)."""
        m = qk_llama_memory()
        check(lib().qk_llama_batch_memory_bytes(self.handle, ctypes.byref(m)), "memory")
        return {k: int(getattr(m, k)) for k, _ in m._fields_}

    def forward(self, tokens, pos, kv_row, need_logits: bool = True, seq=None, logit_rows=None):
        """tokens, pos, kv_row: per-token sequences (several tokens of one
        sequence share its kv_row: a prefill chunk).  Returns the greedy next
        tokens (list) or None.  logit_rows: the token indices whose logits
        and successors are computed (qk_llama_batch_forward_rows); by default
        every token when need_logits, none otherwise."""
        n = len(tokens)
        tok = (ctypes.c_int32 * n)(*[int(t) for t in tokens])
        desc = (qk_batch_token * n)()
        for i in range(n):
            desc[i].pos, desc[i].kv_row = int(pos[i]), int(kv_row[i])
            desc[i].seq = int(seq[i]) if seq is not None else i
        if logit_rows is None:
            nxt = (ctypes.c_int32 * n)()
            check(lib().qk_llama_batch_forward(self.handle, tok, desc, n, int(need_logits), nxt), "batched forward")
            return list(nxt) if need_logits else None
        r = len(logit_rows)
        rows = (ctypes.c_int32 * max(r, 1))(*[int(i) for i in logit_rows])
        nxt = (ctypes.c_int32 * max(r, 1))()
        check(lib().qk_llama_batch_forward_rows(self.handle, tok, desc, n, rows, r, nxt), "batched forward")
        return list(nxt)[:r]

    def logits(self, n_tokens: int):
        import numpy as np
        p = ctypes.c_void_p()
        check(lib().qk_llama_batch_logits(self.handle, ctypes.byref(p)), "logits")
        return copy_to_host(p.value, n_tokens * self.cfg["vocab"], np.float32).reshape(n_tokens, self.cfg["vocab"])

    def residual(self, n_tokens: int):
        """The residual streams after the last step (host copy, [n_tokens][dim])."""
        import numpy as np
        p = ctypes.c_void_p()
        check(lib().qk_llama_batch_residual(self.handle, ctypes.byref(p)), "residual")
        return copy_to_host(p.value, n_tokens * self.cfg["dim"], np.float32).reshape(n_tokens, self.cfg["dim"])

    def set_trace(self, residuals: "DeviceBuffer | None", quantized: "DeviceBuffer | None" = None) -> None:
        """Per token of each following step, residuals [token][layer][dim] and
        INT8 inputs [token][layer][4][max(dim, hidden)]
        (qk_llama_batch_set_trace); None stops."""
        self._trace = (residuals, quantized)
        check(lib().qk_llama_batch_set_trace(self.handle, residuals.ptr if residuals else None,
                                             quantized.ptr if quantized else None), "set_trace")

    def set_int8(self, q4k: bool = True, q6k: bool = True) -> None:
        """The reference's INT8 batched arithmetic (both types or neither;
        qk_llama_batch_set_int8)."""
        check(lib().qk_llama_batch_set_int8(self.handle, int(q4k), int(q6k)), "set_int8")

    def matrix_calls(self) -> int:
        """Quantized matrix products issued since create (qk_llama_batch_matrix_calls)."""
        n = ctypes.c_uint64()
        check(lib().qk_llama_batch_matrix_calls(self.handle, ctypes.byref(n)), "matrix_calls")
        return n.value

    def load_kv(self, key_cache, value_cache) -> None:
        """Copy fp32 caches laid out [layer][cache_rows][kv_dim] (the
        reference's layout) into the driver's head-major caches."""
        _load_kv(self.kv_cache(), self.cfg, self.cache_rows, key_cache, value_cache)

    def kv_rows(self, n: int):
        """Rows 0..n-1 of every layer of both caches, as host arrays
        [layer][n][kv_dim] (the reference's layout)."""
        return _kv_rows(self.kv_cache(), self.cfg, self.cache_rows, n)

    def load_kv_rows(self, row0: int, key_rows, value_rows) -> None:
        """Write host rows [layer][n][kv_dim] (one sequence's rows) at cache
        rows row0 .. row0 + n - 1 of every layer."""
        _load_kv_rows(self.kv_cache(), self.cfg, self.cache_rows, row0, key_rows, value_rows)


_HIP = None


def _hip() -> ctypes.CDLL:
    """libamdhip64 for plain device<->host copies of buffers the C ABI owns."""
    global _HIP
    if _HIP is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipMemcpy.argtypes = [_vp, _vp, ctypes.c_size_t, _i]
        h.hipMemcpy.restype = _i
        h.hipMemcpy2D.argtypes = [_vp, ctypes.c_size_t, _vp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _i]
        h.hipMemcpy2D.restype = _i
        h.hipDeviceSynchronize.argtypes = []
        h.hipDeviceSynchronize.restype = _i
        h.hipMalloc.argtypes, h.hipMalloc.restype = [ctypes.POINTER(_vp), ctypes.c_size_t], _i
        h.hipFree.argtypes, h.hipFree.restype = [_vp], _i
        h.hipEventCreate.argtypes, h.hipEventCreate.restype = [ctypes.POINTER(_vp)], _i
        h.hipEventDestroy.argtypes, h.hipEventDestroy.restype = [_vp], _i
        h.hipEventRecord.argtypes, h.hipEventRecord.restype = [_vp, _vp], _i
        h.hipEventSynchronize.argtypes, h.hipEventSynchronize.restype = [_vp], _i
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _vp, _vp]
        h.hipEventElapsedTime.restype = _i
        _HIP = h
    return _HIP


class DeviceBuffer:
    """nbytes of device memory owned by this object (hipMalloc / hipFree),
    for buffers the C ABI fills, such as the drivers' traces."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _vp()
        if _hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)) != 0:
            raise QKError("DeviceBuffer", QK_ERR_DEVICE, f"hipMalloc of {self.nbytes} bytes failed")
        self.ptr = p.value

    def host(self, dtype, count: int | None = None):
        """The first count values (all by default) as a host array."""
        import numpy as np
        size = np.dtype(dtype).itemsize
        return copy_to_host(self.ptr, self.nbytes // size if count is None else count, dtype)

    def close(self) -> None:
        if getattr(self, "ptr", None) and _HIP is not None:
            _HIP.hipDeviceSynchronize()
            _HIP.hipFree(self.ptr)
        self.ptr = None

    __del__ = close


class GpuTimer:
    """Device time from start() to stop() on one stream, summed over every
    interval (FastGPU's start_timer / stop_timer, inferencer.cu:1172-1179):
    two HIP events recorded on the stream; stop() waits for the second."""

    def __init__(self, stream=None):
        h = _hip()
        self._stream = stream_handle(stream)
        self._start, self._end = _vp(), _vp()
        if h.hipEventCreate(ctypes.byref(self._start)) != 0 or h.hipEventCreate(ctypes.byref(self._end)) != 0:
            raise QKError("GpuTimer", QK_ERR_DEVICE, "hipEventCreate failed")
        self.seconds = 0.0

    def start(self) -> None:
        if _hip().hipEventRecord(self._start, self._stream) != 0:
            raise QKError("GpuTimer", QK_ERR_DEVICE, "hipEventRecord failed")

    def stop(self) -> None:
        h = _hip()
        ms = ctypes.c_float()
        if h.hipEventRecord(self._end, self._stream) != 0 or h.hipEventSynchronize(self._end) != 0 or \
                h.hipEventElapsedTime(ctypes.byref(ms), self._start, self._end) != 0:
            raise QKError("GpuTimer", QK_ERR_DEVICE, "GPU timer failed")
        self.seconds += ms.value / 1e3

    def close(self) -> None:
        if getattr(self, "_start", None) and _HIP is not None:
            _HIP.hipEventDestroy(self._start)
            _HIP.hipEventDestroy(self._end)
        self._start = self._end = None

    __del__ = close


def _kv_shape(cfg) -> tuple[int, int, int]:
    """(layers, kv_heads, head_dim) of a model config."""
    return cfg["layers"], cfg["kv_heads"], cfg["dim"] // cfg["heads"]


def _load_kv(ptrs, cfg, rows: int, key_cache, value_cache) -> None:
    """Host caches [layer][rows][kv_heads * head_dim] into a driver's
    [layer][kv_heads][rows][head_dim] device caches."""
    import numpy as np
    layers, kvh, hd = _kv_shape(cfg)
    n = layers * rows * kvh * hd
    for dst, a in zip(ptrs, (key_cache, value_cache)):
        a = _cache_array(a, n).reshape(layers, rows, kvh, hd)
        copy_to_device(dst, np.ascontiguousarray(a.transpose(0, 2, 1, 3)), n * 4)


def _kv_rows(ptrs, cfg, rows: int, n: int):
    """Rows 0..n-1 of a driver's head-major caches as two host arrays
    [layer][n][kv_heads * head_dim] (one strided copy per cache)."""
    import numpy as np
    layers, kvh, hd = _kv_shape(cfg)
    if not 0 <= n <= rows:
        raise QKError("kv_rows", QK_ERR_INVALID_ARG, f"{n} rows of a {rows}-row cache")
    out = []
    for src in ptrs:
        a = np.empty((layers, kvh, n, hd), dtype=np.float32)
        if n:
            _copy_2d(a.ctypes.data, n * hd * 4, src, rows * hd * 4, n * hd * 4, layers * kvh, 2)
        out.append(np.ascontiguousarray(a.transpose(0, 2, 1, 3)).reshape(layers, n, kvh * hd))
    return out[0], out[1]


def _load_kv_rows(ptrs, cfg, rows: int, row0: int, key_rows, value_rows) -> None:
    """Host rows [layer][n][kv_heads * head_dim] into rows row0 .. row0+n-1 of
    a driver's head-major caches (one strided copy per cache)."""
    import numpy as np
    layers, kvh, hd = _kv_shape(cfg)
    k = np.asarray(key_rows)
    n = k.shape[1] if k.ndim == 3 else -1
    if n < 0 or not 0 <= row0 <= rows - n:
        raise QKError("load_kv_rows", QK_ERR_INVALID_ARG, f"rows {row0}..{row0 + n - 1} of a {rows}-row cache")
    for dst, a in zip(ptrs, (key_rows, value_rows)):
        a = _cache_array(a, layers * n * kvh * hd).reshape(layers, n, kvh, hd)
        a = np.ascontiguousarray(a.transpose(0, 2, 1, 3))
        if n:
            _copy_2d(dst + row0 * hd * 4, rows * hd * 4, a.ctypes.data, n * hd * 4, n * hd * 4, layers * kvh, 1)


def copy_kv_rows(dst, src, n: int) -> None:
    """Rows 0..n-1 of every layer and KV head of src's caches into dst's (a
    Runner or BatchRunner each; same model), device to device: one strided
    copy per cache."""
    layers, kvh, hd = _kv_shape(dst.cfg)
    rows_of = lambda r: r.cache_rows if hasattr(r, "cache_rows") else r.cfg["context"]
    dr, sr = rows_of(dst), rows_of(src)
    if not 0 <= n <= min(dr, sr):
        raise QKError("copy_kv_rows", QK_ERR_INVALID_ARG, f"{n} rows between caches of {sr} and {dr} rows")
    if n == 0:
        return
    for d, s_ in zip(dst.kv_cache(), src.kv_cache()):
        _copy_2d(d, dr * hd * 4, s_, sr * hd * 4, n * hd * 4, layers * kvh, 3)


def _copy_2d(dst: int, dpitch: int, src: int, spitch: int, width: int, height: int, kind: int) -> None:
    """height rows of width bytes between pitched buffers (hipMemcpy2D; kind
    1 host->device, 2 device->host, 3 device->device), after a device-wide
    synchronisation so no queued step still uses either buffer."""
    h = _hip()
    if h.hipDeviceSynchronize() != 0 or h.hipMemcpy2D(dst, dpitch, src, spitch, width, height, kind) != 0:
        raise QKError("copy_2d", QK_ERR_DEVICE, "hipMemcpy2D failed")


def _cache_array(a, count: int):
    """a as a contiguous float32 array of exactly count values (QKError
    otherwise): caches are copied whole, never partly or past their end."""
    import numpy as np
    a = np.asarray(a)
    if a.dtype != np.float32 or a.size != count:
        raise QKError("load_kv", QK_ERR_INVALID_ARG,
                      f"cache must be float32 with {count} values, got {a.dtype} with {a.size}")
    return np.ascontiguousarray(a)


def copy_to_device(dst: int, host_array, nbytes: int | None = None) -> None:
    """Copy host_array into device memory at dst.  nbytes, when given, is the
    destination's size and must equal the array's.  The device is
    synchronised first, so no queued step on any stream still uses dst."""
    import numpy as np
    a = np.ascontiguousarray(host_array)
    if nbytes is not None and a.nbytes != nbytes:
        raise QKError("copy_to_device", QK_ERR_INVALID_ARG, f"{a.nbytes} bytes for a {nbytes}-byte buffer")
    h = _hip()
    if h.hipDeviceSynchronize() != 0 or h.hipMemcpy(dst, a.ctypes.data, a.nbytes, 1) != 0:
        raise QKError("copy_to_device", QK_ERR_DEVICE, "hipMemcpy host->device failed")


def copy_to_host(src: int, count: int, dtype) -> "object":
    import numpy as np
    out = np.empty(count, dtype=dtype)
    h = _hip()
    if h.hipDeviceSynchronize() != 0 or h.hipMemcpy(out.ctypes.data, src, out.nbytes, 2) != 0:
        raise QKError("copy_to_host", QK_ERR_DEVICE, "hipMemcpy device->host failed")
    return out


def copy_device(dst: int, src: int, nbytes: int) -> None:
    """Device-to-device copy of nbytes (the device is synchronised first)."""
    h = _hip()
    if h.hipDeviceSynchronize() != 0 or h.hipMemcpy(dst, src, nbytes, 3) != 0:
        raise QKError("copy_device", QK_ERR_DEVICE, "hipMemcpy device->device failed")


def _runner_load_kv(self, key_cache, value_cache) -> None:
    """Copy fp32 caches laid out [layer][context][kv_dim] (the reference's
    layout) into the runner's head-major caches."""
    _load_kv(self.kv_cache(), self.cfg, self.cfg["context"], key_cache, value_cache)


def _runner_kv_rows(self, n: int):
    """Rows 0..n-1 of every layer of both caches, host arrays [layer][n][kv_dim]."""
    return _kv_rows(self.kv_cache(), self.cfg, self.cfg["context"], n)


def _runner_logits(self):
    import numpy as np
    return copy_to_host(self.logits_ptr(), self.cfg["vocab"], np.float32)


Runner.load_kv = _runner_load_kv
Runner.kv_rows = _runner_kv_rows
Runner.logits = _runner_logits
