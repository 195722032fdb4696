"""ctypes wrapper of liboqoracle.so: the CPU restatement of inferencer.cu's
Q4_K / Q6_K path.

TEST INFRASTRUCTURE ONLY.  Loaded by tests/, by __graft_entry__.smoke() and by
the cpu_baseline leg of bench.py -- always as the oracle results are compared with, or the reported CPU
baseline, never as the product path.  See qk_oracle.h for how each function is
pinned.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = _HERE / "liboqoracle.so"
Q4_K, Q6_K = 12, 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}
_LIB = None


class LlamaConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("dim", "layers", "heads", "kv_heads", "hidden", "vocab", "context")] + \
               [("eps", ctypes.c_float), ("rope_theta", ctypes.c_float)]


class LlamaLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("q_type", "k_type", "v_type", "o_type", "gate_type", "up_type",
                                             "down_type")] + \
               [(n, ctypes.c_void_p) for n in ("q", "k", "v", "o", "gate", "up", "down", "attn_norm", "ffn_norm")]


class LlamaWeights(ctypes.Structure):
    _fields_ = [("embd_type", ctypes.c_int), ("token_embd", ctypes.c_void_p), ("output_type", ctypes.c_int),
                ("output", ctypes.c_void_p), ("output_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(LlamaLayer))]


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is not built; run `make -C oracle`")
        h = ctypes.CDLL(str(LIB_PATH))
        vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
        h.oq_f16_to_f32.argtypes, h.oq_f16_to_f32.restype = [ctypes.c_uint16], ctypes.c_float
        h.oq_q4k_value.argtypes, h.oq_q4k_value.restype = [vp, i32], ctypes.c_float
        h.oq_q6k_value.argtypes, h.oq_q6k_value.restype = [vp, i32], ctypes.c_float
        h.oq_q4k_scale_min.argtypes = [vp, i32, ctypes.POINTER(i32), ctypes.POINTER(i32)]
        h.oq_q4k_scale_min.restype = None
        h.oq_dequant_rows.argtypes, h.oq_dequant_rows.restype = [i32, vp, vp, i64, i64, i64], i32
        h.oq_embedding.argtypes, h.oq_embedding.restype = [i32, vp, vp, i64, vp, i64], i32
        h.oq_gemv_f64.argtypes, h.oq_gemv_f64.restype = [i32, vp, vp, i64, vp, i64, i64, i64, i64], i32
        h.oq_gemv_f32_ref.argtypes, h.oq_gemv_f32_ref.restype = [i32, vp, vp, vp, i64, i64], i32
        h.oq_quantize_x32.argtypes, h.oq_quantize_x32.restype = [vp, vp, vp, i64], None
        h.oq_subblock_dots_i8.argtypes, h.oq_subblock_dots_i8.restype = [i32, vp, vp, vp, vp, i64, i64], i32
        h.oq_gemv_i8_f64.argtypes, h.oq_gemv_i8_f64.restype = [i32, vp, vp, vp, vp, i64, i64], i32
        h.oq_rmsnorm.argtypes, h.oq_rmsnorm.restype = [vp, vp, vp, i64, ctypes.c_double], None
        h.oq_rope_tables.argtypes, h.oq_rope_tables.restype = [vp, vp, i32, i32, ctypes.c_float], None
        h.oq_rope.argtypes, h.oq_rope.restype = [vp, i64, vp, vp, i32, i32], None
        h.oq_attention.argtypes, h.oq_attention.restype = [vp, vp, vp, vp, i32, i32, i32, i32], None
        h.oq_silu_mul.argtypes, h.oq_silu_mul.restype = [vp, vp, i64], None
        h.oq_argmax_f64.argtypes, h.oq_argmax_f64.restype = [vp, i64], i64
        h.oq_argmax_f32.argtypes, h.oq_argmax_f32.restype = [vp, i64], i64
        h.oq_llama_create.argtypes = [ctypes.POINTER(LlamaConfig), ctypes.POINTER(LlamaWeights)]
        h.oq_llama_create.restype = vp
        h.oq_llama_destroy.argtypes, h.oq_llama_destroy.restype = [vp], None
        h.oq_llama_load_cache.argtypes, h.oq_llama_load_cache.restype = [vp, vp, vp, i32], i32
        h.oq_llama_forward.argtypes = [vp, i32, i32, i32, vp, ctypes.POINTER(i32)]
        h.oq_llama_forward.restype = i32
        h.oq_llama_set_int8.argtypes, h.oq_llama_set_int8.restype = [vp, i32, i32], None
        h.oq_omp_max_threads.argtypes, h.oq_omp_max_threads.restype = [], i32
        _LIB = h
    return _LIB


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def omp_max_threads() -> int:
    """Threads the oracle's OpenMP loops run on (omp_get_max_threads)."""
    return int(lib().oq_omp_max_threads())


def f16_to_f32(bits: int) -> float:
    return lib().oq_f16_to_f32(bits)


def scale_min(scales: np.ndarray, sub: int) -> tuple[int, int]:
    s, m = ctypes.c_int(), ctypes.c_int()
    lib().oq_q4k_scale_min(_p(np.ascontiguousarray(scales, dtype=np.uint8)), sub, ctypes.byref(s), ctypes.byref(m))
    return s.value, m.value


def dequant(qtype: int, w: np.ndarray, cols: int, rows: int, row0: int = 0) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    assert lib().oq_dequant_rows(qtype, _p(w), _p(out), cols, row0, rows) == 0
    return out


def value(qtype: int, block: np.ndarray, i: int) -> float:
    block = np.ascontiguousarray(block, dtype=np.uint8)
    return (lib().oq_q4k_value if qtype == Q4_K else lib().oq_q6k_value)(_p(block), i)


def embedding(qtype: int, w: np.ndarray, tokens, cols: int) -> np.ndarray:
    tok = np.ascontiguousarray(tokens, dtype=np.int32)
    out = np.empty((tok.size, cols), dtype=np.float32)
    assert lib().oq_embedding(qtype, _p(w), _p(tok), tok.size, _p(out), cols) == 0
    return out


def gemv_f64(qtype: int, w: np.ndarray, x: np.ndarray, cols: int, rows: int) -> np.ndarray:
    """y = W x (x: [cols] or [tokens, cols]) with fp64 accumulation."""
    x2 = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    ntok = x2.shape[0]
    y = np.empty((ntok, rows), dtype=np.float64)
    assert lib().oq_gemv_f64(qtype, _p(w), _p(x2), cols, _p(y), rows, cols, rows, ntok) == 0
    return y[0] if np.ndim(x) == 1 else y


def gemv_f32_ref(qtype: int, w: np.ndarray, x: np.ndarray, cols: int, rows: int) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    assert lib().oq_gemv_f32_ref(qtype, _p(w), _p(np.ascontiguousarray(x, dtype=np.float32)), _p(y), cols, rows) == 0
    return y


def quantize_x32(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    xq = np.empty(x.size, dtype=np.int8)
    xs = np.empty((x.size + 31) // 32, dtype=np.float32)
    lib().oq_quantize_x32(_p(x), _p(xq), _p(xs), x.size)
    return xq, xs


def subblock_dots_i8(qtype: int, w: np.ndarray, xq: np.ndarray, cols: int, rows: int):
    nsub = 8 if qtype == Q4_K else 16
    dots = np.empty((rows, cols // 256 * nsub), dtype=np.int32)
    xs = np.empty(cols // 256 * nsub, dtype=np.int32)
    assert lib().oq_subblock_dots_i8(qtype, _p(w), _p(np.ascontiguousarray(xq, dtype=np.int8)), _p(dots), _p(xs),
                                     cols, rows) == 0
    return dots, xs


def gemv_i8_f64(qtype: int, w: np.ndarray, xq: np.ndarray, xscale: np.ndarray, cols: int, rows: int) -> np.ndarray:
    y = np.empty(rows, dtype=np.float64)
    assert lib().oq_gemv_i8_f64(qtype, _p(w), _p(np.ascontiguousarray(xq, dtype=np.int8)),
                                _p(np.ascontiguousarray(xscale, dtype=np.float32)), _p(y), cols, rows) == 0
    return y


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float64)
    out = np.empty_like(x)
    lib().oq_rmsnorm(_p(x), _p(np.ascontiguousarray(weight, dtype=np.float32)), _p(out), x.size, eps)
    return out


def rope_tables(context: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    c = np.empty((context, head_dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().oq_rope_tables(_p(c), _p(s), context, head_dim, theta)
    return c, s


def rope(v: np.ndarray, cosine: np.ndarray, sine: np.ndarray, pos: int, head_dim: int) -> np.ndarray:
    out = np.array(v, dtype=np.float64, copy=True)
    lib().oq_rope(_p(out), out.size, _p(cosine), _p(sine), pos, head_dim)
    return out


def attention(q, key_cache, value_cache, pos: int, heads: int, kv_heads: int, head_dim: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float64)
    kc = np.ascontiguousarray(key_cache, dtype=np.float64)
    vc = np.ascontiguousarray(value_cache, dtype=np.float64)
    out = np.empty(heads * head_dim, dtype=np.float64)
    lib().oq_attention(_p(q), _p(kc), _p(vc), _p(out), pos, heads, kv_heads, head_dim)
    return out


def silu_mul(gate, up) -> np.ndarray:
    g = np.array(gate, dtype=np.float64, copy=True)
    lib().oq_silu_mul(_p(g), _p(np.ascontiguousarray(up, dtype=np.float64)), g.size)
    return g


def argmax(v) -> int:
    v = np.ascontiguousarray(v)
    if v.dtype == np.float32:
        return int(lib().oq_argmax_f32(_p(v), v.size))
    v = np.ascontiguousarray(v, dtype=np.float64)
    return int(lib().oq_argmax_f64(_p(v), v.size))


class Llama:
    """fp64 decode step over host weight arrays (kept referenced here)."""

    def __init__(self, cfg: dict, weights: dict):
        self._keep = weights
        self.cfg = LlamaConfig(**{k: cfg[k] for k in ("dim", "layers", "heads", "kv_heads", "hidden", "vocab",
                                                        "context")}, eps=cfg["eps"], rope_theta=cfg["rope_theta"])
        layers = (LlamaLayer * cfg["layers"])()
        for i, L in enumerate(weights["layers"]):
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                setattr(layers[i], name + "_type", L[name + "_type"])
                setattr(layers[i], name, _p(L[name]))
            layers[i].attn_norm = _p(L["attn_norm"])
            layers[i].ffn_norm = _p(L["ffn_norm"])
        self._layers = layers
        out = weights.get("output")
        self.w = LlamaWeights(embd_type=weights["embd_type"], token_embd=_p(weights["token_embd"]),
                              output_type=weights.get("output_type", 0), output=_p(out) if out is not None else None,
                              output_norm=_p(weights["output_norm"]), layers=layers)
        self.handle = lib().oq_llama_create(ctypes.byref(self.cfg), ctypes.byref(self.w))
        if not self.handle:
            raise ValueError("oracle rejected the llama configuration")

    def __del__(self):
        if getattr(self, "handle", None):
            lib().oq_llama_destroy(self.handle)
            self.handle = None

    def load_cache(self, key_cache: np.ndarray, value_cache: np.ndarray, n_positions: int) -> None:
        assert lib().oq_llama_load_cache(self.handle, _p(np.ascontiguousarray(key_cache, dtype=np.float32)),
                                         _p(np.ascontiguousarray(value_cache, dtype=np.float32)), n_positions) == 0

    def set_int8(self, q4k: bool = True, q6k: bool = True) -> None:
        """INT8 GEMV modes of the decode step (the reference's use_dp4a and
        use_q6_dp4a): each GEMV on a matrix of an enabled type quantizes its
        input per 32 values and takes exact integer sub-block dots."""
        lib().oq_llama_set_int8(self.handle, int(q4k), int(q6k))

    def forward(self, token: int, pos: int, need_logits: bool = True):
        logits = np.empty(self.cfg.vocab, dtype=np.float64) if need_logits else None
        nxt = ctypes.c_int(-1)
        rc = lib().oq_llama_forward(self.handle, token, pos, int(need_logits),
                                    _p(logits) if logits is not None else None, ctypes.byref(nxt))
        assert rc == 0
        return nxt.value, logits
