"""Seeded synthetic inputs for the Q4_K / Q6_K workloads (ctypes over libqksynth.so).

The generator (SplitMix64, Box-Muller, software double->fp16 RNE) is specified
in csrc/qk_synth.h.  Every array returned here is a fresh numpy array.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

_HERE = pathlib.Path(__file__).resolve().parent
_LIB = None

Q4_K = 12
Q6_K = 14
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210}


def _lib():
    global _LIB
    if _LIB is None:
        path = _HERE / "libqksynth.so"
        if not path.exists():
            raise ImportError(f"{path} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(str(path))
        u64, i64, dbl = ctypes.c_uint64, ctypes.c_int64, ctypes.c_double
        vp = ctypes.c_void_p
        for name in ("qs_fill_q4k", "qs_fill_q6k"):
            getattr(lib, name).argtypes = [vp, i64, u64, u64, dbl]
            getattr(lib, name).restype = None
        lib.qs_fill_normal_f32.argtypes = [vp, i64, u64, u64, dbl, dbl]
        lib.qs_fill_normal_f32.restype = None
        lib.qs_fill_uniform_i32.argtypes = [vp, i64, u64, u64, ctypes.c_int32, ctypes.c_int32]
        lib.qs_fill_uniform_i32.restype = None
        lib.qs_fill_bytes.argtypes = [vp, i64, u64, u64]
        lib.qs_fill_bytes.restype = None
        lib.qs_f64_to_f16_array.argtypes = [vp, vp, i64]
        lib.qs_f64_to_f16_array.restype = None
        _LIB = lib
    return _LIB


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def quant_blocks(qtype: int, n_blocks: int, seed: int, stream: int, d_sigma: float | None = None) -> np.ndarray:
    """n_blocks random super-blocks of qtype as a flat uint8 array."""
    if qtype == Q4_K:
        out = np.empty(n_blocks * 144, dtype=np.uint8)
        _lib().qs_fill_q4k(_ptr(out), n_blocks, seed, stream, 0.02 if d_sigma is None else d_sigma)
    elif qtype == Q6_K:
        out = np.empty(n_blocks * 210, dtype=np.uint8)
        _lib().qs_fill_q6k(_ptr(out), n_blocks, seed, stream, 0.01 if d_sigma is None else d_sigma)
    else:
        raise ValueError(f"unsupported storage type {qtype}")
    return out


def quant_matrix(qtype: int, cols: int, rows: int, seed: int, stream: int,
                 d_sigma: float | None = None) -> np.ndarray:
    """A rows x cols quantized matrix, rows contiguous (uint8, rows * row_bytes)."""
    if cols % 256:
        raise ValueError("cols must be a multiple of 256")
    return quant_blocks(qtype, rows * (cols // 256), seed, stream, d_sigma)


def normal_f32(n: int, seed: int, stream: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _lib().qs_fill_normal_f32(_ptr(out), n, seed, stream, mean, sigma)
    return out


def uniform_i32(n: int, seed: int, stream: int, lo: int, hi: int) -> np.ndarray:
    """n integers uniform in [lo, hi] (inclusive)."""
    out = np.empty(n, dtype=np.int32)
    _lib().qs_fill_uniform_i32(_ptr(out), n, seed, stream, lo, hi)
    return out


def random_bytes(n: int, seed: int, stream: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    _lib().qs_fill_bytes(_ptr(out), n, seed, stream)
    return out


def f64_to_f16_bits(values) -> np.ndarray:
    src = np.ascontiguousarray(values, dtype=np.float64)
    out = np.empty(src.shape, dtype=np.uint16)
    _lib().qs_f64_to_f16_array(_ptr(src), _ptr(out), src.size)
    return out
