#!/usr/bin/env python3
"""Writes tests/golden/golden.npz, the committed fixtures of the Q4_K / Q6_K
path (numpy .npz, no pickled objects):

  kat_q4k_blocks / kat_q4k_values   two hand-built Q4_K blocks and their 512
  kat_q6k_blocks / kat_q6k_values   (256 per block) dequantized values, from
                                    the closed forms of inferencer.cu:454-487
                                    evaluated here in exact integer
                                    arithmetic (every value is representable).
  rnd_q4k_blocks / rnd_q4k_values   seeded random blocks (seed 41) and the
  rnd_q6k_blocks / rnd_q6k_values   oracle's bit patterns for them.
  gemv_<type>_512x64_{w,x,y}        64-row GEMVs with fp64 y from the oracle.
  config1_w_sha256 / config1_y      the Q4_K 2048 x 2048 workload (seed 0):
                                    the SHA-256 of its weight bytes and the
                                    fp64 y.

Run from the repository root after building (python3 tests/golden/make_golden.py).
"""
import hashlib
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "tests"))
from conftest import load_oracle, load_package  # noqa: E402

Q4_K, Q6_K = 12, 14


def f16_bits(v: float) -> int:
    return int(np.array([v], dtype=np.float16).view(np.uint16)[0])


def kat_q4k():
    """d = 1, dmin = 0.5: w = sc*q - m/2, a multiple of 1/2 below 1000."""
    blocks, values = [], []
    for variant in range(2):
        b = bytearray(144)
        b[0:2] = f16_bits(1.0).to_bytes(2, "little")
        b[2:4] = f16_bits(0.5).to_bytes(2, "little")
        sc = [(7 * j + 3 + 29 * variant) % 64 for j in range(8)]
        mn = [(11 * j + 5 + 13 * variant) % 64 for j in range(8)]
        s = [0] * 12
        for j in range(4):
            s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
            s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
            s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
        b[4:16] = bytes(s)
        q = [(5 * i + 3 * variant + i // 37) % 16 for i in range(256)]
        for i in range(256):
            lo = (i // 64) * 32 + i % 32
            if (i // 32) % 2 == 0:
                b[16 + lo] = (b[16 + lo] & 0xF0) | q[i]
            else:
                b[16 + lo] = (b[16 + lo] & 0x0F) | (q[i] << 4)
        blocks.append(bytes(b))
        values += [sc[i // 32] * q[i] - mn[i // 32] / 2 for i in range(256)]
    return np.frombuffer(b"".join(blocks), dtype=np.uint8).copy(), np.array(values, dtype=np.float32)


def kat_q6k():
    """d = 0.25: w = 0.25*scale*(code-32), a multiple of 1/4."""
    blocks, values = [], []
    for variant in range(2):
        b = bytearray(210)
        code = [(9 * i + 17 * variant + i // 11) % 64 for i in range(256)]
        scales = [((5 * j + 7 * variant) % 64) - 32 for j in range(16)]
        for i in range(256):
            g, p = divmod(i, 128)
            part, l = divmod(p, 32)
            lo_idx = g * 64 + (part & 1) * 32 + l
            if part < 2:
                b[lo_idx] = (b[lo_idx] & 0xF0) | (code[i] & 15)
            else:
                b[lo_idx] = (b[lo_idx] & 0x0F) | ((code[i] & 15) << 4)
            hi_idx = 128 + g * 32 + l
            b[hi_idx] |= ((code[i] >> 4) & 3) << (2 * part)
        b[192:208] = bytes(s & 0xFF for s in scales)
        b[208:210] = f16_bits(0.25).to_bytes(2, "little")
        blocks.append(bytes(b))
        values += [0.25 * scales[i // 16] * (code[i] - 32) for i in range(256)]
    return np.frombuffer(b"".join(blocks), dtype=np.uint8).copy(), np.array(values, dtype=np.float32)


def main() -> None:
    load_package()
    import inferencer_jetson_amd.synth as synth
    import inferencer_jetson_amd.workloads as wl
    oracle = load_oracle()
    out = {}
    out["kat_q4k_blocks"], out["kat_q4k_values"] = kat_q4k()
    out["kat_q6k_blocks"], out["kat_q6k_values"] = kat_q6k()
    for name, t in (("q4k", Q4_K), ("q6k", Q6_K)):
        blocks = synth.quant_blocks(t, 6, 41, 1 + t)
        out[f"rnd_{name}_blocks"] = blocks
        out[f"rnd_{name}_values"] = oracle.dequant(t, blocks, 256, 6).reshape(-1)
        w = synth.quant_matrix(t, 512, 64, 42, t)
        x = synth.normal_f32(512, 42, 2)
        out[f"gemv_{name}_512x64_w"] = w
        out[f"gemv_{name}_512x64_x"] = x
        out[f"gemv_{name}_512x64_y"] = oracle.gemv_f64(t, w, x, 512, 64)
    w, x = wl.gemv_q4k_2048()
    out["config1_w_sha256"] = np.frombuffer(hashlib.sha256(w.tobytes()).digest(), dtype=np.uint8).copy()
    out["config1_y"] = oracle.gemv_f64(Q4_K, w, x, 2048, 2048)
    path = pathlib.Path(__file__).resolve().parent / "golden.npz"
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
