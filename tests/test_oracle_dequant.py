"""Pins the oracle's fp16 and Q4_K / Q6_K decode (qk_oracle.c, restating
inferencer.cu:453-497) against closed forms and independent encoders.

- fp16: every one of the 65,536 half patterns against numpy's float16.
- Known-answer blocks built by hand (d = 1, dmin = 0, unit scales => w = q).
- Round trips through GGML's published block *packing* (the encoder loops of
  quantize_row_q4_K_ref / quantize_row_q6_K_ref, restated below in numpy):
  random codes and scales are packed, and the decode must return
  d*sc*q - dmin*m (Q4_K) or d*sc*(q-32) (Q6_K) at every element.  A swapped
  nibble, a wrong group stride or a mis-shifted high bit fails here.
- GGML's dequantize_row_q4_K / q6_K loop structure (per 64 / 128 values),
  restated in vectorised numpy, must agree bit for bit on random blocks.
"""
import numpy as np
import pytest

Q4_K, Q6_K = 12, 14


def f16_bytes(value: float) -> np.ndarray:
    return np.frombuffer(np.float16(value).tobytes(), dtype=np.uint8)


def test_f16_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ------------------------------------------------------------ encoders --

def pack_q4k_scales(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """GGML's 6-bit scale/min packing (quantize_row_q4_K_ref)."""
    out = np.zeros(12, dtype=np.uint8)
    for j in range(8):
        ls, lm = int(sc[j]), int(m[j])
        if j < 4:
            out[j] = ls
            out[j + 4] = lm
        else:
            out[j + 4] = (ls & 0xF) | ((lm & 0xF) << 4)
            out[j - 4] |= (ls >> 4) << 6
            out[j] |= (lm >> 4) << 6
    return out


def encode_q4k(d: float, dmin: float, sc, m, codes) -> np.ndarray:
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = f16_bytes(d)
    blk[2:4] = f16_bytes(dmin)
    blk[4:16] = pack_q4k_scales(np.asarray(sc), np.asarray(m))
    L = np.asarray(codes, dtype=np.int64)
    q = blk[16:]
    for j in range(0, 256, 64):
        for l in range(32):
            q[j // 2 + l] = L[j + l] | (L[j + l + 32] << 4)
    return blk


def encode_q6k(d: float, scales, codes) -> np.ndarray:
    """GGML's Q6_K packing (quantize_row_q6_K_ref), codes L in 0..63."""
    blk = np.zeros(210, dtype=np.uint8)
    L = np.asarray(codes, dtype=np.int64)
    for j in range(0, 256, 128):
        ql = blk[j // 2: j // 2 + 64]
        qh = blk[128 + j // 4: 128 + j // 4 + 32]
        for l in range(32):
            q1, q2, q3, q4 = (L[j + l] & 0xF, L[j + l + 32] & 0xF, L[j + l + 64] & 0xF, L[j + l + 96] & 0xF)
            ql[l] = q1 | (q3 << 4)
            ql[l + 32] = q2 | (q4 << 4)
            qh[l] = (L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) | \
                    ((L[j + l + 96] >> 4) << 6)
    blk[192:208] = np.asarray(scales, dtype=np.int8).view(np.uint8)
    blk[208:210] = f16_bytes(d)
    return blk


# ------------------------------------------- GGML dequantize, restated --

def ggml_dequant_q4k(blocks: np.ndarray) -> np.ndarray:
    """dequantize_row_q4_K: per 64 values, two (scale, min) pairs."""
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dmin = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.int64)
    q = b[:, 16:].astype(np.int64)
    sc = np.empty((b.shape[0], 8), dtype=np.int64)
    mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[:, j] = s[:, j] & 63
            mn[:, j] = s[:, j + 4] & 63
        else:
            sc[:, j] = (s[:, j + 4] & 0xF) | ((s[:, j - 4] >> 6) << 4)
            mn[:, j] = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    out = np.empty((b.shape[0], 256), dtype=np.float32)
    for chunk in range(4):
        qq = q[:, chunk * 32:(chunk + 1) * 32]
        for half, codes in ((0, qq & 0xF), (1, qq >> 4)):
            j = 2 * chunk + half
            d1 = d * sc[:, j].astype(np.float32)
            m1 = dmin * mn[:, j].astype(np.float32)
            out[:, chunk * 64 + half * 32: chunk * 64 + half * 32 + 32] = \
                d1[:, None] * codes.astype(np.float32) - m1[:, None]
    return out.reshape(-1)


def ggml_dequant_q6k(blocks: np.ndarray) -> np.ndarray:
    """dequantize_row_q6_K: two halves of 128 values, 32 lanes each."""
    b = blocks.reshape(-1, 210)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float32)[:, 0]
    sc = b[:, 192:208].copy().view(np.int8).astype(np.float32)
    out = np.empty((b.shape[0], 256), dtype=np.float32)
    for n in range(2):
        ql = b[:, 64 * n: 64 * n + 64].astype(np.int64)
        qh = b[:, 128 + 32 * n: 128 + 32 * n + 32].astype(np.int64)
        l = np.arange(32)
        is_ = l // 16
        q1 = ((ql[:, :32] & 0xF) | (((qh >> 0) & 3) << 4)) - 32
        q2 = ((ql[:, 32:] & 0xF) | (((qh >> 2) & 3) << 4)) - 32
        q3 = ((ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4)) - 32
        q4 = ((ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4)) - 32
        s = sc[:, 8 * n:8 * n + 8]
        base = 128 * n
        for k, q in enumerate((q1, q2, q3, q4)):
            out[:, base + 32 * k: base + 32 * k + 32] = \
                (d[:, None] * s[:, is_ + 2 * k]) * q.astype(np.float32)
    return out.reshape(-1)


# ------------------------------------------------------------- tests --

def test_q4k_unit_scales_known_answer(oracle):
    # d = 1, dmin = 0, every scale 1 and min 0: w is the raw nibble.
    sc = np.ones(8, dtype=np.int64)
    m = np.zeros(8, dtype=np.int64)
    blk = np.zeros(144, dtype=np.uint8)
    blk[0:2] = f16_bytes(1.0)
    blk[4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]
    assert np.array_equal(pack_q4k_scales(sc, m), blk[4:16])
    # qs byte k: low nibble k % 16, high nibble 15 - k % 16.
    k = np.arange(128)
    blk[16:] = (k % 16) | ((15 - k % 16) << 4)
    w = oracle.dequant(Q4_K, blk, 256, 1)[0]
    # element 0..31 of each 64-group: low nibbles of bytes l (l%16);
    # element 32..63: high nibbles 15 - l%16.
    i = np.arange(256)
    want = np.where(i % 64 < 32, (i % 32) % 16, 15 - (i % 32) % 16).astype(np.float32)
    assert np.array_equal(w, want)


def test_q4k_scale_min_high_bits(oracle):
    sc = np.array([1, 2, 3, 4, 37, 50, 63, 17])
    m = np.array([5, 6, 7, 8, 33, 44, 55, 60])
    packed = pack_q4k_scales(sc, m)
    for j in range(8):
        assert oracle.scale_min(packed, j) == (sc[j], m[j])
    blk = encode_q4k(0.5, 0.25, sc, m, np.where(np.arange(256) % 64 < 32, 10, 5))
    w = oracle.dequant(Q4_K, blk, 256, 1)[0]
    i = np.arange(256)
    q = np.where(i % 64 < 32, 10, 5)
    want = (0.5 * sc[i // 32] * q - 0.25 * m[i // 32]).astype(np.float32)
    assert np.array_equal(w, want)


def test_q6k_unit_scale_known_answer(oracle):
    # d = 1, scales 1: w = code - 32.  One planted code per position.
    for pos in (0, 1, 15, 16, 31, 32, 63, 64, 95, 96, 127, 128, 200, 255):
        codes = np.full(256, 32)
        codes[pos] = 32 + 7
        blk = encode_q6k(1.0, np.ones(16), codes)
        w = oracle.dequant(Q6_K, blk, 256, 1)[0]
        want = np.zeros(256, dtype=np.float32)
        want[pos] = 7.0
        assert np.array_equal(w, want), pos


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4k_encode_decode_round_trip(oracle, seed):
    rng = np.random.default_rng(seed)
    for _ in range(20):
        sc = rng.integers(0, 64, 8)
        m = rng.integers(0, 64, 8)
        codes = rng.integers(0, 16, 256)
        d, dmin = np.float16(rng.uniform(0, 0.05)), np.float16(rng.uniform(0, 0.05))
        blk = encode_q4k(float(d), float(dmin), sc, m, codes)
        w = oracle.dequant(Q4_K, blk, 256, 1)[0]
        i = np.arange(256)
        df, dminf = np.float32(d), np.float32(dmin)
        want = (df * sc[i // 32].astype(np.float32)) * codes.astype(np.float32) - dminf * m[i // 32].astype(np.float32)
        assert np.array_equal(w.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q6k_encode_decode_round_trip(oracle, seed):
    rng = np.random.default_rng(seed)
    for _ in range(20):
        scales = rng.integers(-128, 128, 16)
        codes = rng.integers(0, 64, 256)
        d = np.float16(rng.uniform(0, 0.05))
        blk = encode_q6k(float(d), scales, codes)
        w = oracle.dequant(Q6_K, blk, 256, 1)[0]
        i = np.arange(256)
        want = (np.float32(d) * scales[i // 16].astype(np.float32)) * (codes - 32).astype(np.float32)
        assert np.array_equal(w.view(np.uint32), want.astype(np.float32).view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_dequant_matches_ggml_loop(oracle, synth, qtype):
    # Random blocks, including full-range scale bytes and qh bits.
    n = 512
    blocks = synth.random_bytes(n * (144 if qtype == Q4_K else 210), 11, 3)
    # Keep d / dmin finite (random bytes can hold inf / nan halves).
    b = blocks.reshape(n, -1)
    hdr = slice(0, 4) if qtype == Q4_K else slice(208, 210)
    b[:, hdr] = synth.f64_to_f16_bits(np.abs(np.random.default_rng(5).normal(0, 0.02, (n, (hdr.stop - hdr.start) // 2)))
                                      ).view(np.uint8).reshape(n, -1)
    got = oracle.dequant(qtype, blocks, 256 * n, 1).reshape(-1)
    want = ggml_dequant_q4k(blocks) if qtype == Q4_K else ggml_dequant_q6k(blocks)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_every_fp16_scale_decodes_exactly(oracle):
    # One Q4_K block per finite fp16 d (subnormals included): sc = 63,
    # q = 15, dmin = 0 => w = d*945 exactly.  Q6_K: scale -128, code 0 =>
    # w = d*4096.
    bits = np.arange(65536, dtype=np.uint16)
    vals = bits.view(np.float16)
    finite = bits[np.isfinite(vals)]
    nq4 = finite.size
    q4 = np.zeros((nq4, 144), dtype=np.uint8)
    q4[:, 0:2] = finite.view(np.uint8).reshape(-1, 2)
    q4[:, 4:16] = pack_q4k_scales(np.full(8, 63), np.zeros(8, dtype=np.int64))
    q4[:, 16:] = 0xFF
    w = oracle.dequant(Q4_K, q4.reshape(-1), 256, nq4)[:, 0]
    want = finite.view(np.float16).astype(np.float32) * np.float32(945.0)
    assert np.array_equal(w.view(np.uint32), want.view(np.uint32))
    q6 = np.zeros((nq4, 210), dtype=np.uint8)
    q6[:, 192:208] = np.uint8(0x80)
    q6[:, 208:210] = finite.view(np.uint8).reshape(-1, 2)
    w6 = oracle.dequant(Q6_K, q6.reshape(-1), 256, nq4)[:, 0]
    want6 = finite.view(np.float16).astype(np.float32) * np.float32(4096.0)
    assert np.array_equal(w6.view(np.uint32), want6.view(np.uint32))


def test_embedding_is_row_gather(oracle, synth):
    w = synth.quant_matrix(Q6_K, 512, 10, 3, 1)
    rows = oracle.dequant(Q6_K, w, 512, 10)
    tokens = np.array([3, 0, 9, 3], dtype=np.int32)
    assert np.array_equal(oracle.embedding(Q6_K, w, tokens, 512), rows[tokens])
