"""Pins the oracle's INT8 mode (qk_oracle.c restating quantize_x32_cuda,
dot_q4_block_dp4a and dot_q6_block_dp4a, inferencer.cu:520-556, 613-643):
the quantizer against its numpy closed form (bit-exact), the integer
sub-block dots against numpy int64 dots of codes extracted GGML-loop style,
and the float combine against a numpy float64 combine."""
import numpy as np
import pytest

from conftest import rel_l2

Q4_K, Q6_K = 12, 14


def quantize_closed_form(x: np.ndarray):
    x = x.astype(np.float32)
    n = x.size
    groups = (n + 31) // 32
    xs = np.empty(groups, dtype=np.float32)
    xq = np.empty(n, dtype=np.int8)
    for g in range(groups):
        v = x[g * 32:(g + 1) * 32]
        amax = np.max(np.abs(v))
        scale = np.float32(amax) / np.float32(127.0) if amax > 0 else np.float32(1.0)
        xs[g] = scale
        xq[g * 32:(g + 1) * 32] = np.clip(np.rint(v / scale), -127, 127).astype(np.int8)
    return xq, xs


def q4k_codes(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 144)
    q = b[:, 16:].astype(np.int64)
    out = np.empty((b.shape[0], 256), dtype=np.int64)
    for chunk in range(4):
        qq = q[:, chunk * 32:(chunk + 1) * 32]
        out[:, chunk * 64: chunk * 64 + 32] = qq & 0xF
        out[:, chunk * 64 + 32: chunk * 64 + 64] = qq >> 4
    return out


def q6k_codes(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 210)
    out = np.empty((b.shape[0], 256), dtype=np.int64)
    for n in range(2):
        ql = b[:, 64 * n: 64 * n + 64].astype(np.int64)
        qh = b[:, 128 + 32 * n: 128 + 32 * n + 32].astype(np.int64)
        out[:, 128 * n + 0: 128 * n + 32] = (ql[:, :32] & 0xF) | (((qh >> 0) & 3) << 4)
        out[:, 128 * n + 32: 128 * n + 64] = (ql[:, 32:] & 0xF) | (((qh >> 2) & 3) << 4)
        out[:, 128 * n + 64: 128 * n + 96] = (ql[:, :32] >> 4) | (((qh >> 4) & 3) << 4)
        out[:, 128 * n + 96: 128 * n + 128] = (ql[:, 32:] >> 4) | (((qh >> 6) & 3) << 4)
    return out - 32


def test_quantize_matches_closed_form(oracle, synth):
    x = synth.normal_f32(4096, 21, 1)
    x[100:132] = 0.0                       # an all-zero group: scale 1
    x[300] = 1e-30                         # tiny values
    x[64:96] = 0.0                         # amax 127 => scale exactly 1,
    x[64] = 127.0                          # so the next values are exact
    x[65:70] = [0.5, 1.5, 2.5, -0.5, -1.5]  # .5 ties: half to even
    xq, xs = oracle.quantize_x32(x)
    wq, ws = quantize_closed_form(x)
    assert np.array_equal(xq, wq)
    assert np.array_equal(xs.view(np.uint32), ws.view(np.uint32))


def test_quantize_ragged_tail(oracle, synth):
    x = synth.normal_f32(100, 22, 1)
    xq, xs = oracle.quantize_x32(x)
    wq, ws = quantize_closed_form(x)
    assert np.array_equal(xq, wq) and np.array_equal(xs, ws)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_subblock_dots_exact(oracle, workloads, qtype):
    cols, rows = 1024, 24
    w, x = workloads.gemv_case(qtype, cols, rows, seed=23)
    xq, xs = oracle.quantize_x32(x)
    dots, xsums = oracle.subblock_dots_i8(qtype, w, xq, cols, rows)
    codes = (q4k_codes(w) if qtype == Q4_K else q6k_codes(w)).reshape(rows, cols)
    sub = 32 if qtype == Q4_K else 16
    prod = (codes * xq.astype(np.int64)[None, :]).reshape(rows, cols // sub, sub).sum(axis=2)
    assert np.array_equal(dots, prod)
    assert np.array_equal(xsums, xq.astype(np.int64).reshape(-1, sub).sum(axis=1))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_gemv_i8_combine(oracle, workloads, qtype):
    cols, rows = 1024, 24
    w, x = workloads.gemv_case(qtype, cols, rows, seed=24)
    xq, xs = oracle.quantize_x32(x)
    got = oracle.gemv_i8_f64(qtype, w, xq, xs, cols, rows)
    b = w.reshape(rows, cols // 256, -1)
    codes = (q4k_codes(w) if qtype == Q4_K else q6k_codes(w)).reshape(rows, cols)
    xqi = xq.astype(np.float64)
    want = np.zeros(rows)
    for r in range(rows):
        for blk in range(cols // 256):
            block = b[r, blk]
            c = codes[r, blk * 256:(blk + 1) * 256].astype(np.float64)
            xv = xqi[blk * 256:(blk + 1) * 256]
            if qtype == Q4_K:
                d = float(block[0:2].copy().view(np.float16)[0])
                dmin = float(block[2:4].copy().view(np.float16)[0])
                for s in range(8):
                    sc, m = oracle.scale_min(block[4:16], s)
                    dot = c[s * 32:(s + 1) * 32] @ xv[s * 32:(s + 1) * 32]
                    sm = xv[s * 32:(s + 1) * 32].sum()
                    want[r] += (d * sc * dot - dmin * m * sm) * float(xs[blk * 8 + s])
            else:
                d = float(block[208:210].copy().view(np.float16)[0])
                scales = block[192:208].copy().view(np.int8).astype(np.float64)
                for j in range(16):
                    dot = c[j * 16:(j + 1) * 16] @ xv[j * 16:(j + 1) * 16]
                    want[r] += d * scales[j] * dot * float(xs[blk * 8 + j // 2])
    assert rel_l2(got, want) < 1e-13
    # INT8 mode approximates the FP32 GEMV to the activation rounding.
    assert rel_l2(got, oracle.gemv_f64(qtype, w, x, cols, rows)) < 2e-2
