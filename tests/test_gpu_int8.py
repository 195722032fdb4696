"""GPU INT8 mode (the reference's default DP4A path): the activation quantizer
is bit-exact against the oracle's closed form; the INT8 GEMV (exact integer
dots, fp32 combine) is within rel-L2 1e-5 of the oracle's fp64 combine of the
same integer dots."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14


@pytest.mark.parametrize("cols", [32, 100, 2048, 3072, 8192])
def test_quantize_bit_exact(qk, torch_gpu, oracle, synth, cols):
    t = torch_gpu
    x = synth.normal_f32(cols, 61, cols) * np.float32(3.0)
    x[: min(32, cols)] = 0.0                       # an all-zero group
    if cols >= 70:
        x[32] = 127.0
        x[33:38] = [0.5, 1.5, 2.5, -0.5, -1.5]     # round-half-even ties
    xq = t.zeros(cols, dtype=t.int8, device="cuda")
    xs = t.zeros((cols + 31) // 32, dtype=t.float32, device="cuda")
    qk.quantize(to_dev(t, x), xq, xs, cols)
    t.cuda.synchronize()
    wq, ws = oracle.quantize_x32(x)
    assert np.array_equal(xq.cpu().numpy(), wq)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), ws.view(np.uint32))


def test_quantize_batched_strides(qk, torch_gpu, oracle, synth):
    # The reference's batch layout: xq stride 8192 bytes, xscale stride 256.
    t = torch_gpu
    cols, ntok = 3072, 5
    x = synth.normal_f32(ntok * cols, 62, 1).reshape(ntok, cols)
    xq = t.zeros((ntok, 8192), dtype=t.int8, device="cuda")
    xs = t.zeros((ntok, 256), dtype=t.float32, device="cuda")
    qk.quantize(to_dev(t, x), xq, xs, cols, n_tokens=ntok, ldx=cols, ldxq=8192, ldscale=256)
    t.cuda.synchronize()
    for k in range(ntok):
        wq, ws = oracle.quantize_x32(x[k])
        assert np.array_equal(xq[k, :cols].cpu().numpy(), wq)
        assert np.array_equal(xs[k, : cols // 32].cpu().numpy(), ws)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("cols,rows", [(2048, 2048), (3072, 1000), (8192, 2048), (256, 33), (4352, 65)])
def test_gemv_i8_matches_integer_oracle(qk, torch_gpu, oracle, workloads, qtype, cols, rows):
    t = torch_gpu
    w, x = workloads.gemv_case(qtype, cols, rows, seed=63)
    xq, xs = oracle.quantize_x32(x)
    y = t.empty(rows, device="cuda")
    qk.matvec_i8(qk.Tensor((cols, rows), qtype, to_dev(t, w)), to_dev(t, xq), to_dev(t, xs), y, cols, rows)
    t.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), oracle.gemv_i8_f64(qtype, w, xq, xs, cols, rows)) < 1e-5


def test_gemv_i8_multi_token(qk, torch_gpu, oracle, workloads):
    t = torch_gpu
    cols, rows, ntok = 2048, 512, 4
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=64, n_tokens=ntok)
    xq = np.zeros((ntok, 8192), dtype=np.int8)
    xs = np.zeros((ntok, 256), dtype=np.float32)
    for k in range(ntok):
        xq[k, :cols], xs[k, : cols // 32] = oracle.quantize_x32(x[k])
    y = t.empty((ntok, rows), device="cuda")
    qk.matvec_i8(qk.Tensor((cols, rows), Q6_K, to_dev(t, w)), to_dev(t, xq), to_dev(t, xs), y, cols, rows,
                 n_tokens=ntok, ldxq=8192, ldscale=256, ldy=rows)
    t.cuda.synchronize()
    for k in range(ntok):
        want = oracle.gemv_i8_f64(Q6_K, w, xq[k, :cols], xs[k, : cols // 32], cols, rows)
        assert rel_l2(y[k].cpu().numpy(), want) < 1e-5


# Long INT8 launches over the split Q6_K layout (at least 32768 wave tiles,
# one matrix of whole tiles) run the LDS-staged kernel, whose weights reach
# the lanes through global -> LDS copies; short launches run the register
# kernel.  Each row's arithmetic is the same in both, so the long launch
# equals short launches over row slices bit for bit, and both are within
# rel-L2 1e-5 of the oracle's fp64 combine of the same integer dots.
@pytest.mark.parametrize("cols,rows,ntok", [(2048, 128256, 1), (2048, 32768, 2), (1024, 131072, 1)])
def test_gemv_i8_split_long_launch(qk, torch_gpu, oracle, workloads, cols, rows, ntok):
    t = torch_gpu
    Q6_K_SPLIT = qk.Q6_K_SPLIT
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=65, n_tokens=ntok)
    x = x.reshape(ntok, cols)
    xq = np.zeros((ntok, cols), dtype=np.int8)
    xs = np.zeros((ntok, cols // 32), dtype=np.float32)
    for k in range(ntok):
        xq[k], xs[k] = oracle.quantize_x32(x[k])
    split = qk.split_q6k(qk.Tensor((cols, rows), Q6_K, to_dev(t, w)))
    xq_d, xs_d = to_dev(t, xq), to_dev(t, xs)
    y = t.full((ntok, rows), float("nan"), device="cuda")
    qk.matvec_i8(split, xq_d, xs_d, y, cols, rows, n_tokens=ntok, ldxq=cols, ldscale=cols // 32, ldy=rows)
    t.cuda.synchronize()
    got = y.cpu().numpy()
    for k in range(ntok):
        assert rel_l2(got[k], oracle.gemv_i8_f64(Q6_K, w, xq[k], xs[k], cols, rows)) < 1e-5
    rb = qk.tensor_bytes(Q6_K_SPLIT, cols, 1)
    n = 4096
    for r0 in (0, rows // 2 - 7 * 16, rows - n):
        part = qk.Tensor((cols, n), Q6_K_SPLIT, split.data[r0 * rb:(r0 + n) * rb])
        ys = t.full((ntok, n), float("nan"), device="cuda")
        qk.matvec_i8(part, xq_d, xs_d, ys, cols, n, n_tokens=ntok, ldxq=cols, ldscale=cols // 32, ldy=n)
        t.cuda.synchronize()
        assert np.array_equal(ys.cpu().numpy().view(np.uint32), got[:, r0:r0 + n].view(np.uint32)), r0
