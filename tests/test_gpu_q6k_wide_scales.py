"""Q6_K blocks with sub-block scales over the whole int8 range.

The workloads draw Q6_K scales from -32..31, but llama.cpp's Q6_K quantizer
maps each block's largest sub-block to about +-128, so real GGUF tensors
carry scales up to 127 and -128 in every block.  The matrix-core path holds
s * (code - 32) in fp16, exact only while |s| <= 62; wider blocks take the
exact W_a + W_b decode.  Every GEMV form is checked on such blocks against
the fp64 oracle (rel-L2 <= 1e-5 per token), on both Q6_K layouts, and at
the boundary scales 62 / 63 / 64 / -128 where the narrow decode stops being
exact."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
TOL = 1e-5
LDXQ, LDSCALE = 8192, 256


def wide_q6k(synth, cols, rows, seed, planted=None):
    """A Q6_K matrix whose 16 int8 scales per block are uniform in -128..127,
    with scale 0 of every block forced to -128 (llama.cpp's extreme), or all
    sixteen set to `planted`."""
    nb = cols // 256
    w = synth.quant_matrix(Q6_K, cols, rows, seed, 1).reshape(rows * nb, 210).copy()
    if planted is None:
        sc = synth.uniform_i32(rows * nb * 16, seed, 2, -128, 127).astype(np.int8).reshape(rows * nb, 16)
        sc[:, 0] = -128
    else:
        sc = np.full((rows * nb, 16), planted, dtype=np.int8)
    w[:, 192:208] = sc.view(np.uint8)
    return w.reshape(-1)


def batched(qk, t, tensor, x, cols, rows):
    ntok = x.shape[0]
    nws = qk.batch_workspace_bytes(cols, rows, ntok)
    ws = t.empty(max(nws, 256), dtype=t.uint8, device="cuda")
    y = t.full((ntok, rows), float("nan"), device="cuda")
    qk.batch_matvec(tensor, to_dev(t, x), y, cols, rows, ntok, ws, nws)
    t.cuda.synchronize()
    return y.cpu().numpy()


def layouts(qk, t, w, cols, rows):
    g = qk.Tensor((cols, rows), Q6_K, to_dev(t, w))
    s = qk.split_q6k(g)
    t.cuda.synchronize()
    return {"gguf": g, "split": s}


@pytest.mark.parametrize("ntok", [8, 32, 100, 256])
@pytest.mark.parametrize("cols,rows", [(2048, 600), (8192, 300)])
def test_batched_f32_wide_scales(qk, torch_gpu, oracle, synth, ntok, cols, rows):
    t = torch_gpu
    w = wide_q6k(synth, cols, rows, 90 + ntok)
    x = synth.normal_f32(ntok * cols, 91, ntok).reshape(ntok, cols)
    want = oracle.gemv_f64(Q6_K, w, x, cols, rows)
    for name, tensor in layouts(qk, t, w, cols, rows).items():
        got = batched(qk, t, tensor, x, cols, rows)
        assert np.isfinite(got).all(), name
        for k in range(ntok):
            assert rel_l2(got[k], want[k]) < TOL, (name, k)


@pytest.mark.parametrize("planted", [62, 63, 64, -62, -63, -64, 127, -128])
def test_batched_f32_boundary_scales(qk, torch_gpu, oracle, synth, planted):
    t = torch_gpu
    cols, rows, ntok = 2048, 256, 32
    w = wide_q6k(synth, cols, rows, 92, planted=planted)
    x = synth.normal_f32(ntok * cols, 93, 1).reshape(ntok, cols)
    got = batched(qk, t, qk.Tensor((cols, rows), Q6_K, to_dev(t, w)), x, cols, rows)
    want = oracle.gemv_f64(Q6_K, w, x, cols, rows)
    for k in range(ntok):
        assert rel_l2(got[k], want[k]) < TOL, k


def test_fused_qkv_with_wide_v(qk, torch_gpu, oracle, workloads, synth):
    """Q4_K q / k and a wide-scale Q6_K v in one matrix-core launch."""
    t = torch_gpu
    dim, kv, ntok = 2048, 512, 40
    wq, _ = workloads.gemv_case(Q4_K, dim, dim, seed=94)
    wk, _ = workloads.gemv_case(Q4_K, dim, kv, seed=95)
    wv = wide_q6k(synth, dim, kv, 96)
    x = synth.normal_f32(ntok * dim, 97, 1).reshape(ntok, dim)
    mats = [(Q4_K, wq, dim), (Q4_K, wk, kv), (Q6_K, wv, kv)]
    arr = (qk.qk_matrix * 3)()
    keep, ys = [], []
    for i, (qt, w, rows) in enumerate(mats):
        wd = to_dev(t, w)
        y = t.full((ntok, rows), float("nan"), device="cuda")
        keep.append(wd)
        ys.append(y)
        arr[i].type, arr[i].rows, arr[i].w, arr[i].y = qt, rows, wd.data_ptr(), y.data_ptr()
    nws = qk.batch_workspace_bytes(dim, dim + 2 * kv, ntok)
    ws = t.empty(max(nws, 256), dtype=t.uint8, device="cuda")
    xd = to_dev(t, x)
    qk.check(qk.lib().qk_gemv_multi_batched_f32(arr, 3, xd.data_ptr(), dim, dim, ntok, ws.data_ptr(), nws, None),
             "multi batched")
    t.cuda.synchronize()
    for y, (qt, w, rows) in zip(ys, mats):
        got = y.cpu().numpy()
        want = oracle.gemv_f64(qt, w, x, dim, rows)
        for k in range(ntok):
            assert rel_l2(got[k], want[k]) < TOL, (qt, k)


@pytest.mark.parametrize("ntok", [8, 32])
def test_batched_int8_wide_scales(qk, torch_gpu, oracle, synth, ntok):
    t = torch_gpu
    L = qk.lib()
    cols, rows = 2048, 500
    w = wide_q6k(synth, cols, rows, 98)
    x = synth.normal_f32(ntok * cols, 99, 1).reshape(ntok, cols)
    xq = np.zeros((ntok, LDXQ), dtype=np.int8)
    xs = np.zeros((ntok, LDSCALE), dtype=np.float32)
    for k in range(ntok):
        xq[k, :cols], xs[k, : cols // 32] = oracle.quantize_x32(x[k])
    for name, tensor in layouts(qk, t, w, cols, rows).items():
        xqd, xsd = to_dev(t, xq), to_dev(t, xs)
        y = t.full((ntok, rows), float("nan"), device="cuda")
        nws = L.qk_gemv_batched_i8_workspace_bytes(cols, rows, ntok)
        ws = t.empty(max(nws, 256), dtype=t.uint8, device="cuda")
        qk.check(L.qk_gemv_batched_i8(tensor.type, tensor.gpu, xqd.data_ptr(), LDXQ, xsd.data_ptr(), LDSCALE,
                                      y.data_ptr(), rows, cols, rows, ntok, ws.data_ptr(), nws, None),
                 "batched INT8 GEMV")
        t.cuda.synchronize()
        got = y.cpu().numpy()
        for k in range(ntok):
            want = oracle.gemv_i8_f64(Q6_K, w, xq[k, :cols], xs[k, : cols // 32], cols, rows)
            assert rel_l2(got[k], want) < TOL, (name, k)


def test_batch1_f32_and_int8_wide_scales(qk, torch_gpu, oracle, synth):
    """The one-token kernels take the scales in fp32: checked on the same
    blocks so every GEMV form is covered."""
    t = torch_gpu
    cols, rows = 2048, 4096
    w = wide_q6k(synth, cols, rows, 100)
    x = synth.normal_f32(cols, 101, 1)
    xq, xs = oracle.quantize_x32(x)
    want = oracle.gemv_f64(Q6_K, w, x[None, :], cols, rows)[0]
    want8 = oracle.gemv_i8_f64(Q6_K, w, xq, xs, cols, rows)
    for name, tensor in layouts(qk, t, w, cols, rows).items():
        y = t.empty(rows, device="cuda")
        qk.matvec(tensor, to_dev(t, x), y, cols, rows)
        t.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), want) < TOL, name
        qk.matvec_i8(tensor, to_dev(t, xq), to_dev(t, xs), y, cols, rows)
        t.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), want8) < TOL, name
