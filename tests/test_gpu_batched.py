"""GPU multi-token FP32 GEMV (qk_gemv_batched_f32, qk_gemv_multi_batched_f32)
against the fp64 oracle, token by token: rel-L2 <= 1e-5 per token."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
TOL = 1e-5


def run_batched(qk, t, qtype, w, x, cols, rows):
    ntok = x.shape[0]
    ws_bytes = qk.batch_workspace_bytes(cols, rows, ntok)
    ws = t.empty(max(ws_bytes, 256), dtype=t.uint8, device="cuda")
    y = t.full((ntok, rows), float("nan"), device="cuda")
    qk.batch_matvec(qk.Tensor((cols, rows), qtype, to_dev(t, w)), to_dev(t, x), y, cols, rows, ntok, ws, ws_bytes)
    t.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("ntok", [1, 2, 5, 16, 33])
def test_batched_tokens(qk, torch_gpu, oracle, workloads, qtype, ntok):
    cols, rows = 2048, 777
    w, x = workloads.gemv_case(qtype, cols, rows, seed=70 + ntok, n_tokens=max(ntok, 2))
    x = x[:ntok]
    y = run_batched(qk, torch_gpu, qtype, w, x, cols, rows)
    want = oracle.gemv_f64(qtype, w, x, cols, rows)
    for k in range(ntok):
        assert rel_l2(y[k], want[k]) < TOL, k


def test_batched_empty_is_noop(qk, torch_gpu, workloads):
    t = torch_gpu
    w, _ = workloads.gemv_case(Q4_K, 512, 8, seed=79)
    y = t.full((8,), 5.0, device="cuda")
    x = t.zeros(512, device="cuda")
    qk.batch_matvec(qk.Tensor((512, 8), Q4_K, to_dev(t, w)), x, y, 512, 8, 0)
    t.cuda.synchronize()
    assert t.all(y == 5.0)


def test_ffn_3b_ragged_batch(qk, torch_gpu, oracle, workloads):
    """32 decode tokens of 32 sequences through the Llama-3.2-3B FFN shapes."""
    t = torch_gpu
    c = workloads.ffn_3b_ragged()
    x = c["x"]
    dim, hidden = c["cfg"]["dim"], c["cfg"]["hidden"]
    yg = run_batched(qk, t, Q4_K, c["gate"], x, dim, hidden)
    yu = run_batched(qk, t, Q4_K, c["up"], x, dim, hidden)
    wg = oracle.gemv_f64(Q4_K, c["gate"], x, dim, hidden)
    wu = oracle.gemv_f64(Q4_K, c["up"], x, dim, hidden)
    for k in range(x.shape[0]):
        assert rel_l2(yg[k], wg[k]) < TOL and rel_l2(yu[k], wu[k]) < TOL
    h = (wg / (1.0 + np.exp(-np.clip(wg, -80, 80))) * wu).astype(np.float32)
    yd = run_batched(qk, t, Q6_K, c["down"], h, hidden, dim)
    wd = oracle.gemv_f64(Q6_K, c["down"], h, hidden, dim)
    for k in range(x.shape[0]):
        assert rel_l2(yd[k], wd[k]) < TOL


def test_multi_batched_gate_up(qk, torch_gpu, oracle, workloads):
    t = torch_gpu
    dim, hidden, ntok = 2048, 1024, 6
    wg, x = workloads.gemv_case(Q4_K, dim, hidden, seed=80, n_tokens=ntok)
    wu, _ = workloads.gemv_case(Q6_K, dim, hidden, seed=81)
    g = t.empty((ntok, hidden), device="cuda")
    u = t.empty((ntok, hidden), device="cuda")
    arr = (qk.qk_matrix * 2)()
    wgd, wud = to_dev(t, wg), to_dev(t, wu)
    arr[0].type, arr[0].rows, arr[0].w, arr[0].y = Q4_K, hidden, wgd.data_ptr(), g.data_ptr()
    arr[1].type, arr[1].rows, arr[1].w, arr[1].y = Q6_K, hidden, wud.data_ptr(), u.data_ptr()
    ws_bytes = qk.batch_workspace_bytes(dim, 2 * hidden, ntok)
    ws = t.empty(max(ws_bytes, 256), dtype=t.uint8, device="cuda")
    xd = to_dev(t, x)
    qk.check(qk.lib().qk_gemv_multi_batched_f32(arr, 2, xd.data_ptr(), dim, dim, ntok, ws.data_ptr(), ws_bytes, None),
             "multi batched")
    t.cuda.synchronize()
    want_g = oracle.gemv_f64(Q4_K, wg, x, dim, hidden)
    want_u = oracle.gemv_f64(Q6_K, wu, x, dim, hidden)
    for k in range(ntok):
        assert rel_l2(g[k].cpu().numpy(), want_g[k]) < TOL
        assert rel_l2(u[k].cpu().numpy(), want_u[k]) < TOL


# ------------------------------------------------ matrix-core path (T >= 8) --

def _fused(qk, t, mats, x, cols, ntok):
    """qk_gemv_multi_batched_f32 over [(type, w, rows)]; returns the outputs."""
    arr = (qk.qk_matrix * len(mats))()
    keep, outs = [], []
    for i, (qtype, w, rows) in enumerate(mats):
        wd = to_dev(t, w)
        y = t.full((ntok, rows), float("nan"), device="cuda")
        keep.append(wd)
        outs.append(y)
        arr[i].type, arr[i].rows, arr[i].w, arr[i].y = qtype, rows, wd.data_ptr(), y.data_ptr()
    ws_bytes = qk.batch_workspace_bytes(cols, sum(r for _, _, r in mats), ntok)
    ws = t.empty(max(ws_bytes, 256), dtype=t.uint8, device="cuda")
    xd = to_dev(t, x)
    qk.check(qk.lib().qk_gemv_multi_batched_f32(arr, len(mats), xd.data_ptr(), cols, cols, ntok, ws.data_ptr(),
                                                ws_bytes, None), "multi batched")
    t.cuda.synchronize()
    return [y.cpu().numpy() for y in outs]


@pytest.mark.parametrize("ntok", [8, 40, 256])
def test_mfma_fused_qkv_mixed_types(qk, torch_gpu, oracle, workloads, ntok):
    """Llama-3.2-1B QKV: Q4_K q/k, Q6_K v in one launch (mixed-type kernel)."""
    dim, kv = 2048, 512
    wq, x = workloads.gemv_case(Q4_K, dim, dim, seed=90, n_tokens=ntok)
    wk, _ = workloads.gemv_case(Q4_K, dim, kv, seed=91)
    wv, _ = workloads.gemv_case(Q6_K, dim, kv, seed=92)
    outs = _fused(qk, torch_gpu, [(Q4_K, wq, dim), (Q4_K, wk, kv), (Q6_K, wv, kv)], x, dim, ntok)
    for (qtype, w, rows), y in zip([(Q4_K, wq, dim), (Q4_K, wk, kv), (Q6_K, wv, kv)], outs):
        want = oracle.gemv_f64(qtype, w, x, dim, rows)
        for k in range(ntok):
            assert rel_l2(y[k], want[k]) < TOL, (qtype, rows, k)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("cols,rows,ntok", [(8192, 300, 8), (3072, 130, 64), (256, 64, 9), (2048, 700, 256),
                                             (8192, 300, 100), (3072, 520, 32)])
def test_mfma_shapes(qk, torch_gpu, oracle, workloads, qtype, cols, rows, ntok):
    w, x = workloads.gemv_case(qtype, cols, rows, seed=93 + ntok, n_tokens=ntok)
    y = run_batched(qk, torch_gpu, qtype, w, x, cols, rows)
    want = oracle.gemv_f64(qtype, w, x, cols, rows)
    for k in range(ntok):
        assert rel_l2(y[k], want[k]) < TOL, k


def test_mfma_scaled_and_zero_tokens(qk, torch_gpu, oracle, workloads):
    """Per-(token, block) scaling: tokens of very different magnitudes, an
    all-zero token (exact zeros) and a token with one huge outlier."""
    cols, rows, ntok = 2048, 256, 12
    w, x = workloads.gemv_case(Q4_K, cols, rows, seed=97, n_tokens=ntok)
    x = x.copy()
    x[1] *= 1e-30
    x[2] *= 1e30
    x[3] = 0.0
    x[4, 77] = 1e6
    x[5, :256] = 0.0
    y = run_batched(qk, torch_gpu, Q4_K, w, x, cols, rows)
    want = oracle.gemv_f64(Q4_K, w, x, cols, rows)
    assert np.all(y[3] == 0.0)
    for k in range(ntok):
        if k != 3:
            assert rel_l2(y[k], want[k]) < TOL, k


def test_mfma_nonfinite_token_is_isolated(qk, torch_gpu, oracle, workloads):
    cols, rows, ntok = 512, 64, 9
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=98, n_tokens=ntok)
    x = x.copy()
    x[4, 300] = np.inf
    y = run_batched(qk, torch_gpu, Q6_K, w, x, cols, rows)
    want = oracle.gemv_f64(Q6_K, w, x, cols, rows)
    assert np.all(np.isnan(y[4]))
    for k in range(ntok):
        if k != 4:
            assert rel_l2(y[k], want[k]) < TOL, k


def test_mfma_deterministic(qk, torch_gpu, workloads):
    cols, rows, ntok = 8192, 200, 32
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=99, n_tokens=ntok)
    a = run_batched(qk, torch_gpu, Q6_K, w, x, cols, rows)
    b = run_batched(qk, torch_gpu, Q6_K, w, x, cols, rows)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_mfma_needs_workspace(qk, torch_gpu, workloads):
    t = torch_gpu
    cols, rows, ntok = 2048, 64, 8
    w, x = workloads.gemv_case(Q4_K, cols, rows, seed=100, n_tokens=ntok)
    need = qk.batch_workspace_bytes(cols, rows, ntok)
    records = 8 * 33920            # one 32-token tile of packed activations per 256 columns
    assert need > records          # 64 rows x 8 blocks: the blocks split over several workgroups
    ws = t.empty(need, dtype=t.uint8, device="cuda")
    y = t.empty((ntok, rows), device="cuda")
    with pytest.raises(qk.QKError) as e:
        qk.batch_matvec(qk.Tensor((cols, rows), Q4_K, to_dev(t, w)), to_dev(t, x), y, cols, rows, ntok, ws,
                        records - 16)
    assert e.value.status == qk.QK_ERR_INVALID_ARG


def run_ffn(qk, t, ws_, types, x, dim, hidden, y0=None, accumulate=False, alias=False):
    """qk_ffn_batched_f32 over host weights; y starts as y0 (NaN if None);
    alias: y is x itself (the residual add in place)."""
    ntok = x.shape[0]
    n = qk.lib().qk_ffn_batched_workspace_bytes(dim, hidden, ntok)
    ws = t.empty(max(n, 256), dtype=t.uint8, device="cuda")
    gd, ud, dd = (to_dev(t, w) for w in ws_)
    xd = to_dev(t, x)
    y = xd if alias else (to_dev(t, y0) if y0 is not None else t.full((ntok, dim), float("nan"), device="cuda"))
    qk.check(qk.lib().qk_ffn_batched_f32(types[0], gd.data_ptr(), types[1], ud.data_ptr(), types[2], dd.data_ptr(),
                                         xd.data_ptr(), dim, y.data_ptr(), dim, dim, hidden, ntok, int(accumulate),
                                         ws.data_ptr(), n, None), "ffn")
    t.cuda.synchronize()
    return y.cpu().numpy()


def ffn_f64(oracle, ws_, types, x, dim, hidden):
    g = oracle.gemv_f64(types[0], ws_[0], x, dim, hidden)
    u = oracle.gemv_f64(types[1], ws_[1], x, dim, hidden)
    h = g / (1.0 + np.exp(-np.clip(g, -80, 80))) * u
    return oracle.gemv_f64(types[2], ws_[2], h.astype(np.float32), hidden, dim)


@pytest.mark.parametrize("ntok", [1, 5, 8, 32, 33, 100])
def test_ffn_entry(qk, torch_gpu, oracle, workloads, ntok):
    """The FFN in one call (chained SiLU * up records from 8 tokens on, the
    GEMV pair below) against gate / up / SiLU / down in fp64."""
    dim, hidden = 1024, 2048
    types = (Q4_K, Q4_K, Q6_K)
    gw, x = workloads.gemv_case(Q4_K, dim, hidden, seed=90 + ntok, n_tokens=max(ntok, 2))
    x = x[:ntok]
    uw, _ = workloads.gemv_case(Q4_K, dim, hidden, seed=91 + ntok)
    dw, _ = workloads.gemv_case(Q6_K, hidden, dim, seed=92 + ntok)
    y = run_ffn(qk, torch_gpu, (gw, uw, dw), types, x, dim, hidden)
    want = ffn_f64(oracle, (gw, uw, dw), types, x, dim, hidden)
    for k in range(ntok):
        assert rel_l2(y[k], want[k]) < TOL, k


@pytest.mark.parametrize("ntok", [4, 32])
def test_ffn_entry_residual_and_types(qk, torch_gpu, oracle, workloads, synth, ntok):
    """accumulate adds into y, in place over x too; Q6_K gate / up, a split
    Q6_K down."""
    t = torch_gpu
    dim, hidden = 512, 1536
    gw, x = workloads.gemv_case(Q6_K, dim, hidden, seed=95, n_tokens=ntok)
    uw, _ = workloads.gemv_case(Q4_K, dim, hidden, seed=96)
    dw, _ = workloads.gemv_case(Q6_K, hidden, dim, seed=97)
    want = ffn_f64(oracle, (gw, uw, dw), (Q6_K, Q4_K, Q6_K), x, dim, hidden)
    split = qk.split_q6k(qk.Tensor((hidden, dim), Q6_K, to_dev(t, dw)))
    dws = split.data.cpu().numpy()
    y0 = synth.normal_f32(ntok * dim, 98, 1).reshape(ntok, dim)
    for types, dwk in (((Q6_K, Q4_K, Q6_K), dw), ((Q6_K, Q4_K, qk.Q6_K_SPLIT), dws)):
        y = run_ffn(qk, t, (gw, uw, dwk), types, x, dim, hidden, y0=y0, accumulate=True)
        for k in range(ntok):
            assert rel_l2(y[k] - y0[k], want[k]) < TOL, (types, k)
        y = run_ffn(qk, t, (gw, uw, dwk), types, x, dim, hidden, accumulate=True, alias=True)
        for k in range(ntok):
            assert rel_l2(y[k] - x[k], want[k]) < TOL, (types, k)


@pytest.mark.parametrize("down_layout", ["gguf", "split"])
def test_ffn_entry_3b_shape(qk, torch_gpu, oracle, workloads, down_layout):
    """The FFN call bench.py times: Llama-3.2-3B shapes (gate / up 8192 x 3072,
    12 blocks a row; down 3072 x 8192, 32 blocks a row) on the seed-3
    workload's 32 decode tokens, down in the GGUF and in the split Q6_K
    layout, against gate / up / SiLU / down in fp64."""
    t = torch_gpu
    c = workloads.ffn_3b_ragged()
    dim, hidden = c["cfg"]["dim"], c["cfg"]["hidden"]
    dw, dtype = c["down"], Q6_K
    if down_layout == "split":
        dw = qk.split_q6k(qk.Tensor((hidden, dim), Q6_K, to_dev(t, c["down"]))).data.cpu().numpy()
        dtype = qk.Q6_K_SPLIT
    want = ffn_f64(oracle, (c["gate"], c["up"], c["down"]), (Q4_K, Q4_K, Q6_K), c["x"], dim, hidden)
    y = run_ffn(qk, t, (c["gate"], c["up"], dw), (Q4_K, Q4_K, dtype), c["x"], dim, hidden)
    errs = [rel_l2(y[k], want[k]) for k in range(c["x"].shape[0])]
    print(f"3B FFN, 32 tokens, {down_layout} down: worst rel-L2 {max(errs):.2e}", flush=True)
    assert max(errs) < TOL
