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
    ws_bytes = qk.batch_workspace_bytes(cols, ntok)
    ws = t.empty(max(ws_bytes, 16), dtype=t.uint8, device="cuda")
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
    h = (wg / (1.0 + np.exp(-wg)) * wu).astype(np.float32)
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
    ws_bytes = qk.batch_workspace_bytes(dim, ntok)
    ws = t.empty(ws_bytes, dtype=t.uint8, device="cuda")
    xd = to_dev(t, x)
    qk.check(qk.lib().qk_gemv_multi_batched_f32(arr, 2, xd.data_ptr(), dim, dim, ntok, ws.data_ptr(), ws_bytes, None),
             "multi batched")
    t.cuda.synchronize()
    want_g = oracle.gemv_f64(Q4_K, wg, x, dim, hidden)
    want_u = oracle.gemv_f64(Q6_K, wu, x, dim, hidden)
    for k in range(ntok):
        assert rel_l2(g[k].cpu().numpy(), want_g[k]) < TOL
        assert rel_l2(u[k].cpu().numpy(), want_u[k]) < TOL
