"""The LM head with its greedy pick folded into the GEMV epilogue
(qk_gemv_argmax_f32; argmax_blocks_cuda / argmax_final_cuda,
inferencer.cu:1063-1099, 1523-1526): y is bit-identical to qk_gemv_f32 and
the token is the lowest index among the maxima of that y.  Exact ties are
planted by copying a row's bytes (identical rows give identical sums); a
NaN row (fp16 d = NaN) must never win."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K, Q6_K_SPLIT = 12, 14, 114


def _run(qk, t, qtype, w, x, cols, rows, split=False):
    wd = to_dev(t, w)
    T = qk.Tensor((cols, rows), qtype, wd)
    if split:
        T = qk.split_q6k(T)
    xd = to_dev(t, x)
    y = t.empty(rows, device="cuda")
    y0 = t.empty(rows, device="cuda")
    tok = t.full((1,), -7, dtype=t.int32, device="cuda")
    ws = t.empty(qk.lib().qk_gemv_argmax_workspace_bytes(), dtype=t.uint8, device="cuda")
    qk.matvec_argmax(T, xd, y, tok, ws)
    qk.matvec(T, xd, y0, cols, rows)
    t.cuda.synchronize()
    yv = y.cpu().numpy()
    assert np.array_equal(yv.view(np.uint32), y0.cpu().numpy().view(np.uint32))
    return yv, int(tok.cpu().item())


def _lowest_max(y):
    v = np.where(np.isnan(y), -np.inf, y)
    return int(np.argmax(v))          # numpy keeps the first of equal maxima


@pytest.mark.parametrize("qtype,cols,rows,split", [
    (Q6_K, 2048, 128256, True),      # the tied LM head, split layout (gemv_wave, long launch)
    (Q6_K, 2048, 128256, False),
    (Q4_K, 2048, 1000, False),
    (Q6_K, 3072, 5003, False),       # gemv_split, C = 3
    (Q4_K, 8192, 700, False),        # gemv_split, C = 2
    (Q6_K, 2048, 1, False),
    (Q4_K, 256, 3, False),
])
def test_pick_matches_gemv_and_oracle(qk, torch_gpu, oracle, workloads, qtype, cols, rows, split):
    if cols == 2048 and rows == 128256:
        w, x = workloads.lm_head_q6k()
    else:
        w, x = workloads.gemv_case(qtype, cols, rows, seed=400 + rows)
    y, tok = _run(qk, torch_gpu, qtype, w, x, cols, rows, split)
    assert tok == _lowest_max(y)
    y64 = oracle.gemv_f64(qtype, w, x, cols, rows)
    assert rel_l2(y, y64) < 1e-5
    top = np.sort(y64)[-2:]
    if rows == 1 or top[1] - top[0] > 1e-4 * abs(top[1]):
        assert tok == int(np.argmax(y64))


@pytest.mark.parametrize("cols", [2048, 3072])
def test_planted_ties_keep_lowest_index(qk, torch_gpu, workloads, cols):
    rows = 4001
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=420)
    rb = cols // 256 * 210
    y, best = _run(qk, torch_gpu, Q6_K, w, x, cols, rows)
    w2 = w.copy().reshape(rows, rb)
    lo, hi = 17, rows - 2
    assert lo < best < hi or best <= lo
    w2[lo] = w2[best]
    w2[hi] = w2[best]
    y2, tok = _run(qk, torch_gpu, Q6_K, w2.reshape(-1), x, cols, rows)
    assert y2[lo] == y2[hi] == y2.max()
    assert tok == min(lo, best)


def test_nan_row_never_wins(qk, torch_gpu, workloads):
    cols, rows = 2048, 3000
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=430)
    rb = cols // 256 * 210
    w2 = w.copy().reshape(rows, rb)
    for b in range(cols // 256):
        w2[1234, b * 210 + 208: b * 210 + 210] = np.frombuffer(np.float16(np.nan).tobytes(), dtype=np.uint8)
    y, tok = _run(qk, torch_gpu, Q6_K, w2.reshape(-1), x, cols, rows)
    assert np.isnan(y[1234])
    assert tok == _lowest_max(y) and tok != 1234


def test_argmax_entry_point_rejects_bad_arguments(qk, torch_gpu):
    t = torch_gpu
    L = qk.lib()
    w = t.zeros(144 * 8, dtype=t.uint8, device="cuda")
    x = t.zeros(2048, device="cuda")
    y = t.zeros(1, device="cuda")
    o = t.zeros(1, dtype=t.int32, device="cuda")
    ws = t.zeros(L.qk_gemv_argmax_workspace_bytes(), dtype=t.uint8, device="cuda")
    assert L.qk_gemv_argmax_f32(12, w.data_ptr(), x.data_ptr(), y.data_ptr(), 2048, 1, o.data_ptr(), None,
                                None) == qk.QK_ERR_INVALID_ARG
    assert L.qk_gemv_argmax_f32(12, w.data_ptr(), x.data_ptr() + 4, y.data_ptr(), 2048, 1, o.data_ptr(),
                                ws.data_ptr(), None) == qk.QK_ERR_ALIGN
    assert L.qk_gemv_argmax_f32(13, w.data_ptr(), x.data_ptr(), y.data_ptr(), 2048, 1, o.data_ptr(),
                                ws.data_ptr(), None) == qk.QK_ERR_TYPE
