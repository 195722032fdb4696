"""qk_gemv_argmax_f32_noalloc (partials in the library's static device array)
against qk_gemv_argmax_f32 (partials in a caller workspace): the same kernels,
so the logits must agree bit for bit and the greedy token exactly, on two
calls in a row -- the LM head 128256 x 2048, then a smaller Q4_K matrix that
leaves fewer partials in the shared array."""
import numpy as np
import pytest

from conftest import to_dev

pytestmark = pytest.mark.gpu


def _pair(qk, t, qtype, w, x, cols, rows):
    L = qk.lib()
    wd, xd = to_dev(t, w), to_dev(t, x)
    y_ws = t.full((rows,), float("nan"), device="cuda")
    y_na = t.full((rows,), float("nan"), device="cuda")
    tok = t.full((2,), -1, dtype=t.int32, device="cuda")
    ws = t.empty(L.qk_gemv_argmax_workspace_bytes(), dtype=t.uint8, device="cuda")
    qk.check(L.qk_gemv_argmax_f32(qtype, wd.data_ptr(), xd.data_ptr(), y_ws.data_ptr(), cols, rows, tok.data_ptr(),
                                  ws.data_ptr(), None), "argmax with workspace")
    qk.check(L.qk_gemv_argmax_f32_noalloc(qtype, wd.data_ptr(), xd.data_ptr(), y_na.data_ptr(), cols, rows,
                                          tok.data_ptr() + 4, None), "argmax without allocation")
    t.cuda.synchronize()
    return y_ws.cpu().numpy(), y_na.cpu().numpy(), tok.cpu().tolist()


def test_noalloc_argmax_matches_workspace_entry(qk, torch_gpu, workloads, oracle):
    t = torch_gpu
    w, x = workloads.lm_head_q6k()
    a, b, tok = _pair(qk, t, qk.Q6_K, w, x, 2048, 128256)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert tok[0] == tok[1] == int(np.argmax(a))
    assert tok[0] == oracle.argmax(a)
    # Second call, smaller: the array still holds the first call's partials
    # beyond the ones this call writes; none of them may leak into its pick.
    w2, x2 = workloads.gemv_case(qk.Q4_K, 3072, 700, seed=91)
    a2, b2, tok2 = _pair(qk, t, qk.Q4_K, w2, x2, 3072, 700)
    assert np.array_equal(a2.view(np.uint32), b2.view(np.uint32))
    assert tok2[0] == tok2[1] == oracle.argmax(a2)


def test_noalloc_argmax_rejects_bad_arguments(qk, torch_gpu):
    t = torch_gpu
    x = t.zeros(2048, device="cuda")
    y = t.zeros(8, device="cuda")
    tok = t.zeros(1, dtype=t.int32, device="cuda")
    L = qk.lib()
    assert L.qk_gemv_argmax_f32_noalloc(qk.Q4_K, None, x.data_ptr(), y.data_ptr(), 2048, 8, tok.data_ptr(),
                                        None) == qk.QK_ERR_INVALID_ARG
    assert L.qk_gemv_argmax_f32_noalloc(qk.Q4_K, x.data_ptr(), x.data_ptr(), y.data_ptr(), 2000, 8,
                                        tok.data_ptr(), None) == qk.QK_ERR_SHAPE
