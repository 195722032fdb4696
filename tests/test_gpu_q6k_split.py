"""The split Q6_K layout (QK_TYPE_Q6_K_SPLIT, made by qk_q6k_split): the same
210 bytes per super-block with each row's ql / qh / scales / d fields in four
16-byte aligned streams.  It must decode bit-exactly like the GGUF layout it
came from (q6_value, inferencer.cu:473-487) and feed every GEMV path with
the same results: batch-1 FP32 and INT8, fused mixed-type QKV, the few-token
and matrix-core batched GEMMs, the embedding gather."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K, Q6_K_SPLIT = 12, 14, 114
TOL = 1e-5


def _split(qk, t, w, cols, rows):
    """(GGUF device copy, split Tensor) of host Q6_K bytes w."""
    wd = to_dev(t, w)
    return wd, qk.split_q6k(qk.Tensor((cols, rows), Q6_K, wd))


@pytest.mark.parametrize("cols,rows", [(256, 1), (256, 7), (512, 3), (2048, 65), (3072, 9), (8192, 4)])
def test_split_dequant_bit_exact(qk, torch_gpu, oracle, workloads, cols, rows):
    """Every value of every row, the row padding zeroed (cols 3072: 2520-byte
    rows padded to 2528)."""
    t = torch_gpu
    w, _ = workloads.gemv_case(Q6_K, cols, rows, seed=140 + rows)
    _, s = _split(qk, t, w, cols, rows)
    assert s.data.numel() == qk.tensor_bytes(Q6_K_SPLIT, cols, rows)
    out = t.empty((rows, cols), device="cuda")
    qk.dequant_rows(s, out, 0, rows)
    t.cuda.synchronize()
    want = oracle.dequant(Q6_K, w, cols, rows)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
    raw = s.data.cpu().numpy().reshape(rows, -1)
    nb = cols // 256
    assert raw.shape[1] == (nb * 210 + 15) // 16 * 16
    assert not raw[:, nb * 210:].any()
    # The streams hold the block fields in order: ql, qh, scales, d.
    blocks = w.reshape(rows, nb, 210)
    assert np.array_equal(raw[:, : nb * 128].reshape(rows, nb, 128), blocks[:, :, :128])
    assert np.array_equal(raw[:, nb * 128: nb * 192].reshape(rows, nb, 64), blocks[:, :, 128:192])
    assert np.array_equal(raw[:, nb * 192: nb * 208].reshape(rows, nb, 16), blocks[:, :, 192:208])
    assert np.array_equal(raw[:, nb * 208: nb * 210].reshape(rows, nb, 2), blocks[:, :, 208:210])


def test_split_embedding_bit_exact(qk, torch_gpu, oracle, workloads):
    t = torch_gpu
    cols, vocab = 2048, 300
    w, _ = workloads.gemv_case(Q6_K, cols, vocab, seed=150)
    _, s = _split(qk, t, w, cols, vocab)
    tokens = np.array([0, 299, 17, 17, 150], dtype=np.int32)
    out = t.empty((len(tokens), cols), device="cuda")
    td = to_dev(t, tokens)
    qk.embedding(s, td, out, len(tokens))
    t.cuda.synchronize()
    want = oracle.dequant(Q6_K, w, cols, vocab)[tokens]
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("nb", [1, 3, 8, 12, 16, 32, 56])
def test_split_gemv_shapes(qk, torch_gpu, oracle, workloads, nb):
    """Batch-1 GEMV on the split layout (every launch shape: one-wave tiles,
    split tiles, long rows) against fp64, and equal to the GGUF-layout
    result: the same bytes in the same lanes."""
    t = torch_gpu
    cols = 256 * nb
    for rows in (1, 3, 65, 257):
        w, x = workloads.gemv_case(Q6_K, cols, rows, seed=160 + nb, x_stream=rows)
        wd, s = _split(qk, t, w, cols, rows)
        xd = to_dev(t, x)
        y = t.empty(rows, device="cuda")
        y0 = t.empty(rows, device="cuda")
        qk.matvec(s, xd, y, cols, rows)
        qk.matvec(qk.Tensor((cols, rows), Q6_K, wd), xd, y0, cols, rows)
        t.cuda.synchronize()
        assert rel_l2(y.cpu().numpy(), oracle.gemv_f64(Q6_K, w, x, cols, rows)) < TOL, (nb, rows)
        assert np.array_equal(y.cpu().numpy(), y0.cpu().numpy()), (nb, rows)


def test_split_lm_head(qk, torch_gpu, oracle, workloads):
    t = torch_gpu
    w, x = workloads.lm_head_q6k()
    _, s = _split(qk, t, w, 2048, 128256)
    y = t.empty(128256, device="cuda")
    qk.matvec(s, to_dev(t, x), y, 2048, 128256)
    t.cuda.synchronize()
    y64 = oracle.gemv_f64(Q6_K, w, x, 2048, 128256)
    assert rel_l2(y.cpu().numpy(), y64) < TOL
    assert int(np.argmax(y.cpu().numpy())) == int(np.argmax(y64))


def test_split_fused_qkv_mixed(qk, torch_gpu, oracle, workloads):
    t = torch_gpu
    dim, kv = 2048, 512
    wq, x = workloads.gemv_case(Q4_K, dim, dim, seed=170)
    wk, _ = workloads.gemv_case(Q4_K, dim, kv, seed=171)
    wv, _ = workloads.gemv_case(Q6_K, dim, kv, seed=172)
    _, sv = _split(qk, t, wv, dim, kv)
    q, k, v = t.empty(dim, device="cuda"), t.empty(kv, device="cuda"), t.empty(kv, device="cuda")
    T = qk.Tensor
    qk.qkv(T((dim, dim), Q4_K, to_dev(t, wq)), T((dim, kv), Q4_K, to_dev(t, wk)), sv, to_dev(t, x), q, k, v, dim, kv)
    t.cuda.synchronize()
    assert rel_l2(q.cpu().numpy(), oracle.gemv_f64(Q4_K, wq, x, dim, dim)) < TOL
    assert rel_l2(k.cpu().numpy(), oracle.gemv_f64(Q4_K, wk, x, dim, kv)) < TOL
    assert rel_l2(v.cpu().numpy(), oracle.gemv_f64(Q6_K, wv, x, dim, kv)) < TOL


def test_split_gemv_i8(qk, torch_gpu, oracle, workloads):
    t = torch_gpu
    cols, rows = 3072, 130
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=180)
    wd, s = _split(qk, t, w, cols, rows)
    xq, xs = oracle.quantize_x32(x)
    xqd, xsd = to_dev(t, xq), to_dev(t, xs)
    y = t.empty(rows, device="cuda")
    y0 = t.empty(rows, device="cuda")
    qk.matvec_i8(s, xqd, xsd, y, cols, rows)
    qk.matvec_i8(qk.Tensor((cols, rows), Q6_K, wd), xqd, xsd, y0, cols, rows)
    t.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), oracle.gemv_i8_f64(Q6_K, w, xq, xs, cols, rows)) < TOL
    assert np.array_equal(y.cpu().numpy(), y0.cpu().numpy())


@pytest.mark.parametrize("cols,rows,ntok", [(2048, 777, 3), (8192, 300, 8), (3072, 130, 64), (2048, 700, 256)])
def test_split_batched(qk, torch_gpu, oracle, workloads, cols, rows, ntok):
    """Few-token GEMV (below 8 tokens) and matrix-core GEMM (from 8 on)."""
    t = torch_gpu
    w, x = workloads.gemv_case(Q6_K, cols, rows, seed=190 + ntok, n_tokens=max(ntok, 2))
    x = x[:ntok]
    _, s = _split(qk, t, w, cols, rows)
    ws_bytes = qk.batch_workspace_bytes(cols, rows, ntok)
    ws = t.empty(max(ws_bytes, 256), dtype=t.uint8, device="cuda")
    y = t.full((ntok, rows), float("nan"), device="cuda")
    qk.batch_matvec(s, to_dev(t, x), y, cols, rows, ntok, ws, ws_bytes)
    t.cuda.synchronize()
    want = oracle.gemv_f64(Q6_K, w, x, cols, rows)
    got = y.cpu().numpy()
    for k in range(ntok):
        assert rel_l2(got[k], want[k]) < TOL, k


def test_split_rejects_bad_arguments(qk, torch_gpu, workloads):
    t = torch_gpu
    L = qk.lib()
    w, _ = workloads.gemv_case(Q6_K, 512, 4, seed=200)
    wd = to_dev(t, w)
    dst = t.empty(qk.tensor_bytes(Q6_K_SPLIT, 512, 4) + 16, dtype=t.uint8, device="cuda")
    assert L.qk_q6k_split(wd.data_ptr(), dst.data_ptr() + 8, 512, 4, None) == qk.QK_ERR_ALIGN
    assert L.qk_q6k_split(wd.data_ptr(), wd.data_ptr(), 512, 4, None) == qk.QK_ERR_INVALID_ARG   # overlap
    assert L.qk_q6k_split(wd.data_ptr(), None, 512, 4, None) == qk.QK_ERR_INVALID_ARG
    assert L.qk_q6k_split(wd.data_ptr(), dst.data_ptr(), 500, 4, None) == qk.QK_ERR_SHAPE
