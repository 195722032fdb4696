"""INT8 multi-token GEMV on the matrix cores (qk_gemv_batched_i8): the
reference's batched INT8 semantics (gemv_batch_dp4a, inferencer.cu:678-699)
at the reference's activation strides (8192 bytes of codes and 256 scales
per token, inferencer.cu:687-688).

* With unit block scales (d = 1, dmin = 0, sub-block scales 1) and unit
  activation scales every product and partial sum is an exact integer, so
  the outputs must equal the oracle's exact integer sub-block dots summed
  over the row, bit for bit.
* With random blocks, every token within rel-L2 1e-5 of the oracle's fp64
  combine of the exact integer dots (gemv_i8_f64), and within 1e-6 of the
  one-token INT8 kernel."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
LDXQ, LDSCALE = 8192, 256


def _unit_scales(qtype, w, cols, rows):
    """Blocks with d = 1, dmin = 0 and every sub-block scale 1 (codes kept)."""
    nb = cols // 256
    bpb = 144 if qtype == Q4_K else 210
    blk = w.reshape(rows * nb, bpb).copy()
    one = np.array([0x00, 0x3C], dtype=np.uint8)     # fp16 1.0
    if qtype == Q4_K:
        blk[:, 0:2] = one
        blk[:, 2:4] = 0
        blk[:, 4:16] = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], dtype=np.uint8)
    else:
        blk[:, 192:208] = 1
        blk[:, 208:210] = one
    return blk.reshape(-1)


def _run(qk, t, qtype, w, xq, xs, cols, rows, ntok):
    L = qk.lib()
    wd, xqd, xsd = to_dev(t, w), to_dev(t, xq), to_dev(t, xs)
    y = t.full((ntok, rows), float("nan"), device="cuda")
    nws = L.qk_gemv_batched_i8_workspace_bytes(cols, rows, ntok)
    ws = t.empty(max(nws, 256), dtype=t.uint8, device="cuda")
    qk.check(L.qk_gemv_batched_i8(qtype, wd.data_ptr(), xqd.data_ptr(), LDXQ, xsd.data_ptr(), LDSCALE, y.data_ptr(),
                                  rows, cols, rows, ntok, ws.data_ptr(), nws, None), "batched INT8 GEMV")
    t.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("ntok", [8, 33])
def test_integer_dots_exact(qk, torch_gpu, oracle, workloads, synth, qtype, ntok):
    cols, rows = 2048, 300
    w, _ = workloads.gemv_case(qtype, cols, rows, seed=80)
    w = _unit_scales(qtype, w, cols, rows)
    xq = np.zeros((ntok, LDXQ), dtype=np.int8)
    xq[:, :cols] = (synth.uniform_i32(ntok * cols, 81, 1, -127, 127)).reshape(ntok, cols).astype(np.int8)
    xs = np.zeros((ntok, LDSCALE), dtype=np.float32)
    xs[:, : cols // 32] = 1.0
    got = _run(qk, torch_gpu, qtype, w, xq, xs, cols, rows, ntok)
    for k in range(ntok):
        dots, _ = oracle.subblock_dots_i8(qtype, w, xq[k, :cols], cols, rows)
        want = dots.astype(np.int64).sum(axis=1).astype(np.float64)
        assert np.array_equal(got[k].astype(np.float64), want), k


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("ntok", [8, 32, 100])
@pytest.mark.parametrize("cols,rows", [(2048, 512), (3072, 1000), (8192, 300)])
def test_matches_integer_oracle(qk, torch_gpu, oracle, workloads, qtype, ntok, cols, rows):
    t = torch_gpu
    w, x = workloads.gemv_case(qtype, cols, rows, seed=82, n_tokens=ntok)
    xq = np.zeros((ntok, LDXQ), dtype=np.int8)
    xs = np.zeros((ntok, LDSCALE), dtype=np.float32)
    for k in range(ntok):
        xq[k, :cols], xs[k, : cols // 32] = oracle.quantize_x32(x[k])
    got = _run(qk, t, qtype, w, xq, xs, cols, rows, ntok)
    one = t.empty((ntok, rows), device="cuda")
    qk.matvec_i8(qk.Tensor((cols, rows), qtype, to_dev(t, w)), to_dev(t, xq), to_dev(t, xs), one, cols, rows,
                 n_tokens=ntok, ldxq=LDXQ, ldscale=LDSCALE, ldy=rows)
    t.cuda.synchronize()
    per_token = one.cpu().numpy()
    for k in range(ntok):
        want = oracle.gemv_i8_f64(qtype, w, xq[k, :cols], xs[k, : cols // 32], cols, rows)
        assert rel_l2(got[k], want) < 1e-5, k
        assert rel_l2(got[k], per_token[k]) < 1e-6, k
