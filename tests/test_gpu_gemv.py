"""GPU parity of the batch-1 FP32 dequant-GEMV (qk_gemv_f32, qk_gemv_multi_f32)
against the fp64 oracle.  Bar: relative L2 error <= 1e-5 (fp32 accumulation
against fp64 truth); one-hot activations must reproduce dequantized columns
bit for bit."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
TOL = 1e-5


def run_gemv(qk, torch, qtype, w, x, cols, rows):
    wd, xd = to_dev(torch, w), to_dev(torch, x)
    yd = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
    qk.matvec(qk.Tensor((cols, rows), qtype, wd), xd, yd, cols, rows)
    torch.cuda.synchronize()
    return yd.cpu().numpy()


def test_config1_q4k_2048(qk, torch_gpu, oracle, workloads):
    w, x = workloads.gemv_q4k_2048()
    y = run_gemv(qk, torch_gpu, Q4_K, w, x, 2048, 2048)
    assert rel_l2(y, oracle.gemv_f64(Q4_K, w, x, 2048, 2048)) < TOL


def test_config2_lm_head_q6k(qk, torch_gpu, oracle, workloads):
    w, x = workloads.lm_head_q6k()
    y = run_gemv(qk, torch_gpu, Q6_K, w, x, 2048, 128256)
    y64 = oracle.gemv_f64(Q6_K, w, x, 2048, 128256)
    assert np.all(np.isfinite(y))
    assert rel_l2(y, y64) < TOL
    assert int(np.argmax(y)) == int(np.argmax(y64))


# Block counts covering every launch shape: chunk count 1 (P | 64), split
# tiles with LDS (C = 2..16, incl. odd nb), and rows too long for chunks.
NB = [1, 2, 3, 4, 5, 7, 8, 12, 16, 17, 24, 32, 56]


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("nb", NB)
def test_shapes(qk, torch_gpu, oracle, workloads, qtype, nb):
    cols = 256 * nb
    for rows in (1, 3, 65, 257):
        w, x = workloads.gemv_case(qtype, cols, rows, seed=100 + nb, x_stream=rows)
        y = run_gemv(qk, torch_gpu, qtype, w, x, cols, rows)
        assert rel_l2(y, oracle.gemv_f64(qtype, w, x, cols, rows)) < TOL, (nb, rows)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_one_hot_is_exact_column(qk, torch_gpu, oracle, workloads, qtype):
    # Exact equality of values: the single non-zero product is rounded once,
    # as in q4_value / q6_value; the other lanes add zeros (so a -0.0 weight
    # comes back as +0.0, equal in value).
    cols, rows = 2048, 130
    w, _ = workloads.gemv_case(qtype, cols, rows, seed=41)
    W = oracle.dequant(qtype, w, cols, rows)
    for c in (0, 17, 31, 32, 100, 255, 256, 1023, 2047):
        e = np.zeros(cols, dtype=np.float32)
        e[c] = 1.0
        y = run_gemv(qk, torch_gpu, qtype, w, e, cols, rows)
        assert np.array_equal(y, W[:, c]), c


def test_multi_qkv_mixed_types(qk, torch_gpu, oracle, workloads, synth):
    dim, kv = 2048, 512
    wq, x = workloads.gemv_case(Q4_K, dim, dim, seed=42)
    wk, _ = workloads.gemv_case(Q4_K, dim, kv, seed=43)
    wv, _ = workloads.gemv_case(Q6_K, dim, kv, seed=44)
    t = torch_gpu
    q = t.empty(dim, device="cuda")
    k = t.empty(kv, device="cuda")
    v = t.empty(kv, device="cuda")
    T = qk.Tensor
    qk.qkv(T((dim, dim), Q4_K, to_dev(t, wq)), T((dim, kv), Q4_K, to_dev(t, wk)), T((dim, kv), Q6_K, to_dev(t, wv)),
           to_dev(t, x), q, k, v, dim, kv)
    t.cuda.synchronize()
    assert rel_l2(q.cpu().numpy(), oracle.gemv_f64(Q4_K, wq, x, dim, dim)) < TOL
    assert rel_l2(k.cpu().numpy(), oracle.gemv_f64(Q4_K, wk, x, dim, kv)) < TOL
    assert rel_l2(v.cpu().numpy(), oracle.gemv_f64(Q6_K, wv, x, dim, kv)) < TOL


def test_multi_gate_up(qk, torch_gpu, oracle, workloads):
    dim, hidden = 2048, 8192
    wg, x = workloads.gemv_case(Q4_K, dim, hidden, seed=45)
    wu, _ = workloads.gemv_case(Q4_K, dim, hidden, seed=46)
    t = torch_gpu
    g = t.empty(hidden, device="cuda")
    u = t.empty(hidden, device="cuda")
    T = qk.Tensor
    qk.gate_up(T((dim, hidden), Q4_K, to_dev(t, wg)), T((dim, hidden), Q4_K, to_dev(t, wu)), to_dev(t, x), g, u,
               dim, hidden)
    t.cuda.synchronize()
    assert rel_l2(g.cpu().numpy(), oracle.gemv_f64(Q4_K, wg, x, dim, hidden)) < TOL
    assert rel_l2(u.cpu().numpy(), oracle.gemv_f64(Q4_K, wu, x, dim, hidden)) < TOL


def test_ffn_down_q6k_8192(qk, torch_gpu, oracle, workloads):
    w, x = workloads.gemv_case(Q6_K, 8192, 2048, seed=47)
    assert rel_l2(run_gemv(qk, torch_gpu, Q6_K, w, x, 8192, 2048), oracle.gemv_f64(Q6_K, w, x, 8192, 2048)) < TOL


def test_output_overwritten_and_bounded(qk, torch_gpu, workloads):
    # y is overwritten (never accumulated) and nothing past rows is written.
    t = torch_gpu
    w, x = workloads.gemv_case(Q4_K, 512, 70, seed=48)
    wd, xd = to_dev(t, w), to_dev(t, x)
    y = t.full((80,), 12345.0, device="cuda")
    qk.matvec(qk.Tensor((512, 70), Q4_K, wd), xd, y, 512, 70)
    first = y.clone()
    qk.matvec(qk.Tensor((512, 70), Q4_K, wd), xd, y, 512, 70)
    t.cuda.synchronize()
    assert t.equal(first, y)
    assert t.all(y[70:] == 12345.0)


def test_validation_errors(qk, torch_gpu):
    t = torch_gpu
    x = t.zeros(256, device="cuda")
    y = t.zeros(4, device="cuda")
    w = t.zeros(144 * 4, dtype=t.uint8, device="cuda")
    with pytest.raises(qk.QKError):
        qk.matvec(qk.Tensor((256, 4), 13, w), x, y, 256, 4)
    with pytest.raises(qk.QKError):
        qk.matvec(qk.Tensor((256, 4), Q4_K, w), x, y, 256, 5)
    rc = qk.lib().qk_gemv_f32(Q4_K, w.data_ptr() + 2, x.data_ptr(), y.data_ptr(), 256, 4, None)
    assert rc == qk.QK_ERR_ALIGN


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_wide_range_within_groups(qk, torch_gpu, oracle, workloads, qtype):
    """Every 16-column activation group holds one value ~1e3 and fifteen
    ~1e-3 (10^6 apart).  The FP32 kernels carry each group as 22-bit block
    fixed point: X = rint(x * 2^(21-e)), e = ilogb(max|x|) of the group, so
    each value is rounded to within 2^(e-22) and the small ones keep ~2
    bits.  Pinned three ways: the device equals the fp64 product of that
    rounded x to fp32 rounding (rel-L2 1e-6), the rounding moves each row by
    at most sum_k |W_rk| 2^(e_k - 22) (the documented bound, computed from
    the dequantized weights), and the whole output meets the 1e-5 bar
    against the exact fp64 product because the large values dominate."""
    cols, rows = 2048, 515
    w, _ = workloads.gemv_case(qtype, cols, rows, seed=43)
    rng = np.random.default_rng(44)
    x = (rng.standard_normal(cols) * 1e-3).astype(np.float32)
    big = np.arange(0, cols, 16) + rng.integers(0, 16, cols // 16)
    x[big] = (rng.standard_normal(big.size) * 1e3).astype(np.float32)
    y = run_gemv(qk, torch_gpu, qtype, w, x, cols, rows)
    y64 = oracle.gemv_f64(qtype, w, x, cols, rows)
    assert rel_l2(y, y64) < TOL
    # The block fixed point in fp64: e = ilogb of each group's max.
    gmax = np.abs(x.astype(np.float64)).reshape(-1, 16).max(axis=1)
    e = (np.frexp(gmax)[1] - 1).astype(np.float64)
    step = np.repeat(np.exp2(e - 21), 16)
    xf = np.rint(x.astype(np.float64) / step) * step
    yf = oracle.gemv_f64(qtype, w, xf.astype(np.float32), cols, rows)
    assert np.array_equal(xf.astype(np.float32).astype(np.float64), xf)   # the rounded x is exact in fp32
    assert rel_l2(y, yf) < 1e-6
    W = oracle.dequant(qtype, w, cols, rows).astype(np.float64).reshape(rows, cols)
    bound = np.abs(W) @ (step / 2)
    assert np.all(np.abs(yf - y64) <= bound * (1 + 1e-9))
    xs = x.copy()
    xs[big] = 0.0
    small = oracle.gemv_f64(qtype, w, xs, cols, rows)
    print(f"rel-L2 {rel_l2(y, y64):.2e}, against the rounded x {rel_l2(y, yf):.2e}; error / norm of the small "
          f"values' share {np.linalg.norm(y - y64) / np.linalg.norm(small):.2e}; largest row error / bound "
          f"{np.max(np.abs(yf - y64) / bound):.2f}", flush=True)


# One matrix whose rows fill whole tiles (64 / gcd(4 * nb, 64) rows) is read
# through a scalar tile base with buffer loads: gemv_whole for nb <= 16
# blocks per row, gemv_split's whole-tile form for the multi-wave tiles of
# nb = 3, 12 or 32.  One more row leaves a partial tile and runs the
# per-lane-address kernels.  Both compute every row with the same
# arithmetic, so the shared rows agree bit for bit, and both are within
# 1e-5 of the oracle.  Covers every single-wave tile height (16, 8, 4, 2,
# 1 rows), three multi-wave tiles and the three storage layouts.
@pytest.mark.parametrize("layout", ["q4k", "q6k", "q6k_split"])
@pytest.mark.parametrize("nb", [1, 2, 3, 4, 8, 12, 16, 32])
def test_whole_tiles_match_partial_tiles(qk, torch_gpu, oracle, workloads, layout, nb):
    t = torch_gpu
    qtype = Q4_K if layout == "q4k" else Q6_K
    cols, rows = 256 * nb, 272
    w, x = workloads.gemv_case(qtype, cols, rows + 1, seed=140 + nb, x_stream=3)
    xd = to_dev(t, x)
    full = qk.Tensor((cols, rows + 1), qtype, to_dev(t, w))
    if layout == "q6k_split":
        full = qk.split_q6k(full)
    rb = qk.tensor_bytes(full.type, cols, 1)
    whole = qk.Tensor((cols, rows), full.type, full.data[: rows * rb])
    y_whole = t.full((rows,), float("nan"), device="cuda")
    y_part = t.full((rows + 1,), float("nan"), device="cuda")
    qk.matvec(whole, xd, y_whole, cols, rows)
    qk.matvec(full, xd, y_part, cols, rows + 1)
    t.cuda.synchronize()
    a, b = y_whole.cpu().numpy(), y_part.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b[:rows].view(np.uint32))
    assert rel_l2(b, oracle.gemv_f64(qtype, w, x, cols, rows + 1)) < TOL


# Long launches of the multi-wave-tile kernel (cols 3072: three waves share a
# four-row tile; at least 16 tiles per wave-group at two workgroups per CU)
# run four workgroups per CU.  FP32 and INT8 against the oracle, and bit for
# bit against a short launch over a row slice.
@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_split_long_launch(qk, torch_gpu, oracle, workloads, qtype):
    t = torch_gpu
    cols, rows, n = 3072, 32768, 2048
    w, x = workloads.gemv_case(qtype, cols, rows, seed=150, x_stream=4)
    mat = qk.Tensor((cols, rows), qtype, to_dev(t, w))
    if qtype == Q6_K:
        mat = qk.split_q6k(mat)
    xd = to_dev(t, x)
    xq, xs = oracle.quantize_x32(x)
    xq_d, xs_d = to_dev(t, xq), to_dev(t, xs)
    y = t.full((rows,), float("nan"), device="cuda")
    yi = t.full((rows,), float("nan"), device="cuda")
    qk.matvec(mat, xd, y, cols, rows)
    qk.matvec_i8(mat, xq_d, xs_d, yi, cols, rows)
    t.cuda.synchronize()
    got, goti = y.cpu().numpy(), yi.cpu().numpy()
    assert rel_l2(got, oracle.gemv_f64(qtype, w, x, cols, rows)) < TOL
    assert rel_l2(goti, oracle.gemv_i8_f64(qtype, w, xq, xs, cols, rows)) < TOL
    rb = qk.tensor_bytes(mat.type, cols, 1)
    r0 = rows // 2 + 4 * 37
    part = qk.Tensor((cols, n), mat.type, mat.data[r0 * rb:(r0 + n) * rb])
    ys = t.full((n,), float("nan"), device="cuda")
    ysi = t.full((n,), float("nan"), device="cuda")
    qk.matvec(part, xd, ys, cols, n)
    qk.matvec_i8(part, xq_d, xs_d, ysi, cols, n)
    t.cuda.synchronize()
    assert np.array_equal(ys.cpu().numpy().view(np.uint32), got[r0:r0 + n].view(np.uint32))
    assert np.array_equal(ysi.cpu().numpy().view(np.uint32), goti[r0:r0 + n].view(np.uint32))
