"""The INT8 multi-token product on the integer matrix cores
(qk_gemv_batched_i8, qk_gemv_multi_batched_i8, qk_ffn_batched_i8): the
reference's batched INT8 arithmetic (gemv_batch_dp4a, qkv_batch_cuda,
gate_up_batch_cuda, inferencer.cu:678-751; the sub-block combines of
dot_q4_block_dp4a / dot_q6_block_dp4a, 520-542, 613-643).

* Integer blocks (d = dmin = 1 for Q4_K with its real 6-bit scales and
  mins, d = 1 with full-range int8 scales for Q6_K) and unit activation
  scales: every product and partial sum is an exact integer below 2^24, so
  the outputs equal the oracle's integer formula bit for bit -- the
  sub-block dots, the Q4_K min term and the Q6_K scale pairs all pinned.
* Random blocks with activation scales spanning 2^20 inside one 256-column
  block: within rel-L2 1e-5 of the oracle's fp64 combine (gemv_i8_f64).
* Fused matrices of mixed types, the split Q6_K layout, and the FFN call
  (SiLU(gate) * up quantized in the gate / up product's epilogue) against
  the oracle's quantizer and fp64 products.
* Launches larger than one round of workgroups (20010 rows, or the FFN at
  520 tokens), which walk their row tiles with the next tile's weights in
  flight, against the same fp64 bars."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14
LDXQ, LDSCALE = 8192, 256
ONE = np.array([0x00, 0x3C], dtype=np.uint8)      # fp16 1.0


def _integer_blocks(qtype, w, cols, rows):
    nb = cols // 256
    bpb = 144 if qtype == Q4_K else 210
    blk = w.reshape(rows * nb, bpb).copy()
    if qtype == Q4_K:
        blk[:, 0:2] = ONE
        blk[:, 2:4] = ONE
    else:
        blk[:, 208:210] = ONE
        blk[:, 192:208] = np.random.default_rng(7).integers(0, 256, (rows * nb, 16), dtype=np.uint8)
    return blk.reshape(-1)


def _integer_want(oracle, qtype, w, xq, cols, rows):
    """sum over sub-blocks of sc * dot - m * sum(xq) (Q4_K) or scale * dot
    (Q6_K), in int64."""
    nb = cols // 256
    dots, sums = oracle.subblock_dots_i8(qtype, w, xq, cols, rows)
    dots = dots.astype(np.int64).reshape(rows, nb, -1)
    bpb = 144 if qtype == Q4_K else 210
    blk = w.reshape(rows, nb, bpb)
    if qtype == Q6_K:
        sc = blk[:, :, 192:208].view(np.int8).astype(np.int64)
        return (sc * dots).sum(axis=(1, 2))
    sc = np.empty((rows, nb, 8), dtype=np.int64)
    mn = np.empty_like(sc)
    for r in range(rows):
        for b in range(nb):
            for s in range(8):
                sc[r, b, s], mn[r, b, s] = oracle.scale_min(blk[r, b, 4:16], s)
    return (sc * dots).sum(axis=(1, 2)) - (mn * sums.astype(np.int64).reshape(1, nb, 8)).sum(axis=(1, 2))


def _run(qk, t, qtype, w, xq, xs, cols, rows, ntok, ldxq=LDXQ, ldscale=LDSCALE):
    y = t.full((ntok, rows), float("nan"), device="cuda")
    wd, xqd, xsd = to_dev(t, w), to_dev(t, xq), to_dev(t, xs)
    L = qk.lib()
    nws = L.qk_gemv_batched_i8_workspace_bytes(cols, rows, ntok)
    ws = t.empty(max(nws, 16), dtype=t.uint8, device="cuda")
    qk.check(L.qk_gemv_batched_i8(qtype, wd.data_ptr(), xqd.data_ptr(), ldxq, xsd.data_ptr(), ldscale, y.data_ptr(),
                                  rows, cols, rows, ntok, ws.data_ptr() if nws else None, nws, None), "batched INT8")
    t.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, 114])
@pytest.mark.parametrize("cols", [2048, 3072, 8192])
@pytest.mark.parametrize("ntok", [8, 33])
def test_integer_combine_exact(qk, torch_gpu, oracle, workloads, synth, qtype, cols, ntok):
    t = torch_gpu
    base = Q4_K if qtype == Q4_K else Q6_K
    rows = 96
    w, _ = workloads.gemv_case(base, cols, rows, seed=110)
    w = _integer_blocks(base, w, cols, rows)
    lim = 2 if base == Q4_K else 1      # every partial sum stays below 2^24
    xq = np.zeros((ntok, LDXQ), dtype=np.int8)
    xq[:, :cols] = synth.uniform_i32(ntok * cols, 111, 1, -lim, lim).reshape(ntok, cols).astype(np.int8)
    xs = np.zeros((ntok, LDSCALE), dtype=np.float32)
    xs[:, : cols // 32] = 1.0
    wk = w
    if qtype == 114:
        wk = qk.split_q6k(qk.Tensor((cols, rows), Q6_K, to_dev(t, w))).data.cpu().numpy()
    got = _run(qk, t, qtype, wk, xq, xs, cols, rows, ntok)
    for k in range(ntok):
        want = _integer_want(oracle, base, w, xq[k, :cols], cols, rows).astype(np.float64)
        assert np.array_equal(got[k].astype(np.float64), want), (k, np.abs(got[k] - want).max())


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
@pytest.mark.parametrize("ntok", [8, 32, 100])
def test_wide_activation_scales(qk, torch_gpu, oracle, workloads, synth, qtype, ntok):
    """Per-32 scales 2^-10 .. 2^10 inside every block: each sub-block's scale
    is applied to its own exact integer dot, as the reference does."""
    cols, rows = 2048, 500
    w, _ = workloads.gemv_case(qtype, cols, rows, seed=112)
    xq = np.zeros((ntok, LDXQ), dtype=np.int8)
    xq[:, :cols] = synth.uniform_i32(ntok * cols, 113, 1, -127, 127).reshape(ntok, cols).astype(np.int8)
    xs = np.zeros((ntok, LDSCALE), dtype=np.float32)
    xs[:, : cols // 32] = np.exp2(synth.uniform_i32(ntok * cols // 32, 113, 2, -10, 10)).reshape(ntok, -1)
    got = _run(qk, torch_gpu, qtype, w, xq, xs, cols, rows, ntok)
    for k in range(ntok):
        want = oracle.gemv_i8_f64(qtype, w, xq[k, :cols], xs[k, : cols // 32], cols, rows)
        assert rel_l2(got[k], want) < 1e-5, k


@pytest.mark.parametrize("ntok", [8, 32, 77])
@pytest.mark.parametrize("split_v", [False, True])
@pytest.mark.parametrize("cols", [2048, 3072])
def test_fused_qkv_mixed_types(qk, torch_gpu, oracle, workloads, ntok, split_v, cols):
    """Q4_K q / k and Q6_K v (GGUF or split layout) in one launch over the
    reference's quantizer outputs (qkv_batch_cuda's row routing); at 3072
    columns the rows split over two workgroups and a reduction launch."""
    t = torch_gpu
    shapes = [(Q4_K, cols), (Q4_K, 512), (Q6_K, 520)]
    ws = [workloads.gemv_case(ty, cols, rows, seed=120 + i)[0] for i, (ty, rows) in enumerate(shapes)]
    _, x = workloads.gemv_case(Q4_K, cols, 8, seed=123, n_tokens=ntok)
    xq = np.zeros((ntok, cols), dtype=np.int8)
    xs = np.zeros((ntok, cols // 32), dtype=np.float32)
    for k in range(ntok):
        xq[k], xs[k] = oracle.quantize_x32(x[k])
    dev = [to_dev(t, w) for w in ws]
    types = [ty for ty, _ in shapes]
    if split_v:
        dev[2] = qk.split_q6k(qk.Tensor((cols, 520), Q6_K, dev[2])).data
        types[2] = 114
    outs = [t.full((ntok, rows), float("nan"), device="cuda") for _, rows in shapes]
    mats = (qk.qk_matrix * 3)(*[qk.qk_matrix(types[i], shapes[i][1], dev[i].data_ptr(), outs[i].data_ptr())
                                for i in range(3)])
    xqd, xsd = to_dev(t, xq), to_dev(t, xs)
    L = qk.lib()
    nws = L.qk_gemv_batched_i8_workspace_bytes(cols, sum(r for _, r in shapes), ntok)
    wsd = t.empty(max(nws, 16), dtype=t.uint8, device="cuda")
    qk.check(L.qk_gemv_multi_batched_i8(mats, 3, xqd.data_ptr(), cols, xsd.data_ptr(), cols // 32, cols, ntok,
                                        wsd.data_ptr() if nws else None, nws, None), "fused INT8")
    t.cuda.synchronize()
    for i, (ty, rows) in enumerate(shapes):
        got = outs[i].cpu().numpy()
        for k in range(ntok):
            want = oracle.gemv_i8_f64(ty, ws[i], xq[k], xs[k], cols, rows)
            assert rel_l2(got[k], want) < 1e-5, (i, k)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, 114])
@pytest.mark.parametrize("cols,ntok", [(2048, 32), (3072, 70)])
def test_tile_walking_launch(qk, torch_gpu, oracle, workloads, synth, qtype, cols, ntok):
    """More (row tile, token tile) units than the chip holds at once: the
    workgroups walk the row tiles with the next tile's weights in flight
    (3072 columns: two splits and the reduction too).  20010 rows, so the
    last row tile is partial; three tokens of every token tile against the
    fp64 oracle at rel-L2 1e-5."""
    t = torch_gpu
    base = Q6_K if qtype == 114 else qtype
    rows = 20010
    w, x = workloads.gemv_case(base, cols, rows, seed=140, n_tokens=ntok)
    xq = np.zeros((ntok, LDXQ), dtype=np.int8)
    xs = np.zeros((ntok, LDSCALE), dtype=np.float32)
    for k in range(ntok):
        xq[k, :cols], xs[k, : cols // 32] = oracle.quantize_x32(x[k])
    wk = w
    if qtype == 114:
        wk = qk.split_q6k(qk.Tensor((cols, rows), Q6_K, to_dev(t, w))).data.cpu().numpy()
    got = _run(qk, t, qtype, wk, xq, xs, cols, rows, ntok)
    for k in sorted({0, 31, ntok // 2, ntok - 1}):
        want = oracle.gemv_i8_f64(base, w, xq[k, :cols], xs[k, : cols // 32], cols, rows)
        assert rel_l2(got[k], want) < 1e-5, k


@pytest.mark.parametrize("ntok", [4, 8, 32, 40, 520])
@pytest.mark.parametrize("accumulate", [False, True])
def test_ffn_int8(qk, torch_gpu, oracle, workloads, synth, ntok, accumulate):
    """gate / up, SiLU(gate) * up quantized per 32, down: the hidden rows the
    call quantized (in its workspace) match the oracle's quantizer applied to
    SiLU * up of the oracle's gate and up (up to the rare value within fp32
    rounding of a rounding boundary), and the output matches the oracle's
    down product over those hidden rows."""
    t = torch_gpu
    dim, hidden = 1024, 2048
    gw, x = workloads.gemv_case(Q4_K, dim, hidden, seed=130, n_tokens=max(ntok, 2))
    x = x[:ntok]
    uw, _ = workloads.gemv_case(Q4_K, dim, hidden, seed=131)
    dw, _ = workloads.gemv_case(Q6_K, hidden, dim, seed=132)
    xq = np.zeros((ntok, dim), dtype=np.int8)
    xs = np.zeros((ntok, dim // 32), dtype=np.float32)
    for k in range(ntok):
        xq[k], xs[k] = oracle.quantize_x32(x[k])
    L = qk.lib()
    nws = L.qk_ffn_batched_i8_workspace_bytes(dim, hidden, ntok)
    wsd = t.zeros(nws, dtype=t.uint8, device="cuda")
    y0 = synth.normal_f32(ntok * dim, 133, 1).reshape(ntok, dim)
    y = to_dev(t, y0)
    gd, ud, dd = to_dev(t, gw), to_dev(t, uw), to_dev(t, dw)
    xqd, xsd = to_dev(t, xq), to_dev(t, xs)
    qk.check(L.qk_ffn_batched_i8(Q4_K, gd.data_ptr(), Q4_K, ud.data_ptr(), Q6_K, dd.data_ptr(), xqd.data_ptr(), dim,
                                 xsd.data_ptr(), dim // 32, y.data_ptr(), dim, dim, hidden, ntok, int(accumulate),
                                 wsd.data_ptr(), nws, None), "INT8 FFN")
    t.cuda.synchronize()
    got = y.cpu().numpy() - (y0 if accumulate else 0)
    raw = wsd.cpu().numpy()
    hq = raw[: ntok * hidden].view(np.int8).reshape(ntok, hidden)
    off = (ntok * hidden + 255) // 256 * 256
    hs = raw[off: off + ntok * hidden // 32 * 4].view(np.float32).reshape(ntok, hidden // 32)
    flips = 0
    for k in range(ntok):
        g = oracle.gemv_i8_f64(Q4_K, gw, xq[k], xs[k], dim, hidden)
        u = oracle.gemv_i8_f64(Q4_K, uw, xq[k], xs[k], dim, hidden)
        # silu_cuda's fp32 arithmetic: exp(-g) overflows to inf below g = -88.7
        # and the product is then 0 (at 520 tokens whole groups of 32 lie there).
        g32, u32 = g.astype(np.float32), u.astype(np.float32)
        with np.errstate(over="ignore"):
            h = g32 / (np.float32(1.0) + np.exp(-g32)) * u32
        wq, wsc = oracle.quantize_x32(h)
        assert np.max(np.abs(hq[k].astype(int) - wq.astype(int))) <= 1, k
        flips += int(np.count_nonzero(hq[k] != wq))
        assert rel_l2(hs[k], wsc) < 1e-5, k
        want = oracle.gemv_i8_f64(Q6_K, dw, hq[k], hs[k], hidden, dim)
        assert rel_l2(got[k], want) < 1e-5, k
    print(f"{ntok} tokens: {flips} of {ntok * hidden} hidden codes one step off the oracle's", flush=True)
    assert flips <= max(2, ntok * hidden // 10000)
