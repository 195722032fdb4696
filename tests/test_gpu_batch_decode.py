"""Ragged decode batches on the GPU: the batched RoPE / KV write and
attention kernels per token against the oracle's fp64 restatements
(rope_cache_batch_cuda, attention_batch_cuda, inferencer.cu:953-1041,
generalised to one sequence per token), the per-row argmax, and the batched
decode step (qk_llama_batch_forward) against one fp64 oracle model per
sequence: identical greedy tokens, logits within rel-L2 1e-4 on the small
model (teacher-forced on the oracle's tokens, with the top-2 margin printed
per token like --compare-prefill, inferencer.cu:1814-1825)."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu

SMALL = dict(dim=512, layers=2, heads=8, kv_heads=2, hidden=1024, vocab=1000, context=64, eps=1e-5,
             rope_theta=10000.0)


def _desc(qk, t, pos, kv_row):
    arr = np.zeros(len(pos), dtype=[("pos", "<i4"), ("seq", "<i4"), ("kv_row", "<i8")])
    arr["pos"], arr["seq"], arr["kv_row"] = pos, np.arange(len(pos)), kv_row
    return t.from_numpy(arr.view(np.uint8).copy()).to("cuda")


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(32, 8, 64), (24, 8, 128)])
def test_batched_rope_and_attention(qk, torch_gpu, oracle, synth, heads, kv_heads, head_dim):
    t = torch_gpu
    layers, layer, ctx = 2, 1, 300
    pos = np.array([0, 5, 77, 150, 299, 31, 200], dtype=np.int64)
    n = len(pos)
    kv_row = np.arange(n, dtype=np.int64) * ctx           # sequence s owns rows s*ctx .. s*ctx + ctx - 1
    rows = n * ctx
    kv = kv_heads * head_dim
    cos, sin = oracle.rope_tables(ctx, head_dim, 500000.0)
    kc = synth.normal_f32(layers * rows * kv, 60, 1).reshape(layers, rows, kv)
    vc = synth.normal_f32(layers * rows * kv, 60, 2).reshape(layers, rows, kv)
    q = synth.normal_f32(n * heads * head_dim, 60, 3).reshape(n, heads * head_dim)
    k = synth.normal_f32(n * kv, 60, 4).reshape(n, kv)
    v = synth.normal_f32(n * kv, 60, 5).reshape(n, kv)
    qd, kd, vd, cd, sd = (to_dev(t, a) for a in (q, k, v, cos, sin))
    kcd, vcd = to_dev(t, kc), to_dev(t, vc)
    dd = _desc(qk, t, pos, kv_row)
    out = t.empty((n, heads * head_dim), device="cuda")
    L = qk.lib()
    qk.check(L.qk_rope_kv_write_batched(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cd.data_ptr(), sd.data_ptr(),
                                        kcd.data_ptr(), vcd.data_ptr(), layer, rows, dd.data_ptr(), n, ctx, heads,
                                        kv_heads, head_dim, None), "rope batched")
    qk.check(L.qk_attention_batched_f32(qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out.data_ptr(), layer, rows,
                                        dd.data_ptr(), n, int(pos.max()), heads, kv_heads, head_dim, None),
             "attention batched")
    t.cuda.synchronize()
    got_k = kcd.cpu().numpy()
    got = out.cpu().numpy()
    for i in range(n):
        qr = oracle.rope(q[i], cos, sin, int(pos[i]), head_dim)
        kr = oracle.rope(k[i], cos, sin, int(pos[i]), head_dim)
        r0 = int(kv_row[i])
        assert np.max(np.abs(got_k[layer, r0 + pos[i]] - kr)) < 1e-5
        kseq = kc[layer, r0:r0 + ctx].copy()
        vseq = vc[layer, r0:r0 + ctx].copy()
        kseq[pos[i]], vseq[pos[i]] = kr, v[i]
        want = oracle.attention(qr, kseq[: pos[i] + 1], vseq[: pos[i] + 1], int(pos[i]), heads, kv_heads, head_dim)
        assert rel_l2(got[i], want) < 1e-5, i
    # other layers untouched
    assert np.array_equal(got_k[0], kc[0])


def test_batched_attention_rejects_out_of_range_tokens(qk, torch_gpu, synth):
    """A descriptor beyond max_pos or the cache yields NaN outputs, never an
    out-of-bounds read."""
    t = torch_gpu
    heads, kv_heads, hd, rows = 4, 2, 64, 100
    kv = kv_heads * hd
    kcd = t.zeros((1, rows, kv), device="cuda")
    vcd = t.zeros((1, rows, kv), device="cuda")
    q = t.ones((3, heads * hd), device="cuda")
    dd = _desc(qk, t, np.array([10, 60, 5]), np.array([0, 50, 98]))   # ok; beyond max_pos; beyond the cache
    out = t.zeros((3, heads * hd), device="cuda")
    qk.check(qk.lib().qk_attention_batched_f32(q.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out.data_ptr(), 0, rows,
                                               dd.data_ptr(), 3, 40, heads, kv_heads, hd, None), "attention")
    t.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isfinite(o[0])) and np.all(np.isnan(o[1])) and np.all(np.isnan(o[2]))


def _split_case(qk, t, oracle, synth, heads, kv_heads, head_dim, pos, seed):
    """Caches with each token's sequence at its own rows, rotated queries, and
    the oracle's attention per token."""
    layers, layer = 2, 1
    n = len(pos)
    ctx = int(pos.max()) + 1
    kv_row = np.arange(n, dtype=np.int64) * ctx
    rows = n * ctx
    kv = kv_heads * head_dim
    kc = synth.normal_f32(layers * rows * kv, seed, 1).reshape(layers, rows, kv)
    vc = synth.normal_f32(layers * rows * kv, seed, 2).reshape(layers, rows, kv)
    q = synth.normal_f32(n * heads * head_dim, seed, 3).reshape(n, heads * head_dim)
    want = [oracle.attention(q[i], kc[layer, kv_row[i]:kv_row[i] + pos[i] + 1],
                             vc[layer, kv_row[i]:kv_row[i] + pos[i] + 1], int(pos[i]), heads, kv_heads, head_dim)
            for i in range(n)]
    dev = dict(q=to_dev(t, q), kc=to_dev(t, kc), vc=to_dev(t, vc), desc=_desc(qk, t, pos, kv_row),
               out=t.empty((n, heads * head_dim), device="cuda"))
    return dev, want, layer, rows


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(32, 8, 64), (24, 8, 128), (8, 1, 32), (4, 2, 256),
                                                     (48, 8, 128), (16, 2, 256), (12, 3, 16)])
@pytest.mark.parametrize("split_rows", [0, 7, 64])
def test_split_attention(qk, torch_gpu, oracle, synth, heads, kv_heads, head_dim, split_rows):
    """Rows spread over splits of 7 (ragged last splits, splits shorter than
    one load round), 64 and the batch's own choice, partials merged by the
    second kernel: the oracle's attention per token within rel-L2 1e-5."""
    t = torch_gpu
    pos = np.array([0, 6, 7, 63, 64, 130, 299, 1, 200], dtype=np.int64)
    dev, want, layer, rows = _split_case(qk, t, oracle, synth, heads, kv_heads, head_dim, pos, 62)
    L = qk.lib()
    n, max_pos = len(pos), int(pos.max())
    wsb = L.qk_attention_split_workspace_bytes(n, heads, kv_heads, head_dim, max_pos, split_rows)
    if split_rows:
        assert wsb == n * kv_heads * (max_pos // split_rows + 1) * \
            ((2 * (heads // kv_heads) + 3) // 4 * 4 + heads // kv_heads * head_dim) * 4
    ws = t.empty(max(wsb, 16), dtype=t.uint8, device="cuda")
    qk.check(L.qk_attention_split_f32(dev["q"].data_ptr(), dev["kc"].data_ptr(), dev["vc"].data_ptr(),
                                      dev["out"].data_ptr(), layer, rows, dev["desc"].data_ptr(), n, max_pos, heads,
                                      kv_heads, head_dim, split_rows, ws.data_ptr(), wsb, None), "split attention")
    t.cuda.synchronize()
    got = dev["out"].cpu().numpy()
    for i in range(n):
        assert rel_l2(got[i], want[i]) < 1e-5, (i, int(pos[i]))


@pytest.mark.parametrize("room", ["none", "short"])
def test_split_attention_short_workspace(qk, torch_gpu, oracle, synth, room):
    """With no workspace the call runs one split per token; with a workspace
    shorter than the splits ask for, fewer and longer splits: the same
    results either way."""
    t = torch_gpu
    heads, kv_heads, head_dim = 32, 8, 64
    pos = np.array([500, 3, 257, 64], dtype=np.int64)
    dev, want, layer, rows = _split_case(qk, t, oracle, synth, heads, kv_heads, head_dim, pos, 63)
    L = qk.lib()
    n, max_pos = len(pos), int(pos.max())
    full = L.qk_attention_split_workspace_bytes(n, heads, kv_heads, head_dim, max_pos, 16)
    wsb = 0 if room == "none" else full // 5
    ws = t.empty(max(full, 16), dtype=t.uint8, device="cuda")
    qk.check(L.qk_attention_split_f32(dev["q"].data_ptr(), dev["kc"].data_ptr(), dev["vc"].data_ptr(),
                                      dev["out"].data_ptr(), layer, rows, dev["desc"].data_ptr(), n, max_pos, heads,
                                      kv_heads, head_dim, 16, ws.data_ptr() if wsb else None, wsb, None),
             "split attention")
    t.cuda.synchronize()
    got = dev["out"].cpu().numpy()
    for i in range(n):
        assert rel_l2(got[i], want[i]) < 1e-5, i


def test_split_attention_rejects_out_of_range_tokens(qk, torch_gpu, synth):
    """Descriptors beyond max_pos or the cache give NaN rows with several
    splits too, and never read outside the cache."""
    t = torch_gpu
    heads, kv_heads, hd, rows = 4, 2, 64, 100
    kv = kv_heads * hd
    kcd = t.zeros((1, rows, kv), device="cuda")
    vcd = t.zeros((1, rows, kv), device="cuda")
    q = t.ones((3, heads * hd), device="cuda")
    dd = _desc(qk, t, np.array([30, 60, 5]), np.array([0, 30, 98]))   # ok; beyond max_pos; beyond the cache
    out = t.zeros((3, heads * hd), device="cuda")
    L = qk.lib()
    wsb = L.qk_attention_split_workspace_bytes(3, heads, kv_heads, hd, 40, 8)
    ws = t.empty(wsb, dtype=t.uint8, device="cuda")
    qk.check(L.qk_attention_split_f32(q.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), out.data_ptr(), 0, rows,
                                      dd.data_ptr(), 3, 40, heads, kv_heads, hd, 8, ws.data_ptr(), wsb, None),
             "split attention")
    t.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isfinite(o[0])) and np.all(np.isnan(o[1])) and np.all(np.isnan(o[2]))


def test_argmax_rows(qk, torch_gpu, oracle, synth):
    t = torch_gpu
    rows, n, ld = 5, 128256, 128300
    v = synth.normal_f32(rows * ld, 61, 1).reshape(rows, ld)
    v[1, [3, 90000]] = 40.0                # tie: lowest index wins
    v[2, n:] = 1e9                         # beyond n: ignored
    vd = to_dev(t, v)
    ws = t.empty(qk.lib().qk_argmax_rows_workspace_bytes(n, rows), dtype=t.uint8, device="cuda")
    out = t.full((rows,), -1, dtype=t.int32, device="cuda")
    qk.check(qk.lib().qk_argmax_rows_f32(vd.data_ptr(), n, ld, rows, out.data_ptr(), ws.data_ptr(), None), "argmax rows")
    t.cuda.synchronize()
    assert out.cpu().tolist() == [oracle.argmax(v[r, :n]) for r in range(rows)]


def batch_case(wl, synth, cfg, seed, positions):
    """Per-sequence caches [layer][context][kv_dim] (N(0,1) below pos, zero
    above) and the packed [layer][S*context][kv_dim] caches of the batch."""
    S, ctx = len(positions), cfg["context"]
    kv = cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    seqs = []
    for s, p in enumerate(positions):
        kc = np.zeros((cfg["layers"], ctx, kv), dtype=np.float32)
        vc = np.zeros_like(kc)
        kc[:, :p] = synth.normal_f32(cfg["layers"] * p * kv, seed, 10 + 2 * s).reshape(cfg["layers"], p, kv)
        vc[:, :p] = synth.normal_f32(cfg["layers"] * p * kv, seed, 11 + 2 * s).reshape(cfg["layers"], p, kv)
        seqs.append((kc, vc))
    packed_k = np.concatenate([k for k, _ in seqs], axis=1)
    packed_v = np.concatenate([v for _, v in seqs], axis=1)
    return seqs, packed_k, packed_v


def run_batch_decode(qk, oracle, wl, synth, cfg, seed, positions, steps, logits_tol):
    W = wl.llama_weights(cfg, seed)
    S, ctx = len(positions), cfg["context"]
    seqs, pk, pv = batch_case(wl, synth, cfg, seed, positions)
    br = qk.BatchRunner(cfg, W, max_tokens=S, cache_rows=S * ctx)
    br.load_kv(pk, pv)
    orcs = []
    for s, p in enumerate(positions):
        om = oracle.Llama(cfg, W)
        om.load_cache(seqs[s][0], seqs[s][1], p)
        orcs.append(om)
    tokens = [int(x) for x in synth.uniform_i32(S, seed, 30, 0, cfg["vocab"] - 1)]
    pos = list(positions)
    kv_row = [s * ctx for s in range(S)]
    for step in range(steps):
        got = br.forward(tokens, pos, kv_row, True)
        lg = br.logits(S)
        want = []
        for s in range(S):
            o, ref = orcs[s].forward(tokens[s], pos[s], True)
            top = np.sort(ref)[-2:]
            err = rel_l2(lg[s], ref)
            print(f"step {step} seq {s} pos {pos[s]}: gpu {got[s]} ref {o} top2 margin {top[1] - top[0]:.4f} "
                  f"logits rel-L2 {err:.2e}", flush=True)
            assert err < logits_tol
            want.append(o)
        assert got == want
        tokens = want                      # teacher-forced on the oracle's tokens
        pos = [p + 1 for p in pos]
    br.close()


@pytest.mark.parametrize("positions", [[3, 10, 21, 33, 58], [3, 10, 21, 33, 40, 47, 52, 58]])
def test_small_llama_ragged_batch(qk, torch_gpu, oracle, workloads, synth, positions):
    """5 tokens (GEMV path) and 8 tokens (matrix-core path), one per sequence."""
    run_batch_decode(qk, oracle, workloads, synth, SMALL, seed=12, positions=positions, steps=4, logits_tol=1e-4)


def test_llama_1b_ragged_batch(qk, torch_gpu, oracle, workloads, synth):
    """Random-init Llama-3.2-1B, 8 sequences at ragged positions 64..599."""
    cfg = dict(workloads.LLAMA_1B, context=640)
    positions = [64, 599, 130, 257, 401, 88, 512, 333]
    run_batch_decode(qk, oracle, workloads, synth, cfg, seed=2, positions=positions, steps=2, logits_tol=1e-2)


def test_driver_cache_layout_round_trip(qk, torch_gpu, workloads, synth):
    """The drivers' caches are head-major ([layer][kv_heads][rows][head_dim]):
    load_kv converts the reference's [layer][rows][kv_dim], kv_rows converts
    back, and copy_kv_rows moves rows between a BatchRunner and a Runner."""
    cfg = SMALL
    W = workloads.llama_weights(cfg, 5)
    layers, kvh, hd = cfg["layers"], cfg["kv_heads"], cfg["dim"] // cfg["heads"]
    rows = 3 * cfg["context"]
    k = synth.normal_f32(layers * rows * kvh * hd, 70, 1).reshape(layers, rows, kvh * hd)
    v = synth.normal_f32(layers * rows * kvh * hd, 70, 2).reshape(layers, rows, kvh * hd)
    br = qk.BatchRunner(cfg, W, max_tokens=2, cache_rows=rows)
    br.load_kv(k, v)
    kp, _ = br.kv_cache()
    raw = qk.copy_to_host(kp, layers * rows * kvh * hd, np.float32).reshape(layers, kvh, rows, hd)
    assert np.array_equal(raw, k.reshape(layers, rows, kvh, hd).transpose(0, 2, 1, 3))
    gk, gv = br.kv_rows(rows)
    assert np.array_equal(gk, k) and np.array_equal(gv, v)
    gk, gv = br.kv_rows(17)
    assert np.array_equal(gk, k[:, :17]) and np.array_equal(gv, v[:, :17])
    r = qk.Runner(cfg, W)
    qk.copy_kv_rows(r, br, 40)
    rk, rv = r.kv_rows(40)
    assert np.array_equal(rk, k[:, :40]) and np.array_equal(rv, v[:, :40])
    with pytest.raises(qk.QKError):
        qk.copy_kv_rows(r, br, cfg["context"] + 1)
    r.close()
    br.close()


def test_llama_1b_32_sequences_bench_shape(qk, torch_gpu, oracle, workloads, synth):
    """The batch bench.py times: 32 sequences of the random-init Llama-3.2-1B
    decoding at positions ctx - 1, ctx ~ U[64, 2048] (seed-3 descriptor), each
    sequence's rows packed in one cache (the timed step's multi-split
    attention, its merge writing the o projection's records, and the
    32-token matrix-core chain).  Every cache row holds N(0,1) values; the
    checked sequences' rows come from the workload generator and feed one
    fp64 oracle model each: the 8 longest contexts and 4 others, greedy
    tokens identical, logits rel-L2 and top-2 margin printed per sequence
    (--compare-prefill's report, inferencer.cu:1814-1825)."""
    t = torch_gpu
    case = workloads.batch_decode_1b(extra_rows=1)
    cfg, n, rows = case["cfg"], case["n"], case["rows"]
    W = workloads.llama_weights(cfg, case["weights_seed"])
    br = qk.BatchRunner(cfg, W, max_tokens=n, cache_rows=rows)
    layers, kv = cfg["layers"], cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    g = t.Generator(device="cuda")
    g.manual_seed(2)
    for dst in br.kv_cache():
        for layer in range(layers):
            blk = t.randn(rows * kv, device="cuda", generator=g)
            qk.copy_device(dst + layer * rows * kv * 4, blk.data_ptr(), rows * kv * 4)
            del blk
    pos, kv_row = case["pos"], case["kv_row"]
    order = [int(i) for i in np.argsort(pos, kind="stable")]
    checked = order[-8:] + order[0:24:6]
    host = {}
    for s in checked:
        p = pos[s]
        k = synth.normal_f32(layers * p * kv, 80, 10 + 2 * s).reshape(layers, p, kv)
        v = synth.normal_f32(layers * p * kv, 80, 11 + 2 * s).reshape(layers, p, kv)
        br.load_kv_rows(kv_row[s], k, v)
        host[s] = (k, v)
    print(f"32 sequences, positions {min(pos)}..{max(pos)}, checking {sorted(checked)}", flush=True)
    got = br.forward(case["tokens"], pos, kv_row, True)
    lg = br.logits(n)
    br.close()
    for s in checked:
        p = pos[s]
        kc = np.zeros((layers, cfg["context"], kv), dtype=np.float32)
        vc = np.zeros_like(kc)
        kc[:, :p], vc[:, :p] = host[s]
        om = oracle.Llama(cfg, W)
        om.load_cache(kc, vc, p)
        o, ref = om.forward(case["tokens"][s], p, True)
        del om
        top = np.sort(ref)[-2:]
        err = rel_l2(lg[s], ref)
        print(f"seq {s} pos {p}: gpu {got[s]} ref {o} top2 margin {top[1] - top[0]:.4f} logits rel-L2 {err:.2e}",
              flush=True)
        assert got[s] == o, s
        assert err < 1e-2, s
