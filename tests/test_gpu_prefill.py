"""Continuous batches with prefill chunks on the GPU: several tokens of one
sequence in one step of the batched driver (qk_llama_batch_forward), causal
within the chunk, against the oracle's sequential decode steps
(FastRunner::prefill's contract, inferencer.cu:1279-1423: rope_cache_batch_cuda
writes every row before attention_batch_cuda reads them, 953-1041), and the
mixed continuous-batch workload's projections at 256 tokens against fp64.

Bars: projections rel-L2 <= 1e-5 per token; decode steps greedy tokens
identical to the oracle's at every position, logits within rel-L2 1e-4 on
the 2-layer model and 1e-2 on the random-init 1B model (whose O(1e4)
attention scores make fp32 score rounding move softmax weights by ~1e-3; see
test_gpu_decode.py), with the oracle's top-2 margin printed per token like
--compare-prefill (inferencer.cu:1814-1825)."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu

SMALL = dict(dim=512, layers=2, heads=8, kv_heads=2, hidden=1024, vocab=1000, context=64, eps=1e-5,
             rope_theta=10000.0)


def test_mixed_1b_256_projections(qk, torch_gpu, oracle, workloads):
    """The seed-4 mixed batch (2 prefill chunks of 96 + 64 decodes, 256 packed
    tokens): fused QKV (Q4_K q/k, Q6_K v), o, fused gate/up at K = 2048 and
    the Q6_K down projection at K = 8192, every token within rel-L2 1e-5 of
    the fp64 oracle."""
    t = torch_gpu
    case = workloads.mixed_1b_256()
    cfg, W, mix = case["cfg"], case["weights"], workloads.MIX_1B
    x, x_ffn = case["x"], case["x_ffn"]
    ntok = x.shape[0]
    assert ntok == 256 and case["desc"].n_tokens == 256
    L = qk.lib()
    dev = {n: to_dev(t, W[n]) for n in workloads.TENSORS}
    xd, xfd = to_dev(t, x), to_dev(t, x_ffn)
    out = {}

    def run(names, xin, cols):
        shapes = [workloads.tensor_shape(cfg, n) for n in names]
        ys = [t.empty((ntok, rows), device="cuda") for _, rows in shapes]
        arr = qk._matrices([(qk.Tensor((c, r), mix[n], dev[n]), y) for n, (c, r), y in zip(names, shapes, ys)])
        nb = L.qk_gemv_batched_workspace_bytes(cols, sum(r for _, r in shapes), ntok)
        ws = t.empty(max(nb, 256), dtype=t.uint8, device="cuda")
        qk.check(L.qk_gemv_multi_batched_f32(arr, len(names), xin.data_ptr(), cols, cols, ntok, ws.data_ptr(), nb,
                                             None), "mixed-256 projections")
        t.cuda.synchronize()
        for n, y in zip(names, ys):
            out[n] = y.cpu().numpy()

    run(["q", "k", "v"], xd, cfg["dim"])
    run(["o"], xd, cfg["dim"])
    run(["gate", "up"], xd, cfg["dim"])
    run(["down"], xfd, cfg["hidden"])
    for n in workloads.TENSORS:
        cols, rows = workloads.tensor_shape(cfg, n)
        ref = oracle.gemv_f64(mix[n], W[n], x_ffn if n == "down" else x, cols, rows)
        errs = [rel_l2(out[n][i], ref[i]) for i in range(ntok)]
        print(f"{n}: {rows}x{cols} worst token rel-L2 {max(errs):.2e}", flush=True)
        assert max(errs) < 1e-5, n


def _sequences(synth, cfg, seed, specs):
    """Per-sequence caches: spec (prefilled rows, chunk length); rows below
    the prefill are N(0,1), the rest zero."""
    kv = cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    out = []
    for s, (pre, _) in enumerate(specs):
        kc = np.zeros((cfg["layers"], cfg["context"], kv), dtype=np.float32)
        vc = np.zeros_like(kc)
        if pre:
            kc[:, :pre] = synth.normal_f32(cfg["layers"] * pre * kv, seed, 40 + 2 * s).reshape(cfg["layers"], pre, kv)
            vc[:, :pre] = synth.normal_f32(cfg["layers"] * pre * kv, seed, 41 + 2 * s).reshape(cfg["layers"], pre, kv)
        out.append((kc, vc))
    return out


def run_chunked(qk, oracle, wl, synth, cfg, seed, specs, logits_tol, order_seed=None, split_calls=1,
                logit_rows="all", followups=1):
    """One batched step holding, per sequence s, specs[s] = (prefilled rows,
    tokens) -- a chunk of consecutive positions from the prefill on -- in a
    shuffled token order (order_seed), optionally cut into split_calls
    consecutive calls; then `followups` decode steps of every sequence from
    its greedy successor.  Compared with one oracle model per sequence
    stepping through the same tokens one at a time."""
    W = wl.llama_weights(cfg, seed)
    ctx, S = cfg["context"], len(specs)
    seqs = _sequences(synth, cfg, seed, specs)
    br = qk.BatchRunner(cfg, W, max_tokens=sum(n for _, n in specs), cache_rows=S * ctx)
    br.load_kv(np.concatenate([k for k, _ in seqs], axis=1), np.concatenate([v for _, v in seqs], axis=1))
    orcs = []
    for s, (pre, _) in enumerate(specs):
        om = oracle.Llama(cfg, W)
        om.load_cache(seqs[s][0], seqs[s][1], pre)
        orcs.append(om)
    prompts = [[int(v) for v in synth.uniform_i32(n, seed, 70 + s, 0, cfg["vocab"] - 1)] for s, (_, n) in
               enumerate(specs)]
    entries = [(s, i) for s, (_, n) in enumerate(specs) for i in range(n)]   # (sequence, index in chunk)
    if order_seed is not None:
        perm = np.random.default_rng(order_seed).permutation(len(entries))
        entries = [entries[i] for i in perm]
    # The oracle, one token at a time per sequence.
    ref = {}
    for s, (pre, n) in enumerate(specs):
        for i in range(n):
            ref[(s, i)] = orcs[s].forward(prompts[s][i], pre + i, True)
    calls = np.array_split(np.arange(len(entries)), split_calls)
    if split_calls > 1:
        # Consecutive calls must see earlier positions first: order each
        # sequence's tokens across calls by position.
        entries = sorted(entries, key=lambda e: e[1])
    for c, idx in enumerate(calls):
        part = [entries[i] for i in idx]
        tokens = [prompts[s][i] for s, i in part]
        pos = [specs[s][0] + i for s, i in part]
        kv_row = [s * ctx for s, _ in part]
        rows = list(range(len(part))) if logit_rows == "all" else \
            [j for j, (s, i) in enumerate(part) if i == specs[s][1] - 1]
        got = br.forward(tokens, pos, kv_row, seq=[s for s, _ in part], logit_rows=rows)
        lg = br.logits(len(rows))
        for j, r in enumerate(rows):
            s, i = part[r]
            o, want = ref[(s, i)]
            top = np.sort(want)[-2:]
            err = rel_l2(lg[j], want)
            print(f"call {c} seq {s} pos {specs[s][0] + i}: gpu {got[j]} ref {o} top2 margin {top[1] - top[0]:.4f} "
                  f"logits rel-L2 {err:.2e}", flush=True)
            assert err < logits_tol, (s, i)
            assert got[j] == o, (s, i)
    # Decode steps on the caches the chunk wrote.
    tokens = [ref[(s, n - 1)][0] for s, (_, n) in enumerate(specs)]
    pos = [pre + n for pre, n in specs]
    for step in range(followups):
        got = br.forward(tokens, pos, [s * ctx for s in range(S)], True)
        lg = br.logits(S)
        want = []
        for s in range(S):
            o, r = orcs[s].forward(tokens[s], pos[s], True)
            err = rel_l2(lg[s], r)
            print(f"decode {step} seq {s} pos {pos[s]}: gpu {got[s]} ref {o} logits rel-L2 {err:.2e}", flush=True)
            assert err < logits_tol
            want.append(o)
        assert got == want
        tokens = want
        pos = [p + 1 for p in pos]
    br.close()


@pytest.mark.parametrize("order_seed", [None, 7])
def test_small_llama_prefill_chunks_in_one_step(qk, torch_gpu, oracle, workloads, synth, order_seed):
    """A fresh 12-token chunk, an 8-token chunk continuing 10 prefilled rows
    and two single decode tokens in one step (26 tokens, matrix-core path),
    in packed order and shuffled."""
    specs = [(0, 12), (10, 8), (20, 1), (33, 1)]
    run_chunked(qk, oracle, workloads, synth, SMALL, seed=13, specs=specs, logits_tol=1e-4, order_seed=order_seed)


def test_small_llama_prefill_chunk_few_tokens(qk, torch_gpu, oracle, workloads, synth):
    """A 5-token chunk with one decode (6 tokens: the few-token GEMV path)."""
    run_chunked(qk, oracle, workloads, synth, SMALL, seed=14, specs=[(0, 5), (9, 1)], logits_tol=1e-4)


def test_small_llama_prefill_chunk_over_two_calls(qk, torch_gpu, oracle, workloads, synth):
    """The same chunks cut into two consecutive calls: the second call's
    tokens read rows the first wrote."""
    specs = [(0, 12), (10, 8), (20, 1), (33, 1)]
    run_chunked(qk, oracle, workloads, synth, SMALL, seed=13, specs=specs, logits_tol=1e-4, split_calls=2)


def test_llama_1b_prefill_chunk_with_decodes(qk, torch_gpu, oracle, workloads, synth):
    """Random-init Llama-3.2-1B: a fresh 96-token prefill chunk and three
    decode tokens of prefilled sequences in one step (99 tokens), every
    position's logits and greedy successor against the oracle's sequential
    steps, then one decode step of all four sequences."""
    cfg = dict(workloads.LLAMA_1B, context=640)
    specs = [(0, 96), (64, 1), (511, 1), (300, 1)]
    run_chunked(qk, oracle, workloads, synth, cfg, seed=2, specs=specs, logits_tol=1e-2, order_seed=3)


def test_batch_rejects_tokens_writing_one_row(qk, torch_gpu, workloads):
    """Two tokens at the same (kv_row, pos) would write one cache row from
    two workgroups: QK_ERR_INVALID_ARG before any launch.  So is a kv_row
    whose sum with pos overflows, and a logit row outside the batch."""
    W = workloads.llama_weights(SMALL, 5)
    br = qk.BatchRunner(SMALL, W, max_tokens=4, cache_rows=4 * SMALL["context"])
    with pytest.raises(qk.QKError) as e:
        br.forward([1, 2, 3], [5, 6, 5], [0, 0, 0], True)
    assert e.value.status == qk.QK_ERR_INVALID_ARG
    with pytest.raises(qk.QKError) as e:
        br.forward([1, 2], [5, 6], [0, 2 ** 63 - 3], True)
    assert e.value.status == qk.QK_ERR_INVALID_ARG
    with pytest.raises(qk.QKError) as e:
        br.forward([1, 2], [5, 6], [0, 64], logit_rows=[2])
    assert e.value.status == qk.QK_ERR_INVALID_ARG
    # The rejected calls left the runner usable.
    assert len(br.forward([1, 2], [5, 6], [0, 64], True)) == 2
    br.close()
