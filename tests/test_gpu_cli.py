"""Prefill comparison and command line on the GPU, over a small random-init
Llama with Llama 3's 128256-token vocabulary written to a GGUF file.

* compare_prefill (the reference's --compare-prefill, inferencer.cu:1707-1833):
  the batched driver's prefill chunks against the one-sequence driver's
  token-by-token prompt, both then decoding greedily -- identical tokens
  wherever the baseline's top-2 margin is clear of the logit difference,
  logits within rel-L2 1e-4, residual and per-layer cache rows within
  1e-3 relative.
* The command line's text equals the one-sequence driver's greedy tokens
  decoded, with sequential and with batched prefill (the prompt's cache
  rows handed from the batched to the one-sequence driver), and the fp64
  oracle's greedy tokens decoded, over the same weights (up to the first
  step whose top-2 margin is within fp32 roundoff of a tie)."""
import io
import importlib.util

import numpy as np
import pytest

import gguf_writer as gw
import llama3_vocab as V
from conftest import ROOT, rel_l2

pytestmark = pytest.mark.gpu

CFG = dict(dim=256, layers=2, heads=4, kv_heads=2, hidden=512, vocab=128256, context=128, eps=1e-5,
           rope_theta=500000.0)
PROMPT = "the quantized matrix, naïve GPU cache: 12345 tokens"


def _weights(workloads, synth):
    W = workloads.llama_weights(CFG, 31)
    for l, L in enumerate(W["layers"]):
        L["attn_norm"] = 1.0 + 0.2 * synth.normal_f32(CFG["dim"], 31, 600 + 2 * l)
        L["ffn_norm"] = 1.0 + 0.2 * synth.normal_f32(CFG["dim"], 31, 601 + 2 * l)
    return W


@pytest.fixture(scope="module")
def model(qk, workloads, synth, tmp_path_factory):
    pytest.importorskip("tokenizers")
    import inferencer_jetson_amd.tokenizer as T
    tokens, merges = V.trained_vocab(T.LLAMA3_SPLIT)
    W = _weights(workloads, synth)
    path = tmp_path_factory.mktemp("gguf") / "llama3_small.gguf"
    gw.llama_writer(CFG, W, workloads.tensor_shape, tokens=list(tokens), merges=list(merges)).write(path)
    g = qk.GGUF(path)
    g.upload()
    tok = T.Tokenizer.from_gguf(g)
    return path, g, tok, T


def _greedy(qk, g, ids, n, int8=False):
    r = qk.Runner.from_gguf(g, CFG["context"])
    r.set_int8(int8, int8)
    nxt = 0
    for i, t in enumerate(ids):
        nxt = r.forward(t, i, i + 1 == len(ids))
    out = []
    for i in range(n):
        out.append(nxt)
        nxt = r.forward(nxt, len(ids) + i, True)
    r.close()
    return out


@pytest.mark.parametrize("chunk,int8", [(4, False), (8, False), (32, False), (8, True), (32, True)])
def test_compare_prefill(qk, torch_gpu, model, chunk, int8):
    import inferencer_jetson_amd.compare as cmp
    _, g, tok, T = model
    ids = T.chat_prompt(tok, PROMPT)
    assert len(ids) > 8
    r = qk.Runner.from_gguf(g, CFG["context"])
    b = qk.BatchRunner.from_gguf(g, CFG["context"], chunk, CFG["context"])
    rep = cmp.compare_prefill(qk, r, b, ids, 6, chunk, int8=int8)
    r.close()
    b.close()
    assert rep["tokens"] == len(ids) and len(rep["layers"]) == CFG["layers"]
    # Random-init weights make activations and attention scores large, so
    # the two drivers' roundoff (different kernels, ~1e-7 relative) is
    # amplified through the softmax from layer to layer; in the INT8 mode a
    # code on a rounding midpoint can go either way as well.  Relative bars
    # on the diagnostics the reference prints, strict on the tokens.
    bar = 2e-2 if int8 else 1e-3
    assert rep["residual_rms"] < bar * rep["residual_ref_rms"]
    for L in rep["layers"]:
        assert L["residual_rms"] < bar * L["residual_ref_rms"], L
        if int8:
            assert sum(L["int8_mismatches"]) <= 0.02 * (3 * CFG["dim"] + CFG["hidden"]), L
        else:
            assert "int8_mismatches" not in L
    for s in rep["steps"]:
        if s["top2_margin"] > 100 * s["logit_max"]:
            assert s["baseline_token"] == s["batched_token"], s
    assert rep["steps"][0]["baseline_token"] == rep["steps"][0]["batched_token"]
    lines = cmp.format_report(1, rep)
    assert lines[0].startswith("Prompt 1: residual max abs difference") and len(lines) >= 1 + CFG["layers"] + 6
    layer_lines = [l for l in lines if l.startswith("  layer ")]
    assert len(layer_lines) == CFG["layers"]
    assert all(("INT8 differences [QKV, attention output, gate/up, down]" in l) == int8 for l in layer_lines)


def test_compare_prefill_logits_close(qk, torch_gpu, model):
    """The prompt's last-token logits of both drivers within rel-L2 1e-4."""
    _, g, tok, T = model
    ids = T.chat_prompt(tok, PROMPT)
    r = qk.Runner.from_gguf(g, CFG["context"])
    b = qk.BatchRunner.from_gguf(g, CFG["context"], 32, CFG["context"])
    for i, t in enumerate(ids):
        r.forward(t, i, i + 1 == len(ids))
    n = len(ids)
    b.forward(ids, list(range(n)), [0] * n, seq=[0] * n, logit_rows=[n - 1])
    la, lb = r.logits(), b.logits(1)[0]
    assert rel_l2(lb, la) < 1e-4
    assert rel_l2(b.residual(n)[n - 1], r.residual()) < 1e-4
    r.close()
    b.close()


def _cli():
    spec = importlib.util.spec_from_file_location("qk_cli", ROOT / "inferencer-jetson_amd" / "__main__.py")
    cli = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(cli)
    return cli


def _run(cli, args):
    out, err = io.BytesIO(), io.StringIO()
    rc = cli.run(args, stdout=out, stderr=err, stdin=io.StringIO(""))
    return rc, out.getvalue(), err.getvalue()


@pytest.mark.parametrize("prefill", [1, 8])
def test_cli_generates_the_drivers_tokens(qk, torch_gpu, model, prefill):
    path, g, tok, T = model
    ids = T.chat_prompt(tok, PROMPT)
    n = 6
    want = _greedy(qk, g, ids, n)
    stop = tok.stop_ids()
    text = b""
    for t in want:
        if t in stop:
            break
        text += tok.decode(t)
    cli = _cli()
    rc, out, err = _run(cli, ["--model", str(path), "--context", "128", "--max-tokens", str(n), "--float-gemv",
                              "--prefill-batch", str(prefill), "--stats", PROMPT])
    assert rc == 0, err
    assert out == text + b"\n", (out, text)
    assert "steady decode" in err and "Total:" in err
    # Matrix products counted as FastGPU::calls counts them: seven per layer
    # and token of the prompt plus its one LM head, then seven per layer and
    # one LM head per decode step (a stop token ends the loop after its step).
    shown = 0
    while shown < n and want[shown] not in stop:
        shown += 1
    steps = n - 1 if shown == n else shown
    calls = 7 * CFG["layers"] * len(ids) + 1 + steps * (7 * CFG["layers"] + 1)
    assert f"s across {calls} quantized matrix calls" in err, err
    assert "  GPU pipeline: " in err and "Model: " in err


def test_cli_int8_default_and_compare_output(qk, torch_gpu, model):
    path, g, tok, T = model
    ids = T.chat_prompt(tok, PROMPT)
    want = _greedy(qk, g, ids, 4, int8=True)
    stop = tok.stop_ids()
    text = b""
    for t in want:
        if t in stop:
            break
        text += tok.decode(t)
    cli = _cli()
    rc, out, err = _run(cli, ["--model", str(path), "--context", "128", "--max-tokens", "4", PROMPT])
    assert rc == 0, err
    assert out == text + b"\n"
    assert "Q4_K matrix path: INT8; Q6_K matrix path: INT8" in err
    # INT8 batched prefill (the reference's only batched mode) runs and
    # counts the prompt's products the same way.
    rc, out2, err2 = _run(cli, ["--model", str(path), "--context", "128", "--max-tokens", "4", "--prefill-batch", "8",
                                "--stats", PROMPT])
    assert rc == 0, err2
    assert out2.endswith(b"\n") and "quantized matrix calls" in err2
    rc, out, err = _run(cli, ["--model", str(path), "--context", "128", "--max-tokens", "5", "--prefill-batch", "6",
                              "--compare-prefill", PROMPT])
    assert rc == 0, err
    lines = out.decode().splitlines()
    assert lines[0].startswith("Prompt 1: residual max abs difference")
    assert sum("INT8 differences [QKV, attention output, gate/up, down]" in l for l in lines) == CFG["layers"]
    steps = [l for l in lines if l.startswith("  step ")]
    assert len(steps) == 5
    assert all("baseline token" in l and "batched token" in l and "top-2 margin" in l for l in steps)


@pytest.mark.parametrize("int8", [False, True])
def test_cli_text_matches_the_oracle(qk, torch_gpu, oracle, workloads, synth, model, int8):
    """The command line (sequential prefill; FP32 GEMVs, or the reference's
    default INT8 modes) against the fp64 oracle model in the same mode,
    built from the same weights the GGUF file holds: the oracle's greedy
    tokens, decoded, are a prefix of the printed text up to the first step
    whose top-2 margin is below 1e-3 (FP32: where fp32 roundoff may pick the
    other token) or 0.5 (INT8: where a code one step off a quantization
    midpoint may), and at least three steps are compared."""
    path, g, tok, T = model
    W = _weights(workloads, synth)
    ids = T.chat_prompt(tok, PROMPT)
    n = 8
    om = oracle.Llama(CFG, W)
    om.set_int8(int8, int8)
    nxt = lg = None
    for i, t in enumerate(ids):
        nxt, lg = om.forward(int(t), i, i + 1 == len(ids))
    want, margins = [], []
    for i in range(n):
        top = np.sort(lg)[-2:]
        want.append(int(nxt))
        margins.append(float(top[1] - top[0]))
        if i + 1 < n:
            nxt, lg = om.forward(int(nxt), len(ids) + i, True)
    del om
    stop = tok.stop_ids()
    clear = 0
    while clear < n and margins[clear] > (0.5 if int8 else 1e-3) and want[clear] not in stop:
        clear += 1
    print("oracle tokens", want, "margins", [f"{m:.3g}" for m in margins], flush=True)
    assert clear >= 3
    text = b"".join(tok.decode(t) for t in want[:clear])
    rc, out, err = _run(_cli(), ["--model", str(path), "--context", "128", "--max-tokens", str(n)] +
                        ([] if int8 else ["--float-gemv"]) + [PROMPT])
    assert rc == 0, err
    assert out.startswith(text), (out, text)
