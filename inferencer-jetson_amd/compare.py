"""Sequential against batched prefill: the reference's --compare-prefill
(inferencer.cu:1707-1833) over this package's two drivers.

The baseline runs the prompt one token per step through the one-sequence
driver (Runner, FastRunner::forward), the batched run feeds it as prefill
chunks of `chunk` tokens through the batched driver (BatchRunner; several
tokens of one sequence per step, causal within the chunk), both in one
arithmetic mode (the reference's INT8 modes, or FP32), and both then decode
`steps` greedy tokens.  Both drivers trace every prompt token's residual
after each layer, and in the INT8 mode the quantized inputs of each layer's
four products (qk_llama_set_trace, qk_llama_batch_set_trace).  Reported, as
the reference does:

* the residual stream after the prompt (max abs and RMS difference,
  inferencer.cu:1764-1767);
* per prompt token, the first layer whose residual differs by more than
  1e-6 (1768-1782);
* INT8: the first layer where the first token's quantized inputs differ,
  with the mismatch counts [QKV, attention output, gate/up, down]
  (1783-1797);
* per layer, the last token's residual difference and, INT8, its mismatch
  counts (1798-1813);
* per decode step, both greedy tokens, the baseline's top-2 logit margin
  and the logits' max abs / RMS difference (1814-1825).
"""
from __future__ import annotations

import numpy as np

STAGES = "[QKV, attention output, gate/up, down]"


def _diff(a, b) -> tuple[float, float]:
    d = np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)
    if d.size == 0:
        return 0.0, 0.0
    return float(np.max(np.abs(d))), float(np.sqrt(np.mean(d * d)))


def _rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a))) if a.size else 0.0


def _counts(a, b, dim: int, hidden: int) -> list[int]:
    """Mismatching codes per stage; a, b: [4][max(dim, hidden)] int8."""
    widths = (dim, dim, dim, hidden)
    return [int(np.count_nonzero(a[s, :w] != b[s, :w])) for s, w in enumerate(widths)]


def compare_prefill(qk, runner, batch, input_ids, steps: int, chunk: int, int8: bool = False) -> dict:
    """Run both prefills of input_ids and `steps` greedy steps each.

    runner: a Runner with context >= len(input_ids) + steps; batch: a
    BatchRunner with max_tokens >= chunk and cache_rows >= len(input_ids) +
    steps (the sequence's rows start at row 0); int8: both run the
    reference's INT8 modes (set_int8), else FP32."""
    ids = [int(t) for t in input_ids]
    n = len(ids)
    if n < 1 or steps < 1 or chunk < 1:
        raise ValueError("compare_prefill needs a prompt, steps >= 1 and chunk >= 1")
    c = runner.cfg
    layers, dim, hidden = c["layers"], c["dim"], c["hidden"]
    qs = max(dim, hidden)
    runner.set_int8(int8, int8)
    batch.set_int8(int8, int8)

    # Baseline: one token per step (inferencer.cu:1731-1740), each step's
    # per-layer residuals and quantized inputs traced.
    tx = qk.DeviceBuffer(layers * dim * 4)
    tq = qk.DeviceBuffer(layers * 4 * qs)
    runner.set_trace(tx, tq)
    base_layers = np.empty((n, layers, dim), dtype=np.float32)
    base_q = {}
    nxt = 0
    for i, t in enumerate(ids):
        nxt = runner.forward(t, i, i + 1 == n)
        base_layers[i] = tx.host(np.float32).reshape(layers, dim)
        if int8 and i in (0, n - 1):
            base_q[i] = tq.host(np.int8).reshape(layers, 4, qs)
    runner.set_trace(None, None)
    base_res = runner.residual()
    base_ids, base_logits = [], []
    for i in range(steps):
        base_ids.append(nxt)
        base_logits.append(runner.logits())
        if i + 1 < steps:
            nxt = runner.forward(nxt, n + i, True)

    # Batched: prefill chunks of one sequence (kv_row 0), logits for the
    # prompt's last token only, every chunk's tokens traced.
    bx = qk.DeviceBuffer(chunk * layers * dim * 4)
    bq = qk.DeviceBuffer(chunk * layers * 4 * qs)
    batch.set_trace(bx, bq)
    bat_layers = np.empty((n, layers, dim), dtype=np.float32)
    bat_q = {}
    for c0 in range(0, n, chunk):
        part = ids[c0:c0 + chunk]
        m = len(part)
        if c0 + m == n:
            nxt = batch.forward(part, list(range(c0, c0 + m)), [0] * m, seq=[0] * m, logit_rows=[m - 1])[0]
        else:
            batch.forward(part, list(range(c0, c0 + m)), [0] * m, False, seq=[0] * m)
        bat_layers[c0:c0 + m] = bx.host(np.float32, m * layers * dim).reshape(m, layers, dim)
        if int8:
            q = bq.host(np.int8, m * layers * 4 * qs).reshape(m, layers, 4, qs)
            for i in (0, n - 1):
                if c0 <= i < c0 + m:
                    bat_q[i] = q[i - c0]
    batch.set_trace(None, None)
    bat_res = batch.residual(len(ids[(n - 1) // chunk * chunk:]))[-1]
    bat_ids, bat_logits = [], []
    for i in range(steps):
        bat_ids.append(nxt)
        bat_logits.append(batch.logits(1)[0])
        if i + 1 < steps:
            nxt = batch.forward([nxt], [n + i], [0], True, seq=[0])[0]

    token_first = []
    for t in range(n):
        for layer in range(layers):
            mx, rms = _diff(base_layers[t, layer], bat_layers[t, layer])
            if mx > 1e-6:
                token_first.append({"token": t, "id": ids[t], "layer": layer, "max": mx, "rms": rms})
                break
    first_int8 = None
    if int8:
        for layer in range(layers):
            cnt = _counts(base_q[0][layer], bat_q[0][layer], dim, hidden)
            if any(cnt):
                first_int8 = {"layer": layer, "counts": cnt}
                break
    layer_rows = []
    for layer in range(layers):
        mx, rms = _diff(base_layers[n - 1, layer], bat_layers[n - 1, layer])
        row = {"layer": layer, "residual_max": mx, "residual_rms": rms,
               "residual_ref_rms": _rms(base_layers[n - 1, layer])}
        if int8:
            row["int8_mismatches"] = _counts(base_q[n - 1][layer], bat_q[n - 1][layer], dim, hidden)
        layer_rows.append(row)
    step_rows = []
    for i in range(steps):
        lg = base_logits[i]
        tid = base_ids[i]
        second = float(np.max(np.delete(lg, tid))) if lg.size > 1 else float("-inf")
        mx, rms = _diff(lg, bat_logits[i])
        step_rows.append({"step": i + 1, "baseline_token": tid, "batched_token": bat_ids[i],
                          "top2_margin": float(lg[tid]) - second, "logit_max": mx, "logit_rms": rms})
    rm, rr = _diff(base_res, bat_res)
    return {"tokens": n, "chunk": chunk, "int8": int8, "residual_max": rm, "residual_rms": rr,
            "residual_ref_rms": _rms(base_res), "token_first_over_1e-6": token_first,
            "first_int8_difference": first_int8, "layers": layer_rows, "steps": step_rows}


def format_report(index: int, rep: dict) -> list[str]:
    """The report as text lines in the reference's format (inferencer.cu:1766-1825)."""
    out = [f"Prompt {index}: residual max abs difference {rep['residual_max']:.9g}, "
           f"RMS difference {rep['residual_rms']:.9g}"]
    for t in rep["token_first_over_1e-6"]:
        out.append(f"  input token {t['token']} (id {t['id']}): first residual difference >1e-6 at layer "
                   f"{t['layer']}, max {t['max']:.9g}, RMS {t['rms']:.9g}")
    f = rep["first_int8_difference"]
    if f is not None:
        out.append(f"  input token 0 first INT8 differences at layer {f['layer']} {STAGES} "
                   + "/".join(str(x) for x in f["counts"]))
    for L in rep["layers"]:
        line = (f"  layer {L['layer']}: residual max abs difference {L['residual_max']:.9g}, RMS difference "
                f"{L['residual_rms']:.9g}")
        if "int8_mismatches" in L:
            line += f", INT8 differences {STAGES} " + "/".join(str(x) for x in L["int8_mismatches"])
        out.append(line)
    for s in rep["steps"]:
        out.append(f"  step {s['step']}: baseline token {s['baseline_token']}, batched token {s['batched_token']}, "
                   f"baseline top-2 margin {s['top2_margin']:.9g}, logit max abs difference {s['logit_max']:.9g}, "
                   f"RMS difference {s['logit_rms']:.9g}")
    return out
