"""Sequential against batched prefill: the reference's --compare-prefill
(inferencer.cu:1707-1833) over this package's two drivers.

The baseline runs the prompt one token per step through the one-sequence
driver (Runner, FastRunner::forward), the batched run feeds it as prefill
chunks of `chunk` tokens through the batched driver (BatchRunner; several
tokens of one sequence per step, causal within the chunk), and both then
decode `steps` greedy tokens.  Reported, as the reference does:

* the residual stream after the prompt (max abs and RMS difference,
  inferencer.cu:1764-1767);
* per layer, the prompt's key and value cache rows (the reference traces the
  per-layer residuals of every prompt token and names the first layer
  differing by more than 1e-6, inferencer.cu:1768-1782; the cache rows are
  what both drivers keep per layer);
* per decode step, both greedy tokens, the baseline's top-2 logit margin
  and the logits' max abs / RMS difference (inferencer.cu:1814-1825).

The reference's INT8 mismatch counts (inferencer.cu:1783-1813) have no
counterpart: the batched driver computes in FP32 (block fixed point), so the
comparison is run with the one-sequence driver in its FP32 mode.
"""
from __future__ import annotations

import numpy as np


def _diff(a, b) -> tuple[float, float]:
    d = np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64)
    if d.size == 0:
        return 0.0, 0.0
    return float(np.max(np.abs(d))), float(np.sqrt(np.mean(d * d)))


def _rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a))) if a.size else 0.0


def compare_prefill(qk, runner, batch, input_ids, steps: int, chunk: int) -> dict:
    """Run both prefills of input_ids and `steps` greedy steps each.

    runner: a Runner (FP32 mode) with context >= len(input_ids) + steps;
    batch: a BatchRunner with max_tokens >= chunk and cache_rows >=
    len(input_ids) + steps (the sequence's rows start at row 0)."""
    ids = [int(t) for t in input_ids]
    n = len(ids)
    if n < 1 or steps < 1 or chunk < 1:
        raise ValueError("compare_prefill needs a prompt, steps >= 1 and chunk >= 1")
    c = runner.cfg

    # Baseline: one token per step (inferencer.cu:1731-1740).
    nxt = 0
    for i, t in enumerate(ids):
        nxt = runner.forward(t, i, i + 1 == n)
    base_res = runner.residual()
    base_k, base_v = runner.kv_rows(n)
    base_ids, base_logits = [], []
    for i in range(steps):
        base_ids.append(nxt)
        base_logits.append(runner.logits())
        if i + 1 < steps:
            nxt = runner.forward(nxt, n + i, True)

    # Batched: prefill chunks of one sequence (kv_row 0), logits for the
    # prompt's last token only.
    for c0 in range(0, n, chunk):
        part = ids[c0:c0 + chunk]
        m = len(part)
        last = c0 + m == n
        if last:
            nxt = batch.forward(part, list(range(c0, c0 + m)), [0] * m, seq=[0] * m, logit_rows=[m - 1])[0]
        else:
            batch.forward(part, list(range(c0, c0 + m)), [0] * m, False, seq=[0] * m)
    bat_res = batch.residual(len(ids[(n - 1) // chunk * chunk:]))[-1]
    bat_k, bat_v = batch.kv_rows(n)
    bat_ids, bat_logits = [], []
    for i in range(steps):
        bat_ids.append(nxt)
        bat_logits.append(batch.logits(1)[0])
        if i + 1 < steps:
            nxt = batch.forward([nxt], [n + i], [0], True, seq=[0])[0]

    layers = []
    first = None
    for layer in range(c["layers"]):
        km, kr = _diff(base_k[layer], bat_k[layer])
        vm, vr = _diff(base_v[layer], bat_v[layer])
        layers.append({"layer": layer, "key_max": km, "key_rms": kr, "value_max": vm, "value_rms": vr,
                       "key_ref_rms": _rms(base_k[layer]), "value_ref_rms": _rms(base_v[layer])})
        if first is None and max(km, vm) > 1e-6:
            first = layer
    step_rows = []
    for i in range(steps):
        lg = base_logits[i]
        tid = base_ids[i]
        second = float(np.max(np.delete(lg, tid))) if lg.size > 1 else float("-inf")
        mx, rms = _diff(lg, bat_logits[i])
        step_rows.append({"step": i + 1, "baseline_token": tid, "batched_token": bat_ids[i],
                          "top2_margin": float(lg[tid]) - second, "logit_max": mx, "logit_rms": rms})
    rm, rr = _diff(base_res, bat_res)
    return {"tokens": n, "chunk": chunk, "residual_max": rm, "residual_rms": rr, "residual_ref_rms": _rms(base_res),
            "layers": layers,
            "first_layer_over_1e-6": first, "steps": step_rows}


def format_report(index: int, rep: dict) -> list[str]:
    """The report as text lines in the reference's wording (inferencer.cu:1766-1825)."""
    out = [f"Prompt {index}: residual max abs difference {rep['residual_max']:.9g}, "
           f"RMS difference {rep['residual_rms']:.9g}"]
    if rep["first_layer_over_1e-6"] is not None:
        out.append(f"  first key/value cache difference >1e-6 at layer {rep['first_layer_over_1e-6']}")
    for L in rep["layers"]:
        out.append(f"  layer {L['layer']}: key cache max abs difference {L['key_max']:.9g}, RMS difference "
                   f"{L['key_rms']:.9g}; value cache max abs difference {L['value_max']:.9g}, RMS difference "
                   f"{L['value_rms']:.9g}")
    for s in rep["steps"]:
        out.append(f"  step {s['step']}: baseline token {s['baseline_token']}, batched token {s['batched_token']}, "
                   f"baseline top-2 margin {s['top2_margin']:.9g}, logit max abs difference {s['logit_max']:.9g}, "
                   f"RMS difference {s['logit_rms']:.9g}")
    return out
