#!/usr/bin/env python3
"""Benchmark of the Q4_K / Q6_K dequant-GEMV hot path on one MI355X.

A step is one pass of the hot path over one batch of synthetic input: one
Q6_K GEMV over the tied LM head, 128256 x 2048 (215.5 MB of super-blocks),
batch 1, fp32 activations, weights in the split Q6_K layout that the model
drivers repack them into at load time (qk_q6k_split: the same bytes, fields
16-byte aligned); the GGUF-layout time is reported beside it.  Four weight
copies of that matrix (862 MB) rotate from step to step so that the ~256 MB
last-level cache cannot serve them; all inputs are resident in HBM before
timing starts.

value = algorithmic bytes per step (weights + x + y) * steps / wall time of
the timed region (synchronize on both sides).  roofline.achieved divides the
same bytes by the average kernel duration: the span of a HIP event pair
recorded on the launch stream around the timed launches, divided by the
number of launches.  cpu_baseline times the
oracle's OpenMP restatement of the reference's FP32 GEMV (inferencer.cu:
645-661) on the host cores over a bounded row sample of the same matrix.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import pathlib
import re
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
PKG_NAME = "inferencer_jetson_amd"
HBM_PEAK_GBPS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0   # dense fp16 / bf16 matrix-core peak of MI355X
METRIC = "Q4_K/Q6_K GEMV HBM GB/s (% of peak); batched decode tokens/s (1 GPU)"


def load_package():
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    pkg_dir = ROOT / "inferencer-jetson_amd"
    spec = importlib.util.spec_from_file_location(PKG_NAME, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def profile_value(name: str, key: str):
    """A figure from a committed rocprofv3 summary (profiles/<name>.md, a line
    '<key>: N'), or None."""
    path = ROOT / "profiles" / f"{name}.md"
    if not path.exists():
        return None
    m = re.search(re.escape(key) + r":\s*([0-9.eE+]+)", path.read_text())
    return float(m.group(1)) if m else None


def measured_traffic(name: str):
    """HBM bytes per launch from a committed rocprofv3 PMC summary
    (profiles/<name>.md, a line 'traffic_bytes_per_launch: N'), or None."""
    return profile_value(name, "traffic_bytes_per_launch")


def time_launches(torch, launch, steps: int, warmup: int, stream):
    """Runs warmup + timed launches; returns (wall seconds of the timed
    region, mean ms per launch from one pair of HIP events recorded on
    `stream` around the timed launches).  The launches are queued faster
    than they run, so the event span is the kernels back to back plus the
    dispatch gaps between them."""
    for i in range(warmup):
        launch(i)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        launch(warmup + i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) / steps


def cpu_baseline_lm_head(workloads, sample_rows: int, target_s: float) -> dict:
    """The oracle's OpenMP restatement of gemv_quant<14> on a row sample of
    the LM-head matrix: warm-up, then timed repetitions for about target_s
    seconds (at least 20); the median repetition is reported."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle  # noqa: E402  (the CPU baseline leg only)
    import numpy as np
    w, x = workloads.lm_head_q6k()
    row_bytes = 8 * 210
    ws = np.ascontiguousarray(w[: sample_rows * row_bytes])
    for _ in range(3):
        oracle.gemv_f32_ref(14, ws, x, 2048, sample_rows)           # warm
    times, t0 = [], time.perf_counter()
    while len(times) < 20 or time.perf_counter() - t0 < target_s:
        t = time.perf_counter()
        oracle.gemv_f32_ref(14, ws, x, 2048, sample_rows)
        times.append(time.perf_counter() - t)
    med = float(np.median(times))
    sample_bytes = sample_rows * row_bytes + 2048 * 4 + sample_rows * 4
    threads = oracle.omp_max_threads()
    return {"value": round(sample_bytes / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"Q6_K GEMV over the first {sample_rows} rows (x 2048) of the LM-head matrix; median of "
                      f"{len(times)} timed repetitions ({sum(times):.1f} s); OpenMP static rows, "
                      f"omp_get_max_threads()={threads}, nproc={os.cpu_count()}"}


def bench_small_gemvs(torch, qk, wl, stream) -> dict:
    """Q4_K 2048x2048 (launch-bound) and the fused 1B gate/up over 16 layers."""
    sec = {}
    w1, x1 = wl.gemv_q4k_2048()
    w1d, x1d = torch.from_numpy(w1).to("cuda"), torch.from_numpy(x1).to("cuda")
    y1 = torch.empty(2048, device="cuda")
    t1 = qk.Tensor((2048, 2048), qk.Q4_K, w1d)
    _, k1 = time_launches(torch, lambda i: qk.matvec(t1, x1d, y1, 2048, 2048, stream), 200, 20, stream)
    b1 = qk.tensor_bytes(qk.Q4_K, 2048, 2048) + 2048 * 8
    sec["gemv_q4k_2048x2048"] = {"kernel_us": round(k1 * 1e3, 2), "GBps_kernel": round(b1 / (k1 * 1e-3) / 1e9, 1)}
    gu = []
    for l in range(16):
        wg = wl.synth.quant_matrix(qk.Q4_K, 2048, 8192, 2, 100 + 16 * l + 4, 0.02)
        wu = wl.synth.quant_matrix(qk.Q4_K, 2048, 8192, 2, 100 + 16 * l + 5, 0.02)
        gu.append((qk.Tensor((2048, 8192), qk.Q4_K, torch.from_numpy(wg).to("cuda")),
                   qk.Tensor((2048, 8192), qk.Q4_K, torch.from_numpy(wu).to("cuda"))))
    g = torch.empty(8192, device="cuda")
    u = torch.empty(8192, device="cuda")
    xg = torch.from_numpy(wl.synth.normal_f32(2048, 2, 7)).to("cuda")
    _, k2 = time_launches(
        torch, lambda i: qk.gate_up(gu[i % 16][0], gu[i % 16][1], xg, g, u, 2048, 8192, stream), 320, 32, stream)
    b2 = 2 * qk.tensor_bytes(qk.Q4_K, 2048, 8192) + 2048 * 4 + 2 * 8192 * 4
    sec["gemv_q4k_gate_up_1b_2x8192x2048"] = {
        "kernel_us": round(k2 * 1e3, 2), "GBps_kernel": round(b2 / (k2 * 1e-3) / 1e9, 1),
        "frac_of_peak": round(b2 / (k2 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
    return sec


def bench_q4k_lm_shape(torch, qk, wl, stream, copies: int) -> dict:
    """Q4_K GEMV at the LM-head shape 128256 x 2048 (147.7 MB of super-blocks,
    rotating copies): the Q4_K kernel's sustained rate, which the 1B / 3B
    Q4_K projections (2.4-14 MB each) are too small to show in one launch."""
    cols, rows = 2048, 128256
    ts = [qk.Tensor((cols, rows), qk.Q4_K,
                    torch.from_numpy(wl.synth.quant_matrix(qk.Q4_K, cols, rows, 6, 1 + 16 * c, 0.02)).to("cuda"))
          for c in range(copies)]
    x = torch.from_numpy(wl.synth.normal_f32(cols, 6, 2)).to("cuda")
    y = torch.empty(rows, device="cuda")
    _, k = time_launches(torch, lambda i: qk.matvec(ts[i % copies], x, y, cols, rows, stream), 2000, 2000, stream)
    b = qk.tensor_bytes(qk.Q4_K, cols, rows) + cols * 4 + rows * 4
    # The reference's default INT8 mode on the same copies (gemv_q4_dp4a,
    # inferencer.cu:518-569): x quantized once outside the timed launches.
    xq = torch.empty(cols, dtype=torch.int8, device="cuda")
    xs = torch.empty(cols // 32, dtype=torch.float32, device="cuda")
    qk.quantize(x, xq, xs, cols, stream=stream)
    _, ki = time_launches(torch, lambda i: qk.matvec_i8(ts[i % copies], xq, xs, y, cols, rows, stream=stream),
                          2000, 2000, stream)
    bi = qk.tensor_bytes(qk.Q4_K, cols, rows) + cols + cols // 32 * 4 + rows * 4
    return {"kernel_us": round(k * 1e3, 2), "GBps_kernel": round(b / (k * 1e-3) / 1e9, 1),
            "frac_of_peak": round(b / (k * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4), "bytes_per_launch": b,
            "int8": {"kernel_us": round(ki * 1e3, 2), "bytes_per_launch": bi,
                     "frac_of_peak": round(bi / (ki * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}


def bench_lm_head_3b(torch, qk, wl, stream, copies: int) -> dict:
    """The Llama-3.2-3B tied LM head: split Q6_K 128256 x 3072 (323 MB of
    super-blocks, rotating copies), batch 1, FP32 and INT8 (x quantized once
    outside the timed launches).  Three waves share each four-row tile here
    (the multi-wave-tile GEMV kernel)."""
    cols, rows = 3072, 128256
    ts = []
    for c in range(copies):
        g = qk.Tensor((cols, rows), qk.Q6_K,
                      torch.from_numpy(wl.synth.quant_matrix(qk.Q6_K, cols, rows, 9, 1 + 16 * c, 0.02)).to("cuda"))
        ts.append(qk.split_q6k(g, stream))
        del g
    x = torch.from_numpy(wl.synth.normal_f32(cols, 9, 2)).to("cuda")
    y = torch.empty(rows, device="cuda")
    _, k = time_launches(torch, lambda i: qk.matvec(ts[i % copies], x, y, cols, rows, stream), 1000, 500, stream)
    b = qk.tensor_bytes(qk.Q6_K_SPLIT, cols, rows) + cols * 4 + rows * 4
    xq = torch.empty(cols, dtype=torch.int8, device="cuda")
    xs = torch.empty(cols // 32, dtype=torch.float32, device="cuda")
    qk.quantize(x, xq, xs, cols, stream=stream)
    _, ki = time_launches(torch, lambda i: qk.matvec_i8(ts[i % copies], xq, xs, y, cols, rows, stream=stream),
                          1000, 500, stream)
    bi = qk.tensor_bytes(qk.Q6_K_SPLIT, cols, rows) + cols + cols // 32 * 4 + rows * 4
    return {"kernel_us": round(k * 1e3, 2), "bytes_per_launch": b,
            "frac_of_peak": round(b / (k * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "int8": {"kernel_us": round(ki * 1e3, 2), "bytes_per_launch": bi,
                     "frac_of_peak": round(bi / (ki * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}


def _workspace(torch, qk, cols, rows, ntok):
    n = qk.batch_workspace_bytes(cols, rows, ntok)
    return torch.empty(max(n, 256), dtype=torch.uint8, device="cuda"), n


def bench_ffn_3b_ragged(torch, qk, wl, stream, copies: int = 8, steps: int = 200, warmup: int = 16,
                        int8: bool = False) -> dict:
    """Llama-3.2-3B FFN for 32 decode tokens of 32 sequences (ragged context
    lengths 64..2048 in the batch descriptor; the FFN reads only the token
    count): fused gate/up (Q4_K 2 x 8192 x 3072), SiLU * up, down (Q6_K
    3072 x 8192).  `copies` weight sets rotate so the last-level cache cannot
    hold them (8 x 49 MB).  With int8, the reference's INT8 mode
    (FastRunner's batched INT8 FFN, inferencer.cu:1362-1380): x quantized
    per 32, then qk_ffn_batched_i8 (3 launches, quantization included in
    the timed step)."""
    dim, hidden, ntok = 3072, 8192, 32
    sets = []
    x_host = None
    for c in range(copies):
        case = wl.ffn_3b_ragged(copy=c)
        x_host = case["x"] if x_host is None else x_host
        sets.append(tuple(torch.from_numpy(case[k]).to("cuda") for k in ("gate", "up", "down")))
    x = torch.from_numpy(x_host).to("cuda")
    gate = torch.empty((ntok, hidden), device="cuda")
    up = torch.empty((ntok, hidden), device="cuda")
    y = torch.empty((ntok, dim), device="cuda")
    L = qk.lib()
    s = qk.stream_handle(stream)

    if int8:
        # x quantized per 32 (quantize_batch_cuda), then one call
        # (qk_ffn_batched_i8): gate / up on the integer matrix cores with
        # SiLU(gate) * up quantized in their epilogue, and down.
        xq = torch.empty((ntok, dim), dtype=torch.int8, device="cuda")
        xs = torch.empty((ntok, dim // 32), dtype=torch.float32, device="cuda")
        n_i = L.qk_ffn_batched_i8_workspace_bytes(dim, hidden, ntok)
        ws_i = torch.empty(n_i, dtype=torch.uint8, device="cuda")
        split_down = [qk.split_q6k(qk.Tensor((hidden, dim), qk.Q6_K, wd), stream).data for _, _, wd in sets]

        def run(i, down_type, downs):
            wg, wu, _ = sets[i % copies]
            qk.quantize(x, xq, xs, dim, n_tokens=ntok, stream=stream)
            qk.check(L.qk_ffn_batched_i8(qk.Q4_K, wg.data_ptr(), qk.Q4_K, wu.data_ptr(), down_type,
                                         downs[i % copies].data_ptr(), xq.data_ptr(), dim, xs.data_ptr(), dim // 32,
                                         y.data_ptr(), dim, dim, hidden, ntok, 0, ws_i.data_ptr(), n_i, s), "INT8 FFN")

        wall, ms = time_launches(torch, lambda i: run(i, qk.Q6_K, [d for _, _, d in sets]), steps, warmup, stream)
        _, ms_split = time_launches(torch, lambda i: run(i, qk.Q6_K_SPLIT, split_down), steps, warmup, stream)
        weights = 2 * qk.tensor_bytes(qk.Q4_K, dim, hidden) + qk.tensor_bytes(qk.Q6_K, hidden, dim)
        # Per token: x in (4 dim), its codes and scales out and in again
        # (dim + dim/8 each way), the hidden codes and scales out and in
        # again (hidden + hidden/8 each way), y out (4 dim).
        act = ntok * (4 * dim + 2 * (dim + dim // 8) + 2 * (hidden + hidden // 8) + 4 * dim)
        return {"tokens": ntok, "ms_per_step": round(ms, 4), "tokens_per_s": round(ntok / (ms * 1e-3), 1),
                "bytes_per_step": weights + act, "GBps": round((weights + act) / (ms * 1e-3) / 1e9, 1),
                "frac_of_peak": round((weights + act) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                "weight_copies": copies, "calls_per_step": 2, "launches_per_step": 3,
                "split_q6k_down": {"ms_per_step": round(ms_split, 4),
                                   "frac_of_peak": round((weights + act) / (ms_split * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}

    # One call (qk_ffn_batched_f32): x packed once, gate / up on the matrix
    # cores with SiLU(gate) * up packed by their reduction straight into the
    # down projection's input records, down and its reduction.
    n_f = L.qk_ffn_batched_workspace_bytes(dim, hidden, ntok)
    ws_f = torch.empty(n_f, dtype=torch.uint8, device="cuda")

    def step(i):
        wg, wu, wd = sets[i % copies]
        qk.check(L.qk_ffn_batched_f32(qk.Q4_K, wg.data_ptr(), qk.Q4_K, wu.data_ptr(), qk.Q6_K, wd.data_ptr(),
                                      x.data_ptr(), dim, y.data_ptr(), dim, dim, hidden, ntok, 0, ws_f.data_ptr(), n_f,
                                      s), "ffn")

    wall, ms = time_launches(torch, step, steps, warmup, stream)
    # The same call with down in the split Q6_K layout, as the decode drivers
    # hold it (a copy made once at load time by qk_q6k_split).
    split_down = [qk.split_q6k(qk.Tensor((hidden, dim), qk.Q6_K, wd), stream).data for _, _, wd in sets]

    def step_split(i):
        wg, wu, _ = sets[i % copies]
        qk.check(L.qk_ffn_batched_f32(qk.Q4_K, wg.data_ptr(), qk.Q4_K, wu.data_ptr(), qk.Q6_K_SPLIT,
                                      split_down[i % copies].data_ptr(), x.data_ptr(), dim, y.data_ptr(), dim, dim,
                                      hidden, ntok, 0, ws_f.data_ptr(), n_f, s), "ffn")

    _, ms_split = time_launches(torch, step_split, steps, warmup, stream)
    weights = 2 * qk.tensor_bytes(qk.Q4_K, dim, hidden) + qk.tensor_bytes(qk.Q6_K, hidden, dim)
    # x in, the SiLU * up product (4 bytes a value as fp16 high / low
    # records), y out.
    act = 4 * ntok * (dim + hidden + dim)
    return {"tokens": ntok, "ms_per_step": round(ms, 4), "tokens_per_s": round(ntok / (ms * 1e-3), 1),
            "bytes_per_step": weights + act, "GBps": round((weights + act) / (ms * 1e-3) / 1e9, 1),
            "frac_of_peak": round((weights + act) / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            "weight_copies": copies, "calls_per_step": 1, "launches_per_step": 5,
            "split_q6k_down": {"ms_per_step": round(ms_split, 4),
                               "frac_of_peak": round((weights + act) / (ms_split * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}}


def bench_mixed_1b_256(torch, qk, wl, stream, steps: int = 20, warmup: int = 3) -> dict:
    """256 packed tokens (2 prefill chunks of 96 + 64 decodes) through the
    seven projections of all 16 Llama-3.2-1B layers on the matrix cores:
    fused QKV (Q4_K q/k, Q6_K v), o (Q4_K), fused gate/up (Q4_K), SiLU * up,
    down (Q6_K).  Useful flops = 2 * 256 * (weights per layer) * 16."""
    cfg = wl.LLAMA_1B
    dim, hidden, ntok = cfg["dim"], cfg["hidden"], 256
    kv = dim // cfg["heads"] * cfg["kv_heads"]
    case = wl.mixed_1b_256()
    layers = []
    for l in range(cfg["layers"]):
        W = {}
        for j, name in enumerate(wl.TENSORS):
            cols, rows = wl.tensor_shape(cfg, name)
            host = case["weights"][name] if l == 0 else wl.synth.quant_matrix(
                wl.MIX_1B[name], cols, rows, 4, 1 + 16 * l + j, wl.SIGMA[wl.MIX_1B[name]])
            W[name] = torch.from_numpy(host).to("cuda")
        layers.append(W)
    x = torch.from_numpy(case["x"]).to("cuda")
    q = torch.empty((ntok, dim), device="cuda")
    k = torch.empty((ntok, kv), device="cuda")
    v = torch.empty((ntok, kv), device="cuda")
    o = torch.empty((ntok, dim), device="cuda")
    gate = torch.empty((ntok, hidden), device="cuda")
    up = torch.empty((ntok, hidden), device="cuda")
    y = torch.empty((ntok, dim), device="cuda")
    ws_qkv, n_qkv = _workspace(torch, qk, dim, dim + 2 * kv, ntok)
    ws_o, n_o = _workspace(torch, qk, dim, dim, ntok)
    ws_gu, n_gu = _workspace(torch, qk, dim, 2 * hidden, ntok)
    ws_d, n_d = _workspace(torch, qk, hidden, dim, ntok)
    L = qk.lib()
    s = qk.stream_handle(stream)
    mix = wl.MIX_1B

    def T(name, W):
        cols, rows = wl.tensor_shape(cfg, name)
        return qk.Tensor((cols, rows), mix[name], W[name])

    def step(i):
        for W in layers:
            arr = qk._matrices([(T("q", W), q), (T("k", W), k), (T("v", W), v)])
            qk.check(L.qk_gemv_multi_batched_f32(arr, 3, x.data_ptr(), dim, dim, ntok, ws_qkv.data_ptr(), n_qkv, s),
                     "qkv")
            qk.check(L.qk_gemv_batched_f32(mix["o"], W["o"].data_ptr(), q.data_ptr(), dim, o.data_ptr(), dim, dim,
                                           dim, ntok, ws_o.data_ptr(), n_o, s), "o")
            arr = qk._matrices([(T("gate", W), gate), (T("up", W), up)])
            qk.check(L.qk_gemv_multi_batched_f32(arr, 2, x.data_ptr(), dim, dim, ntok, ws_gu.data_ptr(), n_gu, s),
                     "gate/up")
            qk.check(L.qk_silu_mul_f32(gate.data_ptr(), up.data_ptr(), ntok * hidden, s), "silu")
            qk.check(L.qk_gemv_batched_f32(mix["down"], W["down"].data_ptr(), gate.data_ptr(), hidden, y.data_ptr(),
                                           dim, hidden, dim, ntok, ws_d.data_ptr(), n_d, s), "down")

    wall, ms = time_launches(torch, step, steps, warmup, stream)
    per_layer = sum(wl.tensor_shape(cfg, n)[0] * wl.tensor_shape(cfg, n)[1] for n in wl.TENSORS)
    flops = 2.0 * ntok * per_layer * cfg["layers"]
    tflops = flops / (ms * 1e-3) / 1e12
    return {"tokens": ntok, "packing": "2 prefill chunks x 96 + 64 decodes", "ms_per_step": round(ms, 4),
            "tokens_per_s": round(ntok / (ms * 1e-3), 1), "useful_TFLOPs": round(tflops, 1),
            "mfma_util_of_fp16_dense_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "mfma_ops_per_useful_product": 2,
            # SQ_VALU_MFMA_BUSY_CYCLES over the summed dispatch time, from the
            # committed rocprofv3 counter run of this workload.
            "mfma_busy_counters": profile_value("batched_gemm_mfma_counters", "mfma_busy_mixed_256"),
            "launches_per_step": 5 * cfg["layers"]}


def bench_decode_1b(torch, qk, wl, int8: bool = False) -> dict:
    """Random-init Llama-3.2-1B decode, one sequence: KV prefilled at 0..511,
    16 prompt tokens at 512..527, then 64 greedy tokens, each step ending in
    the 4-byte token download (FastRunner::forward, inferencer.cu:1424-1531).
    int8: the reference's default INT8 GEMVs (use_dp4a, use_q6_dp4a) with
    --fused-norm-quant.  Timed: the 64 greedy steps, wall clock."""
    w = wl.LLAMA_1B_DECODE
    cfg = w.cfg
    W = wl.llama_weights(cfg, w.seed)
    kc, vc = wl.llama_kv_prefill(cfg, w.seed, w.prefill_positions)
    run = qk.Runner(cfg, W)
    if int8:
        run.set_int8(True, True)
    run.load_kv(kc, vc)
    prompt = wl.llama_prompt(cfg, w.seed, w.prompt_tokens)
    pos = w.prefill_positions
    for i, tok in enumerate(prompt):
        nxt = run.forward(int(tok), pos, i == len(prompt) - 1)
        pos += 1
    torch.cuda.synchronize()
    start_pos = pos
    t0 = time.perf_counter()
    for _ in range(w.greedy_tokens):
        nxt = run.forward(nxt, pos, True)
        pos += 1
    el = time.perf_counter() - t0
    mem = run.memory()
    run.close()
    kv_dim = cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    weights = sum(qk.tensor_bytes(wl.MIX_1B[n], *wl.tensor_shape(cfg, n)) for n in wl.TENSORS) * cfg["layers"] + \
        qk.tensor_bytes(qk.Q6_K, cfg["dim"], cfg["vocab"])
    kv_bytes = sum(cfg["layers"] * (p + 1) * kv_dim * 4 * 2 for p in range(start_pos, pos))
    per_tok = el / w.greedy_tokens
    gbps = (weights * w.greedy_tokens + kv_bytes) / el / 1e9
    return {"tokens": w.greedy_tokens, "ms_per_token": round(per_tok * 1e3, 4),
            "tokens_per_s": round(1.0 / per_tok, 1), "weight_bytes_per_token": weights,
            "GBps": round(gbps, 1), "frac_of_peak": round(gbps / HBM_PEAK_GBPS, 4),
            # FP32 (activation records), per layer: QKV, attention (rows
            # split), o (merging the splits, +add), gate/up, down; then the
            # embedding, the LM head and the greedy pick.  INT8, per layer:
            # QKV (RMSNorm + quantize staged), attention (rows split), o
            # (merging the splits, +add), gate/up (RMSNorm + quantize staged,
            # SiLU*up quantized in the epilogue), down (+add); then the LM
            # head (RMSNorm + quantize staged, greedy partials) and the final
            # pick, which also writes the next token's embedding row (no
            # embedding launch in a greedy step).
            "kernels_per_token": 5 * cfg["layers"] + (2 if int8 else 3),
            "device_bytes": mem}


def _fill_caches(torch, runner, cfg, rows: int, seed: int) -> None:
    """N(0,1) in every row of the runner's packed caches, drawn on the device."""
    import ctypes
    kv_dim = cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    kp, vp = runner.kv_cache()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    per_layer = rows * kv_dim
    for dst in (kp, vp):
        for l in range(cfg["layers"]):
            blk = torch.randn(per_layer, device="cuda", generator=g)
            if hip.hipMemcpy(dst + l * per_layer * 4, blk.data_ptr(), per_layer * 4, 3) != 0:
                raise RuntimeError("device copy failed")
            del blk
    torch.cuda.synchronize()


def bench_mixed_1b_step(torch, qk, wl, steps: int = 10, warmup: int = 3) -> dict:
    """The mixed continuous batch end to end: one step of the random-init
    Llama-3.2-1B (seed 4) over 256 packed tokens -- two fresh 96-token
    prefill chunks (positions 0..95, causal within the chunk) and 64 decode
    tokens at positions ctx - 1, ctx ~ U[64, 2048] -- through
    qk_llama_batch_forward_rows: embedding, 16 layers (projections on the
    matrix cores, RoPE + KV write, attention), and the LM head plus greedy
    pick for the 66 tokens that produce logits (each chunk's last token and
    every decode).  Every step repeats the same positions."""
    import numpy as np
    cfg = dict(wl.LLAMA_1B, context=2048)
    W = wl.llama_weights(cfg, 4)
    d = wl.mixed_1b_256()["desc"]
    seq, pos = d.seq_id.astype(int), d.pos.astype(int)
    n_seq = int(seq.max()) + 1
    cap = [int(d.ctx_len[np.flatnonzero(seq == s)[0]]) for s in range(n_seq)]
    start = np.concatenate([[0], np.cumsum(cap[:-1])]).astype(int)
    rows = int(sum(cap))
    runner = qk.BatchRunner(cfg, W, max_tokens=d.n_tokens, cache_rows=rows)
    _fill_caches(torch, runner, cfg, rows, 4)
    tokens = [int(x) for x in wl.synth.uniform_i32(d.n_tokens, 4, 7, 0, cfg["vocab"] - 1)]
    kv_row = [int(start[s]) for s in seq]
    last = {s: i for i, s in enumerate(seq)}
    logit_rows = sorted(last.values())
    for _ in range(warmup):
        runner.forward(tokens, pos, kv_row, seq=seq, logit_rows=logit_rows)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        runner.forward(tokens, pos, kv_row, seq=seq, logit_rows=logit_rows)
    el = time.perf_counter() - t0
    runner.close()
    ms = el / steps * 1e3
    per_layer = sum(wl.tensor_shape(cfg, n)[0] * wl.tensor_shape(cfg, n)[1] for n in wl.TENSORS)
    proj = 2.0 * d.n_tokens * per_layer * cfg["layers"]
    head = 2.0 * len(logit_rows) * cfg["dim"] * cfg["vocab"]
    tflops = (proj + head) / (ms * 1e-3) / 1e12
    return {"tokens": d.n_tokens, "logit_tokens": len(logit_rows),
            "packing": "2 prefill chunks x 96 (positions 0..95) + 64 decodes (ctx ~ U[64, 2048])",
            "ms_per_step": round(ms, 4), "tokens_per_s": round(d.n_tokens / (ms * 1e-3), 1),
            "useful_matrix_TFLOPs": round(tflops, 1),
            "mfma_util_of_fp16_dense_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "mfma_ops_per_useful_product": 2}


def bench_batch_decode_1b(torch, qk, wl, steps: int = 8, warmup: int = 2, int8: bool = False) -> dict:
    """Random-init Llama-3.2-1B decode step for 32 ragged sequences at once:
    sequence s decodes at position ctx_s - 1 with ctx_s ~ U[64, 2048] (the
    ragged descriptor of the 3B FFN workload, seed 3), its KV rows packed in
    one cache and filled with N(0,1) on the device.  Timed: `steps` steps,
    each ending in the 32 greedy tokens' download; positions advance."""
    case = wl.batch_decode_1b(extra_rows=steps + warmup)
    cfg, n, kv_row, rows = case["cfg"], case["n"], case["kv_row"], case["rows"]
    W = wl.llama_weights(cfg, case["weights_seed"])
    runner = qk.BatchRunner(cfg, W, max_tokens=n, cache_rows=rows)
    if int8:
        runner.set_int8(True, True)
    kv_dim = cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    _fill_caches(torch, runner, cfg, rows, 2)
    tokens, pos = list(case["tokens"]), list(case["pos"])
    for _ in range(warmup):
        tokens = runner.forward(tokens, pos, kv_row, True)
        pos = [p + 1 for p in pos]
    torch.cuda.synchronize()
    kv_read = 0
    t0 = time.perf_counter()
    for _ in range(steps):
        tokens = runner.forward(tokens, pos, kv_row, True)
        kv_read += sum(cfg["layers"] * (p + 1) * kv_dim * 4 * 2 for p in pos)
        pos = [p + 1 for p in pos]
    el = time.perf_counter() - t0
    mem = runner.memory()
    runner.close()
    weights = sum(qk.tensor_bytes(wl.MIX_1B[t], *wl.tensor_shape(cfg, t)) for t in wl.TENSORS) * cfg["layers"] + \
        qk.tensor_bytes(qk.Q6_K, cfg["dim"], cfg["vocab"])
    moved = weights * steps + kv_read
    ms = el / steps * 1e3
    return {"sequences": n, "ms_per_step": round(ms, 4), "tokens_per_s": round(n * steps / el, 1),
            "weight_bytes_per_step": weights, "kv_bytes_per_step": int(kv_read / steps),
            "GBps": round(moved / el / 1e9, 1), "frac_of_peak": round(moved / el / 1e9 / HBM_PEAK_GBPS, 4),
            "context": "ctx ~ U[64, 2048] per sequence (seed 3)", "device_bytes": mem}

def bandwidth_kernel(torch, kind: str, nbytes: int, steps: int, warmup: int) -> tuple[float, int]:
    """Times libqkbench's plain copy or streaming read over nbytes from 4
    rotating sources; returns (mean us per launch, bytes moved per launch)."""
    import ctypes
    lib = ctypes.CDLL(str(ROOT / "inferencer-jetson_amd" / "libqkbench.so"))
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    lib.qkb_copy.argtypes, lib.qkb_copy.restype = [vp, vp, sz, vp], ctypes.c_int
    lib.qkb_stream_read.argtypes, lib.qkb_stream_read.restype = [vp, sz, vp, vp], ctypes.c_int
    lib.qkb_sink_words.restype = ctypes.c_int
    srcs = [torch.full((nbytes // 4,), float(i + 1), device="cuda") for i in range(4)]
    dst = torch.empty(nbytes // 4, device="cuda") if kind == "copy" else None
    sink = torch.zeros(lib.qkb_sink_words(), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def launch(i):
        if kind == "copy":
            rc = lib.qkb_copy(srcs[i % 4].data_ptr(), dst.data_ptr(), nbytes, stream.cuda_stream)
        else:
            rc = lib.qkb_stream_read(srcs[i % 4].data_ptr(), nbytes, sink.data_ptr(), stream.cuda_stream)
        if rc:
            raise RuntimeError(f"bench kernel failed ({rc})")

    _, kern_ms = time_launches(torch, launch, steps, warmup, stream)
    return kern_ms * 1e3, nbytes * (2 if kind == "copy" else 1)


def reference_kernels(torch, args) -> int:
    """Plain copy / streaming read of 256 MiB buffers (4 rotating sources)."""
    nbytes = 256 << 20
    us, moved = bandwidth_kernel(torch, args.only, nbytes, args.steps, args.warmup)
    print(json.dumps({"kernel": args.only, "bytes_per_launch": moved, "read_bytes": nbytes,
                      "write_bytes": nbytes if args.only == "copy" else 0,
                      "kernel_us": round(us, 2), "GBps": round(moved / (us * 1e-6) / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=2000,
                    help="untimed launches first: the clocks settle over the first ~40 ms of a run")
    ap.add_argument("--copies", type=int, default=4, help="rotating weight copies (>= 2x the last-level cache)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--secondary", action=argparse.BooleanOptionalAction, default=True)
    ap.add_argument("--only", choices=["gemv", "copy", "stream", "ffn", "ffn_int8", "mixed", "mixed_step", "decode",
                                       "decode_int8", "batch_decode", "batch_decode_int8"],
                    default="gemv",
                    help="copy / stream: time the reference bandwidth kernels of libqkbench.so instead "
                         "(a plain 256 MiB copy calibrates FETCH_SIZE / WRITE_SIZE; a streaming read gives "
                         "the practical read ceiling); ffn / mixed / decode / batch_decode: run one secondary "
                         "workload alone (for profiling) and print its result")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              "(the GEMV shards by rows with no communication between GPUs).", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    qk = load_package()
    import inferencer_jetson_amd.workloads as wl

    torch.cuda.set_device(0)
    if args.only in ("copy", "stream"):
        return reference_kernels(torch, args)
    if args.only != "gemv":
        stream = torch.cuda.current_stream()
        run = {"ffn": lambda: bench_ffn_3b_ragged(torch, qk, wl, stream),
               "ffn_int8": lambda: bench_ffn_3b_ragged(torch, qk, wl, stream, int8=True),
               "mixed": lambda: bench_mixed_1b_256(torch, qk, wl, stream),
               "mixed_step": lambda: bench_mixed_1b_step(torch, qk, wl),
               "decode": lambda: bench_decode_1b(torch, qk, wl),
               "decode_int8": lambda: bench_decode_1b(torch, qk, wl, int8=True),
               "batch_decode": lambda: bench_batch_decode_1b(torch, qk, wl),
               "batch_decode_int8": lambda: bench_batch_decode_1b(torch, qk, wl, int8=True)}[args.only]
        print(json.dumps({args.only: run()}), flush=True)
        return 0
    stream = torch.cuda.current_stream()
    cols, rows = 2048, 128256
    log(f"[bench] building {args.copies} LM-head copies ({rows}x{cols} Q6_K)")
    copies = []
    x_host = None
    for c in range(args.copies):
        w, x_host = wl.lm_head_q6k(copy=c)
        copies.append(torch.from_numpy(w).to("cuda"))
    x = torch.from_numpy(x_host).to("cuda")
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    gguf = [qk.Tensor((cols, rows), qk.Q6_K, wc) for wc in copies]
    # The layout the model drivers run: each copy repacked once by
    # qk_q6k_split (same 210 bytes per block, every field 16-byte aligned).
    tensors = [qk.split_q6k(t, stream) for t in gguf]
    torch.cuda.synchronize()

    def launch(i):
        qk.matvec(tensors[i % len(tensors)], x, y, cols, rows, stream)

    weight_bytes = qk.tensor_bytes(qk.Q6_K_SPLIT, cols, rows)
    assert weight_bytes == qk.tensor_bytes(qk.Q6_K, cols, rows)   # 2048 columns: no row padding
    step_bytes = weight_bytes + cols * 4 + rows * 4
    log(f"[bench] timing {args.steps} steps after {args.warmup} warmup")
    wall, kern_ms = time_launches(torch, launch, args.steps, args.warmup, stream)
    value = step_bytes * args.steps / wall / 1e9
    achieved = step_bytes / (kern_ms * 1e-3) / 1e9
    traffic = measured_traffic("gemv_q6k_lm_head_128256x2048")
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        # fp32 in and out; inside the kernel each 16-value activation group
        # is 22-bit fixed point (exact int8-limb dots), combined in fp32.
        "dtype": "f32 (activations as 22-bit block fixed point)",
        "data": "synthetic (seeded random Q6_K super-blocks, x ~ N(0,1))",
        "config": {"workload": "lm_head_q6k: Q6_K GEMV 128256x2048 (tied LM head), batch 1, "
                               f"{args.copies} rotating weight copies, split Q6_K layout",
                   "rows": rows, "cols": cols, "bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBPS, 4), "traffic": traffic},
    }
    log(f"[bench] lm_head_q6k: {value:.1f} GB/s wall, kernel {kern_ms * 1e3:.2f} us = {achieved:.1f} GB/s")

    if args.secondary:
        sec = {}
        _, kg = time_launches(torch, lambda i: qk.matvec(gguf[i % len(gguf)], x, y, cols, rows, stream),
                              200, 20, stream)
        sec["lm_head_q6k_gguf_layout"] = {"kernel_us": round(kg * 1e3, 2),
                                          "GBps_kernel": round(step_bytes / (kg * 1e-3) / 1e9, 1),
                                          "frac_of_peak": round(step_bytes / (kg * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        # The INT8 mode's kernel on the same split copies (gemv_q6_dp4a,
        # inferencer.cu:597-643): x quantized once outside the timed launches.
        xq = torch.empty(cols, dtype=torch.int8, device="cuda")
        xs = torch.empty(cols // 32, dtype=torch.float32, device="cuda")
        qk.quantize(x, xq, xs, cols, stream=stream)
        _, ki = time_launches(torch, lambda i: qk.matvec_i8(tensors[i % len(tensors)], xq, xs, y, cols, rows,
                                                           stream=stream), 2000, 2000, stream)
        i8_bytes = weight_bytes + cols + cols // 32 * 4 + rows * 4
        sec["lm_head_q6k_int8"] = {"kernel_us": round(ki * 1e3, 2), "bytes_per_launch": i8_bytes,
                                   "GBps_kernel": round(i8_bytes / (ki * 1e-3) / 1e9, 1),
                                   "frac_of_peak": round(i8_bytes / (ki * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4)}
        log(f"[bench] lm_head_q6k_int8: {json.dumps(sec['lm_head_q6k_int8'])}")
        log(f"[bench] lm_head_q6k_gguf_layout: {json.dumps(sec['lm_head_q6k_gguf_layout'])}")
        # The practical ceiling of a read-only kernel: a plain streaming read of
        # the headline's weight bytes from 4 rotating buffers.
        sr_us, sr_bytes = bandwidth_kernel(torch, "stream", weight_bytes // 16 * 16, 500, 200)
        sr_gbps = sr_bytes / (sr_us * 1e-6) / 1e9
        sec["stream_read_ceiling"] = {"bytes_per_launch": sr_bytes, "kernel_us": round(sr_us, 2),
                                      "GBps": round(sr_gbps, 1), "frac_of_peak": round(sr_gbps / HBM_PEAK_GBPS, 4),
                                      "lm_head_q6k_frac_of_ceiling": round(achieved / sr_gbps, 4)}
        log(f"[bench] stream_read_ceiling: {json.dumps(sec['stream_read_ceiling'])}")
        sec["gemv_q4k_128256x2048"] = bench_q4k_lm_shape(torch, qk, wl, stream, args.copies)
        sec["lm_head_q6k_3b_128256x3072"] = bench_lm_head_3b(torch, qk, wl, stream, args.copies)
        log(f"[bench] gemv_q4k_128256x2048: {json.dumps(sec['gemv_q4k_128256x2048'])}")
        log(f"[bench] lm_head_q6k_3b_128256x3072: {json.dumps(sec['lm_head_q6k_3b_128256x3072'])}")
        sec.update(bench_small_gemvs(torch, qk, wl, stream))
        sec["ffn_3b_ragged_t32"] = bench_ffn_3b_ragged(torch, qk, wl, stream)
        log(f"[bench] ffn_3b_ragged_t32: {json.dumps(sec['ffn_3b_ragged_t32'])}")
        sec["ffn_3b_ragged_t32_int8"] = bench_ffn_3b_ragged(torch, qk, wl, stream, int8=True)
        log(f"[bench] ffn_3b_ragged_t32_int8: {json.dumps(sec['ffn_3b_ragged_t32_int8'])}")
        sec["mixed_1b_256"] = bench_mixed_1b_256(torch, qk, wl, stream)
        log(f"[bench] mixed_1b_256: {json.dumps(sec['mixed_1b_256'])}")
        sec["mixed_1b_256_step"] = bench_mixed_1b_step(torch, qk, wl)
        log(f"[bench] mixed_1b_256_step: {json.dumps(sec['mixed_1b_256_step'])}")
        sec["llama_1b_decode"] = bench_decode_1b(torch, qk, wl)
        log(f"[bench] llama_1b_decode: {json.dumps(sec['llama_1b_decode'])}")
        sec["llama_1b_decode_int8"] = bench_decode_1b(torch, qk, wl, int8=True)
        log(f"[bench] llama_1b_decode_int8: {json.dumps(sec['llama_1b_decode_int8'])}")
        sec["llama_1b_batch_decode_32"] = bench_batch_decode_1b(torch, qk, wl)
        log(f"[bench] llama_1b_batch_decode_32: {json.dumps(sec['llama_1b_batch_decode_32'])}")
        sec["llama_1b_batch_decode_32_int8"] = bench_batch_decode_1b(torch, qk, wl, int8=True)
        log(f"[bench] llama_1b_batch_decode_32_int8: {json.dumps(sec['llama_1b_batch_decode_32_int8'])}")
        result["secondary"] = sec

    if not args.no_cpu_baseline:
        log(f"[bench] CPU baseline (~{args.cpu_seconds:.0f} s)")
        result["cpu_baseline"] = cpu_baseline_lm_head(wl, sample_rows=65536, target_s=args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
