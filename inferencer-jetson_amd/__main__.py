"""Command line of the package: `python3 inferencer-jetson_amd [options] [prompt ...]`.

The counterpart of the reference's main (inferencer.cu:1595-1979): load a
GGUF Llama, tokenize each prompt with the Llama 3 chat template, prefill it
(one token per step, or in batched chunks with --prefill-batch), decode
greedily until a stop token or --max-tokens, print the text, and with
--stats the per-prompt and average timings.  --tokenize-only prints token
ids without touching the GPU; --compare-prefill runs the sequential /
batched prefill comparison.

Differences from the reference, each because the kernels here differ:
* --gate-warps and --q6-warps are validated as the reference does but have
  no effect: every launch here is sized per shape by the library.
* --fused-norm-quant, --fused-rope-cache and --fused-small-kernels are
  accepted; the decode step here always runs fused.
* --prefill-batch N > 1 runs the batched driver in the decode mode: INT8
  for both types (the default; the reference's only batched mode) or, with
  --float-gemv, FP32 for both (an addition).  Like the reference, a mixed
  mode (--float-q6) is rejected with batched prefill.  The prompt's cache
  rows are then handed to the one-sequence driver for decoding.
* There is no board power meter (the reference reads Jetson's VDD_IN), so
  no energy figures are printed.
"""
from __future__ import annotations

import importlib.util
import pathlib
import sys
import time

_HERE = pathlib.Path(__file__).resolve().parent
_PKG = "inferencer_jetson_amd"

OPTIONS_HELP = """Options:
  --model FILE         Llama GGUF to load (llama3.2-3b/model.gguf when omitted)
  --max-tokens N       end a response after N generated tokens (128)
  --context N          KV rows per sequence, 128 or more (1024)
  --prompts-file FILE  take the prompts from FILE, one per non-empty line
  --stats              report timings for each prompt and for the whole run
  --q6-dp4a            Q6_K matrices take INT8 activations (on by default)
  --float-q6           Q6_K matrices take FP32 activations
  --float-gemv         every quantized matrix takes FP32 activations
  --fused-norm-quant, --fused-rope-cache, --fused-small-kernels
                       kept for old scripts; no effect, the step is always fused
  --gate-warps N, --q6-warps N
                       checked for 2, 4, 8 or 16, then ignored: this library
                       chooses each launch's shape from the matrix
  --prefill-batch N    feed the prompt N tokens per step, 1 to 32 (1)
  --tokenize-only      print the prompt's token ids; the GPU is not used
  --compare-prefill    run the prompt token by token and in batches and print
                       where the two differ (needs --prefill-batch 2 or more)
  --help               this text
Prompts are the remaining arguments; without any, stdin is read as one prompt.
"""


def _package():
    if _PKG in sys.modules:
        return sys.modules[_PKG]
    spec = importlib.util.spec_from_file_location(_PKG, _HERE / "__init__.py",
                                                  submodule_search_locations=[str(_HERE)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[_PKG] = mod
    spec.loader.exec_module(mod)
    return mod


class Options:
    def __init__(self):
        self.model = "llama3.2-3b/model.gguf"
        self.prompts: list[str] = []
        self.max_tokens, self.context = 128, 1024
        self.tokenize_only = self.stats = self.compare_prefill = False
        self.prompts_file = False
        self.use_dp4a = self.use_q6_dp4a = True
        self.gate_warps = self.q6_warps = 4
        self.prefill_batch = 1


def parse(argv: list[str], stdin) -> Options | None:
    """The reference's argument loop and checks (inferencer.cu:1604-1670);
    None after --help.  Errors raise ValueError."""
    o = Options()
    i = 0

    def value():
        nonlocal i
        i += 1
        return argv[i]

    while i < len(argv):
        a = argv[i]
        has_value = i + 1 < len(argv)
        if a == "--model" and has_value:
            o.model = value()
        elif a in ("--max-tokens", "--context", "--gate-warps", "--q6-warps", "--prefill-batch") and has_value:
            v = int(value())
            setattr(o, {"--max-tokens": "max_tokens", "--context": "context", "--gate-warps": "gate_warps",
                        "--q6-warps": "q6_warps", "--prefill-batch": "prefill_batch"}[a], v)
        elif a == "--prompts-file" and has_value:
            o.prompts_file = True
            try:
                with open(value(), "r", encoding="utf-8", newline="") as f:
                    for line in f.read().split("\n"):
                        line = line[:-1] if line.endswith("\r") else line
                        if line:
                            o.prompts.append(line)
            except OSError:
                raise ValueError("Cannot open prompts file")
        elif a == "--tokenize-only":
            o.tokenize_only = True
        elif a == "--compare-prefill":
            o.compare_prefill = True
        elif a == "--stats":
            o.stats = True
        elif a == "--q6-dp4a":
            o.use_q6_dp4a = True
        elif a == "--float-q6":
            o.use_q6_dp4a = False
        elif a == "--float-gemv":
            o.use_dp4a = o.use_q6_dp4a = False
        elif a in ("--fused-norm-quant", "--fused-rope-cache", "--fused-small-kernels"):
            pass
        elif a == "--help":
            return None
        elif a.startswith("-"):
            raise ValueError("Unknown option: " + a)
        elif a:
            o.prompts.append(a)
        i += 1
    if not o.prompts and not o.prompts_file:
        text = stdin.read()
        if text:
            o.prompts.append(text)
    if not o.prompts or o.max_tokens < 1 or o.context < 128:
        raise ValueError("Provide prompts, positive --max-tokens, and --context >= 128")
    if o.gate_warps not in (2, 4, 8, 16) or o.q6_warps not in (2, 4, 8, 16):
        raise ValueError("--gate-warps and --q6-warps must be 2, 4, 8, or 16")
    if not 1 <= o.prefill_batch <= 32:
        raise ValueError("--prefill-batch must be in 1..32")
    if o.prefill_batch > 1 and o.use_dp4a != o.use_q6_dp4a:
        raise ValueError("Batched prefill runs Q4_K and Q6_K in one mode: INT8 (the default) or FP32 (--float-gemv)")
    if o.compare_prefill and (o.tokenize_only or o.prefill_batch == 1):
        raise ValueError("--compare-prefill requires --prefill-batch 2..32 and GPU inference")
    if len(o.prompts) > 1:
        o.stats = True
    return o


def _prefill_batched(qk, runner, batch, ids: list[int]) -> int:
    """The prompt in chunks through the batched driver, its cache rows
    copied into the one-sequence driver; returns the greedy next token."""
    n, chunk = len(ids), batch.max_tokens
    nxt = 0
    for c0 in range(0, n, chunk):
        part = ids[c0:c0 + chunk]
        m = len(part)
        if c0 + m == n:
            nxt = batch.forward(part, list(range(c0, c0 + m)), [0] * m, seq=[0] * m, logit_rows=[m - 1])[0]
        else:
            batch.forward(part, list(range(c0, c0 + m)), [0] * m, False, seq=[0] * m)
    qk.copy_kv_rows(runner, batch, n)
    return nxt


STORAGE_NAMES = {0: "FP32", 1: "FP16", 12: "Q4_K", 14: "Q6_K"}


def storage_summary(model, q4k_int8: bool, q6k_int8: bool) -> str:
    """One line on the model's tensors: parameter count, each storage type's
    share of the parameters (in type-id order), bits per parameter and
    tensor bytes, and the arithmetic each quantized type runs in -- the facts
    the reference prints at load (GGUF::print_storage, inferencer.cu:296-315)."""
    params: dict[int, int] = {}
    nbytes = 0
    for t in model.tensors():
        n = 1
        for d in range(t.n_dims):
            n *= int(t.dims[d])
        params[t.type] = params.get(t.type, 0) + n
        nbytes += int(t.bytes)
    total = max(sum(params.values()), 1)
    shares = []
    for ty in sorted(params):
        pct = 100.0 * params[ty] / total
        shares.append(f"{STORAGE_NAMES.get(ty, 'unknown')} {'<0.1' if pct < 0.05 else f'{pct:.1f}'}%")
    mode = lambda on: "INT8" if on else "FP32"
    return (f"Model: {total / 1e9:.3f}B parameters ({', '.join(shares)}), {8.0 * nbytes / total:.2f} bits per "
            f"parameter, {nbytes / 2**30:.2f} GiB of tensor data; Q4_K products in {mode(q4k_int8)}, Q6_K "
            f"products in {mode(q6k_int8)}, accumulation in FP32\n")


def run(argv: list[str], stdout=None, stderr=None, stdin=None) -> int:
    stdout = stdout or sys.stdout.buffer
    stderr = stderr or sys.stderr
    try:
        o = parse(argv, stdin or sys.stdin)
        if o is None:
            stdout.write(b"Usage: python3 inferencer-jetson_amd [options] [prompt ...]\n" + OPTIONS_HELP.encode())
            return 0
        qk = _package()
        import inferencer_jetson_amd.tokenizer as tk
        import inferencer_jetson_amd.compare as cmp

        t_start = time.perf_counter()
        model = qk.GGUF(o.model)
        t_loaded = time.perf_counter()
        tok = tk.Tokenizer.from_gguf(model)
        t_tok = time.perf_counter()
        stderr.write(storage_summary(model, o.use_dp4a, o.use_q6_dp4a))
        runner = batch = timer = None
        t_up0 = t_up1 = t_ready = t_tok
        if not o.tokenize_only:
            t_up0 = time.perf_counter()
            model.upload()
            t_up1 = time.perf_counter()
            _, nbytes, _ = model.data()
            stderr.write(f"GPU device 0; uploaded {nbytes / 2**30:.2f} GiB of model weights to GPU memory\n")
            if not o.compare_prefill:
                runner = qk.Runner.from_gguf(model, o.context)
                runner.set_int8(o.use_dp4a, o.use_q6_dp4a)
                if o.prefill_batch > 1:
                    batch = qk.BatchRunner.from_gguf(model, o.context, o.prefill_batch, o.context)
                    batch.set_int8(o.use_dp4a, o.use_q6_dp4a)
                timer = qk.GpuTimer()
            t_ready = time.perf_counter()
            stderr.write(f"Q4_K matrix path: {'INT8' if o.use_dp4a else 'FP32'}; Q6_K matrix path: "
                         f"{'INT8' if o.use_q6_dp4a else 'FP32'}\n")
            stderr.write(f"Prompt prefill batch: {o.prefill_batch} token(s)\n")

        if o.compare_prefill:
            steps = min(o.max_tokens, 8)
            for p, prompt in enumerate(o.prompts):
                ids = tk.chat_prompt(tok, prompt)
                if len(ids) + steps > o.context:
                    raise ValueError("Comparison prompt exceeds --context")
                # Fresh drivers per prompt: both start from empty caches, as
                # runner->reset() does.
                r = qk.Runner.from_gguf(model, o.context)
                b = qk.BatchRunner.from_gguf(model, o.context, o.prefill_batch, o.context)
                rep = cmp.compare_prefill(qk, r, b, ids, steps, o.prefill_batch, int8=o.use_dp4a)
                r.close()
                b.close()
                stdout.write(("\n".join(cmp.format_report(p + 1, rep)) + "\n").encode())
            stdout.flush()
            return 0

        stop = tok.stop_ids()
        sums = dict(tokenize=0.0, prefill=0.0, decode=0.0, prompt=0.0, compute=0.0, gpu=0.0)
        calls = lambda: runner.matrix_calls() + (batch.matrix_calls() if batch is not None else 0)
        n_in = n_out = n_steps = 0
        for p, prompt in enumerate(o.prompts):
            t0 = time.perf_counter()
            ids = tk.chat_prompt(tok, prompt)
            t1 = time.perf_counter()
            if len(ids) + o.max_tokens > o.context:
                raise ValueError(f"Prompt {p + 1} and response exceed --context")
            sums["tokenize"] += t1 - t0
            n_in += len(ids)
            if len(o.prompts) > 1:
                stdout.write(f"[{p + 1}/{len(o.prompts)}] ".encode())
                stdout.flush()
            if o.tokenize_only:
                stdout.write((" ".join(str(i) for i in ids) + " \n").encode())
                sums["prompt"] += time.perf_counter() - t0
                continue
            gpu_before, calls_before = timer.seconds, calls()
            tp = time.perf_counter()
            timer.start()
            if batch is not None:
                nxt = _prefill_batched(qk, runner, batch, ids)
            else:
                nxt = 0
                for i, t in enumerate(ids):
                    nxt = runner.forward(t, i, i + 1 == len(ids))
            timer.stop()
            td = time.perf_counter()
            generated = steps = 0
            compute = 0.0
            for i in range(o.max_tokens):
                if nxt in stop:
                    break
                stdout.write(tok.decode(nxt))
                stdout.flush()
                generated += 1
                if i + 1 == o.max_tokens or len(ids) + i >= o.context:
                    break
                ts = time.perf_counter()
                timer.start()
                nxt = runner.forward(nxt, len(ids) + i, True)
                timer.stop()
                compute += time.perf_counter() - ts
                steps += 1
            stdout.write(b"\n")
            stdout.flush()
            tf = time.perf_counter()
            sums["prefill"] += td - tp
            sums["decode"] += tf - td
            sums["prompt"] += tf - t0
            sums["compute"] += compute
            gpu = timer.seconds - gpu_before
            sums["gpu"] += gpu
            n_out += generated
            n_steps += steps
            if o.stats:
                stderr.write(f"Prompt {p + 1}/{len(o.prompts)}: {len(ids)} input tokens, {generated} output tokens\n"
                             f"  tokenization {t1 - t0:.3f} s; prompt computation {td - tp:.3f} s; response "
                             f"generation {tf - td:.3f} s; total {tf - t0:.3f} s\n"
                             f"  output throughput {generated / max(tf - t0, 1e-9):.3f} tokens/s; steady decode "
                             f"{steps / max(compute, 1e-9):.3f} tokens/s\n"
                             f"  GPU pipeline {gpu:.3f} s across {calls() - calls_before} quantized matrix calls\n")
        if o.stats:
            t_end = time.perf_counter()
            n = len(o.prompts)
            stderr.write(f"One-time GGUF metadata and mmap: {t_loaded - t_start:.3f} s\n"
                         f"One-time tokenizer setup: {t_tok - t_loaded:.3f} s\n")
            if not o.tokenize_only:
                stderr.write(f"One-time GPU weight allocation and upload: {t_up1 - t_up0:.3f} s\n"
                             f"One-time runtime buffer setup: {t_ready - t_up1:.3f} s\n")
            stderr.write(f"Average over {n} prompts:\n  tokenization: {sums['tokenize'] / n:.3f} s\n")
            if not o.tokenize_only:
                stderr.write(f"  prompt computation: {sums['prefill'] / n:.3f} s\n"
                             f"  response generation: {sums['decode'] / n:.3f} s\n"
                             f"  inference per prompt (including tokenization): {sums['prompt'] / n:.3f} s\n"
                             f"  input processing: {n_in / max(sums['prefill'], 1e-9):.3f} tokens/s\n"
                             f"  output throughput: {n_out / max(sums['prompt'], 1e-9):.3f} tokens/s\n"
                             f"  steady decode: {n_steps / max(sums['compute'], 1e-9):.3f} tokens/s\n"
                             f"  GPU pipeline: {sums['gpu'] / n:.3f} s\n")
            stderr.write(f"Total: {n_in} input tokens, {n_out} output tokens, {t_end - t_start:.3f} s elapsed\n")
        stdout.flush()
        return 0
    except (ValueError, OSError, RuntimeError) as e:
        stderr.write(f"Error: {e}\n")
        return 1


if __name__ == "__main__":
    sys.exit(run(sys.argv[1:]))
