"""Seeded synthetic workloads of the quantized GEMV path, as host numpy arrays.

Each workload fixes its seed; the (seed, stream) pairs below are the whole
specification of its inputs (generator: csrc/qk_synth.h).

  gemv_q4k_2048      Q4_K 2048 x 2048 (Llama-3.2-1B attn_q), x ~ N(0,1); seed 0.
  lm_head_q6k        Q6_K 128256 x 2048 (tied LM head), x ~ N(0,1); seed 1.
  llama_1b_decode    random-init Llama-3.2-1B, Q4_K_M-style mix, fp32 KV cache
                     prefilled at positions 0..511, 16 prompt ids, 64 greedy
                     tokens; seed 2.
  ffn_3b_ragged      Llama-3.2-3B FFN (Q4_K gate/up 8192 x 3072, Q6_K down
                     3072 x 8192) on 32 decode tokens of 32 sequences with
                     context lengths uniform 64..2048; seed 3.
  mixed_1b_256       256 packed tokens on Llama-3.2-1B shapes: 2 prefill chunks
                     of 96 plus 64 single-token decodes; seed 4.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import synth

Q4_K, Q6_K = synth.Q4_K, synth.Q6_K

# Block-scale sigmas of the workloads: |N(0, 0.02)| for Q4_K d / dmin,
# |N(0, 0.01)| for Q6_K d.
SIGMA = {Q4_K: 0.02, Q6_K: 0.01}


def gemv_case(qtype: int, cols: int, rows: int, seed: int, w_stream: int = 1, x_stream: int = 2,
              n_tokens: int = 1):
    """(weights uint8[rows*row_bytes], x float32[n_tokens, cols] or [cols])."""
    w = synth.quant_matrix(qtype, cols, rows, seed, w_stream, SIGMA[qtype])
    x = synth.normal_f32(cols * n_tokens, seed, x_stream)
    return w, (x if n_tokens == 1 else x.reshape(n_tokens, cols))


def gemv_q4k_2048():
    return gemv_case(Q4_K, 2048, 2048, seed=0)


def lm_head_q6k(copy: int = 0):
    """The LM-head GEMV; copy > 0 gives further weight sets of the same
    distribution (streams 16*copy + 1) for cache-rotation in timing."""
    w = synth.quant_matrix(Q6_K, 2048, 128256, 1, 1 + 16 * copy, SIGMA[Q6_K])
    x = synth.normal_f32(2048, 1, 2)
    return w, x


# ------------------------------------------------------------------ Llama --

LLAMA_1B = dict(dim=2048, layers=16, heads=32, kv_heads=8, hidden=8192, vocab=128256, context=1024,
                eps=1e-5, rope_theta=500000.0)
LLAMA_3B = dict(dim=3072, layers=28, heads=24, kv_heads=8, hidden=8192, vocab=128256, context=1024,
                eps=1e-5, rope_theta=500000.0)

# Q4_K_M-style mix of the 1B decode workload.
MIX_1B = dict(q=Q4_K, k=Q4_K, v=Q6_K, o=Q4_K, gate=Q4_K, up=Q4_K, down=Q6_K)
TENSORS = ("q", "k", "v", "o", "gate", "up", "down")


def tensor_shape(cfg: dict, name: str) -> tuple[int, int]:
    """(cols, rows) of a layer tensor."""
    dim, hidden = cfg["dim"], cfg["hidden"]
    kv_dim = dim // cfg["heads"] * cfg["kv_heads"]
    return {"q": (dim, dim), "k": (dim, kv_dim), "v": (dim, kv_dim), "o": (dim, dim),
            "gate": (dim, hidden), "up": (dim, hidden), "down": (hidden, dim)}[name]


def llama_weights(cfg: dict, seed: int, mix: dict | None = None, embd_type: int = Q6_K) -> dict:
    """Random-init weights: token_embd (tied LM head) on stream 1, layer l
    tensor j on stream 100 + 16*l + j, RMSNorm gains 1.0."""
    mix = MIX_1B if mix is None else mix
    dim = cfg["dim"]
    layers = []
    for l in range(cfg["layers"]):
        L = {}
        for j, name in enumerate(TENSORS):
            cols, rows = tensor_shape(cfg, name)
            L[name] = synth.quant_matrix(mix[name], cols, rows, seed, 100 + 16 * l + j, SIGMA[mix[name]])
            L[name + "_type"] = mix[name]
        L["attn_norm"] = np.ones(dim, dtype=np.float32)
        L["ffn_norm"] = np.ones(dim, dtype=np.float32)
        layers.append(L)
    embd = synth.quant_matrix(embd_type, dim, cfg["vocab"], seed, 1, SIGMA[embd_type])
    return dict(embd_type=embd_type, token_embd=embd, output=None, output_type=0,
                output_norm=np.ones(dim, dtype=np.float32), layers=layers)


def llama_kv_prefill(cfg: dict, seed: int, n_positions: int) -> tuple[np.ndarray, np.ndarray]:
    """fp32 caches [layer][context][kv_dim], N(0,1) at positions < n_positions
    (K on stream 3, V on stream 4, layer-major), zeros elsewhere."""
    kv_dim = cfg["dim"] // cfg["heads"] * cfg["kv_heads"]
    shape = (cfg["layers"], cfg["context"], kv_dim)
    kc = np.zeros(shape, dtype=np.float32)
    vc = np.zeros(shape, dtype=np.float32)
    n = cfg["layers"] * n_positions * kv_dim
    kc[:, :n_positions] = synth.normal_f32(n, seed, 3).reshape(cfg["layers"], n_positions, kv_dim)
    vc[:, :n_positions] = synth.normal_f32(n, seed, 4).reshape(cfg["layers"], n_positions, kv_dim)
    return kc, vc


def llama_prompt(cfg: dict, seed: int, n: int = 16) -> np.ndarray:
    return synth.uniform_i32(n, seed, 5, 0, cfg["vocab"] - 1)


@dataclass
class DecodeWorkload:
    cfg: dict
    seed: int
    prefill_positions: int = 512
    prompt_tokens: int = 16
    greedy_tokens: int = 64


LLAMA_1B_DECODE = DecodeWorkload(cfg=LLAMA_1B, seed=2)


# ------------------------------------------------------- batched tokens --

@dataclass
class BatchDescriptor:
    """Ragged batch metadata, one entry per packed token: the sequence it
    belongs to, its position, that sequence's context length after the token,
    and the first KV row of the sequence in a packed cache."""
    seq_id: np.ndarray
    pos: np.ndarray
    ctx_len: np.ndarray
    kv_offset: np.ndarray = field(default=None)

    @property
    def n_tokens(self) -> int:
        return int(self.seq_id.size)


def ffn_3b_ragged(seed: int = 3, n_tokens: int = 32, copy: int = 0):
    """3B FFN on n_tokens decode tokens of distinct sequences; copy > 0 gives
    further weight sets (streams 16*copy + 1..3) for cache rotation in timing."""
    cfg = LLAMA_3B
    base = 16 * copy
    gate = synth.quant_matrix(Q4_K, cfg["dim"], cfg["hidden"], seed, base + 1, SIGMA[Q4_K])
    up = synth.quant_matrix(Q4_K, cfg["dim"], cfg["hidden"], seed, base + 2, SIGMA[Q4_K])
    down = synth.quant_matrix(Q6_K, cfg["hidden"], cfg["dim"], seed, base + 3, SIGMA[Q6_K])
    x = synth.normal_f32(n_tokens * cfg["dim"], seed, 4).reshape(n_tokens, cfg["dim"])
    ctx = synth.uniform_i32(n_tokens, seed, 5, 64, 2048)
    desc = BatchDescriptor(seq_id=np.arange(n_tokens, dtype=np.int32), pos=(ctx - 1).astype(np.int32),
                           ctx_len=ctx.astype(np.int32),
                           kv_offset=np.concatenate([[0], np.cumsum(ctx[:-1])]).astype(np.int64))
    return dict(gate=gate, up=up, down=down, x=x, desc=desc, cfg=cfg)


def mixed_1b_256(seed: int = 4):
    """2 prefill chunks of 96 tokens + 64 decodes packed into 256 tokens, with
    one layer's seven projections of the 1B shapes."""
    cfg = LLAMA_1B
    chunk, decodes = 96, 64
    seq = np.concatenate([np.zeros(chunk), np.ones(chunk), 2 + np.arange(decodes)]).astype(np.int32)
    ctx_dec = synth.uniform_i32(decodes, seed, 6, 64, 2048)
    pos = np.concatenate([np.arange(chunk), np.arange(chunk), ctx_dec - 1]).astype(np.int32)
    ctx = np.concatenate([np.full(chunk, chunk), np.full(chunk, chunk), ctx_dec]).astype(np.int32)
    desc = BatchDescriptor(seq_id=seq, pos=pos, ctx_len=ctx)
    weights = {}
    for j, name in enumerate(TENSORS):
        cols, rows = tensor_shape(cfg, name)
        weights[name] = synth.quant_matrix(MIX_1B[name], cols, rows, seed, 1 + j, SIGMA[MIX_1B[name]])
    x = synth.normal_f32(256 * cfg["dim"], seed, 8).reshape(256, cfg["dim"])
    x_ffn = synth.normal_f32(256 * cfg["hidden"], seed, 9).reshape(256, cfg["hidden"])
    return dict(weights=weights, x=x, x_ffn=x_ffn, desc=desc, cfg=cfg)


def batch_decode_1b(extra_rows: int, seed: int = 3):
    """The 32-sequence decode batch on the random-init Llama-3.2-1B (weights
    seed 2): sequence s decodes at position ctx_s - 1, ctx_s ~ U[64, 2048]
    from the 3B FFN workload's descriptor (seed 3), its KV rows packed after
    the previous sequence's with extra_rows rows to spare (the steps that
    follow).  First tokens uniform in the vocabulary (seed 3, stream 6)."""
    desc = ffn_3b_ragged(seed)["desc"]
    n = desc.n_tokens
    cap = desc.ctx_len.astype(np.int64) + extra_rows
    kv_row = np.concatenate([[0], np.cumsum(cap[:-1])]).astype(np.int64)
    cfg = dict(LLAMA_1B, context=2048 + extra_rows)
    tokens = [int(x) for x in synth.uniform_i32(n, seed, 6, 0, cfg["vocab"] - 1)]
    return dict(cfg=cfg, weights_seed=2, n=n, cap=cap, kv_row=[int(r) for r in kv_row], rows=int(cap.sum()),
                pos=[int(c) - 1 for c in desc.ctx_len], tokens=tokens)
