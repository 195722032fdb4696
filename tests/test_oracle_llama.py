"""Pins the oracle's decode step (qk_oracle.c oq_llama_*, restating the
operation order of FastRunner::forward, inferencer.cu:1424-1531) against an
independent, vectorised torch float64 restatement on a small configuration:
RMSNorm as mean/rsqrt, RoPE as a complex multiply, attention as one
softmax-matmul per head, SiLU through torch.sigmoid, all on the oracle's
dequantized weights (bit-exact, pinned by test_oracle_dequant)."""
import numpy as np
import pytest
import torch

from conftest import rel_l2

CFG = dict(dim=512, layers=2, heads=8, kv_heads=2, hidden=1024, vocab=1000, context=32, eps=1e-5,
           rope_theta=10000.0)


def _rms(x, w, eps):
    return x * torch.rsqrt(x.pow(2).mean() + eps) * w


def _rope(v, cos_row, sin_row, head_dim):
    z = torch.view_as_complex(v.reshape(-1, 2).contiguous())
    f = torch.arange(z.numel()) % (head_dim // 2)
    rot = torch.complex(cos_row[f], sin_row[f])
    return torch.view_as_real(z * rot).reshape(-1)


class TorchStep:
    def __init__(self, oracle, cfg, weights, kc, vc):
        self.cfg = cfg
        dq = lambda t, a, cols, rows: torch.from_numpy(oracle.dequant(t, a, cols, rows).astype(np.float64))
        dim, hidden = cfg["dim"], cfg["hidden"]
        self.hd = dim // cfg["heads"]
        kv = self.hd * cfg["kv_heads"]
        self.layers = []
        for L in weights["layers"]:
            self.layers.append(dict(
                q=dq(L["q_type"], L["q"], dim, dim), k=dq(L["k_type"], L["k"], dim, kv),
                v=dq(L["v_type"], L["v"], dim, kv), o=dq(L["o_type"], L["o"], dim, dim),
                gate=dq(L["gate_type"], L["gate"], dim, hidden), up=dq(L["up_type"], L["up"], dim, hidden),
                down=dq(L["down_type"], L["down"], hidden, dim),
                attn_norm=torch.from_numpy(L["attn_norm"].astype(np.float64)),
                ffn_norm=torch.from_numpy(L["ffn_norm"].astype(np.float64))))
        self.embd = dq(weights["embd_type"], weights["token_embd"], dim, cfg["vocab"])
        self.out_norm = torch.from_numpy(weights["output_norm"].astype(np.float64))
        c, s = oracle.rope_tables(cfg["context"], self.hd, cfg["rope_theta"])
        self.cos, self.sin = torch.from_numpy(c.astype(np.float64)), torch.from_numpy(s.astype(np.float64))
        self.kc = torch.from_numpy(kc.astype(np.float64)).clone()
        self.vc = torch.from_numpy(vc.astype(np.float64)).clone()

    def forward(self, token, pos):
        cfg, hd = self.cfg, self.hd
        group = cfg["heads"] // cfg["kv_heads"]
        x = self.embd[token].clone()
        for l, L in enumerate(self.layers):
            xn = _rms(x, L["attn_norm"], cfg["eps"])
            q = _rope(L["q"] @ xn, self.cos[pos], self.sin[pos], hd)
            k = _rope(L["k"] @ xn, self.cos[pos], self.sin[pos], hd)
            self.kc[l, pos] = k
            self.vc[l, pos] = L["v"] @ xn
            keys = self.kc[l, : pos + 1].reshape(pos + 1, cfg["kv_heads"], hd)
            vals = self.vc[l, : pos + 1].reshape(pos + 1, cfg["kv_heads"], hd)
            heads = []
            for h in range(cfg["heads"]):
                kvh = h // group
                p = torch.softmax(keys[:, kvh] @ q[h * hd:(h + 1) * hd] / np.sqrt(hd), dim=0)
                heads.append(p @ vals[:, kvh])
            x = x + L["o"] @ torch.cat(heads)
            xn = _rms(x, L["ffn_norm"], cfg["eps"])
            g = L["gate"] @ xn
            x = x + L["down"] @ (g * torch.sigmoid(g) * (L["up"] @ xn))
        return self.embd @ _rms(x, self.out_norm, cfg["eps"])


@pytest.mark.parametrize("seed", [21, 22])
def test_llama_step_matches_torch_restatement(oracle, workloads, seed):
    cfg = CFG
    weights = workloads.llama_weights(cfg, seed)
    n_prefill = 9
    kc, vc = workloads.llama_kv_prefill(cfg, seed, n_prefill)
    ref = oracle.Llama(cfg, weights)
    ref.load_cache(kc, vc, n_prefill)
    tstep = TorchStep(oracle, cfg, weights, kc, vc)
    token = int(workloads.llama_prompt(cfg, seed, 1)[0])
    for pos in range(n_prefill, n_prefill + 4):
        nxt, logits = ref.forward(token, pos)
        want = tstep.forward(token, pos).numpy()
        assert rel_l2(logits, want) < 1e-12, pos
        assert nxt == int(np.argmax(want))
        token = nxt


def test_llama_step_without_logits_still_writes_cache(oracle, workloads):
    cfg = CFG
    weights = workloads.llama_weights(cfg, 5)
    kc, vc = workloads.llama_kv_prefill(cfg, 5, 3)
    a, b = oracle.Llama(cfg, weights), oracle.Llama(cfg, weights)
    a.load_cache(kc, vc, 3)
    b.load_cache(kc, vc, 3)
    nxt, lg = a.forward(7, 3, need_logits=False)
    assert nxt == -1 and lg is None
    # Position 3 now holds token 7's K/V in `a`: both models agree at pos 4
    # only if `b` also processes token 7 first.
    b.forward(7, 3)
    n_a, la = a.forward(11, 4)
    n_b, lb = b.forward(11, 4)
    assert n_a == n_b and np.array_equal(la, lb)
