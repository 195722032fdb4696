"""Pins the oracle's decode-step operations (qk_oracle.c restating
inferencer.cu:821-834, 906-1009, 1053-1099, 1218-1226) against torch /
numpy float64 library routines and closed forms."""
import numpy as np
import pytest
import torch

from conftest import rel_l2


def test_rmsnorm_vs_torch(oracle, synth):
    x = synth.normal_f32(2048, 31, 1).astype(np.float64) * 3.0
    w = synth.normal_f32(2048, 31, 2)
    got = oracle.rmsnorm(x, w, 1e-5)
    t = torch.from_numpy(x)
    want = (t * torch.rsqrt(t.pow(2).mean() + 1e-5) * torch.from_numpy(w.astype(np.float64))).numpy()
    assert rel_l2(got, want) < 1e-14


def test_rope_tables(oracle):
    c, s = oracle.rope_tables(1024, 64, 500000.0)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)
    freq = np.power(np.float64(500000.0), -2.0 * np.arange(32) / 64.0)
    ang = np.arange(1024)[:, None] * freq[None, :]
    # float32 powf / cosf / sinf of a float32 angle: within float32 rounding
    # of the angle (|angle| <= 1023) of the exact values.
    assert np.max(np.abs(c - np.cos(ang))) < 2e-4
    assert np.max(np.abs(s - np.sin(ang))) < 2e-4
    assert np.max(np.abs(c[:, 20:] - np.cos(ang[:, 20:]))) < 1e-6


def test_rope_is_pairwise_complex_rotation(oracle, synth):
    c, s = oracle.rope_tables(64, 64, 10000.0)
    v = synth.normal_f32(512, 32, 1).astype(np.float64)
    pos = 37
    got = oracle.rope(v, c, s, pos, 64)
    z = v[0::2] + 1j * v[1::2]
    f = np.arange(256) % 32
    rot = c[pos, f].astype(np.float64) + 1j * s[pos, f].astype(np.float64)
    want = np.empty_like(v)
    want[0::2] = (z * rot).real
    want[1::2] = (z * rot).imag
    assert np.max(np.abs(got - want)) < 1e-12
    assert np.array_equal(oracle.rope(v, c, s, 0, 64), v)


@pytest.mark.parametrize("heads,kv_heads,head_dim,pos", [(32, 8, 64, 100), (4, 4, 128, 0), (8, 2, 64, 300)])
def test_attention_vs_torch(oracle, synth, heads, kv_heads, head_dim, pos):
    kv_dim = kv_heads * head_dim
    q = synth.normal_f32(heads * head_dim, 33, 1).astype(np.float64)
    kc = synth.normal_f32((pos + 1) * kv_dim, 33, 2).astype(np.float64).reshape(pos + 1, kv_dim)
    vc = synth.normal_f32((pos + 1) * kv_dim, 33, 3).astype(np.float64).reshape(pos + 1, kv_dim)
    got = oracle.attention(q, kc, vc, pos, heads, kv_heads, head_dim)
    Q = torch.from_numpy(q).view(heads, 1, head_dim)
    K = torch.from_numpy(kc).view(pos + 1, kv_heads, head_dim).transpose(0, 1)
    V = torch.from_numpy(vc).view(pos + 1, kv_heads, head_dim).transpose(0, 1)
    group = heads // kv_heads
    K = K.repeat_interleave(group, dim=0).contiguous()
    V = V.repeat_interleave(group, dim=0).contiguous()
    p = torch.softmax(torch.matmul(Q, K.transpose(1, 2).contiguous()) / np.sqrt(head_dim), dim=-1)
    want = torch.matmul(p, V).reshape(-1).numpy()
    assert rel_l2(got, want) < 1e-13


def test_silu_mul_vs_torch(oracle, synth):
    g = synth.normal_f32(1000, 34, 1).astype(np.float64) * 4
    u = synth.normal_f32(1000, 34, 2).astype(np.float64)
    want = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    assert rel_l2(oracle.silu_mul(g, u), want) < 1e-14


def test_argmax_lowest_index_on_ties(oracle, synth):
    v = synth.normal_f32(128256, 35, 1)
    assert oracle.argmax(v) == int(np.argmax(v))
    v[[5, 700, 90000]] = 100.0
    assert oracle.argmax(v) == 5
    assert oracle.argmax(v.astype(np.float64)) == 5
    v[:] = -np.inf
    assert oracle.argmax(v) == 0
