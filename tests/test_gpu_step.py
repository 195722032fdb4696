"""GPU decode-step kernels against the oracle's fp64 restatements
(inferencer.cu:821-834, 930-1009, 1043-1099)."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [3072, 2048, 1001])
def test_rmsnorm(qk, torch_gpu, oracle, synth, n):
    t = torch_gpu
    ntok = 3
    x = synth.normal_f32(n * ntok, 91, 1).reshape(ntok, n) * np.float32(50.0)
    w = synth.normal_f32(n, 91, 2)
    out = t.empty((ntok, n), device="cuda")
    # Device copies stay bound to names until the launch has finished: a
    # temporary freed before the kernel runs lets the allocator reuse it.
    xd, wd = to_dev(t, x), to_dev(t, w)
    qk.check(qk.lib().qk_rmsnorm_f32(xd.data_ptr(), wd.data_ptr(), out.data_ptr(), n, ntok, 1e-5, None), "rmsnorm")
    t.cuda.synchronize()
    for k in range(ntok):
        assert rel_l2(out[k].cpu().numpy(), oracle.rmsnorm(x[k], w, 1e-5)) < 1e-6


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(32, 8, 64), (24, 8, 128)])
def test_rope_kv_write(qk, torch_gpu, oracle, synth, heads, kv_heads, head_dim):
    t = torch_gpu
    ctx, layer, pos, layers = 600, 1, 537, 3
    cos, sin = oracle.rope_tables(ctx, head_dim, 500000.0)
    kv = kv_heads * head_dim
    q = synth.normal_f32(heads * head_dim, 92, 1)
    k = synth.normal_f32(kv, 92, 2)
    v = synth.normal_f32(kv, 92, 3)
    kc = t.zeros((layers, ctx, kv), device="cuda")
    vc = t.zeros((layers, ctx, kv), device="cuda")
    qd, kd, vd, cd, sd = (to_dev(t, a) for a in (q, k, v, cos, sin))
    qk.check(qk.lib().qk_rope_kv_write(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cd.data_ptr(), sd.data_ptr(),
                                       kc.data_ptr(), vc.data_ptr(), layer, pos, ctx, heads, kv_heads, head_dim,
                                       None), "rope")
    t.cuda.synchronize()
    assert np.max(np.abs(qd.cpu().numpy() - oracle.rope(q, cos, sin, pos, head_dim))) < 1e-5
    assert np.max(np.abs(kc[layer, pos].cpu().numpy() - oracle.rope(k, cos, sin, pos, head_dim))) < 1e-5
    assert np.array_equal(vc[layer, pos].cpu().numpy(), v)
    # nothing else written
    kc[layer, pos] = 0
    vc[layer, pos] = 0
    assert float(kc.abs().sum()) == 0.0 and float(vc.abs().sum()) == 0.0


@pytest.mark.parametrize("heads,kv_heads,head_dim,pos", [(32, 8, 64, 591), (24, 8, 128, 100), (4, 4, 64, 0),
                                                          (32, 8, 64, 1023), (8, 1, 32, 300), (4, 2, 256, 77)])
def test_attention(qk, torch_gpu, oracle, synth, heads, kv_heads, head_dim, pos):
    t = torch_gpu
    ctx, layer, layers = 1024, 2, 3
    kv = kv_heads * head_dim
    q = synth.normal_f32(heads * head_dim, 93, 1)
    kc = synth.normal_f32(layers * ctx * kv, 93, 2).reshape(layers, ctx, kv)
    vc = synth.normal_f32(layers * ctx * kv, 93, 3).reshape(layers, ctx, kv)
    out = t.empty(heads * head_dim, device="cuda")
    qd, kd, vd = to_dev(t, q), to_dev(t, kc), to_dev(t, vc)
    qk.check(qk.lib().qk_attention_f32(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), out.data_ptr(), layer, pos, ctx,
                                       heads, kv_heads, head_dim, None), "attention")
    t.cuda.synchronize()
    want = oracle.attention(q, kc[layer, : pos + 1], vc[layer, : pos + 1], pos, heads, kv_heads, head_dim)
    assert rel_l2(out.cpu().numpy(), want) < 1e-5


def test_add_and_silu(qk, torch_gpu, synth):
    t = torch_gpu
    n = 8192
    a = synth.normal_f32(n, 94, 1)
    b = synth.normal_f32(n, 94, 2)
    ad, bd = to_dev(t, a), to_dev(t, b)
    qk.check(qk.lib().qk_add_f32(ad.data_ptr(), bd.data_ptr(), n, None), "add")
    t.cuda.synchronize()
    assert np.array_equal(ad.cpu().numpy(), a + b)
    g = synth.normal_f32(n, 94, 3) * np.float32(6.0)
    gd = to_dev(t, g)
    qk.check(qk.lib().qk_silu_mul_f32(gd.data_ptr(), bd.data_ptr(), n, None), "silu")
    t.cuda.synchronize()
    g64 = g.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * b
    assert rel_l2(gd.cpu().numpy(), want) < 1e-6


@pytest.mark.parametrize("n", [1, 1000, 128256])
def test_argmax_lowest_index(qk, torch_gpu, oracle, synth, n):
    t = torch_gpu
    v = synth.normal_f32(n, 95, 1)
    if n > 10:
        v[[7, n // 2, n - 1]] = 50.0
    ws = t.empty(max(qk.lib().qk_argmax_workspace_bytes(n), 8), dtype=t.uint8, device="cuda")
    out = t.full((1,), -1, dtype=t.int32, device="cuda")
    vd = to_dev(t, v)
    qk.check(qk.lib().qk_argmax_f32(vd.data_ptr(), n, out.data_ptr(), ws.data_ptr(), None), "argmax")
    t.cuda.synchronize()
    assert int(out.item()) == oracle.argmax(v)
