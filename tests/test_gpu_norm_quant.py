"""GPU fused RMSNorm + per-32 quantization (qk_rmsnorm_quantize_x32) against
the two-launch composition qk_rmsnorm_f32 + qk_quantize_x32 (bit for bit)
and the oracle: rmsnorm (inferencer.cu:821-834) in fp64 within 1e-6, and
quantize_x32 (inferencer.cu:544-556) of the kernel's own fp32 output,
bit-exact -- the contract of rmsnorm_quantize_cuda / _batch_cuda
(inferencer.cu:839-889)."""
import numpy as np
import pytest

from conftest import rel_l2, to_dev

pytestmark = pytest.mark.gpu


def _run_fused(qk, t, xd, wd, cols, ntok, ldx, ldxq, ldscale, with_out=True):
    out = t.full((ntok, cols), float("nan"), device="cuda") if with_out else None
    xq = t.zeros((ntok, ldxq), dtype=t.int8, device="cuda")
    xs = t.full((ntok, ldscale), -1.0, device="cuda")
    qk.rmsnorm_quantize(xd, wd, out, xq, xs, cols, ntok, 1e-5, ldx=ldx, ldxq=ldxq, ldscale=ldscale)
    t.cuda.synchronize()
    return out, xq, xs


@pytest.mark.parametrize("cols,ntok,ldx,ldxq,ldscale", [
    (2048, 1, 2048, 2048, 64),
    (3072, 3, 3072, 8192, 256),      # the reference's batch strides
    (8192, 5, 8200, 8192, 256),
    (2080, 2, 2080, 2080, 65),       # last loop round partly idle
    (32, 4, 36, 32, 1),
])
def test_fused_matches_two_launches_and_oracle(qk, torch_gpu, oracle, synth, cols, ntok, ldx, ldxq, ldscale):
    t = torch_gpu
    x = np.zeros((ntok, ldx), dtype=np.float32)
    x[:, :cols] = synth.normal_f32(ntok * cols, 300 + cols, 1).reshape(ntok, cols) * np.float32(20.0)
    w = synth.normal_f32(cols, 300 + cols, 2)
    xd, wd = to_dev(t, x), to_dev(t, w)
    out, xq, xs = _run_fused(qk, t, xd, wd, cols, ntok, ldx, ldxq, ldscale)

    # The same values through the two separate launches.
    xc = to_dev(t, np.ascontiguousarray(x[:, :cols]))
    out2 = t.empty((ntok, cols), device="cuda")
    xq2 = t.zeros((ntok, cols), dtype=t.int8, device="cuda")
    xs2 = t.empty((ntok, cols // 32), device="cuda")
    qk.check(qk.lib().qk_rmsnorm_f32(xc.data_ptr(), wd.data_ptr(), out2.data_ptr(), cols, ntok, 1e-5, None), "rms")
    qk.quantize(out2, xq2, xs2, cols, ntok)
    t.cuda.synchronize()

    o, q, s = out.cpu().numpy(), xq.cpu().numpy(), xs.cpu().numpy()
    assert np.array_equal(o.view(np.uint32), out2.cpu().numpy().view(np.uint32))
    assert np.array_equal(q[:, :cols], xq2.cpu().numpy())
    assert np.array_equal(s[:, : cols // 32].view(np.uint32), xs2.cpu().numpy().view(np.uint32))
    for k in range(ntok):
        assert rel_l2(o[k], oracle.rmsnorm(x[k, :cols], w, 1e-5)) < 1e-6
        wq, wsc = oracle.quantize_x32(o[k])
        assert np.array_equal(q[k, :cols], wq)
        assert np.array_equal(s[k, : cols // 32].view(np.uint32), wsc.view(np.uint32))
    # Nothing is written past the row in the strided buffers.
    assert not q[:, cols:].any()
    assert (s[:, cols // 32:] == -1.0).all()


def test_fused_without_fp32_copy_and_zero_row(qk, torch_gpu, oracle, synth):
    t = torch_gpu
    cols, ntok = 2048, 2
    x = synth.normal_f32(ntok * cols, 310, 1).reshape(ntok, cols)
    x[1] = 0.0                                   # rms 0: scale 1/sqrt(eps), values 0
    w = synth.normal_f32(cols, 310, 2)
    xd, wd = to_dev(t, x), to_dev(t, w)
    _, xq, xs = _run_fused(qk, t, xd, wd, cols, ntok, cols, cols, cols // 32, with_out=False)
    out, xq2, xs2 = _run_fused(qk, t, xd, wd, cols, ntok, cols, cols, cols // 32)
    assert np.array_equal(xq.cpu().numpy(), xq2.cpu().numpy())
    assert np.array_equal(xs.cpu().numpy(), xs2.cpu().numpy())
    assert not xq.cpu().numpy()[1].any()
    assert (xs.cpu().numpy()[1] == 1.0).all()    # amax 0 -> scale 1 (inferencer.cu:551)


def test_fused_rounds_half_to_even(qk, torch_gpu, oracle):
    """x = 1 everywhere with eps 0 makes the RMS scale exactly 1, so the
    normalised values are the planted weights: a group with amax 127 has
    quantization scale 1.0 and planted halves must round to even."""
    t = torch_gpu
    cols = 64
    x = np.ones((1, cols), dtype=np.float32)
    w = np.zeros(cols, dtype=np.float32)
    w[:8] = [127.0, 2.5, 3.5, -2.5, 0.5, -0.5, 1.5, -126.5]
    w[32:36] = [-300.0, 150.0, 1e-3, 299.0]
    xd, wd = to_dev(t, x), to_dev(t, w)
    out = t.empty((1, cols), device="cuda")
    xq = t.zeros((1, cols), dtype=t.int8, device="cuda")
    xs = t.empty((1, 2), device="cuda")
    qk.rmsnorm_quantize(xd, wd, out, xq, xs, cols, 1, 0.0)
    t.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy()[0], w)
    q, s = xq.cpu().numpy()[0], xs.cpu().numpy()[0]
    assert s[0] == 1.0
    assert q[:8].tolist() == [127, 2, 4, -2, 0, 0, 2, -126]
    wq, wsc = oracle.quantize_x32(w)
    assert np.array_equal(q, wq) and np.array_equal(s.view(np.uint32), wsc.view(np.uint32))
    assert q[32:36].tolist() == [-127, 64, 0, 127]
