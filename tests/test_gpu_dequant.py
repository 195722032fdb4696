"""GPU dequant (qk_dequant_rows, qk_embedding): bit-exact against the oracle's
q4_value / q6_value restatement, including every finite fp16 block scale."""
import numpy as np
import pytest

from conftest import to_dev
from test_oracle_dequant import pack_q4k_scales

pytestmark = pytest.mark.gpu
Q4_K, Q6_K = 12, 14


def gpu_dequant(qk, torch, qtype, w, cols, rows, row0=0):
    out = torch.full((rows, cols), float("nan"), device="cuda")
    qk.dequant_rows(qk.Tensor((cols, row0 + rows), qtype, to_dev(torch, w)), out, row0, rows)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_random_blocks_bit_exact(qk, torch_gpu, oracle, synth, qtype):
    cols, rows = 2048, 300
    w = synth.quant_matrix(qtype, cols, rows, 51, 1)
    got = gpu_dequant(qk, torch_gpu, qtype, w, cols, rows)
    want = oracle.dequant(qtype, w, cols, rows)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # A row window.
    got = gpu_dequant(qk, torch_gpu, qtype, w, cols, 7, row0=101)
    assert np.array_equal(got.view(np.uint32), want[101:108].view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_full_range_bytes_bit_exact(qk, torch_gpu, oracle, synth, qtype):
    # Uniform random bytes everywhere except finite fp16 scales.
    n = 4096
    bpb = 144 if qtype == Q4_K else 210
    w = synth.random_bytes(n * bpb, 52, 1).reshape(n, bpb)
    hdr = slice(0, 4) if qtype == Q4_K else slice(208, 210)
    k = (hdr.stop - hdr.start) // 2
    w[:, hdr] = synth.f64_to_f16_bits(np.random.default_rng(1).normal(0, 0.05, (n, k))).view(np.uint8).reshape(n, -1)
    w = w.reshape(-1)
    got = gpu_dequant(qk, torch_gpu, qtype, w, 256 * 16, n // 16)
    want = oracle.dequant(qtype, w, 256 * 16, n // 16)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_every_fp16_scale(qk, torch_gpu, oracle):
    bits = np.arange(65536, dtype=np.uint16)
    finite = bits[np.isfinite(bits.view(np.float16))]
    n = finite.size - finite.size % 8
    finite = finite[:n]
    q4 = np.zeros((n, 144), dtype=np.uint8)
    q4[:, 0:2] = finite.view(np.uint8).reshape(-1, 2)
    q4[:, 2:4] = finite[::-1].copy().view(np.uint8).reshape(-1, 2)
    q4[:, 4:16] = pack_q4k_scales(np.arange(56, 64), np.arange(1, 9))
    q4[:, 16:] = np.arange(128, dtype=np.uint8)[None, :] * 2 + 1
    w = q4.reshape(-1)
    got = gpu_dequant(qk, torch_gpu, Q4_K, w, 2048, n // 8)
    want = oracle.dequant(Q4_K, w, 2048, n // 8)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    q6 = np.zeros((n, 210), dtype=np.uint8)
    q6[:, :192] = np.arange(192, dtype=np.uint8)[None, :] * 7
    q6[:, 192:208] = np.arange(-128, 128, 16, dtype=np.int8).view(np.uint8)[None, :]
    q6[:, 208:210] = finite.view(np.uint8).reshape(-1, 2)
    w6 = q6.reshape(-1)
    got6 = gpu_dequant(qk, torch_gpu, Q6_K, w6, 2048, n // 8)
    want6 = oracle.dequant(Q6_K, w6, 2048, n // 8)
    assert np.array_equal(got6.view(np.uint32), want6.view(np.uint32))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_embedding_gather(qk, torch_gpu, oracle, synth, qtype):
    t = torch_gpu
    cols, vocab = 2048, 1000
    w = synth.quant_matrix(qtype, cols, vocab, 53, 1)
    tokens = np.array([0, 999, 17, 17, 512], dtype=np.int32)
    out = t.empty((tokens.size, cols), device="cuda")
    qk.embedding(qk.Tensor((cols, vocab), qtype, to_dev(t, w)), to_dev(t, tokens), out, tokens.size)
    t.cuda.synchronize()
    want = oracle.embedding(qtype, w, tokens, cols)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_embedding_out_of_range_token_reads_nothing(qk, torch_gpu, synth):
    t = torch_gpu
    w = synth.quant_matrix(Q6_K, 512, 10, 54, 1)
    tokens = np.array([3, 10, -1], dtype=np.int32)
    out = t.zeros((3, 512), device="cuda")
    qk.embedding(qk.Tensor((512, 10), Q6_K, to_dev(t, w)), to_dev(t, tokens), out, 3)
    t.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.all(np.isfinite(o[0])) and np.all(np.isnan(o[1])) and np.all(np.isnan(o[2]))
