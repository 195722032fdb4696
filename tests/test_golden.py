"""Committed fixtures (tests/golden/golden.npz, written by
tests/golden/make_golden.py).  On the CPU: the oracle reproduces the
hand-built known-answer blocks (closed forms of inferencer.cu:454-487 in
exact arithmetic) and its own recorded outputs, and the seeded generator
reproduces the Q4_K 2048 x 2048 workload byte for byte.  On the GPU: the HIP
dequant is bit-exact and the HIP GEMV within rel-L2 1e-5 of the fixtures."""
import hashlib
import pathlib

import numpy as np
import pytest

from conftest import rel_l2, to_dev

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "golden.npz"
Q4_K, Q6_K = 12, 14
TYPES = (("q4k", Q4_K), ("q6k", Q6_K))


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name,qtype", TYPES)
def test_oracle_known_answer_blocks(oracle, golden, name, qtype):
    blocks, want = golden[f"kat_{name}_blocks"], golden[f"kat_{name}_values"]
    got = oracle.dequant(qtype, blocks, 256, blocks.size // (144 if qtype == Q4_K else 210)).reshape(-1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name,qtype", TYPES)
def test_oracle_reproduces_recorded_outputs(oracle, golden, name, qtype):
    blocks = golden[f"rnd_{name}_blocks"]
    got = oracle.dequant(qtype, blocks, 256, 6).reshape(-1)
    assert np.array_equal(got.view(np.uint32), golden[f"rnd_{name}_values"].view(np.uint32))
    w, x = golden[f"gemv_{name}_512x64_w"], golden[f"gemv_{name}_512x64_x"]
    assert np.array_equal(oracle.gemv_f64(qtype, w, x, 512, 64), golden[f"gemv_{name}_512x64_y"])


def test_generator_reproduces_config1(oracle, workloads, golden):
    w, x = workloads.gemv_q4k_2048()
    assert hashlib.sha256(w.tobytes()).digest() == golden["config1_w_sha256"].tobytes()
    assert np.array_equal(oracle.gemv_f64(Q4_K, w, x, 2048, 2048), golden["config1_y"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,qtype", TYPES)
def test_gpu_dequant_matches_fixtures(qk, torch_gpu, golden, name, qtype):
    torch = torch_gpu
    for kind in ("kat", "rnd"):
        blocks = golden[f"{kind}_{name}_blocks"]
        n = blocks.size // (144 if qtype == Q4_K else 210)
        out = torch.full((n, 256), float("nan"), device="cuda")
        qk.dequant_rows(qk.Tensor((256, n), qtype, to_dev(torch, blocks)), out, 0, n)
        torch.cuda.synchronize()
        got = out.cpu().numpy().reshape(-1)
        assert np.array_equal(got.view(np.uint32), golden[f"{kind}_{name}_values"].view(np.uint32)), kind


@pytest.mark.gpu
@pytest.mark.parametrize("name,qtype", TYPES)
def test_gpu_gemv_matches_fixtures(qk, torch_gpu, golden, name, qtype):
    torch = torch_gpu
    w, x = golden[f"gemv_{name}_512x64_w"], golden[f"gemv_{name}_512x64_x"]
    y = torch.full((64,), float("nan"), device="cuda")
    qk.matvec(qk.Tensor((512, 64), qtype, to_dev(torch, w)), to_dev(torch, x), y, 512, 64)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), golden[f"gemv_{name}_512x64_y"]) <= 1e-5


@pytest.mark.gpu
def test_gpu_config1_matches_fixture(qk, torch_gpu, workloads, golden):
    torch = torch_gpu
    w, x = workloads.gemv_q4k_2048()
    y = torch.full((2048,), float("nan"), device="cuda")
    qk.matvec(qk.Tensor((2048, 2048), Q4_K, to_dev(torch, w)), to_dev(torch, x), y, 2048, 2048)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), golden["config1_y"]) <= 1e-5
