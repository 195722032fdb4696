"""Pins the oracle's GEMV (qk_oracle.c: oq_gemv_f64 restating the maths of
gemv_quant, inferencer.cu:645-661; oq_gemv_f32_ref restating its fp32 lane
order) against numpy's float64 matmul of the dequantized matrix and against
closed-form invariants."""
import numpy as np
import pytest

from conftest import rel_l2

Q4_K, Q6_K = 12, 14


@pytest.mark.parametrize("qtype,cols,rows", [(Q4_K, 512, 64), (Q6_K, 512, 64), (Q4_K, 3072, 17), (Q6_K, 2048, 33)])
def test_gemv_f64_matches_numpy(oracle, workloads, qtype, cols, rows):
    w, x = workloads.gemv_case(qtype, cols, rows, seed=7)
    W = oracle.dequant(qtype, w, cols, rows).astype(np.float64)
    want = W @ x.astype(np.float64)
    got = oracle.gemv_f64(qtype, w, x, cols, rows)
    assert rel_l2(got, want) < 1e-13


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_gemv_invariants(oracle, workloads, qtype):
    cols, rows = 1024, 40
    w, x = workloads.gemv_case(qtype, cols, rows, seed=8)
    W = oracle.dequant(qtype, w, cols, rows).astype(np.float64)
    # One-hot x selects a dequantized column exactly.
    for c in (0, 31, 32, 255, 256, 777, 1023):
        e = np.zeros(cols, dtype=np.float32)
        e[c] = 1.0
        assert np.array_equal(oracle.gemv_f64(qtype, w, e, cols, rows), W[:, c])
    # All-ones x gives the row sums.
    ones = np.ones(cols, dtype=np.float32)
    assert rel_l2(oracle.gemv_f64(qtype, w, ones, cols, rows), W.sum(axis=1)) < 1e-14
    # Scaling x by 2^k scales y exactly.
    y = oracle.gemv_f64(qtype, w, x, cols, rows)
    assert np.array_equal(oracle.gemv_f64(qtype, w, (x * np.float32(8.0)).astype(np.float32), cols, rows), y * 8.0)


def test_gemv_batched_tokens(oracle, workloads):
    w, x = workloads.gemv_case(Q4_K, 768, 20, seed=9, n_tokens=5)
    y = oracle.gemv_f64(Q4_K, w, x, 768, 20)
    for t in range(5):
        assert np.array_equal(y[t], oracle.gemv_f64(Q4_K, w, x[t], 768, 20))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_gemv_f32_ref_tolerance(oracle, workloads, qtype):
    # The fp32 restatement of the reference kernel's order stays within
    # fp32 rounding of the fp64 truth.
    w, x = workloads.gemv_case(qtype, 2048, 256, seed=10)
    assert rel_l2(oracle.gemv_f32_ref(qtype, w, x, 2048, 256), oracle.gemv_f64(qtype, w, x, 2048, 256)) < 2e-6


def test_config1_reference_semantics(oracle, workloads):
    w, x = workloads.gemv_q4k_2048()
    y64 = oracle.gemv_f64(Q4_K, w, x, 2048, 2048)
    assert rel_l2(oracle.gemv_f32_ref(Q4_K, w, x, 2048, 2048), y64) < 2e-6
