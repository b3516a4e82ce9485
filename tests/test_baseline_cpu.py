"""The timed CPU baseline (oracle/refcpu_simd.c: the reference's AVX2/AVX-VNNI
kernels and worker pool restated) computes what the scalar oracle computes."""
import numpy as np
import pytest

import oracle
from sllm_qmm import synth

from _helpers import make_raw, make_x, term_abs_sum


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5", "q5k1"])
def test_baseline_matches_oracle(qtype):
    N, K, M = 300, 1024, 3
    raw = make_raw(qtype, N, K, 17)
    x = make_x(M, K, 18)
    got = oracle.baseline_matmul(qtype, raw, N, x).astype(np.float64)
    ref = oracle.matmul(qtype, raw, N, x).astype(np.float64)
    # q8 / q4_1 / q5 / q5k1 take the same per-group term and sequential order as
    # the oracle; q4 uses the fused kernel's 4 FMA lane accumulators.
    if qtype == "q4":
        assert np.all(np.abs(got - ref) <= 1e-5 * term_abs_sum(qtype, raw, N, x) + 1e-30)
    else:
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("groups", [1, 2, 7, 18, 48])
def test_fused_q4_vs_scalar_decode(groups):
    # q4q8_test.go:62-91 (makeQ4Row pattern), tolerance 1e-3 * (|ref| + 1)
    raw = np.zeros((groups, 18), np.uint8)
    sb = oracle.f64_to_f16(0.04)
    raw[:, 0], raw[:, 1] = sb & 0xFF, sb >> 8
    g = np.arange(groups)[:, None]
    j = np.arange(16)[None, :]
    raw[:, 2:] = ((g * 13 + j * 5) % 256).astype(np.uint8)
    x = (((np.arange(groups * 32) % 23) - 11) * 0.017).astype(np.float32)[None]
    fused = oracle.baseline_matmul("q4", raw.reshape(-1), 1, x)[0, 0]
    scalar = oracle.matmul("q4", raw.reshape(-1), 1, x)[0, 0]
    assert abs(float(fused) - float(scalar)) <= 1e-3 * (abs(float(scalar)) + 1)


def test_worker_rule():
    # parallel.go:35-43
    w = oracle.baseline().bl_workers()
    import os
    n = len(os.sched_getaffinity(0))
    assert w == (n if n <= 8 else (n - 2 if n <= 18 else 16))


def test_synthetic_generator_is_deterministic():
    a = synth.normal(3, 1001)
    b = synth.normal(3, 1001)
    assert np.array_equal(a, b) and a.dtype == np.float32
    assert abs(float(a.mean())) < 0.1 and abs(float(a.std()) - 1) < 0.1
    assert np.array_equal(synth.q4k_blocks(1, 4, 256), synth.q4k_blocks(1, 4, 256))
    assert not np.array_equal(synth.q4k_blocks(1, 4, 256), synth.q4k_blocks(2, 4, 256))
