"""Seeded sweep of matmul shapes against the oracle: weight rows from 1 to a
few hundred (not multiples of the tile sizes), K from one block up (GEMM
stages of 128 columns or not), activation rows on both sides of every
GEMV / GEMM switch and tile edge, every int8 format and Q5_0. Each case is the
reference's modelMatmulQuantIntoF32 (float32_ops.go:379-460) on the same
bytes, held to the 1e-5 bar, with the same argmax wherever the bar cannot
swap the top two."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import sllm_qmm as sq

from _helpers import assert_fp32_parity, make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu

M_VALUES = [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 128, 129, 200]


def _cases():
    rng = np.random.default_rng(20260)
    cases = []
    for qtype in ("q8", "q4", "q4_1", "q5", "q5k1"):
        for _ in range(24):
            N = int(rng.integers(1, 700))
            if qtype == "q5k1":
                K = 256 * int(rng.integers(1, 9))
            else:
                K = 32 * int(rng.integers(1, 80))
            M = int(rng.choice(M_VALUES))
            cases.append((qtype, N, K, M))
    return cases


@pytest.mark.parametrize("qtype,N,K,M", _cases())
def test_shape_sweep(qtype, N, K, M):
    raw = make_raw(qtype, N, K, seed=N * 7 + K + M)
    x = make_x(M, K, seed=N + M)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    got, rows, cols = sq.model_matmul_quant_into_f32(w, x, M, K)
    assert (rows, cols) == (M, N)
    ref = oracle.matmul(qtype, raw, N, x)
    got = got.reshape(M, N)
    bound = term_abs_sum(qtype, raw, N, x)
    assert_fp32_parity(got, ref, bound, f"{qtype} {N}x{K} M={M}")
    for m in range(M):
        # the same winner wherever the reference's top two are further apart
        # than the bar lets the outputs move
        top = np.sort(ref[m].astype(np.float64))[::-1]
        if N == 1 or top[0] - top[1] > 2e-5 * bound[m].max():
            assert int(np.argmax(got[m])) == oracle.argmax(ref[m])


def _multi_cases():
    rng = np.random.default_rng(20261)
    cases = []
    for qtype in ("q8", "q4_1", "q5", "q5k1"):
        for _ in range(6):
            n = int(rng.integers(2, 5))
            Ns = tuple(int(v) for v in rng.integers(1, 500, n))
            K = 256 * int(rng.integers(1, 9)) if qtype == "q5k1" else 32 * int(rng.integers(1, 80))
            M = int(rng.choice(M_VALUES))
            cases.append((qtype, Ns, K, M))
    return cases


@pytest.mark.parametrize("qtype,Ns,K,M", _multi_cases())
def test_multi_shape_sweep(qtype, Ns, K, M):
    # consecutive matmuls on one input (q/k/v, gate/up) in one call: each
    # weight's output as its own modelMatmulQuantIntoF32 gives it
    raws = [make_raw(qtype, N, K, seed=N + 13 * i + K) for i, N in enumerate(Ns)]
    ws = [sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, r, K // 32, N, K)) for r, N in zip(raws, Ns)]
    x = make_x(M, K, seed=M + K)
    outs = sq.model_matmul_multi_quant_into_f32(ws, x, M, K)
    for r, N, got in zip(raws, Ns, outs):
        ref = oracle.matmul(qtype, r, N, x)
        assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, r, N, x), f"{qtype} multi {Ns}x{K} M={M}")
