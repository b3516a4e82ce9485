"""GEMV launch shapes against the oracle and against each other.

The tuning knobs only change how rows are streamed:
- ring depth D, through `gemv_inflight_kb` (D = 1, 2, 4 or 8);
- blocks per lane per unit, through `gemv_max_nb` (including a partial last chunk);
- waves per workgroup, through `gemv_waves` (rows per wave, so consecutive or strided rows).

A row's lane split and summation order depend only on K, so every setting
must give the same bits. Those bits must match the oracle's matmul within the
reassociation bound.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import sllm_qmm as sq

from _helpers import assert_fp32_parity, make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu

DEFAULTS = {"gemv_inflight_kb": 32768, "gemv_max_nb": 8, "gemv_waves": 16}
KNOBS = [("gemv_inflight_kb", (64, 4096, 1 << 20)), ("gemv_max_nb", (1, 2, 3)), ("gemv_waves", (4, 8))]
CASES = [("q4_1", 4096, 4096), ("q8", 1024, 14336), ("q5k1", 2048, 4096), ("q5", 1536, 2048), ("q4", 3000, 576)]


@pytest.mark.parametrize("qtype,N,K", CASES)
@pytest.mark.parametrize("M", [1, 3])
def test_launch_shapes_give_the_same_bits(qtype, N, K, M):
    raw = make_raw(qtype, N, K, seed=N + 7)
    x = make_x(M, K, seed=11 + M)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    for k, v in DEFAULTS.items():
        sq.set_param(k, v)
    base, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    base = base.reshape(M, N)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(base, ref, term_abs_sum(qtype, raw, N, x), f"{qtype} {N}x{K} M={M}")
    try:
        for knob, vals in KNOBS:
            for v in vals:
                sq.set_param(knob, v)
                got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
                assert np.array_equal(got.reshape(M, N).view(np.uint32), base.view(np.uint32)), \
                    f"{qtype} {N}x{K} M={M}: {knob}={v} changed the bits"
            sq.set_param(knob, DEFAULTS[knob])
    finally:
        for k, v in DEFAULTS.items():
            sq.set_param(k, v)
