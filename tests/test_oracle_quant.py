"""Pins the oracle's quantizers: quantizeActivationsQ8 (q8q8.go:96-125),
quantizeQ8RowsF32 (gguf.go:1136-1186) and quantizeQ8Rows (gguf.go:1080-1134)."""
import math

import numpy as np

import oracle
from sllm_qmm import synth


def _act_closed_form(x: np.ndarray):
    """Per-element closed form with numpy float32 ops (IEEE division and product)."""
    b = x.reshape(-1, 32).astype(np.float32)
    a = np.abs(b)
    a[np.isnan(a)] = 0
    amax = a.max(axis=1)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        s = np.where(amax > 0, amax / np.float32(127.0), np.float32(0)).astype(np.float32)
        inv = np.where(amax > 0, np.float32(1.0) / s, np.float32(0)).astype(np.float32)
        p = (b * inv[:, None]).astype(np.float32)
        ok = (p >= -2147483648.0) & (p < 2147483648.0)
        q = np.where(ok, np.trunc(np.where(ok, p, 0)), -2147483648.0)
    q = np.clip(q, -128, 127).astype(np.int8)
    return q.reshape(x.shape), s


def test_activation_quantizer_closed_form():
    x = synth.normal(5, 64 * 32 * 9, 1.0).reshape(9, -1)
    x[1] *= np.float32(1e-38)          # denormal scales
    x[2, :32] = 0                      # all-zero block
    x[3, 5] = np.nan                   # NaN ignored by the max; its code is -128 (CVTTSS2SL)
    x[4, 7] = np.inf
    x[5] = np.float32(1e-45)           # scale underflows to 0, 1/scale = +Inf
    q, s = oracle.quantize_act_q8(x)
    rq, rs = _act_closed_form(x)
    assert np.array_equal(q, rq)
    assert np.array_equal(s.reshape(-1).view(np.uint32), rs.view(np.uint32))
    assert q[3, 5] == -128 and q[5, 0] == -128
    assert np.all(q[2, :32] == 0) and s[2, 0] == 0


def test_activation_quantizer_roundtrip():
    # q8q8_test.go:88-105
    x = np.sin(np.arange(4 * 32) * 0.3).astype(np.float32)
    q, s = oracle.quantize_act_q8(x)
    recon = q.reshape(4, 32).astype(np.float32) * s[:, None]
    assert np.all(np.abs(recon - x.reshape(4, 32)) <= s[:, None])


def test_activation_quantizer_invariants():
    x = synth.normal(6, 32 * 200, 3.0)
    q, s = oracle.quantize_act_q8(x)
    qn, sn = oracle.quantize_act_q8(-x)
    assert np.array_equal(s, sn) and np.array_equal(qn, -q)          # sign symmetry
    b = x.reshape(-1, 32)
    top = np.abs(b).argmax(axis=1)
    assert set(np.abs(q.reshape(-1, 32)[np.arange(200), top]).tolist()) <= {126, 127}  # truncation of ~127
    # truncation, not rounding: every code is at most |x|/scale in magnitude
    assert np.all(np.abs(q.reshape(-1, 32).astype(np.float64)) <= np.abs(b) / s[:, None] * (1 + 1e-6))


def _f16_trunc_bits(v: np.ndarray) -> np.ndarray:
    return np.array([oracle.f64_to_f16(float(t)) for t in v], np.uint16)


def _round_half_away(v: np.ndarray) -> np.ndarray:
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def test_quantize_q8_rows_f32_closed_form():
    rows, cols = 12, 256
    w = synth.normal(7, rows * cols, 0.02).reshape(rows, cols)
    w[2] = 0
    raw = oracle.quantize_q8_rows_f32(w).reshape(-1, 34)
    b = w.reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    s = np.where(amax > 0, amax / np.float32(127), 0).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = (np.float32(1) / s).astype(np.float32)
        val = (b * inv[:, None]).astype(np.float32).astype(np.float64)
    val = np.clip(val, -128, 127)
    q = np.where(np.isnan(val), 0, _round_half_away(np.nan_to_num(val))).astype(np.int8)
    assert np.array_equal(raw[:, 0].astype(np.uint16) | (raw[:, 1].astype(np.uint16) << 8), _f16_trunc_bits(s.astype(np.float64)))
    assert np.array_equal(raw[:, 2:].view(np.int8), q)
    assert np.all(raw.reshape(rows, -1, 34)[2] == 0)  # all-zero rows stay zero (NaN codes -> 0)


def test_quantize_q8_rows_f64_round_half_away_and_bound():
    # maxAbs 127 -> scale 1, inv 1: x = +-2.5 must round away from zero (math.Round)
    w = np.zeros((1, 32))
    w[0, 0] = 127.0
    w[0, 1], w[0, 2], w[0, 3] = 2.5, -2.5, 3.5
    raw = oracle.quantize_q8_rows_f64(w)
    assert int(raw[0]) | (int(raw[1]) << 8) == 0x3C00
    assert raw[2:6].view(np.int8).tolist() == [127, 3, -3, 4]
    # gguf_test.go:331-367 style reconstruction bound
    x = (np.arange(64) - 32) * 0.1
    raw = oracle.quantize_q8_rows_f64(x.reshape(2, 32)).reshape(2, 34)
    scale = np.array([oracle.f16_to_f64(int(r[0]) | (int(r[1]) << 8)) for r in raw])
    rec = raw[:, 2:].view(np.int8).astype(np.float64) * scale[:, None]
    assert np.abs(rec.reshape(-1) - x).max() < 0.5
    assert math.isclose(scale[0], 3.2 / 127, rel_tol=2 ** -9)
