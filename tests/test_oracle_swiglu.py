"""The oracle's SwiGLU (model_f32.go:486-489) against the formula evaluated
independently in Python: fp64 exp and division, float32 rounding of s, then
(gate * s) * up in float32."""
import math
import struct

import numpy as np

import oracle


def f32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def py_swiglu(g: float, u: float) -> float:
    try:
        e = math.exp(-g)
    except OverflowError:
        e = math.inf
    s = f32(1.0 / (1.0 + e)) if not math.isnan(e) else math.nan
    return f32(f32(g * s) * u)


def test_swiglu_matches_formula():
    rng = np.random.default_rng(3)
    g = np.concatenate([rng.normal(0, 3, 4000), [0.0, -0.0, 1e-30, -1e-30, 88.0, -88.0, 700.0, -700.0, 800.0,
                                                 -800.0]]).astype(np.float32)
    u = rng.normal(0, 2, g.size).astype(np.float32)
    got = oracle.swiglu(g, u)
    want = np.array([py_swiglu(float(a), float(b)) for a, b in zip(g, u)], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_swiglu_special_values():
    g = np.array([np.nan, np.inf, -np.inf, 0.0], np.float32)
    u = np.array([1.0, 2.0, 1.0, 5.0], np.float32)
    h = oracle.swiglu(g, u)
    assert np.isnan(h[0])                  # exp(NaN) = NaN
    assert h[1] == np.inf                  # s = 1: inf * 1 * 2
    assert np.isnan(h[2])                  # s = 0: -inf * 0 = NaN
    assert h[3] == 0.0                     # s = 0.5: 0 * 0.5 * 5
