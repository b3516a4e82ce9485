"""Pins the oracle's f16 codecs (refcpu.c) independently of their code.

Each check uses a route the oracle does not: numpy's IEEE half conversion, the
reference tests' own encode tables, or a closed-form property.
"""
import math

import numpy as np
import pytest

import oracle


def _all_halves():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    return bits, bits.view(np.float16).astype(np.float32)


def test_cvtph_decode_exhaustive_matches_ieee():
    # VCVTPH2PS is the exact IEEE conversion; numpy's float16 -> float32 is too.
    bits, ref = _all_halves()
    got = np.array([oracle.f16_to_f32_cvtph(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_lut_decode_flushes_subnormals_like_the_go_code():
    # dot_scalar.go:53-55 builds float32 bits frac<<13 and divides by 2^24 in
    # float32: compute that with numpy float32 arithmetic, independently.
    bits, exact = _all_halves()
    got = np.array([oracle.f16_to_f32_lut(int(b)) for b in bits], np.float32)
    sub = ((bits & 0x7C00) == 0) & ((bits & 0x3FF) != 0)
    frac = (bits[sub] & 0x3FF).astype(np.uint32)
    sign = (bits[sub] & 0x8000).astype(np.uint32) << 16
    with np.errstate(under="ignore"):
        go = (sign | (frac << 13)).view(np.float32) / np.float32(1 << 24)
    assert np.all(go == 0.0)
    assert np.array_equal(got[sub].view(np.uint32), go.view(np.uint32))  # signed zeros
    normal = ~sub & ~np.isnan(exact)
    assert np.array_equal(got[normal].view(np.uint32), exact[normal].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(exact)]))


def test_f16_to_f64_exact():
    bits, _ = _all_halves()
    ref = bits.view(np.float16).astype(np.float64)
    got = np.array([oracle.f16_to_f64(int(b)) for b in bits])
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan], ref[~nan])


@pytest.mark.parametrize("v,want", [
    (0.0, 0x0000), (1.0, 0x3C00), (-1.0, 0xBC00), (2.0, 0x4000), (0.5, 0x3800), (4.0, 0x4400),  # quantize_test.go:174-196
    (65504.0, 0x7BFF), (-65504.0, 0xFBFF),                                                      # gguf_test.go:297-316
    (math.nan, 0), (math.inf, 0), (-math.inf, 0),                                                # quantize_test.go:199-213
])
def test_f64_to_f16_reference_table(v, want):
    assert oracle.f64_to_f16(v) == want


def _trunc_f16_numpy(v: float) -> int:
    """Round-toward-zero f16 via numpy's round-to-nearest plus a one-ulp correction."""
    h = np.float16(v)
    if abs(float(h)) > abs(v):
        hb = int(np.array([h]).view(np.uint16)[0])
        hb = (hb & 0x8000) | ((hb & 0x7FFF) - 1)
        return hb
    return int(np.array([h]).view(np.uint16)[0])


def test_f64_to_f16_truncates_in_normal_range():
    rng = np.random.default_rng(1)
    e = rng.uniform(-14, 15.99, 20000)
    v = np.sign(rng.standard_normal(20000)) * np.exp2(e)
    for x in v:
        assert oracle.f64_to_f16(float(x)) == _trunc_f16_numpy(float(x)), x
    # a value just below 1 + 2^-10 truncates to 1.0 where rounding would not
    assert oracle.f64_to_f16(1.0 + 2 ** -10 - 2 ** -30) == 0x3C00


def test_f64_to_f16_flush_and_overflow():
    assert oracle.f64_to_f16(2.0 ** -14) == 0x0400          # smallest normal kept
    assert oracle.f64_to_f16(2.0 ** -15) == 0x0000          # below normal range -> +0 (no subnormals)
    assert oracle.f64_to_f16(-(2.0 ** -20)) == 0x8000       # -> -0
    assert oracle.f64_to_f16(-0.0) == 0x8000
    assert oracle.f64_to_f16(5e-324) == 0x0000              # fp64 subnormal
    assert oracle.f64_to_f16(65535.9) == 0x7BFF             # truncation stays finite
    assert oracle.f64_to_f16(65536.0) == 0x7C00             # exponent overflow -> +Inf
    assert oracle.f64_to_f16(-1e300) == 0xFC00


def test_f16_roundtrip_bound():
    # gguf_test.go:319-330
    for v in [0.0, 1.0, -1.0, 0.5, 127.0, 0.12345, 10000.0]:
        r = oracle.f16_to_f64(oracle.f64_to_f16(v))
        assert abs(r - v) / max(abs(v), 1e-10) <= 0.01
