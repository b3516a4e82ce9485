"""Pins the oracle's block dots, row dots and matmul drivers.

- integer block dots against brute-force numpy int64 sums (and the reference's
  pattern vectors, q8q8_test.go:24-43);
- the reference tests' known answers (32, 32, 64, -16, nibble order);
- row results against an exact fp64 evaluation of the same quantized operands
  (a dropped term, a wrong sign or index, a swapped nibble half fails this);
- the reference's tolerance tests of the int8 path against its float path.
"""
import numpy as np
import pytest

import oracle
from sllm_qmm import synth

from _helpers import make_raw, make_x


@pytest.mark.parametrize("n", [32, 64, 32 * 18, 32 * 48])
def test_int8_dot_reference_pattern(n):
    i = np.arange(n)
    a = (i % 37 - 18).astype(np.int8)
    b = ((i * 7) % 51 - 25).astype(np.int8)
    assert oracle.int8_dot(a, b) == int((a.astype(np.int64) * b.astype(np.int64)).sum())


def _nibbles(raw_blocks: np.ndarray, off: int) -> np.ndarray:
    q = raw_blocks[:, off:off + 16]
    return np.concatenate([q & 0x0F, q >> 4], axis=1).astype(np.int64)  # elements 0..15, 16..31


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5k1", "q5"])
def test_block_dots_brute_force(qtype):
    N, K, M = 9, 512, 2
    raw = make_raw(qtype, N, K, seed=3)
    x = make_x(M, K, 4)
    got = oracle.block_dots(qtype, raw, N, K, x)
    xq, _ = oracle.quantize_act_q8(x)
    xq = xq.reshape(M, 1, K // 32, 32).astype(np.int64)
    G = K // 32
    if qtype == "q8":
        w = raw.reshape(N, G, 34)[..., 2:].view(np.int8).astype(np.int64)
        ref = (w[None] * xq).sum(-1)
    elif qtype == "q4":
        w = _nibbles(raw.reshape(N * G, 18), 2).reshape(N, G, 32) - 8
        ref = (w[None] * xq).sum(-1)
    elif qtype == "q4_1":
        w = _nibbles(raw.reshape(N * G, 20), 4).reshape(N, G, 32)
        ref = (w[None] * xq).sum(-1)
    elif qtype == "q5k1":
        lo = _nibbles(raw[: N * G * 20].reshape(N * G, 20), 4).reshape(N, G, 32)
        hi = _nibbles(raw[N * G * 20:].reshape(N * G, 20), 4).reshape(N, G, 32)
        ref = np.stack([(lo[None] * xq).sum(-1), (hi[None] * xq).sum(-1)], -1)
    else:
        # q5: the fp32 in-block partial in the reference's pair order
        b = raw.reshape(N * G, 22)
        qh = b[:, 2:6].copy().view(np.uint32)[:, 0]
        nib = _nibbles(b, 6)
        hb = ((qh[:, None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int64)
        v = ((nib | (hb << 4)) - 16).astype(np.float32).reshape(N, G, 32)
        xf = x.reshape(M, 1, G, 32)
        s = np.zeros((M, N, G), np.float32)
        for j in range(16):
            pair = (v[None, ..., j] * xf[..., j]).astype(np.float32) + (v[None, ..., j + 16] * xf[..., j + 16]).astype(np.float32)
            s = (s + pair).astype(np.float32)
        ref = s.view(np.int32)
    assert np.array_equal(got, ref)


def _q8_group(scale_bits, q):
    g = np.zeros(34, np.uint8)
    g[0], g[1] = scale_bits & 0xFF, scale_bits >> 8
    g[2:] = np.asarray(q, np.int8).view(np.uint8)
    return g


def test_known_answers():
    ones = np.ones((1, 32), np.float32)
    # float32_ops_test.go:304-346, 658-676: Q8 group, scale 1.0, q = 1, x = 1 -> 32
    assert oracle.matmul("q8", _q8_group(0x3C00, np.ones(32)), 1, ones)[0, 0] == pytest.approx(32.0, abs=0.01)
    # float32_ops_test.go:238-254, 582-602: Q4_0 nibbles 0x99 (both +1) -> 32
    g = np.zeros(18, np.uint8); g[1] = 0x3C; g[2:] = 0x99
    assert oracle.matmul("q4", g, 1, ones)[0, 0] == pytest.approx(32.0, abs=0.01)
    # q8_fast_test.go:121-143: Q4_1 d = 1, m = 1, nibbles 0, x = 2 -> 64
    g = np.zeros(20, np.uint8); g[1] = 0x3C; g[3] = 0x3C
    assert oracle.matmul("q4_1", g, 1, 2 * ones)[0, 0] == pytest.approx(64.0, abs=0.01)
    # q5_test.go:94-112: zero nibbles and high bits decode to -16
    g = np.zeros(22, np.uint8); g[1] = 0x3C
    assert np.all(oracle.dequant("q5_0", g, 32) == -16.0)
    assert oracle.matmul("q5", g, 1, ones)[0, 0] == -512.0


def test_q4_nibble_order():
    # quantize_test.go:215-248 and q8_fast_test.go:145-188
    g = np.zeros(18, np.uint8); g[1] = 0x3C; g[2:] = 0x09
    d = oracle.dequant("q4_0", g, 32)
    assert np.all(d[:16] == 1.0) and np.all(d[16:] == -8.0)
    g[2:] = 0xA3
    x = np.zeros(32); x[3], x[19] = 3.0, 7.0
    assert float(oracle.dequant("q4_0", g, 32) @ x) == -5.0 * 3.0 + 2.0 * 7.0
    g[2:] = [(j << 4) | (j + 1) for j in range(16)]
    d = oracle.dequant("q4_0", g, 32)
    assert d[:16].tolist() == [((j + 1) & 15) - 8 for j in range(16)]
    assert d[16:].tolist() == [j - 8 for j in range(16)]


def _exact_rows(qtype, raw, N, x):
    """fp64 evaluation of the same quantized operands (scales as each kernel decodes them)."""
    K = x.shape[1]
    G = K // 32
    xq, xs = oracle.quantize_act_q8(x)
    xa = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32, axis=1)
    if qtype == "q5":
        w = oracle.dequant("q5_0", raw, N * K).reshape(N, K)
        return x.astype(np.float64) @ w.T
    if qtype == "q5k1":
        w = (oracle.dequant("q4_1", raw[: N * G * 20], N * K) + oracle.dequant("q4_1", raw[N * G * 20:], N * K))
        return xa @ w.reshape(N, K).T
    kind = {"q8": "q8_0", "q4": "q4_0", "q4_1": "q4_1"}[qtype]
    return xa @ oracle.dequant(kind, raw, N * K).reshape(N, K).T


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5", "q5k1"])
def test_rows_match_exact_fp64_of_same_operands(qtype):
    N, K, M = 64, 1024, 3
    raw = make_raw(qtype, N, K, 8)
    x = make_x(M, K, 9)
    got = oracle.matmul(qtype, raw, N, x).astype(np.float64)
    ref = _exact_rows(qtype, raw, N, x)
    assert np.abs(got - ref).max() <= 1e-5 * np.abs(ref).max()


def test_q5k1_is_low_plus_high():
    N, K = 16, 512
    raw = make_raw("q5k1", N, K, 2)
    x = make_x(2, K, 3)
    half = N * (K // 32) * 20
    lo = oracle.matmul("q4_1", raw[:half], N, x)
    hi = oracle.matmul("q4_1", raw[half:], N, x)
    assert np.array_equal(oracle.matmul("q5k1", raw, N, x), (lo + hi).astype(np.float32))


def _pattern_x(n):
    return (((np.arange(n) % 23) - 11) * 0.017).astype(np.float32)


def test_q8q8_int8_path_vs_float_path():
    # q8q8_test.go:48-86: 64 x 576, pattern weights, <= 2% of the vector scale
    out_f, cols = 64, 576
    w = (((np.arange(out_f * cols) % 29) - 14) * 0.021).astype(np.float32).reshape(out_f, cols)
    raw = oracle.quantize_q8_rows_f32(w)
    wd = oracle.dequant("q8_0", raw, out_f * cols).reshape(out_f, cols)
    for rows in (1, 3):
        x = _pattern_x(rows * cols).reshape(rows, cols)
        ref = x.astype(np.float64) @ wd.T
        got = oracle.matmul("q8", raw, out_f, x)
        assert np.abs(got - ref).max() / np.abs(ref).max() <= 0.02


@pytest.mark.parametrize("qtype,bb,dm", [("q4", 18, None), ("q4_1", 20, (0.05, -0.3))])
def test_q4_int8_paths_vs_float_path(qtype, bb, dm):
    # q4q8_test.go:25-60 and q41q8_test.go:11-51: <= 5% of the vector scale
    out_f, cols = 48, 576
    groups = cols // 32
    raw = np.zeros((out_f, groups, bb), np.uint8)
    r = np.arange(out_f)[:, None, None]
    g = np.arange(groups)[None, :, None]
    j = np.arange(16)[None, None, :]
    off = 2 if qtype == "q4" else 4
    raw[..., off:] = ((r * 13 + g * 7 + j * 5) % 256).astype(np.uint8)
    d_bits = oracle.f64_to_f16(0.04 if qtype == "q4" else dm[0])
    raw[..., 0], raw[..., 1] = d_bits & 0xFF, d_bits >> 8
    if qtype == "q4_1":
        m_bits = oracle.f64_to_f16(dm[1])
        raw[..., 2], raw[..., 3] = m_bits & 0xFF, m_bits >> 8
    raw = raw.reshape(-1)
    x = _pattern_x(cols).reshape(1, cols)
    wd = oracle.dequant("q4_0" if qtype == "q4" else "q4_1", raw, out_f * cols).reshape(out_f, cols)
    ref = x.astype(np.float64) @ wd.T
    got = oracle.matmul(qtype, raw, out_f, x)
    assert np.abs(got - ref).max() / np.abs(ref).max() <= 0.05


def test_argmax_rules():
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1            # first of ties
    assert oracle.argmax(np.array([np.nan, 5, 6], np.float32)) == 0          # NaN at 0 is never replaced
    assert oracle.argmax(np.array([1, np.nan, 0.5, 7, 7], np.float32)) == 3  # later NaNs never win
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
