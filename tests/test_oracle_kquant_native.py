"""Pins the oracle's Q2_K / Q3_K dequantizers (dequantizeQ2KNative /
dequantizeQ3KNative, kquants.go:147-245) and the dense float32 matmul
(modelMatmulFloatIntoF32, float32_ops.go:462-482). The reference's tests hold
no fixtures for these types, so the checks are by construction: blocks are
encoded here from chosen codes, scales, mins and high bits - element e of a
super-block belongs to 16-element sub-block e // 16; within a 128-element
half, the code of sub-block pair p sits at bit pair 2 (p % 4) of code byte
(16 * (e // 16 % 2) + e % 16); the Q3_K high bit at bit 4 * half + p % 4 of
mask byte (16 * (e // 16 % 2) + e % 16); the 6-bit Q3_K scales packed with low
nibbles in bytes 0..7 and high bit pairs in bytes 8..11 - and the decoded
values must equal d * sc * q - dmin * m (Q2_K) and d * (sc - 32) * (q - 4 (1 -
h)) (Q3_K) exactly."""
from __future__ import annotations

import numpy as np
import pytest

import oracle


def f16_bits(v: float) -> int:
    return int(np.array(v, np.float16).view(np.uint16))


def place_codes(qs: np.ndarray, codes: np.ndarray) -> None:
    for e in range(256):
        half, r = divmod(e, 128)
        sub = e // 16                      # 0..15
        pair = (sub % 8) // 2              # sub-block pair within the half
        byte = 32 * half + 16 * (sub % 2) + e % 16
        qs[byte] |= int(codes[e]) << (2 * pair)


def encode_q2k(codes, sc, mn, d, dmin) -> np.ndarray:
    blk = np.zeros(84, np.uint8)
    blk[0:16] = (np.asarray(sc) & 15) | ((np.asarray(mn) & 15) << 4)
    qs = np.zeros(64, np.int64)
    place_codes(qs, codes)
    blk[16:80] = qs.astype(np.uint8)
    blk[80:82] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    blk[82:84] = np.frombuffer(np.uint16(f16_bits(dmin)).tobytes(), np.uint8)
    return blk


def encode_q3k(codes, hbits, scales6, d) -> np.ndarray:
    blk = np.zeros(110, np.uint8)
    hm = np.zeros(32, np.int64)
    for e in range(256):
        half = e // 128
        sub = e // 16
        pair = (sub % 8) // 2
        hm[16 * (sub % 2) + e % 16] |= int(hbits[e]) << (4 * half + pair)
    blk[0:32] = hm.astype(np.uint8)
    qs = np.zeros(64, np.int64)
    place_codes(qs, codes)
    blk[32:96] = qs.astype(np.uint8)
    v = [int(s) for s in scales6]
    sc = np.zeros(12, np.int64)
    for i in range(4):
        sc[i] = (v[i] & 15) | ((v[8 + i] & 15) << 4)
        sc[4 + i] = (v[4 + i] & 15) | ((v[12 + i] & 15) << 4)
        sc[8 + i] = (v[i] >> 4) | ((v[4 + i] >> 4) << 2) | ((v[8 + i] >> 4) << 4) | ((v[12 + i] >> 4) << 6)
    blk[96:108] = sc.astype(np.uint8)
    blk[108:110] = np.frombuffer(np.uint16(f16_bits(d)).tobytes(), np.uint8)
    return blk


@pytest.mark.parametrize("seed", range(4))
def test_q2k_decodes_what_was_encoded(seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 4, 256)
    sc, mn = rng.integers(0, 16, 16), rng.integers(0, 16, 16)
    d, dmin = float(np.float16(rng.uniform(1e-3, 0.1))), float(np.float16(rng.uniform(1e-3, 0.05)))
    got = oracle.dequant("q2_k", encode_q2k(codes, sc, mn, d, dmin), 256)
    sub = np.arange(256) // 16
    want = d * sc[sub].astype(np.float64) * codes - dmin * mn[sub].astype(np.float64)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(4))
def test_q3k_decodes_what_was_encoded(seed):
    rng = np.random.default_rng(10 + seed)
    codes = rng.integers(0, 4, 256)
    hb = rng.integers(0, 2, 256)
    s6 = rng.integers(0, 64, 16)
    d = float(np.float16(rng.uniform(1e-3, 0.1)))
    got = oracle.dequant("q3_k", encode_q3k(codes, hb, s6, d), 256)
    sub = np.arange(256) // 16
    want = d * (s6[sub].astype(np.float64) - 32) * (codes - 4 * (1 - hb)).astype(np.float64)
    assert np.array_equal(got, want)


def test_special_cases():
    # zero codes leave only the minimum; all high bits set remove the -4 offset;
    # scale 32 in Q3_K zeroes the sub-block
    z = np.zeros(256, np.int64)
    got = oracle.dequant("q2_k", encode_q2k(z, np.full(16, 5), np.arange(16), 0.5, 0.25), 256)
    assert np.array_equal(got, -0.25 * (np.arange(256) // 16))
    ones = np.ones(256, np.int64)
    got = oracle.dequant("q3_k", encode_q3k(np.full(256, 3), ones, np.full(16, 33), 2.0), 256)
    assert np.array_equal(got, np.full(256, 6.0))
    got = oracle.dequant("q3_k", encode_q3k(np.full(256, 3), z, np.full(16, 32), 2.0), 256)
    assert np.all(got == 0.0)


def test_dense_matmul_is_the_sequential_float32_loop():
    # float64 product within the bound of a sequential float32 sum
    rng = np.random.default_rng(3)
    N, K = 7, 1000
    w = rng.normal(size=(N, K)).astype(np.float32)
    x = rng.normal(size=(2, K)).astype(np.float32)
    got = oracle.matmul_dense(w, x).astype(np.float64)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    bound = (K + 1) * 2.0 ** -24 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    assert np.all(np.abs(got - want) <= bound)
    # one row of length 1: exactly the float32 product
    assert oracle.matmul_dense(w[:, :1], x[:, :1])[0, 0] == np.float32(x[0, 0] * w[0, 0])
    # block sums add up (in float64) to the float64 product
    bs = oracle.dense_block_sums(w[:, :992], x[:, :992]).astype(np.float64)
    want = x[:, :992].astype(np.float64) @ w[:, :992].astype(np.float64).T
    assert np.all(np.abs(bs.sum(axis=2) - want) <= 40 * 2.0 ** -24 * (np.abs(x[:, :992]).astype(np.float64) @ np.abs(w[:, :992]).astype(np.float64).T))


def test_dense_weights_are_the_float32_rounding():
    rng = np.random.default_rng(4)
    raw = np.concatenate([encode_q2k(rng.integers(0, 4, 256), rng.integers(0, 16, 16), rng.integers(0, 16, 16),
                                     0.013, 0.007) for _ in range(4)])
    w = oracle.dense_weights(10, raw, 2, 512)
    assert w.dtype == np.float32 and w.shape == (2, 512)
    assert np.array_equal(w.reshape(-1), oracle.dequant("q2_k", raw, 1024).astype(np.float32))


def _round_f32(fr) -> float:
    """Correctly rounded float32 (nearest, ties to even) of an exact nonzero
    rational in float32's normal range, by integer arithmetic."""
    from fractions import Fraction
    sign = -1.0 if fr < 0 else 1.0
    a = abs(fr)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if a < Fraction(2) ** e:
        e -= 1
    elif a >= Fraction(2) ** (e + 1):
        e += 1
    scaled = a / Fraction(2) ** (e - 23)  # in [2^23, 2^24)
    q, r = divmod(scaled.numerator, scaled.denominator)
    if 2 * r > scaled.denominator or (2 * r == scaled.denominator and q & 1):
        q += 1
    return sign * q * 2.0 ** (e - 23)


def test_q2k_fp64_difference_rounds_like_one_float32_rounding():
    # The reference forms d*sc*q - dmin*m in float64 and the dense loader
    # rounds it to float32 (kquants.go:163-172, gguf.go:907-911); the GPU
    # rounds the exact difference once (a fused multiply-add: d*sc*q has at
    # most 17 significant bits, dmin*m at most 15, both exact in float32).
    # Both operands are integer multiples of 2^-24 (f16's finest step) below
    # 2^22, so the float64 difference is always exact and the two routes
    # round the same value once. Checked against exact rational arithmetic
    # over scales from the ends of the f16 range, with float32 roundings that
    # are inexact, also just below powers of two (where float32's spacing
    # halves).
    from fractions import Fraction
    rng = np.random.default_rng(11)
    classes = []
    for i in range(240):
        kind = i % 4
        if kind == 0:    # large d, subnormal dmin
            db, mb = int(rng.integers(0x7000, 0x7C00)), int(rng.integers(0x0001, 0x0400))
        elif kind == 1:  # subnormal d, large dmin
            db, mb = int(rng.integers(0x0001, 0x0400)), int(rng.integers(0x7000, 0x7C00))
        elif kind == 2:  # d a power of two, dmin tiny and positive
            db, mb = int(rng.integers(0x18, 0x1F)) << 10, int(rng.integers(0x0001, 0x0100))
        else:            # anywhere in the finite f16 range
            db, mb = int(rng.integers(0x0001, 0x7C00)), int(rng.integers(0x0001, 0x7C00))
        if kind != 2:
            db |= int(rng.integers(0, 2)) << 15
            mb |= int(rng.integers(0, 2)) << 15
        classes.append((db, mb))
    f16 = lambda b: float(np.array(b, np.uint16).view(np.float16))
    blocks, expect = [], []
    for db, mb in classes:
        codes = rng.integers(0, 4, 256)
        sc = rng.integers(0, 16, 16)
        mn = rng.integers(0, 16, 16)
        if db & 0x3FF == 0:  # scales 1, 2, 4, 8 (and codes 1, 2) keep d*sc*q a power of two
            sc = np.array([1, 2, 4, 8])[rng.integers(0, 4, 16)]
        d, dm = f16(db), f16(mb)
        blocks.append(encode_q2k(codes, sc, mn, d, dm))
        expect.append((d, dm, codes, sc, mn))
    raw = np.concatenate(blocks)
    got = oracle.dequant("q2_k", raw, 256 * len(blocks)).astype(np.float32).reshape(len(blocks), 256)
    inexact64 = inexact32 = pow2_inexact = 0
    for bi, (d, dm, codes, sc, mn) in enumerate(expect):
        memo = {}
        for e in range(256):
            key = (int(sc[e // 16]), int(codes[e]), int(mn[e // 16]))
            if key not in memo:
                s, q, m = key
                exact = Fraction(d) * s * q - Fraction(dm) * m
                if exact == 0:
                    memo[key] = None
                else:
                    memo[key] = _round_f32(exact)
                    inexact64 += int(Fraction(float(np.float64(d * s * q) - np.float64(dm * m))) != exact)
                    if Fraction(memo[key]) != exact:
                        inexact32 += 1
                        pow2_inexact += int(d * s * q > 0 and (d * s * q).hex().startswith("0x1.0000000000000p"))
            want = memo[key]
            if want is None:
                assert got[bi, e] == 0.0
            else:
                assert np.float32(want).view(np.uint32) == got[bi, e].view(np.uint32), (bi, e, key)
    assert inexact64 == 0      # the float64 difference never rounds
    assert inexact32 > 1000    # the float32 rounding does
    assert pow2_inexact > 10   # ... also just below powers of two
