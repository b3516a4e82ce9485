"""The oracle's rmsNormFlatF32 (float32_ops.go:159-172): the reference order
against a pure-Python float32 restatement, and the library's association of
the sum of squares against an independent numpy restatement of that order."""
import math
import struct

import numpy as np

import oracle


def f32(v: float) -> float:
    return struct.unpack("<f", struct.pack("<f", v))[0]


def py_rmsnorm(x, w, eps):
    ss = 0.0
    for v in x:
        ss = f32(ss + f32(float(v) * float(v)))
    inv = f32(1.0 / f32(math.sqrt(ss / len(x) + float(np.float32(eps)))))
    return np.array([f32(f32(float(a) * inv) * float(b)) for a, b in zip(x, w)], np.float32)


def test_reference_order():
    rng = np.random.default_rng(1)
    for K in (32, 96, 576):
        x = rng.normal(0, 2, K).astype(np.float32)
        w = rng.normal(1, 0.1, K).astype(np.float32)
        got = oracle.rmsnorm(x[None], w, 1e-5)[0]
        assert np.array_equal(got.view(np.uint32), py_rmsnorm(x, w, 1e-5).view(np.uint32))


def np_lib_ss(x: np.ndarray) -> np.float32:
    K = x.size
    slots = np.zeros(256, np.float32)
    for s in range(256):
        p = np.float32(0)
        for i in range(s, K, 256):
            p = np.float32(p + np.float32(x[i] * x[i]))
        slots[s] = p
    def tree16(v):
        a = list(v)
        w = 1
        while w < 16:
            for i in range(0, 16, 2 * w):
                a[i] = np.float32(a[i] + a[i + w])
            w *= 2
        return a[0]
    waves = []
    for q in range(4):
        r = [tree16(slots[64 * q + 16 * k: 64 * q + 16 * k + 16]) for k in range(4)]
        waves.append(np.float32(np.float32(np.float32(r[0] + r[1]) + r[2]) + r[3]))
    return np.float32(np.float32(np.float32(waves[0] + waves[1]) + waves[2]) + waves[3])


def test_library_order():
    rng = np.random.default_rng(2)
    for K in (512, 4096, 1000 * 32):
        x = rng.normal(0, 1, K).astype(np.float32)
        w = rng.normal(1, 0.1, K).astype(np.float32)
        ss = np_lib_ss(x)
        inv = np.float32(1.0) / np.float32(math.sqrt(float(ss) / K + float(np.float32(1e-6))))
        want = (x * inv) * w
        got = oracle.rmsnorm(x[None], w, 1e-6, lib_order=True)[0]
        assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32))
        ref = oracle.rmsnorm(x[None], w, 1e-6)[0]
        # only the sum's association differs: a sequential float32 sum of K
        # squares is within K * 2^-24 of the exact one (relative), so are the
        # normed values, up to a few ulp of the scaling itself
        tol = (K + 4) * 2.0 ** -24 * np.abs(ref)
        assert np.all(np.abs(got - ref) <= tol)
