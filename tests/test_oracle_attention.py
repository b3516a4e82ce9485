"""Pins the oracle's restatement of the attention step of a decode / prefill
step (applyRopeInPlaceF32 float32_ops.go:174-188, fusedAttentionHeadF32
float32_ops.go:190-235, forwardBlock's head handling model_f32.go:398-466)
against the reference's own test expectations (float32_ops_test.go:53-120,
169-190) and against what the mathematics fixes: identities that hold
exactly, and float64 evaluations of the definitions within stated
floating-point bounds. A wrong sign, pair layout, position, mask limit, kv
head mapping or cache offset changes outputs by O(1) and fails these."""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle

U = 2.0 ** -24  # float32 unit roundoff


def freqs_for(d_k, half_dim=None, base=10000.0):
    # model_f32.go:256-260: float32(1 / base^(2i / ropeDim)), ropeDim = 2 * half_dim
    half_dim = half_dim or d_k // 2
    rope_dim = 2 * half_dim
    return np.array([1.0 / math.pow(base, 2.0 * i / rope_dim) for i in range(half_dim)], np.float32)


# ------------------------------------------------------------------ RoPE ----

def test_rope_reference_known_answer():
    # float32_ops_test.go:53-88: dK 4, halfDim 2, rows at positions 5 and 6
    data = np.array([[1.0, 0.0, 0.0, 1.0], [0.5, 0.5, -0.5, 0.5]], np.float32)
    freqs = np.array([1.0 / math.pow(10000.0, 0.0 / 4), 1.0 / math.pow(10000.0, 2.0 / 4)], np.float32)
    got = oracle.rope(data, 5, freqs, 2)
    for r in range(2):
        pos = 5 + r
        for i in range(2):
            ang = float(freqs[i]) * float(pos)
            c, s = np.float32(math.cos(ang)), np.float32(math.sin(ang))
            x0, x1 = data[r, 2 * i], data[r, 2 * i + 1]
            assert abs(float(got[r, 2 * i]) - float(x0 * c - x1 * s)) < 1e-5
            assert abs(float(got[r, 2 * i + 1]) - float(x0 * s + x1 * c)) < 1e-5


def test_rope_identity_at_position_zero_and_tail_untouched():
    rng = np.random.default_rng(1)
    x = rng.normal(size=(1, 10)).astype(np.float32)
    fr = freqs_for(10, 3)  # partial rotary: pairs 0..2, elements 6..9 pass through
    assert np.array_equal(oracle.rope(x, 0, fr, 3), x)
    y = oracle.rope(x, 7, fr, 3)
    assert np.array_equal(y[:, 6:], x[:, 6:])
    assert not np.array_equal(y[:, :6], x[:, :6])


def test_rope_is_a_rotation_of_each_pair():
    rng = np.random.default_rng(2)
    d_k = 64
    x = rng.normal(size=(9, d_k)).astype(np.float32)
    fr = freqs_for(d_k)
    y = oracle.rope(x, 100, fr, d_k // 2).astype(np.float64)
    xd = x.astype(np.float64)
    n0 = np.hypot(xd[:, 0::2], xd[:, 1::2])
    n1 = np.hypot(y[:, 0::2], y[:, 1::2])
    assert np.all(np.abs(n1 - n0) <= 8 * U * n0 + 1e-30)
    # and the rotation angle is freqs[i] * pos, the float32 product (float64
    # rotation by that angle, within the rounding of cos / sin and two products)
    for r in range(9):
        pos = 100 + r
        ang = (fr * np.float32(pos)).astype(np.float64)
        c, s = np.cos(ang), np.sin(ang)
        e0 = xd[r, 0::2] * c - xd[r, 1::2] * s
        e1 = xd[r, 0::2] * s + xd[r, 1::2] * c
        tol = 6 * U * (np.abs(xd[r, 0::2]) + np.abs(xd[r, 1::2]))
        assert np.all(np.abs(y[r, 0::2] - e0) <= tol)
        assert np.all(np.abs(y[r, 1::2] - e1) <= tol)


# ------------------------------------------------------------- attention ----

def f64_attention(q, k, v, causal, cache_len):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    d_k = q.shape[1]
    s = q @ k.T / math.sqrt(d_k)
    if causal:
        for qi in range(q.shape[0]):
            s[qi, cache_len + qi + 1:] = -np.inf
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    return p @ v, p


def attention_bound(q, k, v, p, score_rel=0.0):
    """|oracle - exact| per output element: the float32 dot (d_k + 2 roundings
    of sum |q_d k_d| scaled), the exp (score error + 2u), the sequential sum of
    kv_len exps and of the weighted values (kv_len + 4 roundings each) - all
    weighted by p |v|. score_rel adds an input error relative to sum |q||k|."""
    qa, ka, va = (np.abs(a.astype(np.float64)) for a in (q, k, v))
    d_k, kv = q.shape[1], k.shape[0]
    ds = (qa @ ka.T).max(axis=1) / math.sqrt(d_k) * ((d_k + 2) * U + score_rel)
    per = 2 * ds[:, None] + (2 * kv + 8) * U
    return (p @ va) * per + 1e-30


def test_attention_reference_known_answers():
    # float32_ops_test.go:90-105 and 107-120
    out = oracle.attention_head(np.array([[1.0, 0.0]]), np.array([[1.0, 0.0], [0.0, 1.0]]),
                                np.array([[1.0, 0.0], [0.0, 1.0]]), causal=False)
    assert 0.99 <= out[0].sum() <= 1.01 and out[0, 0] >= 0.5
    eye = np.eye(2, dtype=np.float32)
    out = oracle.attention_head(eye, eye, eye, causal=True, cache_len=0)
    assert out[0, 0] >= 0.99


def test_attention_one_key_returns_its_value_exactly():
    rng = np.random.default_rng(3)
    q, k, v = (rng.normal(size=(1, 32)).astype(np.float32) for _ in range(3))
    assert np.array_equal(oracle.attention_head(q, k, v), v)


def test_attention_identical_keys_average_the_values():
    rng = np.random.default_rng(4)
    n, d_k = 37, 16
    q = rng.normal(size=(1, d_k)).astype(np.float32)
    k = np.repeat(rng.normal(size=(1, d_k)).astype(np.float32), n, axis=0)
    v = rng.normal(size=(n, d_k)).astype(np.float32)
    got = oracle.attention_head(q, k, v, causal=False).astype(np.float64)
    mean = v.astype(np.float64).mean(axis=0)
    assert np.all(np.abs(got[0] - mean) <= (n + 4) * U * np.abs(v).astype(np.float64).mean(axis=0) * 2)


@pytest.mark.parametrize("q_rows,kv,cache_len", [(1, 1, 0), (1, 7, 6), (1, 300, 299), (3, 40, 37), (5, 5, 0)])
def test_attention_matches_float64_softmax(q_rows, kv, cache_len):
    rng = np.random.default_rng(kv + q_rows)
    d_k = 64
    q = (rng.normal(size=(q_rows, d_k)) * 2).astype(np.float32)
    k = (rng.normal(size=(kv, d_k))).astype(np.float32)
    v = rng.normal(size=(kv, d_k)).astype(np.float32)
    got = oracle.attention_head(q, k, v, causal=True, cache_len=cache_len).astype(np.float64)
    want, p = f64_attention(q, k, v, True, cache_len)
    assert np.all(np.abs(got - want) <= attention_bound(q, k, v, p))


def test_causal_mask_limit():
    # row qi sees keys 0 .. cache_len + qi; what lies beyond changes nothing
    rng = np.random.default_rng(5)
    q = rng.normal(size=(3, 16)).astype(np.float32)
    k = rng.normal(size=(10, 16)).astype(np.float32)
    v = rng.normal(size=(10, 16)).astype(np.float32)
    a = oracle.attention_head(q, k, v, causal=True, cache_len=6)
    k2, v2 = k.copy(), v.copy()
    k2[7:], v2[7:] = 50.0, -9.0  # beyond row 0's limit (6 + 0 + 1)
    b = oracle.attention_head(q, k2, v2, causal=True, cache_len=6)
    assert np.array_equal(a[0], b[0])
    assert not np.array_equal(a[1], b[1])  # row 1 sees key 7


# ------------------------------------------------------ the whole section ----

def f64_layer(q, k, v, n_heads, n_kv, d_k, cache_k, cache_v, cache_len, start_pos, freqs, half_dim,
              qb, kb, vb, qn, kn, eps):
    seq = q.shape[0]
    q, k, v = (a.astype(np.float64).copy() for a in (q, k, v))
    for a, b in ((q, qb), (k, kb), (v, vb)):
        if b is not None:
            n = min(b.size, a.shape[1])
            a[:, :n] += b[:n]

    def heads(a, n):
        return [a[:, h * d_k:(h + 1) * d_k].copy() for h in range(n)]

    def norm(x, w):
        return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)

    def rope(x):
        x = x.copy()
        for r in range(x.shape[0]):
            ang = (freqs * np.float32(start_pos + r)).astype(np.float64)
            c, s = np.cos(ang), np.sin(ang)
            x0, x1 = x[r, 0:2 * half_dim:2].copy(), x[r, 1:2 * half_dim:2].copy()
            x[r, 0:2 * half_dim:2] = x0 * c - x1 * s
            x[r, 1:2 * half_dim:2] = x0 * s + x1 * c
        return x

    qh, kh, vh = heads(q, n_heads), heads(k, n_kv), heads(v, n_kv)
    if qn is not None:
        qh = [norm(x, qn) for x in qh]
    if kn is not None:
        kh = [norm(x, kn) for x in kh]
    qh, kh = [rope(x) for x in qh], [rope(x) for x in kh]
    ck = cache_k.astype(np.float64).copy()
    cv = cache_v.astype(np.float64).copy()
    for g in range(n_kv):
        ck[g, cache_len:cache_len + seq] = kh[g]
        cv[g, cache_len:cache_len + seq] = vh[g]
    kv = cache_len + seq
    rep = n_heads // n_kv
    out = np.zeros((seq, n_heads * d_k))
    bounds = np.zeros_like(out)
    for h in range(n_heads):
        g = h // rep
        o, p = f64_attention(qh[h], ck[g, :kv], cv[g, :kv], True, cache_len)
        out[:, h * d_k:(h + 1) * d_k] = o
        # inputs of the score carry the norm and RoPE roundings: about d_k + 16 u
        bounds[:, h * d_k:(h + 1) * d_k] = attention_bound(qh[h], ck[g, :kv], cv[g, :kv], p,
                                                           score_rel=2 * (d_k + 16) * U)
    return out, ck, cv, bounds


@pytest.mark.parametrize("opts", [
    dict(n_heads=8, n_kv=2, d_k=16, seq=1, cache_len=11, half_dim=8, bias=False, qk=False),
    dict(n_heads=8, n_kv=2, d_k=16, seq=3, cache_len=5, half_dim=6, bias=True, qk=True),
    dict(n_heads=4, n_kv=4, d_k=32, seq=4, cache_len=0, half_dim=16, bias=True, qk=False),
])
def test_attention_layer_matches_float64(opts):
    rng = np.random.default_rng(opts["seq"] * 31 + opts["cache_len"])
    H, KV, dk, seq, cl = opts["n_heads"], opts["n_kv"], opts["d_k"], opts["seq"], opts["cache_len"]
    cap = cl + seq + 3
    q = rng.normal(size=(seq, H * dk)).astype(np.float32)
    k = rng.normal(size=(seq, KV * dk)).astype(np.float32)
    v = rng.normal(size=(seq, KV * dk)).astype(np.float32)
    ck = rng.normal(size=(KV, cap, dk)).astype(np.float32)
    cv = rng.normal(size=(KV, cap, dk)).astype(np.float32)
    fr = freqs_for(dk, opts["half_dim"])
    qb = kb = vb = qn = kn = None
    if opts["bias"]:
        qb = rng.normal(size=H * dk - 3).astype(np.float32)  # shorter than the row: only its length is added
        kb = rng.normal(size=KV * dk + 5).astype(np.float32)  # longer: only the row's width is added
        vb = rng.normal(size=KV * dk).astype(np.float32)
    if opts["qk"]:
        qn = rng.normal(1, 0.2, dk).astype(np.float32)
        kn = rng.normal(1, 0.2, dk).astype(np.float32)
    start = cl
    out, nk, nv = oracle.attention_layer(q, k, v, H, KV, dk, ck, cv, cl, start, fr, opts["half_dim"],
                                         qb, kb, vb, qn, kn, 1e-5)
    want, wk, wv, bound = f64_layer(q, k, v, H, KV, dk, ck, cv, cl, start, fr, opts["half_dim"],
                                    qb, kb, vb, qn, kn, 1e-5)
    assert np.all(np.abs(out - want) <= bound)
    # rows outside [cache_len, cache_len + seq) are untouched; the new ones are
    # the biased (v) and normed + rotated (k) rows
    assert np.array_equal(nk[:, :cl], ck[:, :cl]) and np.array_equal(nk[:, cl + seq:], ck[:, cl + seq:])
    assert np.array_equal(nv[:, :cl], cv[:, :cl])
    tol = 8 * (dk + 16) * U * np.abs(wk[:, cl:cl + seq]) + 1e-6 * (qn is not None)
    assert np.all(np.abs(nk[:, cl:cl + seq] - wk[:, cl:cl + seq]) <= tol + 4 * U)
    assert np.all(np.abs(nv[:, cl:cl + seq] - wv[:, cl:cl + seq]) <= 2 * U * np.abs(wv[:, cl:cl + seq]))


def test_gqa_head_mapping():
    # repeatKVDataF32 (float32_ops.go:252-260, tested at float32_ops_test.go:169-190):
    # q head h reads kv head h / nRep. kv head g's values are all g + 1.
    H, KV, dk, seq = 6, 2, 8, 1
    rng = np.random.default_rng(6)
    q = rng.normal(size=(seq, H * dk)).astype(np.float32)
    k = rng.normal(size=(seq, KV * dk)).astype(np.float32)
    v = np.concatenate([np.full((seq, dk), g + 1.0, np.float32) for g in range(KV)], axis=1)
    ck = np.zeros((KV, 4, dk), np.float32)
    cv = np.zeros((KV, 4, dk), np.float32)
    for g in range(KV):
        cv[g, :2] = g + 1.0
    out, _, _ = oracle.attention_layer(q, k, v, H, KV, dk, ck, cv, 2, 2, freqs_for(dk), dk // 2)
    for h in range(H):
        np.testing.assert_allclose(out[0, h * dk:(h + 1) * dk], h // 3 + 1.0, rtol=1e-6)
