"""GPU tests of the RMSNorm fused into the GEMV prologue (rmsNormFlatF32,
float32_ops.go:159-172, in front of forwardBlock's and outputLogits'
matmuls). The fused launches must give, bit for bit, what the plain
entry points give on rows normed by the oracle in the library's
sum-of-squares association; against the reference's sequential order the
normed inputs differ by a few ulp, so an activation code can move by one
step and the outputs agree only to that looser level."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq

from _helpers import make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu
EPS = 1e-5


def _w(qtype, N, K, seed):
    raw = make_raw(qtype, N, K, seed=seed)
    return raw, sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def _bits(t):
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("M", [1, 3, 64])
def test_norm_multi(M):
    K = 1024
    specs = [("q4_1", 384), ("q4_1", 96), ("q8", 96), ("q5", 64)]
    ws = [_w(q, n, K, seed=i + 3 * M)[1] for i, (q, n) in enumerate(specs)]
    x = make_x(M, K, seed=M) * np.float32(3.0)
    nw = np.random.default_rng(M).normal(1, 0.2, K).astype(np.float32)
    xd, nwd = _dev(x), _dev(nw)
    outs = [torch.empty(M * w.rows, device="cuda") for w in ws]
    sq.rmsnorm_matmul_multi_dev(ws, xd.data_ptr(), nwd.data_ptr(), EPS, M, K, [o.data_ptr() for o in outs])
    normed = _dev(oracle.rmsnorm(x, nw, EPS, lib_order=True))
    plain = [torch.empty(M * w.rows, device="cuda") for w in ws]
    sq.matmul_multi_dev(ws, normed.data_ptr(), M, K, [o.data_ptr() for o in plain])
    torch.cuda.synchronize()
    for w, a, b in zip(ws, outs, plain):
        assert np.array_equal(_bits(a), _bits(b)), (w.qtype, M)
    # against the reference order end to end (oracle norm + oracle matmul):
    # the two normed inputs differ by ulps, which can move an activation code
    # by a whole step; the outputs then differ by at most |W| |x_hat_a - x_hat_b|
    # (x_hat: the activations as the kernel multiplies them) plus the
    # reassociation bound
    ref_norm = oracle.rmsnorm(x, nw, EPS)
    lib_norm = oracle.rmsnorm(x, nw, EPS, lib_order=True)
    for (q, n), w, a in zip(specs, ws, outs):
        raw = w.export()
        ref = oracle.matmul(q, raw, n, ref_norm).astype(np.float64)
        kind = {"q8": "q8_0", "q4": "q4_0", "q4_1": "q4_1", "q5": "q5_0"}[q]
        W = np.abs(oracle.dequant(kind, raw, n * K).reshape(n, K).astype(np.float64))
        dx = np.abs(_act_hat(q, ref_norm) - _act_hat(q, lib_norm))
        bound = 1e-5 * term_abs_sum(q, raw, n, ref_norm) + dx @ W.T * 1.001 + 1e-30
        got = a.cpu().numpy().reshape(M, n).astype(np.float64)
        assert np.all(np.abs(got - ref) <= bound), q


def _act_hat(qtype, v):
    """The activations the kernel multiplies the weights by: fp32 for Q5_0,
    the Q8_0 codes times their block scale otherwise."""
    if qtype == "q5":
        return v.astype(np.float64)
    q, s = oracle.quantize_act_q8(v)
    M, K = v.shape
    return (q.astype(np.float64).reshape(M, K // 32, 32) * s.astype(np.float64)[..., None]).reshape(M, K)


@pytest.mark.parametrize("M", [1, 70])
def test_norm_swiglu(M):
    K, N = 512, 256
    _, wg = _w("q4_1", N, K, seed=1)
    _, wu = _w("q4_1", N, K, seed=2)
    x = make_x(M, K, seed=9)
    nw = np.random.default_rng(9).normal(1, 0.2, K).astype(np.float32)
    xd, nwd = _dev(x), _dev(nw)
    h = torch.empty(M * N, device="cuda")
    sq.rmsnorm_matmul_swiglu_dev(wg, wu, xd.data_ptr(), nwd.data_ptr(), EPS, M, K, h.data_ptr())
    normed = _dev(oracle.rmsnorm(x, nw, EPS, lib_order=True))
    h2 = torch.empty(M * N, device="cuda")
    sq.matmul_swiglu_dev(wg, wu, normed.data_ptr(), M, K, h2.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(_bits(h), _bits(h2))


def test_norm_argmax():
    K, N = 512, 3000
    _, w = _w("q8", N, K, seed=4)
    x = make_x(1, K, seed=5)
    nw = np.random.default_rng(5).normal(1, 0.2, K).astype(np.float32)
    xd, nwd = _dev(x), _dev(nw)
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    logits = torch.empty(N, device="cuda")
    sq.rmsnorm_matmul_argmax_dev(w, xd.data_ptr(), nwd.data_ptr(), EPS, idx.data_ptr(), logits.data_ptr())
    normed = _dev(oracle.rmsnorm(x, nw, EPS, lib_order=True))
    plain = torch.empty(N, device="cuda")
    sq.matmul_dev(w, normed.data_ptr(), 1, K, plain.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(_bits(logits), _bits(plain))
    lg = plain.cpu().numpy()
    assert int(idx.item()) == int(np.argmax(lg))


@pytest.mark.parametrize("K", [96, 800, 14336])
def test_norm_row_lengths(K):
    # fewer blocks than statistics slots, a row that ends inside the last load
    # batch, and a row that takes several prologue passes
    specs = [("q8", 200), ("q4_1", 72)]
    ws = [_w(q, n, K, seed=30 + i)[1] for i, (q, n) in enumerate(specs)]
    x = make_x(1, K, seed=K) * np.float32(2.5)
    nw = np.random.default_rng(K).normal(1, 0.2, K).astype(np.float32)
    xd, nwd = _dev(x), _dev(nw)
    outs = [torch.empty(w.rows, device="cuda") for w in ws]
    sq.rmsnorm_matmul_multi_dev(ws, xd.data_ptr(), nwd.data_ptr(), EPS, 1, K, [o.data_ptr() for o in outs])
    normed = _dev(oracle.rmsnorm(x, nw, EPS, lib_order=True))
    plain = [torch.empty(w.rows, device="cuda") for w in ws]
    sq.matmul_multi_dev(ws, normed.data_ptr(), 1, K, [o.data_ptr() for o in plain])
    torch.cuda.synchronize()
    for w, a, b in zip(ws, outs, plain):
        assert np.array_equal(_bits(a), _bits(b)), (w.qtype, K)


def test_norm_llama_shapes():
    # the 8B layer's norm + q/k/v and norm + gate/up/SwiGLU at decode
    from sllm_qmm import synth
    H, KV, F = 4096, 1024, 14336
    q = [sq.load_weight_f32_direct(12, synth.q4k_blocks(70 + i, n, H), n, H) for i, n in enumerate((H, KV, KV))]
    g = [sq.load_weight_f32_direct(12, synth.q4k_blocks(80 + i, F, H), F, H) for i in range(2)]
    x = make_x(1, H, seed=11) * np.float32(5)
    nw = np.random.default_rng(11).normal(1, 0.1, H).astype(np.float32)
    xd, nwd = _dev(x), _dev(nw)
    outs = [torch.empty(w.rows, device="cuda") for w in q]
    sq.rmsnorm_matmul_multi_dev(q, xd.data_ptr(), nwd.data_ptr(), EPS, 1, H, [o.data_ptr() for o in outs])
    h = torch.empty(F, device="cuda")
    sq.rmsnorm_matmul_swiglu_dev(g[0], g[1], xd.data_ptr(), nwd.data_ptr(), EPS, 1, H, h.data_ptr())
    normed = _dev(oracle.rmsnorm(x, nw, EPS, lib_order=True))
    plain = [torch.empty(w.rows, device="cuda") for w in q]
    sq.matmul_multi_dev(q, normed.data_ptr(), 1, H, [o.data_ptr() for o in plain])
    h2 = torch.empty(F, device="cuda")
    sq.matmul_swiglu_dev(g[0], g[1], normed.data_ptr(), 1, H, h2.data_ptr())
    torch.cuda.synchronize()
    for a, b in zip(outs, plain):
        assert np.array_equal(_bits(a), _bits(b))
    assert np.array_equal(_bits(h), _bits(h2))
