"""GPU tests of the native Q2_K / Q3_K weights (sllm_weight_from_gguf types
10 and 11). The reference loads these types as dense float32 weights
(gguf.go:907-911) and multiplies with the sequential float32 loop
(modelMatmulFloatIntoF32, float32_ops.go:462-482); the library rebuilds each
of those float32 weights from the native blocks inside the GEMV.

* Per 32-element block, the GPU's sum of x * w from zero in element order is
  bit-identical to the oracle's over its dense weights (this pins every
  rebuilt weight and every product).
* Whole rows differ from the reference's sequential sum only in association:
  |got - ref| <= (K + K/32 + 64) u sum |x w|, u = 2^-24 (both sums' worst
  case; the block-level check above is the exact one).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq

from _helpers import make_raw, make_x

pytestmark = pytest.mark.gpu
U = 2.0 ** -24
PER = {10: 84, 11: 110}


def make_kq(t: int, rows: int, cols: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    nsb = rows * cols // 256
    raw = rng.integers(0, 256, (nsb, PER[t]), dtype=np.uint8)

    def f16(lo, hi):
        return np.frombuffer(rng.uniform(lo, hi, nsb).astype(np.float16).tobytes(), np.uint8).reshape(nsb, 2)

    if t == 10:
        raw[:, 80:82] = f16(1e-3, 3e-2)
        raw[:, 82:84] = f16(1e-3, 2e-2)
    else:
        raw[:, 108:110] = f16(1e-3, 3e-2)
    return raw.reshape(-1)


def load(t, N, K, seed):
    raw = make_kq(t, N, K, seed)
    return raw, sq.load_weight_f32_direct(t, raw, N, K), oracle.dense_weights(t, raw, N, K)


@pytest.mark.parametrize("t", [10, 11])
def test_export_round_trip(t):
    raw, w, _ = load(t, 40, 1024, 1)
    assert w.qtype == {10: "q2k", 11: "q3k"}[t]
    assert w.raw_bytes == raw.size
    assert np.array_equal(w.export(), raw)


@pytest.mark.parametrize("t", [10, 11])
def test_block_sums_bit_exact(t):
    N, K, M = 24, 768, 2
    raw, w, W = load(t, N, K, 2)
    x = make_x(M, K, seed=3)
    got = sq.debug_block_dots(w, x).view(np.float32)
    want = oracle.dense_block_sums(W, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t", [10, 11])
def test_block_sums_bit_exact_special_scales(t):
    # super-block scales d (and Q2_K's dmin) of +-inf, NaN, +-0 and the
    # smallest f16 subnormal among ordinary ones: the rebuilt weights follow
    # IEEE rules as the reference's fp64 dequantization rounded to float32 does
    N, K, M = 24, 768, 2
    raw = make_kq(t, N, K, 4).reshape(-1, PER[t])
    special = [0x7C00, 0xFC00, 0x7E00, 0x0000, 0x8000, 0x0001, 0x8001]
    at = 80 if t == 10 else 108
    for i, bits in enumerate(special):
        raw[3 * i, at:at + 2] = [bits & 0xFF, bits >> 8]
        if t == 10:
            raw[3 * i + 1, 82:84] = [bits & 0xFF, bits >> 8]
    raw = raw.reshape(-1)
    w = sq.load_weight_f32_direct(t, raw, N, K)
    W = oracle.dense_weights(t, raw, N, K)
    x = make_x(M, K, seed=5)
    got = sq.debug_block_dots(w, x).view(np.float32)
    want = oracle.dense_block_sums(W, x)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn)
    assert gn.any()  # the infinite and NaN scales were reached
    assert np.array_equal(got[~gn].view(np.uint32), want[~wn].view(np.uint32))


def test_q2k_block_sums_bit_exact_at_the_ends_of_the_f16_range():
    # d and dmin from opposite ends of the f16 range (largest normals against
    # subnormals, both ways, both signs): the GPU's one-rounding rebuild of
    # d*sc*q - dmin*m must give the reference's float32 of its float64
    # difference where the two products' magnitudes are furthest apart
    N, K, M = 64, 1024, 2
    raw = make_kq(10, N, K, 6).reshape(-1, PER[10])
    rng = np.random.default_rng(7)
    for i in range(raw.shape[0]):
        big, small = int(rng.integers(0x7000, 0x7C00)), int(rng.integers(0x0001, 0x0400))
        db, mb = (big, small) if i % 2 == 0 else (small, big)
        db |= int(rng.integers(0, 2)) << 15
        mb |= int(rng.integers(0, 2)) << 15
        raw[i, 80:82] = [db & 0xFF, db >> 8]
        raw[i, 82:84] = [mb & 0xFF, mb >> 8]
    raw = raw.reshape(-1)
    w = sq.load_weight_f32_direct(10, raw, N, K)
    W = oracle.dense_weights(10, raw, N, K)
    assert np.all(np.isfinite(W))
    x = make_x(M, K, seed=8)
    got = sq.debug_block_dots(w, x).view(np.float32)
    want = oracle.dense_block_sums(W, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,N,K,M", [(10, 300, 4096, 1), (11, 300, 4096, 1), (10, 96, 2048, 3),
                                     (11, 64, 1024, 70), (10, 14336, 4096, 1), (11, 4096, 14336, 1)])
def test_matmul_within_reassociation_bound(t, N, K, M):
    raw, w, W = load(t, N, K, 4 + M)
    x = make_x(M, K, seed=5)
    got = sq.model_matmul_quant_into_f32(w, x, M, K)[0].reshape(M, N).astype(np.float64)
    ref = oracle.matmul_dense(W, x).astype(np.float64)
    terms = np.abs(x).astype(np.float64) @ np.abs(W).astype(np.float64).T
    assert np.all(np.abs(got - ref) <= (K + K // 32 + 64) * U * terms + 1e-30)


def test_shared_launch_and_fused_paths_match_single_calls():
    K = 2048
    _, a, _ = load(10, 256, K, 6)
    _, b, _ = load(11, 128, K, 7)
    c = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", make_raw("q4_1", 96, K, seed=8), K // 32, 96, K))
    x = torch.from_numpy(make_x(1, K, seed=9)).cuda()
    outs = [torch.empty(w.rows, device="cuda") for w in (a, b, c)]
    sq.matmul_multi_dev([a, b, c], x.data_ptr(), 1, K, [o.data_ptr() for o in outs])
    singles = [torch.empty(w.rows, device="cuda") for w in (a, b, c)]
    for w, o in zip((a, b, c), singles):
        sq.matmul_dev(w, x.data_ptr(), 1, K, o.data_ptr())
    torch.cuda.synchronize()
    for o, s in zip(outs, singles):
        assert torch.equal(o.view(torch.int32), s.view(torch.int32))
    # paired gate / up with SwiGLU, and the fused RMSNorm, on Q2_K weights
    _, g, _ = load(10, 512, K, 10)
    _, u, _ = load(10, 512, K, 11)
    nw = np.random.default_rng(12).normal(1, 0.2, K).astype(np.float32)
    nwd = torch.from_numpy(nw).cuda()
    h = torch.empty(512, device="cuda")
    sq.rmsnorm_matmul_swiglu_dev(g, u, x.data_ptr(), nwd.data_ptr(), 1e-5, 1, K, h.data_ptr())
    normed = torch.from_numpy(oracle.rmsnorm(x.cpu().numpy(), nw, 1e-5, lib_order=True)).cuda()
    h2 = torch.empty(512, device="cuda")
    sq.matmul_swiglu_dev(g, u, normed.data_ptr(), 1, K, h2.data_ptr())
    # greedy argmax over a Q3_K head
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    logits = torch.empty(b.rows, device="cuda")
    sq.matmul_argmax_dev(b, x.data_ptr(), idx.data_ptr(), logits.data_ptr())
    torch.cuda.synchronize()
    assert torch.equal(h.view(torch.int32), h2.view(torch.int32))
    lg = logits.cpu().numpy()
    assert np.array_equal(lg.view(np.uint32), singles[1].cpu().numpy().view(np.uint32))
    assert int(idx.item()) == int(np.argmax(lg))


def test_matmul_add_on_native_kquants():
    K, N = 1024, 200
    _, w, W = load(11, N, K, 13)
    x = torch.from_numpy(make_x(1, K, seed=14)).cuda()
    base = np.random.default_rng(15).normal(size=N).astype(np.float32)
    dst = torch.from_numpy(base).cuda()
    sq.matmul_add_dev(w, x.data_ptr(), 1, K, dst.data_ptr())
    plain = torch.empty(N, device="cuda")
    sq.matmul_dev(w, x.data_ptr(), 1, K, plain.data_ptr())
    torch.cuda.synchronize()
    want = base + plain.cpu().numpy()
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), want.view(np.uint32))
