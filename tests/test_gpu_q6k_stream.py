"""GPU tests of Q6_K weights streamed natively (tuning knob gemv_q6k_stream,
off by default). A Q6_K weight loaded with the knob set keeps its 6-bit codes
beside the Q8_0 planes the reference's load computes (dequantizeQ6KBlock +
quantizeQ8Rows, gguf.go:988-1015, 1080-1134), and the decode GEMV, while the
knob is set, rebuilds each block's Q8_0 codes and scale in registers from
them. Its results must be bit-identical to the kernel that reads the Q8_0
planes (which tests/test_gpu_parity.py pins to the oracle byte for byte), on
every entry point: random blocks, blocks built to have exact ties that round
both ways inside one sub-block (left to the kernel's fp64 path), and f16
special values of d."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import make_x

pytestmark = pytest.mark.gpu


def _load(raw: np.ndarray, N: int, K: int) -> sq.DeviceWeight:
    """A Q6_K weight loaded with its streamed planes."""
    sq.set_param("gemv_q6k_stream", 1)
    try:
        return sq.load_weight_f32_direct(synth.GGML_Q6_K, raw, N, K)
    finally:
        sq.set_param("gemv_q6k_stream", 0)


def _both(fn):
    """fn() run with the streamed kernel and with the Q8_0-plane kernel."""
    try:
        sq.set_param("gemv_q6k_stream", 1)
        a = fn()
        sq.set_param("gemv_q6k_stream", 0)
        b = fn()
    finally:
        sq.set_param("gemv_q6k_stream", 0)  # the default
    return a, b


def _bits(t):
    return t.cpu().numpy().view(np.uint32) if isinstance(t, torch.Tensor) else np.asarray(t).view(np.uint32)


def _put_d(raw: np.ndarray, vals) -> np.ndarray:
    """Super-block i takes d = vals[i % len(vals)] (f16 bits)."""
    r = raw.reshape(-1, 210).copy()
    v = np.asarray(vals, np.uint16)[np.arange(r.shape[0]) % len(vals)]
    r[:, 208] = (v & 0xff).astype(np.uint8)
    r[:, 209] = (v >> 8).astype(np.uint8)
    return r.reshape(-1)


def _tie_blocks(seed: int, N: int, K: int) -> np.ndarray:
    """Q6_K super-blocks whose every 32-element block has Mi = 127 * 32 = 254 * 16
    (sub-block scale 127 and a code of -32) and a second sub-block of scale 16
    with odd codes: 127 * 16 |q| / 4064 = |q| / 2 is a half-integer for every
    odd |q|, so each such sub-block has up to 16 exact ties, and with d drawn
    widely some blocks' ties round both ways."""
    rng = np.random.default_rng(seed)
    nsb = N * K // 256
    r = np.zeros((nsb, 210), np.uint8)
    q = rng.integers(-32, 32, size=(nsb, 256))          # element order of the super-block
    odd = 2 * rng.integers(0, 16, size=(nsb, 256)) + 1   # 1..31
    sgn = np.where(rng.random((nsb, 256)) < 0.5, -1, 1)
    for blk in range(8):                                 # 32-element block blk: elements 32 blk ..
        q[:, 32 * blk] = -32                             # in sub-block 2 blk (scale 127)
        q[:, 32 * blk + 16:32 * blk + 32] = np.clip(sgn * odd, -31, 31)[:, 32 * blk + 16:32 * blk + 32]
    sc = np.tile(np.array([127, 16], np.int64), 8)[None, :].repeat(nsb, 0)
    sc[:, 1::2] = np.where(rng.random((nsb, 8)) < 0.2, rng.integers(-128, 128, (nsb, 8)), sc[:, 1::2])
    u = (q + 32).astype(np.uint8)                        # 6-bit codes
    # GGUF Q6_K layout (dequantizeQ6KBlock): element 128 n + 32 k + l takes the
    # low nibble of ql[64 n + 32 (k & 1) + l] (k < 2) or its high nibble, and
    # bits 2k.. of qh[32 n + l]; scale index 8 n + 2 k + l / 16
    for n in range(2):
        for k in range(4):
            e = 128 * n + 32 * k + np.arange(32)
            nib = u[:, e] & 15
            qlo = 64 * n + 32 * (k & 1) + np.arange(32)
            r[:, qlo] |= (nib if k < 2 else nib << 4).astype(np.uint8)
            r[:, 128 + 32 * n + np.arange(32)] |= ((u[:, e] >> 4) << (2 * k)).astype(np.uint8)
    r[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    d = (np.exp(rng.uniform(np.log(1e-5), np.log(10.0), nsb)) * np.where(rng.random(nsb) < 0.5, -1, 1))
    dv = d.astype(np.float16).view(np.uint16)
    r[:, 208] = (dv & 0xff).astype(np.uint8)
    r[:, 209] = (dv >> 8).astype(np.uint8)
    return r.reshape(-1)


def test_tie_blocks_decode_like_the_reference():
    # the load-time planes are the oracle's; exact ties in both directions exist
    N, K = 64, 2048
    raw = _tie_blocks(1, N, K)
    w = _load(raw, N, K)
    qt, ref = oracle.load_weight(14, raw, N, K)
    assert qt == "q8" and np.array_equal(w.export(), ref)
    assert 0 < w.q6k_exact_blocks < N * K // 32  # some blocks need the fp64 path, most do not
    for M in (1, 2, 5):
        x = make_x(M, K, seed=M)
        a, b = _both(lambda: sq.model_matmul_quant_into_f32(w, x, M, K)[0].copy())
        assert np.array_equal(_bits(a), _bits(b)), f"M={M}"


@pytest.mark.parametrize("N,K,M", [(4096, 14336, 1), (300, 1024, 3), (37, 2048, 5), (128, 4096, 4)])
def test_stream_equals_planes(N, K, M):
    raw = synth.q6k_blocks(90 + M, N, K)
    w = _load(raw, N, K)
    x = make_x(M, K, seed=M + 1)
    a, b = _both(lambda: sq.model_matmul_quant_into_f32(w, x, M, K)[0].copy())
    assert np.array_equal(_bits(a), _bits(b))
    assert w.q6k_exact_blocks >= 0
    if N * K <= 1 << 22:
        assert np.array_equal(w.export(), oracle.load_weight(14, raw, N, K)[1])


def test_special_d_values():
    # f16 subnormal, smallest normal, largest, +-0, +-Inf, NaN, negative, one
    N, K = 96, 1024
    vals = [0x0001, 0x03ff, 0x0400, 0x7bff, 0x0000, 0x8000, 0x7c00, 0xfc00, 0x7e00, 0xbc00, 0x3c00, 0x1234]
    raw = _put_d(synth.q6k_blocks(7, N, K), vals)
    raw = raw.reshape(-1, 210)
    raw[3, 192:208] = 0            # every scale zero: Mi = 0
    raw[5, 192:208] = 0x80         # every scale -128
    raw = raw.reshape(-1)
    w = _load(raw, N, K)
    assert np.array_equal(w.export(), oracle.load_weight(14, raw, N, K)[1])
    x = make_x(3, K, seed=4)
    a, b = _both(lambda: sq.model_matmul_quant_into_f32(w, x, 3, K)[0].copy())
    assert np.array_equal(_bits(a), _bits(b))


def test_knob_off_at_load_keeps_q8_planes_only():
    N, K = 64, 1024
    raw = synth.q6k_blocks(3, N, K)
    w = sq.load_weight_f32_direct(synth.GGML_Q6_K, raw, N, K)
    assert w.q6k_exact_blocks == -1
    sq.set_param("gemv_q6k_stream", 1)
    try:
        assert w.plane_bytes == N * K // 32 * 34  # no streamed planes: the Q8_0 kernel
    finally:
        sq.set_param("gemv_q6k_stream", 0)
    s = _load(raw, N, K)
    assert s.plane_bytes == N * K // 32 * 34
    sq.set_param("gemv_q6k_stream", 1)
    try:
        assert s.plane_bytes == N * K // 32 * 28 + N * K // 256 * 2
    finally:
        sq.set_param("gemv_q6k_stream", 0)


def test_stream_on_fused_entries():
    H, F = 4096, 1536
    g = _load(synth.q6k_blocks(80, F, H), F, H)
    u = _load(_tie_blocks(81, F, H), F, H)
    x = torch.from_numpy(make_x(1, H, seed=9)).cuda()
    nw = torch.from_numpy(np.random.default_rng(3).normal(1, 0.1, H).astype(np.float32)).cuda()
    res0 = torch.from_numpy(make_x(1, F, seed=10)).cuda()
    P = lambda t: t.data_ptr()

    def run():
        h = torch.empty(F, device="cuda")
        o = [torch.empty(F, device="cuda") for _ in range(2)]
        idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        r = res0.clone()
        sq.rmsnorm_matmul_swiglu_dev(g, u, P(x), P(nw), 1e-5, 1, H, P(h))
        sq.matmul_multi_dev([g, u], P(x), 1, H, [P(t) for t in o])
        sq.rmsnorm_matmul_argmax_dev(u, P(x), P(nw), 1e-5, P(idx))
        sq.matmul_add_dev(g, P(x), 1, H, P(r))
        torch.cuda.synchronize()
        return h.clone(), o[0].clone(), o[1].clone(), r, int(idx.item())

    a, b = _both(run)
    for ta, tb in zip(a[:4], b[:4]):
        assert torch.equal(ta.view(torch.int32), tb.view(torch.int32))
    assert a[4] == b[4]


def test_head_rmsnorm_argmax_full_size():
    # the Llama-3-8B output head (128256 x 4096, Q6_K) through the fused head
    # entry point, streamed and from the Q8_0 planes
    N, H = 128256, 4096
    w = _load(synth.q6k_blocks(55, N, H), N, H)
    x = torch.from_numpy(make_x(1, H, seed=56)).cuda()
    nw = torch.from_numpy(np.random.default_rng(57).normal(1, 0.1, H).astype(np.float32)).cuda()

    def run():
        logits = torch.empty(N, device="cuda")
        idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        sq.rmsnorm_matmul_argmax_dev(w, x.data_ptr(), nw.data_ptr(), 1e-5, idx.data_ptr(), logits.data_ptr())
        torch.cuda.synchronize()
        return logits.clone(), int(idx.item())

    a, b = _both(run)
    assert torch.equal(a[0].view(torch.int32), b[0].view(torch.int32))
    assert a[1] == b[1]
