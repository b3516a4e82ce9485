"""GPU tests of Q6_K weights streamed natively (load option gemv_q6k_stream,
off by default). A Q6_K weight loaded with the option keeps its 6-bit codes
beside the Q8_0 planes the reference's load computes (dequantizeQ6KBlock +
quantizeQ8Rows, gguf.go:988-1015, 1080-1134), and its decode GEMV rebuilds
each block's Q8_0 codes and scale in registers from them. Its results are
checked against the oracle (oracle.matmul over the requantized Q8_0 Raw) and
must be bit-identical to those of the same weight loaded without the option
(the Q8_0-plane kernel), on every entry point: random blocks, blocks built to
have exact ties that round both ways inside one sub-block (left to the
kernel's fp64 path), f16 special values of d, and the full 128256 x 4096
head."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import assert_fp32_parity, make_x, term_abs_sum

pytestmark = pytest.mark.gpu


def _load(raw: np.ndarray, N: int, K: int, stream: bool = True) -> sq.DeviceWeight:
    """A Q6_K weight loaded with (stream) or without its streamed planes."""
    sq.set_param("gemv_q6k_stream", int(stream))
    try:
        return sq.load_weight_f32_direct(synth.GGML_Q6_K, raw, N, K)
    finally:
        sq.set_param("gemv_q6k_stream", 0)  # the default


def _pair(raw: np.ndarray, N: int, K: int):
    """The weight loaded with its 6-bit planes (streamed) and without (Q8_0 planes)."""
    return _load(raw, N, K, True), _load(raw, N, K, False)


def _check_oracle(got: np.ndarray, raw_q8: np.ndarray, N: int, x: np.ndarray, what: str) -> None:
    """The streamed kernel's output against the oracle (Q8_0 after the reference's requantization)."""
    x = np.asarray(x, np.float32).reshape(-1, x.shape[-1])
    assert_fp32_parity(np.asarray(got).reshape(x.shape[0], N), oracle.matmul("q8", raw_q8, N, x),
                       term_abs_sum("q8", raw_q8, N, x), what)


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
    ws, wp = _pair(raw, N, K)
    qt, ref = oracle.load_weight(14, raw, N, K)
    assert qt == "q8" and np.array_equal(ws.export(), ref)
    assert 0 < ws.q6k_exact_blocks < N * K // 32  # some blocks need the fp64 path, most do not
    for M in (1, 2, 5):
        x = make_x(M, K, seed=M)
        a = sq.model_matmul_quant_into_f32(ws, x, M, K)[0].copy()
        b = sq.model_matmul_quant_into_f32(wp, x, M, K)[0].copy()
        assert np.array_equal(_bits(a), _bits(b)), f"M={M}"
        _check_oracle(a, ref, N, x, f"tie blocks M={M}")


@pytest.mark.parametrize("N,K,M", [(4096, 14336, 1), (14336, 4096, 1), (300, 1024, 3), (37, 2048, 5),
                                   (128, 4096, 4)])
def test_stream_equals_planes_and_oracle(N, K, M):
    raw = synth.q6k_blocks(90 + M, N, K)
    ws, wp = _pair(raw, N, K)
    x = make_x(M, K, seed=M + 1)
    a = sq.model_matmul_quant_into_f32(ws, x, M, K)[0].copy()
    b = sq.model_matmul_quant_into_f32(wp, x, M, K)[0].copy()
    assert np.array_equal(_bits(a), _bits(b))
    assert ws.q6k_exact_blocks >= 0
    ref = oracle.load_weight(14, raw, N, K)[1]
    assert np.array_equal(ws.export(), ref)
    _check_oracle(a, ref, N, x, f"q6k stream {N}x{K} M={M}")


def test_special_d_values():
    # f16 subnormal, smallest normal, largest, +-0, +-Inf, NaN, negative, one
    N, K = 96, 1024
    vals = [0x0001, 0x03ff, 0x0400, 0x7bff, 0x0000, 0x8000, 0x7c00, 0xfc00, 0x7e00, 0xbc00, 0x3c00, 0x1234]
    raw = _put_d(synth.q6k_blocks(7, N, K), vals)
    raw = raw.reshape(-1, 210)
    raw[3, 192:208] = 0            # every scale zero: Mi = 0
    raw[5, 192:208] = 0x80         # every scale -128
    raw = raw.reshape(-1)
    ws, wp = _pair(raw, N, K)
    ref = oracle.load_weight(14, raw, N, K)[1]
    assert np.array_equal(ws.export(), ref)
    x = make_x(3, K, seed=4)
    a = sq.model_matmul_quant_into_f32(ws, x, 3, K)[0].copy()
    b = sq.model_matmul_quant_into_f32(wp, x, 3, K)[0].copy()
    assert np.array_equal(_bits(a), _bits(b))
    _check_oracle(a, ref, N, x, "q6k stream special d")


def test_option_acts_at_load_only():
    N, K = 64, 1024
    raw = synth.q6k_blocks(3, N, K)
    ws, wp = _pair(raw, N, K)
    assert wp.q6k_exact_blocks == -1 and ws.q6k_exact_blocks >= 0
    x = make_x(2, K, seed=3)
    a = sq.model_matmul_quant_into_f32(ws, x, 2, K)[0].copy()
    for opt in (1, 0):
        sq.set_param("gemv_q6k_stream", opt)
        try:
            assert wp.plane_bytes == N * K // 32 * 34  # no streamed planes: the Q8_0 kernel
            assert ws.plane_bytes == N * K // 32 * 28 + N * K // 256 * 2
            assert np.array_equal(_bits(sq.model_matmul_quant_into_f32(ws, x, 2, K)[0]), _bits(a))
        finally:
            sq.set_param("gemv_q6k_stream", 0)


def test_stream_on_fused_entries():
    H, F = 4096, 1536
    g_raw, u_raw = synth.q6k_blocks(80, F, H), _tie_blocks(81, F, H)
    gs, gp = _pair(g_raw, F, H)
    us, up = _pair(u_raw, F, H)
    x = torch.from_numpy(make_x(1, H, seed=9)).cuda()
    nw = torch.from_numpy(np.random.default_rng(3).normal(1, 0.1, H).astype(np.float32)).cuda()
    res0 = torch.from_numpy(make_x(1, F, seed=10)).cuda()
    P = lambda t: t.data_ptr()

    def run(g, u):
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

    a, b = run(gs, us), run(gp, up)
    for ta, tb in zip(a[:4], b[:4]):
        assert torch.equal(ta.view(torch.int32), tb.view(torch.int32))
    assert a[4] == b[4]


def test_head_rmsnorm_argmax_full_size():
    # the Llama-3-8B output head (128256 x 4096, Q6_K) through the fused head
    # entry point, streamed and from the Q8_0 planes, and the streamed logits
    # against the oracle's matmul of the same RMSNorm output
    N, H = 128256, 4096
    raw = synth.q6k_blocks(55, N, H)
    ws, wp = _pair(raw, N, H)
    xh = make_x(1, H, seed=56)
    nwh = np.random.default_rng(57).normal(1, 0.1, H).astype(np.float32)
    x = torch.from_numpy(xh).cuda()
    nw = torch.from_numpy(nwh).cuda()

    def run(w):
        logits = torch.empty(N, device="cuda")
        idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        sq.rmsnorm_matmul_argmax_dev(w, x.data_ptr(), nw.data_ptr(), 1e-5, idx.data_ptr(), logits.data_ptr())
        torch.cuda.synchronize()
        return logits.clone(), int(idx.item())

    a, b = run(ws), run(wp)
    assert torch.equal(a[0].view(torch.int32), b[0].view(torch.int32))
    assert a[1] == b[1]
    normed = oracle.rmsnorm(xh, nwh, 1e-5, lib_order=True).reshape(1, H)
    ref_q8 = wp.export()
    _check_oracle(a[0].cpu().numpy(), ref_q8, N, normed, "q6k stream head")
    assert a[1] == oracle.argmax(oracle.matmul("q8", ref_q8, N, normed)[0])
