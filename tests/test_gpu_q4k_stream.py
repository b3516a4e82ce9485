"""GPU tests of Q4_K weights streamed natively (load option gemv_q4k_stream;
off by default: measured slower): a Q4_K weight loaded with the option keeps
the GGUF Q4_K header beside the Q4_1 planes, and its decode GEMV reads the Q4_1
nibble plane and the headers (18 B / 32 weights), rebuilding each block's Q4_1
scale and min as convertQ4KToQ41 (kquant_kernels.go:30-63) does. Its results
are checked against the oracle (oracle.matmul over the Q4_1 Raw the reference's
load computes) and must be bit-identical to those of the same weight loaded
without the option (the Q4_1-plane kernel), on every entry point, including
headers with f16 special values."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import assert_fp32_parity, make_x, term_abs_sum

pytestmark = pytest.mark.gpu


def _load(raw: np.ndarray, N: int, K: int, stream: bool) -> sq.DeviceWeight:
    sq.set_param("gemv_q4k_stream", int(stream))
    try:
        return sq.load_weight_f32_direct(synth.GGML_Q4_K, raw, N, K)
    finally:
        sq.set_param("gemv_q4k_stream", 0)  # the default


def _pair(raw: np.ndarray, N: int, K: int):
    """The weight loaded with its headers (streamed) and without (Q4_1 planes)."""
    return _load(raw, N, K, True), _load(raw, N, K, False)


def _bits(t):
    return t.cpu().numpy().view(np.uint32) if isinstance(t, torch.Tensor) else np.asarray(t).view(np.uint32)


def _special_headers(raw: np.ndarray) -> np.ndarray:
    raw = raw.reshape(-1, 144).copy()
    vals = [0x0001, 0x03ff, 0x0400, 0x7bff, 0x7c00, 0x7e00, 0x8000, 0x0000, 0xfbff, 0x3c00]
    for i in range(min(len(vals), raw.shape[0])):
        raw[i, 0:2] = [vals[i] & 0xff, vals[i] >> 8]                     # d
        raw[i, 2:4] = [vals[-1 - i] & 0xff, vals[-1 - i] >> 8]           # dmin
    raw[:, 4:16] = np.where(np.arange(raw.shape[0])[:, None] % 3 == 0, 0xff, raw[:, 4:16])  # 63s
    return raw.reshape(-1)


@pytest.mark.parametrize("N,K,M", [(14336, 4096, 1), (4096, 14336, 1), (300, 1024, 3), (37, 2048, 5)])
def test_stream_equals_planes_and_oracle(N, K, M):
    raw = synth.q4k_blocks(70 + M, N, K)
    ws, wp = _pair(raw, N, K)
    assert ws.plane_bytes == N * K // 32 * 18 and wp.plane_bytes == N * K // 32 * 20
    x = make_x(M, K, seed=M)
    a = sq.model_matmul_quant_into_f32(ws, x, M, K)[0].copy()
    b = sq.model_matmul_quant_into_f32(wp, x, M, K)[0].copy()
    assert np.array_equal(_bits(a), _bits(b))
    # the streamed kernel against the oracle directly (Q4_1 after convertQ4KToQ41)
    qt, q41 = oracle.load_weight(12, raw, N, K)
    assert qt == "q4_1" and np.array_equal(ws.export(), q41) and np.array_equal(wp.export(), q41)
    ref = oracle.matmul("q4_1", q41, N, x)
    assert_fp32_parity(a.reshape(M, N), ref, term_abs_sum("q4_1", q41, N, x), f"q4k stream {N}x{K} M={M}")


def test_special_header_values():
    N, K = 64, 2048
    raw = _special_headers(synth.q4k_blocks(5, N, K))
    ws, wp = _pair(raw, N, K)
    q41 = oracle.load_weight(12, raw, N, K)[1]
    assert np.array_equal(ws.export(), q41)
    x = make_x(2, K, seed=6)
    a = sq.model_matmul_quant_into_f32(ws, x, 2, K)[0].copy()
    b = sq.model_matmul_quant_into_f32(wp, x, 2, K)[0].copy()
    assert np.array_equal(_bits(a), _bits(b))
    assert_fp32_parity(a.reshape(2, N), oracle.matmul("q4_1", q41, N, x), term_abs_sum("q4_1", q41, N, x),
                       "q4k stream special headers")


def test_stream_on_fused_entries_and_bytes():
    H, F = 4096, 1536
    g_raw, u_raw = synth.q4k_blocks(80, F, H), synth.q4k_blocks(81, F, H)
    gs, gp = _pair(g_raw, F, H)
    us, up = _pair(u_raw, F, H)
    x = torch.from_numpy(make_x(1, H, seed=9)).cuda()
    nw = torch.from_numpy(np.random.default_rng(3).normal(1, 0.1, H).astype(np.float32)).cuda()
    P = lambda t: t.data_ptr()

    def run(g, u):
        h = torch.empty(F, device="cuda")
        o = [torch.empty(F, device="cuda") for _ in range(2)]
        idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        sq.rmsnorm_matmul_swiglu_dev(g, u, P(x), P(nw), 1e-5, 1, H, P(h))
        sq.matmul_multi_dev([g, u], P(x), 1, H, [P(t) for t in o])
        sq.rmsnorm_matmul_argmax_dev(g, P(x), P(nw), 1e-5, P(idx))
        torch.cuda.synchronize()
        return h.clone(), o[0].clone(), o[1].clone(), int(idx.item())

    a, b = run(gs, us), run(gp, up)
    for ta, tb in zip(a[:3], b[:3]):
        assert torch.equal(ta.view(torch.int32), tb.view(torch.int32))
    assert a[3] == b[3]
    # the option acts at load only: it never changes an existing weight's kernel
    sq.set_param("gemv_q4k_stream", 1)
    try:
        assert gp.plane_bytes == F * H // 32 * 20 and gs.plane_bytes == F * H // 32 * 18
        c = run(gs, us)
    finally:
        sq.set_param("gemv_q4k_stream", 0)
    assert all(torch.equal(ta.view(torch.int32), tc.view(torch.int32)) for ta, tc in zip(a[:3], c[:3]))
