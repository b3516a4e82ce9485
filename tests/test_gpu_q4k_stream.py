"""GPU tests of Q4_K weights streamed natively (tuning knob gemv_q4k_stream;
off by default: measured slower): the decode GEMV reads the Q4_1 nibble plane
and the GGUF Q4_K header per super-block (18 B / 32 weights) and rebuilds each
block's Q4_1 scale and min as convertQ4KToQ41 (kquant_kernels.go:30-63) does.
Its results must be bit-identical to the kernel that reads the d / m planes
the load-time remap wrote (which tests/test_gpu_parity.py pins to the oracle
byte for byte), on every entry point, including headers with f16 special
values."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import make_x

pytestmark = pytest.mark.gpu


def _both(fn):
    """fn() run with the streamed kernel and with the plane kernel."""
    try:
        sq.set_param("gemv_q4k_stream", 1)
        a = fn()
        sq.set_param("gemv_q4k_stream", 0)
        b = fn()
    finally:
        sq.set_param("gemv_q4k_stream", 0)  # the default
    return a, b


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
def test_stream_equals_planes(N, K, M):
    raw = synth.q4k_blocks(70 + M, N, K)
    w = sq.load_weight_f32_direct(synth.GGML_Q4_K, raw, N, K)
    x = make_x(M, K, seed=M)
    a, b = _both(lambda: sq.model_matmul_quant_into_f32(w, x, M, K)[0].copy())
    assert np.array_equal(_bits(a), _bits(b))
    # the plane kernel's result is the oracle's path (Q4_1 after convertQ4KToQ41)
    qt, q41 = oracle.load_weight(12, raw, N, K)
    assert qt == "q4_1" and np.array_equal(w.export(), q41)


def test_special_header_values():
    N, K = 64, 2048
    raw = _special_headers(synth.q4k_blocks(5, N, K))
    w = sq.load_weight_f32_direct(synth.GGML_Q4_K, raw, N, K)
    assert np.array_equal(w.export(), oracle.load_weight(12, raw, N, K)[1])
    x = make_x(2, K, seed=6)
    a, b = _both(lambda: sq.model_matmul_quant_into_f32(w, x, 2, K)[0].copy())
    assert np.array_equal(_bits(a), _bits(b))


def test_stream_on_fused_entries_and_bytes():
    H, F = 4096, 1536
    g = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(80, F, H), F, H)
    u = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(81, F, H), F, H)
    x = torch.from_numpy(make_x(1, H, seed=9)).cuda()
    nw = torch.from_numpy(np.random.default_rng(3).normal(1, 0.1, H).astype(np.float32)).cuda()
    P = lambda t: t.data_ptr()

    def run():
        h = torch.empty(F, device="cuda")
        o = [torch.empty(F, device="cuda") for _ in range(2)]
        idx = torch.zeros(1, dtype=torch.int32, device="cuda")
        sq.rmsnorm_matmul_swiglu_dev(g, u, P(x), P(nw), 1e-5, 1, H, P(h))
        sq.matmul_multi_dev([g, u], P(x), 1, H, [P(t) for t in o])
        sq.rmsnorm_matmul_argmax_dev(g, P(x), P(nw), 1e-5, P(idx))
        torch.cuda.synchronize()
        return h.clone(), o[0].clone(), o[1].clone(), int(idx.item())

    a, b = _both(run)
    for ta, tb in zip(a[:3], b[:3]):
        assert torch.equal(ta.view(torch.int32), tb.view(torch.int32))
    assert a[3] == b[3]
    assert g.plane_bytes == F * H // 32 * 20  # default: the Q4_1 planes
    sq.set_param("gemv_q4k_stream", 1)
    try:
        assert g.plane_bytes == F * H // 32 * 18
    finally:
        sq.set_param("gemv_q4k_stream", 0)
