"""GPU tests of the fused gate / up / SwiGLU entry points (forwardBlock's FFN
input, model_f32.go:479-490). The paired GEMV writes h directly from the two
row sums it holds; h must equal the oracle's SwiGLU of the library's own
gate / up outputs (which are bit-identical to the single matmuls), and stay
within the reassociation bound of the oracle's full path."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq

from _helpers import make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu


def _w(qtype, N, K, seed):
    raw = make_raw(qtype, N, K, seed=seed)
    return raw, sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))


@pytest.mark.parametrize("fmt_g,fmt_u", [("q4_1", "q4_1"), ("q8", "q8"), ("q4", "q4"), ("q5", "q5"),
                                         ("q5k1", "q5k1"), ("q4_1", "q8")])
@pytest.mark.parametrize("M", [1, 3, 64, 70])
def test_swiglu_fused(fmt_g, fmt_u, M):
    N, K = 300, 512
    rg, wg = _w(fmt_g, N, K, seed=M)
    ru, wu = _w(fmt_u, N, K, seed=M + 50)
    x = make_x(M, K, seed=M + 7)
    xd = torch.from_numpy(x).cuda()
    h = torch.empty(M * N, device="cuda")
    gt = torch.empty(M * N, device="cuda")
    up = torch.empty(M * N, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    sq.matmul_swiglu_dev(wg, wu, xd.data_ptr(), M, K, h.data_ptr(), gt.data_ptr(), up.data_ptr(), s)
    g1 = torch.empty(M * N, device="cuda")
    u1 = torch.empty(M * N, device="cuda")
    sq.matmul_dev(wg, xd.data_ptr(), M, K, g1.data_ptr(), s)
    sq.matmul_dev(wu, xd.data_ptr(), M, K, u1.data_ptr(), s)
    torch.cuda.synchronize()
    # gate / up from the paired launch == the single matmuls, bit for bit
    assert torch.equal(gt.view(torch.int32), g1.view(torch.int32))
    assert torch.equal(up.view(torch.int32), u1.view(torch.int32))
    # h == the reference SwiGLU loop over those values
    want = oracle.swiglu(gt.cpu().numpy(), up.cpu().numpy())
    assert np.array_equal(h.cpu().numpy().view(np.uint32), want.view(np.uint32))
    # and the whole path against the oracle's, within the reassociation bound
    gr = oracle.matmul(fmt_g, rg, N, x).reshape(-1).astype(np.float64)
    ur = oracle.matmul(fmt_u, ru, N, x).reshape(-1).astype(np.float64)
    tg = term_abs_sum(fmt_g, rg, N, x).reshape(-1)
    tu = term_abs_sum(fmt_u, ru, N, x).reshape(-1)
    href = oracle.swiglu(gr.astype(np.float32), ur.astype(np.float32)).astype(np.float64)
    bound = 1e-5 * (1.1 * tg * np.abs(ur) + tu * np.abs(gr)) + 1e-6 * np.abs(href) + 1e-30
    assert np.all(np.abs(h.cpu().numpy().astype(np.float64) - href) <= bound)


@pytest.mark.parametrize("N", [1, 7, 2500, 4500, 4501])
@pytest.mark.parametrize("M", [1, 2, 3])
def test_swiglu_row_counts(N, M):
    # paired launches over row counts that give one, two or more rows per wave
    # with strided and consecutive rows, spare waves and a short last wave
    # (4501): each row sum is formed as the single matmul forms it, so the
    # outputs are bit for bit those of the single matmuls and the oracle's
    # SwiGLU of them.
    K = 1024
    _, wg = _w("q4_1", N, K, seed=N + M)
    _, wu = _w("q4_1", N, K, seed=N + M + 1)
    x = make_x(M, K, seed=N)
    xd = torch.from_numpy(x).cuda()
    h, gt, up, g1, u1 = (torch.empty(M * N, device="cuda") for _ in range(5))
    s = torch.cuda.current_stream().cuda_stream
    sq.matmul_swiglu_dev(wg, wu, xd.data_ptr(), M, K, h.data_ptr(), gt.data_ptr(), up.data_ptr(), s)
    sq.matmul_dev(wg, xd.data_ptr(), M, K, g1.data_ptr(), s)
    sq.matmul_dev(wu, xd.data_ptr(), M, K, u1.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(gt.view(torch.int32), g1.view(torch.int32))
    assert torch.equal(up.view(torch.int32), u1.view(torch.int32))
    want = oracle.swiglu(gt.cpu().numpy(), up.cpu().numpy())
    assert np.array_equal(h.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("knob,value", [("gemv_waves", 4), ("gemv_waves", 8), ("gemv_wg_per_cu", 2)])
def test_swiglu_launch_shapes(knob, value):
    # other workgroup shapes of the paired launch (2 or 4 gate waves and as many
    # up waves per workgroup, two workgroups per CU): the same bits
    N, K, M = 4501, 1024, 2
    _, wg = _w("q4_1", N, K, seed=11)
    _, wu = _w("q4_1", N, K, seed=12)
    x = make_x(M, K, seed=13)
    xd = torch.from_numpy(x).cuda()
    h, g1, u1 = (torch.empty(M * N, device="cuda") for _ in range(3))
    s = torch.cuda.current_stream().cuda_stream
    sq.matmul_dev(wg, xd.data_ptr(), M, K, g1.data_ptr(), s)
    sq.matmul_dev(wu, xd.data_ptr(), M, K, u1.data_ptr(), s)
    sq.set_param(knob, value)
    try:
        sq.matmul_swiglu_dev(wg, wu, xd.data_ptr(), M, K, h.data_ptr(), stream=s)
        torch.cuda.synchronize()
    finally:
        sq.set_param(knob, 16 if knob == "gemv_waves" else 1)
    want = oracle.swiglu(g1.cpu().numpy(), u1.cpu().numpy())
    assert np.array_equal(h.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_swiglu_host_entry_equals_device():
    N, K, M = 256, 1024, 2
    _, wg = _w("q4_1", N, K, seed=1)
    _, wu = _w("q4_1", N, K, seed=2)
    x = make_x(M, K, seed=3)
    h_host = sq.model_matmul_swiglu_into_f32(wg, wu, x, M, K)
    xd = torch.from_numpy(x).cuda()
    h = torch.empty(M * N, device="cuda")
    sq.matmul_swiglu_dev(wg, wu, xd.data_ptr(), M, K, h.data_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(h.cpu().numpy().view(np.uint32), h_host.view(np.uint32))


def test_swiglu_llama_ffn_shape():
    from sllm_qmm import synth
    H, F = 4096, 14336
    wg = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(60, F, H), F, H)
    wu = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(61, F, H), F, H)
    x = torch.from_numpy(make_x(1, H, seed=62)).cuda()
    h, g, u = (torch.empty(F, device="cuda") for _ in range(3))
    s = torch.cuda.current_stream().cuda_stream
    sq.matmul_swiglu_dev(wg, wu, x.data_ptr(), 1, H, h.data_ptr(), g.data_ptr(), u.data_ptr(), s)
    torch.cuda.synchronize()
    want = oracle.swiglu(g.cpu().numpy(), u.cpu().numpy())
    assert np.array_equal(h.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_swiglu_errors():
    _, a = _w("q8", 8, 64, 1)
    _, b = _w("q8", 16, 64, 2)
    x = make_x(1, 64, seed=1)
    with pytest.raises(sq.SllmError) as e:
        sq.model_matmul_swiglu_into_f32(a, b, x, 1, 64)     # Rows differ
    assert e.value.status == 1


@pytest.mark.parametrize("N", [9000, 12001, 14336])
def test_paired_row_orders(N):
    # pairs per wave = ceil(N / 4096 wave slots): 3 for 9000 and 12001 rows
    # (consecutive rows per wave, a partly filled last wave, spare waves), 4
    # for 14336 (strided rows); with and without the RMSNorm prologue
    K = 256
    _, wg = _w("q4_1", N, K, seed=N)
    _, wu = _w("q4_1", N, K, seed=N + 1)
    x = make_x(1, K, seed=N % 97)
    xd = torch.from_numpy(x).cuda()
    nw = torch.from_numpy(np.random.default_rng(N).normal(1, 0.1, K).astype(np.float32)).cuda()
    s = torch.cuda.current_stream().cuda_stream
    h = torch.empty(N, device="cuda")
    gt = torch.empty(N, device="cuda")
    up = torch.empty(N, device="cuda")
    sq.matmul_swiglu_dev(wg, wu, xd.data_ptr(), 1, K, h.data_ptr(), gt.data_ptr(), up.data_ptr(), s)
    g1 = torch.empty(N, device="cuda")
    u1 = torch.empty(N, device="cuda")
    sq.matmul_multi_dev([wg, wu], xd.data_ptr(), 1, K, [g1.data_ptr(), u1.data_ptr()], s)
    hn = torch.empty(N, device="cuda")
    sq.rmsnorm_matmul_swiglu_dev(wg, wu, xd.data_ptr(), nw.data_ptr(), 1e-5, 1, K, hn.data_ptr(), s)
    gn = torch.empty(N, device="cuda")
    un = torch.empty(N, device="cuda")
    sq.rmsnorm_matmul_multi_dev([wg, wu], xd.data_ptr(), nw.data_ptr(), 1e-5, 1, K, [gn.data_ptr(), un.data_ptr()], s)
    torch.cuda.synchronize()
    assert torch.equal(gt.view(torch.int32), g1.view(torch.int32))
    assert torch.equal(up.view(torch.int32), u1.view(torch.int32))
    want = oracle.swiglu(gt.cpu().numpy(), up.cpu().numpy())
    assert np.array_equal(h.cpu().numpy().view(np.uint32), want.view(np.uint32))
    wantn = oracle.swiglu(gn.cpu().numpy(), un.cpu().numpy())
    assert np.array_equal(hn.cpu().numpy().view(np.uint32), wantn.view(np.uint32))
