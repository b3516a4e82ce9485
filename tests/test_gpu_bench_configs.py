"""Oracle parity of every BASELINE configuration exactly as bench.py launches
it: the same weights (synth seeds and load path), the same entry points and
the same launch shapes (the fused gate+up launch, several rows per wave, the
Q6_K->Q8_0 down and head, the C2 and C4 shapes at M = 1, 64 and 512), each
checked against oracle.matmul on the oracle's own remap of the same GGUF
bytes. Also weights whose f16 scales / mins are subnormal, the one input
where the reference's two f16 decodes differ (f16LUT flushes them to zero
for Q8_0 / Q5_0, dot_scalar.go:46-64; VCVTPH2PS keeps them for Q4_0 / Q4_1,
q4q8_row_amd64.s:36-38, q41q8_row_amd64.s:58-63).

fp32 bar: |got - ref| <= 1e-5 * sum_g |term_g| per output and 1e-5 of the
vector's scale (reassociation only); argmax equal wherever the top two are
further apart than their bounds."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import REL_TOL, assert_fp32_parity, make_raw, make_x, term_abs_sum
from test_gpu_gemm import slice_rows

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

H, F, V = 4096, 14336, 128256
P = lambda t: t.data_ptr()


def _loaded(ggml_type, raw, N, K):
    """The device weight and the oracle's (qtype, Raw) for the same GGUF bytes;
    the device planes must export to the oracle's Raw byte for byte."""
    w = sq.load_weight_f32_direct(ggml_type, raw, N, K)
    qt, ref = oracle.load_weight(ggml_type, raw, N, K)
    assert w.qtype == qt
    assert np.array_equal(w.export(), ref), f"remap of GGUF type {ggml_type} differs from the oracle"
    return w, ref


def _argmax_agrees(got: np.ndarray, ref: np.ndarray, bound: np.ndarray) -> None:
    top = np.argsort(-ref.astype(np.float64))[:2]
    if ref[top[0]] - ref[top[1]] > REL_TOL * (bound[top[0]] + bound[top[1]]):
        assert int(np.argmax(got)) == oracle.argmax(ref)


def test_c3_gate_up_fused_launch():
    # bench.py gate_up(): one sllm_matmul_multi_dev launch over the two
    # Q4_K->Q4_1 14336x4096 weights (several rows per wave)
    g, graw = _loaded(synth.GGML_Q4_K, synth.q4k_blocks(100, F, H), F, H)
    u, uraw = _loaded(synth.GGML_Q4_K, synth.q4k_blocks(101, F, H), F, H)
    x = synth.normal(1, H).reshape(1, H)
    xd = torch.from_numpy(x).cuda()
    yg, yu = torch.empty(F, device="cuda"), torch.empty(F, device="cuda")
    sq.matmul_multi_dev([g, u], P(xd), 1, H, [P(yg), P(yu)], torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for got, raw, name in ((yg, graw, "gate"), (yu, uraw, "up")):
        got = got.cpu().numpy().reshape(1, F)
        ref = oracle.matmul("q4_1", raw, F, x)
        bound = term_abs_sum("q4_1", raw, F, x)
        assert_fp32_parity(got, ref, bound, f"C3 {name}")
        _argmax_agrees(got[0], ref[0], bound[0])


def test_c3_down_q6k_to_q8():
    # bench.py down(): Q6_K 4096x14336 requantized to Q8_0, on the fp32 h row
    d, draw = _loaded(synth.GGML_Q6_K, synth.q6k_blocks(102, H, F), H, F)
    h = synth.normal(2, F).reshape(1, F)
    hd = torch.from_numpy(h).cuda()
    y = torch.empty(H, device="cuda")
    sq.matmul_dev(d, P(hd), 1, F, P(y))
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(1, H)
    ref = oracle.matmul("q8", draw, H, h)
    bound = term_abs_sum("q8", draw, H, h)
    assert_fp32_parity(got, ref, bound, "C3 down")
    _argmax_agrees(got[0], ref[0], bound[0])


@pytest.mark.parametrize("qtype", ["q4", "q4_1"])
@pytest.mark.parametrize("N,K", [(8192, 2048), (2048, 8192)])
def test_c2_gemv(qtype, N, K):
    # bench.py config_table C2: fp32 N(0, 0.02^2) weights quantized per block
    wf = synth.normal(10 + N // 1024, N * K, 0.02).reshape(N, K)
    raw = {"q4": synth.quantize_q4_0, "q4_1": synth.quantize_q4_1}[qtype](wf)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    x = synth.normal(7, K).reshape(1, K)
    xd = torch.from_numpy(x).cuda()
    y = torch.empty(N, device="cuda")
    sq.matmul_dev(w, P(xd), 1, K, P(y))
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(1, N)
    ref = oracle.matmul(qtype, raw, N, x)
    bound = term_abs_sum(qtype, raw, N, x)
    assert_fp32_parity(got, ref, bound, f"C2 {qtype} {N}x{K}")
    _argmax_agrees(got[0], ref[0], bound[0])


def _c4_weight(kind, N):
    if kind == "q5k1":
        return _loaded(synth.GGML_Q5_K, synth.q5k_blocks(20 + N // 1024, N, H), N, H)
    wf = synth.normal(30 + N // 1024, N * H, 0.02).reshape(N, H)
    raw = synth.quantize_q5_0(wf)
    return sq.DeviceWeight.from_quant(sq.QuantWeight("q5", raw, H // 32, N, H)), raw


@pytest.mark.parametrize("kind", ["q5k1", "q5"])
@pytest.mark.parametrize("N", [4096, 1024, 14336])
@pytest.mark.parametrize("M", [1, 64, 512])
def test_c4_shapes(kind, N, M):
    # bench.py config_table C4: the whole weight runs; for M >= 64 a subset of
    # output columns (first / last 32 rows and 64 random) is compared (weight
    # rows are independent, so their Raw slice is the oracle's input)
    w, raw = _c4_weight(kind, N)
    x = synth.normal(7, M * H).reshape(M, H)
    xd = torch.from_numpy(x).cuda()
    y = torch.empty(M * N, device="cuda")
    sq.matmul_dev(w, P(xd), M, H, P(y))
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(M, N)
    if M == 1:
        rows = np.arange(N)
    else:
        rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 32, N),
                                         np.random.default_rng(N + M).integers(0, N, 64)]))
    sub = raw if M == 1 else slice_rows(kind, raw, N, H // 32, rows)
    ref = oracle.matmul(kind, sub, rows.size, x)
    bound = term_abs_sum(kind, sub, rows.size, x)
    assert_fp32_parity(got[:, rows], ref, bound, f"C4 {kind} {N}x{H} M={M}")
    if M == 1:
        _argmax_agrees(got[0], ref[0], bound[0])


@pytest.mark.parametrize("M", [64, 512])
@pytest.mark.parametrize("which", ["gate", "down"])
def test_c3_prefill_shapes(which, M):
    # bench.py config_table "C3 ... M=64 / 512": the GEMM on the C3 weights
    if which == "gate":
        w, raw = _loaded(synth.GGML_Q4_K, synth.q4k_blocks(100, F, H), F, H)
        N, K = F, H
    else:
        w, raw = _loaded(synth.GGML_Q6_K, synth.q6k_blocks(102, H, F), H, F)
        N, K = H, F
    x = synth.normal(7, M * K).reshape(M, K)
    xd = torch.from_numpy(x).cuda()
    y = torch.empty(M * N, device="cuda")
    sq.matmul_dev(w, P(xd), M, K, P(y))
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(M, N)
    rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 32, N),
                                     np.random.default_rng(M).integers(0, N, 64)]))
    sub = slice_rows(w.qtype, raw, N, K // 32, rows)
    ref = oracle.matmul(w.qtype, sub, rows.size, x)
    assert_fp32_parity(got[:, rows], ref, term_abs_sum(w.qtype, sub, rows.size, x), f"C3 {which} M={M}")


def test_c5_head_rmsnorm_argmax():
    # bench.py decode: the final RMSNorm + Q6_K->Q8_0 head 128256x4096 + greedy
    # argmax in one launch (sllm_rmsnorm_matmul_argmax_dev)
    hw, hraw = _loaded(synth.GGML_Q6_K, synth.q6k_blocks(204, V, H), V, H)
    x = synth.normal(3, H).reshape(1, H)
    nw = (synth.normal(5, H, 0.1) + np.float32(1.0)).astype(np.float32)
    eps = 1e-5
    xd, nwd = torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda()
    logits = torch.empty(V, device="cuda")
    tok = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    sq.rmsnorm_matmul_argmax_dev(hw, P(xd), P(nwd), eps, P(tok), P(logits))
    torch.cuda.synchronize()
    got = logits.cpu().numpy().reshape(1, V)
    # the normed row in the library's sum-of-squares order is the GEMV's input
    # bit for bit (tests/test_gpu_rmsnorm.py); the head against the oracle on it
    normed = oracle.rmsnorm(x, nw, eps, lib_order=True)
    ref = oracle.matmul("q8", hraw, V, normed)
    bound = term_abs_sum("q8", hraw, V, normed)
    assert_fp32_parity(got, ref, bound, "C5 head")
    t = int(tok.item())
    assert t == int(np.argmax(got[0]))  # first maximum of its own logits
    _argmax_agrees(got[0], ref[0], bound[0])


# ---------------------------------------------------------------- f16 subnormal scales

SUB = (0x0001, 0x03FF, 0x8001, 0x83FF)


def _subnormal_raw(qtype: str, N: int, K: int, seed: int) -> np.ndarray:
    """make_raw's weight with the f16 d (and m, Q5K1 dh) of every third block
    set to a subnormal pattern, cycling through SUB."""
    raw = make_raw(qtype, N, K, seed=seed).copy()
    G = K // 32
    nb = N * G
    pat = np.array(SUB, np.uint16)

    def put(view, off, which):
        idx = np.arange(0, nb, 3)
        bits = pat[(idx + which) % 4]
        view[idx, off] = (bits & 0xFF).astype(np.uint8)
        view[idx, off + 1] = (bits >> 8).astype(np.uint8)

    if qtype == "q5k1":
        lo = raw[: nb * 20].reshape(nb, 20)
        hi = raw[nb * 20:].reshape(nb, 20)
        put(lo, 0, 0)
        put(lo, 2, 1)
        put(hi, 0, 2)
    else:
        b = raw.reshape(nb, oracle.BLOCK_BYTES[qtype])
        put(b, 0, 0)
        if qtype == "q4_1":
            put(b, 2, 1)
    return raw


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5", "q5k1"])
@pytest.mark.parametrize("M", [1, 64])
def test_subnormal_scales(qtype, M):
    # every third block's scale (and min) subnormal: 6e-8 .. 6e-5 against
    # about 5e-4 for the other blocks, so a swapped decoder (flush where the
    # reference keeps them, or the reverse) moves outputs far past the bound
    N, K = 96, 512
    raw = _subnormal_raw(qtype, N, K, seed=M + 3)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    assert np.array_equal(w.export(), raw)
    x = make_x(M, K, seed=M + 4)
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} subnormal M={M}")
    # the decode the oracle applies is the one that matters: the same weight
    # with the other decode must differ from what the kernel returned
    flushed = qtype in ("q8", "q5")
    alt = raw.copy()
    G = K // 32
    nb = N * G
    if qtype == "q5k1":
        v = alt[: nb * 20].reshape(nb, 20)
    else:
        v = alt.reshape(nb, oracle.BLOCK_BYTES[qtype])
    bits = v[:, 0].astype(np.uint16) | (v[:, 1].astype(np.uint16) << 8)
    is_sub = ((bits & 0x7C00) == 0) & ((bits & 0x3FF) != 0)
    assert is_sub.any()
    if not flushed:
        # zeroing the subnormal scales must change the exact-decode result
        v[is_sub, 0] = 0
        v[is_sub, 1] = 0
        ref_flush = oracle.matmul(qtype, alt, N, x)
        assert not np.allclose(ref_flush, ref, rtol=0, atol=1e-6 * np.abs(ref).max())
