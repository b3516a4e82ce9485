"""GPU parity of the prefill path (from 8 or 16 activation rows: the int8 MFMA
GEMM for Q8_0 / Q4_0 / Q4_1 / Q5K1, the bf16 MFMA GEMM for Q5_0) against the
oracle, including full BASELINE C4 shapes checked on a row subset (weight rows
are independent, so a row slice of the Raw bytes is the oracle's input for
those output columns), and the GEMM's int32 block dots bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import assert_fp32_parity, make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu

QTYPES = ["q8", "q4", "q4_1", "q5k1", "q5"]


def slice_rows(qtype: str, raw: np.ndarray, N: int, G: int, rows: np.ndarray) -> np.ndarray:
    """Raw bytes of the given weight rows (QuantWeight.Raw layout)."""
    if qtype == "q5k1":
        lo = raw[: N * G * 20].reshape(N, G * 20)[rows]
        hi = raw[N * G * 20:].reshape(N, G * 20)[rows]
        return np.concatenate([lo.reshape(-1), hi.reshape(-1)])
    bb = oracle.BLOCK_BYTES[qtype]
    return raw.reshape(N, G * bb)[rows].reshape(-1)


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("M", [8, 17, 33, 64, 65, 130])
@pytest.mark.parametrize("N,K", [(96, 512), (200, 1024)])
def test_prefill_parity(qtype, M, N, K):
    if qtype == "q5k1" and K % 256:
        pytest.skip("Q5_K rows are whole super-blocks")
    raw = make_raw(qtype, N, K, seed=M + N)
    x = make_x(M, K, seed=K)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} M={M} {N}x{K}")


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5k1"])
@pytest.mark.parametrize("shape,splits", [(1, 1), (1, 3), (2, 5), (2, 8), (1, 2), (2, 1), (3, 1), (3, 3), (3, 8),
                                          (4, 1), (4, 3), (5, 1), (5, 3), (5, 8)])
def test_shape_and_split_overrides(qtype, shape, splits):
    # every workgroup shape and any K split count gives the oracle's result
    # within the bound (K = 1024 is 8 stages: 5 splits of 2 stages leave the
    # last split empty, and it adds a zero tile; 3 splits of 3 stages end on
    # an odd stage count, which the two-stage prefetch handles)
    N, K, M = 320, 1024, 130
    raw = make_raw(qtype, N, K, seed=shape * 10 + splits)
    x = make_x(M, K, seed=splits)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    sq.set_param("gemm_shape", shape)
    sq.set_param("gemm_splits", splits)
    try:
        got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    finally:
        sq.set_param("gemm_shape", 0)
        sq.set_param("gemm_splits", 0)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} shape={shape} S={splits}")


@pytest.mark.parametrize("qtype", ["q8", "q5"])
@pytest.mark.parametrize("splits", [9, 12, 16])
@pytest.mark.parametrize("N,M", [(256, 64), (255, 65)])
def test_split_reduction_layouts(qtype, splits, N, M):
    # the split reduction adds the partial tiles in split order whether it
    # moves four floats per thread (element count a multiple of 4, output
    # 16-byte aligned) or one (odd count, or an output 4 bytes off alignment),
    # with more splits than it loads at once: every layout gives the same bits,
    # within the bound of the oracle's result
    import torch

    K = 4096
    raw = make_raw(qtype, N, K, seed=splits + N)
    x = make_x(M, K, seed=splits)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    torch.cuda.set_device(0)
    s = torch.cuda.current_stream()
    xd = torch.from_numpy(x).cuda()
    buf = torch.zeros(M * N + 8, device="cuda")
    outs = []
    sq.set_param("gemm_splits", splits)
    try:
        for off in (0, 1):
            sq.matmul_dev(w, xd.data_ptr(), M, K, buf.data_ptr() + 4 * off, s.cuda_stream)
            torch.cuda.synchronize()
            outs.append(buf[off:off + M * N].cpu().numpy().copy())
    finally:
        sq.set_param("gemm_splits", 0)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(outs[0].reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"S={splits} {N}x{K} M={M}")


def _block_dots_case(qtype, raw, N, K, x, row0, n_rows, shape=0):
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    sq.set_param("gemm_shape", shape)
    try:
        got = sq.debug_gemm_block_dots(w, x, row0, n_rows)
    finally:
        sq.set_param("gemm_shape", 0)
    sub = slice_rows(qtype, raw, N, K // 32, np.arange(row0, row0 + n_rows))
    ref = oracle.block_dots(qtype, sub, n_rows, K, x)
    assert got.shape == ref.shape
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"{qtype}: {len(bad)} block dots differ, first {bad[0].tolist()}: " \
                          f"{got[tuple(bad[0])]} vs {ref[tuple(bad[0])]}"


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5k1"])
@pytest.mark.parametrize("M", [64, 130])
@pytest.mark.parametrize("shape", [1, 2, 3, 4, 5])
def test_gemm_block_dots_bitexact(qtype, M, shape):
    # the int32 block dots the matrix cores return, read from the registers the
    # epilogue scales, against the oracle's per-(row, block) dots
    N, K = 200, 1024
    raw = make_raw(qtype, N, K, seed=M + shape)
    x = make_x(M, K, seed=3 * M)
    x[1] = 0.0                       # all-zero blocks: xq 0
    x[2, :64] = np.float32(1e30)     # one saturated block: +-127
    _block_dots_case(qtype, raw, N, K, x, 0, N, shape)
    _block_dots_case(qtype, raw, N, K, x, 37, 101, shape)  # a row range starting mid-tile


@pytest.mark.slow
@pytest.mark.parametrize("M", [64, 130])
def test_gemm_block_dots_c3_gate_rows(M):
    # C3 gate (Q4_K -> Q4_1, 14336 x 4096): the GEMM's block dots for the last
    # 256 weight rows, as it computes them inside the full-shape launch plan
    N, K = 14336, 4096
    w = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(11, N, K), N, K)
    raw = w.export()
    x = make_x(M, K, seed=M)
    got = sq.debug_gemm_block_dots(w, x, N - 256, 256)
    sub = slice_rows("q4_1", raw, N, K // 32, np.arange(N - 256, N))
    assert np.array_equal(got, oracle.block_dots("q4_1", sub, 256, K, x))


@pytest.mark.parametrize("qtype", ["q4_1", "q5k1"])
@pytest.mark.parametrize("shape", [0, 4])
def test_gemm_min_term_dominant(qtype, shape):
    # mins far larger than scale x code, of both signs: the min term (added on
    # the fp32 matrix cores two blocks at a time, one block on the 32-row
    # tiles of shape 4) carries most of each output
    N, K, M = 160, 1024, 72
    G = K // 32
    raw = make_raw(qtype, N, K, seed=31).copy()
    blocks = raw[: N * G * 20].reshape(N * G, 20)
    m = np.random.default_rng(5).uniform(-64.0, 64.0, N * G).astype(np.float16)
    blocks[:, 2:4] = m.view(np.uint8).reshape(-1, 2)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, G, N, K))
    x = make_x(M, K, seed=32)
    sq.set_param("gemm_shape", shape)
    try:
        got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    finally:
        sq.set_param("gemm_shape", 0)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} dominant mins")


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5k1"])
def test_gemm_nonfinite_weight_scales(qtype):
    # f16 Inf / NaN / max-finite weight scales and mins: those K stages take the
    # reference's exact operation order, so Inf and NaN outputs match the oracle's
    N, K, M = 96, 512, 64
    raw = make_raw(qtype, N, K, seed=21).copy()
    G = K // 32
    bb = 20 if qtype == "q5k1" else oracle.BLOCK_BYTES[qtype]
    blocks = raw.reshape(-1, bb)
    specials = [0x7c00, 0xfc00, 0x7e00, 0x7bff, 0xfbff]
    for i, v in enumerate(specials):
        r, g = 3 + 17 * i, (5 * i) % G
        blocks[r * G + g, 0:2] = [v & 0xff, v >> 8]
        if qtype in ("q4_1", "q5k1"):
            blocks[(r + 1) * G + g, 2:4] = [v & 0xff, v >> 8]   # min
    if qtype == "q5k1":
        blocks[N * G + 50 * G + 7, 0:2] = [0x00, 0x7c]          # high block scale +Inf
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, G, N, K))
    x = make_x(M, K, seed=22)
    x[5] = 0.0  # zero activation blocks: the reference's scale 0 turns Inf weight scales into NaN
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    ref = oracle.matmul(qtype, raw, N, x)
    assert np.isnan(ref).any() and np.isinf(ref).any()
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} special scales")


@pytest.mark.parametrize("qtype", ["q8", "q4_1", "q5k1", "q5"])
def test_prefill_edge_activations(qtype):
    # zero rows, denormal rows and huge rows through the GEMM's quantize pre-pass
    N, K, M = 64, 512, 64
    raw = make_raw(qtype, N, K, seed=5)
    x = make_x(M, K, seed=6)
    x[0] = 0.0
    x[1] *= np.float32(1e-39)
    x[2] *= np.float32(1e30)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} edges")


@pytest.mark.slow
@pytest.mark.parametrize("ggml_type,N,K,M", [
    (13, 4096, 4096, 64),      # C4 Q5_K q/o projection, M = 64
    (13, 1024, 4096, 512),     # C4 Q5_K k/v projection, M = 512
    (12, 14336, 4096, 64),     # C3 Q4_K gate/up, M = 64
    (6, 4096, 4096, 64),       # C4 Q5_0 (VALU GEMM)
    (6, 1024, 4096, 512),      # C4 Q5_0 k/v, M = 512
])
def test_prefill_full_shapes_on_row_subset(ggml_type, N, K, M):
    raw_gguf = synth.gguf_tensor(ggml_type, 7, N, K)
    w = sq.load_weight_f32_direct(ggml_type, raw_gguf, N, K)
    raw = w.export()
    x = make_x(M, K, seed=9)
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    got = got.reshape(M, N)
    rows = np.unique(np.concatenate([np.arange(32), np.arange(N - 32, N),
                                     np.random.default_rng(0).integers(0, N, 64)]))
    sub = slice_rows(w.qtype, raw, N, K // 32, rows)
    ref = oracle.matmul(w.qtype, sub, rows.size, x)
    assert_fp32_parity(got[:, rows], ref, term_abs_sum(w.qtype, sub, rows.size, x), f"{w.qtype} {N}x{K} M={M}")


def test_gemm_rows_match_gemv_rows():
    # the same activation row through the GEMM (inside a 64-row batch) and the
    # GEMV (alone) gives the same per-block terms; sums may differ only by order
    N, K = 256, 2048
    raw = make_raw("q4_1", N, K, seed=3)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", raw, K // 32, N, K))
    x = make_x(64, K, seed=4)
    big, _, _ = sq.model_matmul_quant_into_f32(w, x, 64, K)
    one = sq.model_matmul_row_quant_into_f32(w, x[17])
    bound = term_abs_sum("q4_1", raw, N, x[17:18])[0]
    assert np.all(np.abs(big.reshape(64, N)[17].astype(np.float64) - one) <= 2e-5 * bound + 1e-30)


@pytest.mark.parametrize("qtype", ["q4_1", "q5"])
def test_gemm_rows_match_gemv_rows_q5(qtype):
    # Q5_0's GEMM forms the same per-block fp32 sums as its GEMV (the reference
    # order); the two may differ only in how the block terms are added up
    N, K = 192, 1024
    raw = make_raw(qtype, N, K, seed=8)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    x = make_x(70, K, seed=9)
    big, _, _ = sq.model_matmul_quant_into_f32(w, x, 70, K)
    for row in (0, 33, 69):
        one = sq.model_matmul_row_quant_into_f32(w, x[row])
        bound = term_abs_sum(qtype, raw, N, x[row:row + 1])[0]
        assert np.all(np.abs(big.reshape(70, N)[row].astype(np.float64) - one) <= 2e-5 * bound + 1e-30), row


def _q5k1_split_scales(raw: np.ndarray, N: int, K: int, blocks) -> np.ndarray:
    """The q5k1 Raw with the given high blocks' scales moved off 16 x the low
    scale (x 1.5), so the weight keeps one MFMA per half."""
    G = K // 32
    out = raw.copy()
    lo = out[: N * G * 20].reshape(N * G, 20)
    hi = out[N * G * 20:].reshape(N * G, 20)
    for b in blocks:
        d = lo[b, 0:2].view(np.float16)[0]
        hi[b, 0:2] = np.array([np.float16(np.float32(d) * 24.0)]).view(np.uint8)
    return out


def test_q5k1_one_mfma_decided_at_load():
    # dh = 16 d in every block (as convertQ5KToTwoQ41 writes it for d sc in the
    # f16 normal range): one MFMA per block; otherwise one per half
    N, K = 64, 512
    raw = make_raw("q5k1", N, K, seed=3)
    assert sq.DeviceWeight.from_quant(sq.QuantWeight("q5k1", raw, K // 32, N, K)).q5k1_one_mfma
    split = _q5k1_split_scales(raw, N, K, [5])
    assert not sq.DeviceWeight.from_quant(sq.QuantWeight("q5k1", split, K // 32, N, K)).q5k1_one_mfma
    w = sq.load_weight_f32_direct(synth.GGML_Q5_K, synth.q5k_blocks(4, N, K), N, K)
    assert w.q5k1_one_mfma
    # a super-block whose 16 d sc overflows f16 (d = 100, sub-block 0's sc =
    # 63): its high block's scale is Inf, not 16 x the low one
    gg = synth.q5k_blocks(5, N, K).reshape(-1, 176).copy()
    gg[7, 0:2] = np.array([np.float16(100.0)]).view(np.uint8)
    gg[7, 4] = (gg[7, 4] & 0xC0) | 63
    w2 = sq.load_weight_f32_direct(synth.GGML_Q5_K, gg.reshape(-1), N, K)
    ex = w2.export()
    G = K // 32
    lo = ex[: N * G * 20].reshape(N * G, 20)[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    hi = ex[N * G * 20:].reshape(N * G, 20)[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    assert w2.q5k1_one_mfma == bool(np.all(hi == 16 * lo))
    assert not w2.q5k1_one_mfma
    assert not sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(6, N, K), N, K).q5k1_one_mfma


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("M", [16, 64, 130, 300])
def test_q5k1_one_and_two_mfma_forms(split, M):
    # both GEMM forms of a Q5K1 weight against the oracle (the two halves'
    # passes, kquant_kernels.go:159-174), on every workgroup shape
    N, K = 192, 1024
    raw = make_raw("q5k1", N, K, seed=M)
    if split:
        raw = _q5k1_split_scales(raw, N, K, [0, 77, N * (K // 32) - 1])
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q5k1", raw, K // 32, N, K))
    assert w.q5k1_one_mfma == (not split)
    x = make_x(M, K, seed=M + 1)
    ref = oracle.matmul("q5k1", raw, N, x)
    bound = term_abs_sum("q5k1", raw, N, x)
    for shape in (0, 1, 2, 3, 4, 5):
        sq.set_param("gemm_shape", shape)
        try:
            got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
        finally:
            sq.set_param("gemm_shape", 0)
        assert_fp32_parity(got.reshape(M, N), ref, bound, f"q5k1 split={split} M={M} shape={shape}")


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("shape", [1, 3, 4, 5])
def test_q5k1_block_dots_both_forms(split, shape):
    # the one-MFMA form's dots (dot + 16 dot_h, split back with one more MFMA
    # of the high bits) and the two-MFMA form's, bit for bit
    N, K, M = 200, 1024, 72
    raw = make_raw("q5k1", N, K, seed=shape + 40)
    if split:
        raw = _q5k1_split_scales(raw, N, K, [3])
    x = make_x(M, K, seed=shape)
    x[1] = 0.0
    x[2, :64] = np.float32(1e30)
    _block_dots_case("q5k1", raw, N, K, x, 0, N, shape)
    _block_dots_case("q5k1", raw, N, K, x, 37, 101, shape)


@pytest.mark.parametrize("scale", ["inf", "nan"])
def test_q5k1_one_mfma_nonfinite_scale(scale):
    # a non-finite low scale with dh = 16 d (inf) keeps the one-MFMA form and
    # takes the exact path for that stage; NaN never equals, so that weight
    # keeps two MFMAs: both give the oracle's result
    N, K, M = 96, 512, 64
    G = K // 32
    raw = make_raw("q5k1", N, K, seed=9).copy()
    lo = raw[: N * G * 20].reshape(N * G, 20)
    hi = raw[N * G * 20:].reshape(N * G, 20)
    v = np.float16(np.inf) if scale == "inf" else np.float16(np.nan)
    lo[10, 0:2] = np.array([v]).view(np.uint8)
    hi[10, 0:2] = np.array([v]).view(np.uint8)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q5k1", raw, G, N, K))
    assert w.q5k1_one_mfma == (scale == "inf")
    x = make_x(M, K, seed=10)
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
    ref = oracle.matmul("q5k1", raw, N, x)
    assert not np.isfinite(ref).all()
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum("q5k1", raw, N, x), f"q5k1 {scale}")
