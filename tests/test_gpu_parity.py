"""GPU parity: the HIP path through the C ABI against the refcpu oracle.

Bit-exact: activation quantization (xq, xs, Σxq), per-block integer dots, the
repack / remap / requantize bytes. fp32 outputs: within 1e-5 of sum|terms|
(reassociation only) and identical argmax.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import assert_fp32_parity, make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu

QTYPES = ["q8", "q4", "q4_1", "q5", "q5k1"]


def _edge_rows(K: int) -> np.ndarray:
    rows = []
    z = np.zeros(K, np.float32)
    rows.append(z.copy())                                   # all-zero blocks: scale 0, q 0
    r = z.copy(); r[::32] = 3.5; rows.append(r)             # one value per block -> q = 127
    r = -np.abs(make_x(1, K, 7)[0]); rows.append(r)         # all negative
    r = make_x(1, K, 8)[0] * np.float32(1e-39); rows.append(r)  # fp32 denormals
    r = make_x(1, K, 9)[0] * np.float32(1e30); rows.append(r)   # large magnitudes
    r = make_x(1, K, 10)[0]; r[1] = np.nan; r[40] = np.inf; r[75] = -np.inf; r[100] = -0.0
    rows.append(r)                                          # NaN / Inf (amd64 int32 semantics)
    r = np.full(K, np.float32(1e-45)); rows.append(r)       # smallest denormal: 1/scale overflows
    return np.stack(rows).astype(np.float32)


def test_quantize_act_bitexact():
    K = 4096
    x = np.concatenate([make_x(5, K, 3), _edge_rows(K)])
    xq, xs, sx = sq.debug_quantize_act(x)
    rq, rs = oracle.quantize_act_q8(x)
    assert np.array_equal(xq, rq)
    assert np.array_equal(xs.view(np.uint32), rs.view(np.uint32))
    assert np.array_equal(sx, rq.reshape(x.shape[0], -1, 32).astype(np.int32).sum(-1))


@pytest.mark.parametrize("qtype", QTYPES)
def test_export_roundtrip(qtype):
    N, K = 67, 512
    raw = make_raw(qtype, N, K, seed=11)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    assert w.qtype == qtype and w.rows == N and w.cols == K
    assert np.array_equal(w.export(), raw)


def test_q5k1_requires_canonical_high_half():
    N, K = 8, 256
    raw = make_raw("q5k1", N, K, seed=5).copy()
    bad = raw.copy()
    bad[N * (K // 32) * 20 + 2] = 1  # non-zero min in the high half
    with pytest.raises(sq.SllmError) as e:
        sq.DeviceWeight.from_quant(sq.QuantWeight("q5k1", bad, K // 32, N, K))
    assert e.value.status == 6
    bad = raw.copy()
    bad[N * (K // 32) * 20 + 4] = 0x22  # nibble 2 in the high half
    with pytest.raises(sq.SllmError):
        sq.DeviceWeight.from_quant(sq.QuantWeight("q5k1", bad, K // 32, N, K))


@pytest.mark.parametrize("ggml_type,expect", [(8, "q8"), (2, "q4"), (3, "q4_1"), (6, "q5"), (12, "q4_1"),
                                              (13, "q5k1"), (14, "q8"), (20, "q8")])
def test_gguf_load_bitexact(ggml_type, expect):
    N, K = 48, 1024
    if ggml_type == 8:
        raw = oracle.quantize_q8_rows_f32(synth.normal(21, N * K, 0.02).reshape(N, K))
    else:
        raw = synth.gguf_tensor(ggml_type, 21, N, K)
    qt, ref = oracle.load_weight(ggml_type, raw, N, K)
    assert qt == expect
    w = sq.load_weight_f32_direct(ggml_type, raw, N, K)
    assert w.qtype == expect
    got = w.export()
    assert np.array_equal(got, ref), f"first diff at byte {np.argmax(got != ref)}"


def test_gguf_unsupported_type():
    with pytest.raises(sq.SllmError) as e:
        sq.load_weight_f32_direct(7, np.zeros(24 * 32, np.uint8), 4, 256)  # Q5_1: dense fp32 in the reference
    assert e.value.status == 2


def test_from_f32_bitexact():
    N, K = 96, 2048
    w = synth.normal(31, N * K, 0.02).reshape(N, K)
    w[3] = 0.0                     # zero row -> zero blocks
    w[5, :64] = 1e-30              # tiny scales: f16 flush to zero
    w[7, :32] = 70000.0            # f16 overflow of the scale
    ref = oracle.quantize_q8_rows_f32(w)
    got = sq.quantize_q8_rows_f32(w, N, K).export()
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("qtype", QTYPES)
def test_block_dots_bitexact(qtype):
    N, K, M = 37, 768 if qtype != "q5k1" else 512, 3
    raw = make_raw(qtype, N, K, seed=41)
    x = make_x(M, K, 42)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    got = sq.debug_block_dots(w, x)
    ref = oracle.block_dots(qtype, raw, N, K, x)
    assert np.array_equal(got, ref)


SHAPES = [(1536, 576), (96, 4096), (40, 14336), (300, 2048)]


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 2, 3, 5])
def test_matmul_parity(qtype, N, K, M):
    if qtype == "q5k1" and K % 256:
        pytest.skip("Q5_K rows are whole 256-element super-blocks")
    raw = make_raw(qtype, N, K, seed=N + K)
    x = make_x(M, K, seed=M)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    got, rows, cols = sq.model_matmul_quant_into_f32(w, x, M, K)
    assert (rows, cols) == (M, N)
    ref = oracle.matmul(qtype, raw, N, x)
    assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} {N}x{K} M={M}")
    for m in range(M):
        assert int(np.argmax(got.reshape(M, N)[m])) == oracle.argmax(ref[m])


def _group(qtype, d_bits, m_bits=0, fill=0, qh=0):
    if qtype == "q8":
        g = np.zeros(34, np.uint8); g[0:2] = [d_bits & 0xFF, d_bits >> 8]; g[2:] = fill
    elif qtype == "q4":
        g = np.zeros(18, np.uint8); g[0:2] = [d_bits & 0xFF, d_bits >> 8]; g[2:] = fill
    elif qtype == "q4_1":
        g = np.zeros(20, np.uint8); g[0:2] = [d_bits & 0xFF, d_bits >> 8]; g[2:4] = [m_bits & 0xFF, m_bits >> 8]
        g[4:] = fill
    else:
        g = np.zeros(22, np.uint8); g[0:2] = [d_bits & 0xFF, d_bits >> 8]
        g[2:6] = np.array([qh], np.uint32).view(np.uint8); g[6:] = fill
    return g


@pytest.mark.parametrize("qtype,group,x,want", [
    ("q8", _group("q8", 0x3C00, fill=1), 1.0, 32.0),            # float32_ops_test.go:304-346
    ("q4", _group("q4", 0x3C00, fill=0x99), 1.0, 32.0),         # float32_ops_test.go:582-602
    ("q4_1", _group("q4_1", 0x3C00, 0x3C00, fill=0), 2.0, 64.0),  # q8_fast_test.go:121-143
    ("q5", _group("q5", 0x3C00, fill=0), 1.0, -512.0),          # q5_test.go:94-112 (every weight -16)
])
def test_known_answers(qtype, group, x, want):
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, group, 1, 1, 32))
    xv = np.full(32, x, np.float32)
    got = sq.model_matmul_row_quant_into_f32(w, xv)
    ref = oracle.matmul(qtype, group, 1, xv[None])
    assert abs(float(got[0]) - want) <= 0.01
    assert got[0] == ref[0, 0]  # one block: no reassociation, bit-exact


def test_row_quant_into_equals_matmul():
    N, K = 513, 1024
    raw = make_raw("q4_1", N, K, 3)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", raw, K // 32, N, K))
    x = make_x(1, K, 4)
    a = sq.model_matmul_row_quant_into_f32(w, x[0])
    b, _, _ = sq.model_matmul_quant_into_f32(w, x, 1, K)
    assert np.array_equal(a, b)


def test_argmax_dev():
    import torch
    rng = np.random.default_rng(0)
    cases = [rng.standard_normal(128256).astype(np.float32)]
    t = rng.standard_normal(5000).astype(np.float32); t[17] = 9.0; t[4000] = 9.0; cases.append(t)
    t = rng.standard_normal(5000).astype(np.float32); t[0] = np.nan; cases.append(t)
    t = rng.standard_normal(5000).astype(np.float32); t[10] = np.nan; t[20] = 50.0; cases.append(t)
    t = np.full(3000, -np.inf, np.float32); cases.append(t)
    for v in cases:
        d = torch.from_numpy(v).cuda()
        assert sq.argmax_f32_dev(d.data_ptr(), v.size) == oracle.argmax(v)


def test_concurrent_callers_match_serial():
    # concurrency_test.go:25-54: concurrent requests must equal the serial results
    N, K = 2048, 2048
    raw = make_raw("q8", N, K, 9)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", raw, K // 32, N, K))
    xs = [make_x(1, K, 100 + i) for i in range(8)]
    serial = [sq.model_matmul_quant_into_f32(w, x, 1, K)[0].copy() for x in xs]
    out = [None] * 8

    def run(i):
        for _ in range(5):
            out[i] = sq.model_matmul_quant_into_f32(w, xs[i], 1, K)[0].copy()

    th = [threading.Thread(target=run, args=(i,)) for i in range(8)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for a, b in zip(serial, out):
        assert np.array_equal(a, b)


def test_errors_are_status_codes():
    raw = make_raw("q8", 4, 64, 1)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", raw, 2, 4, 64))
    with pytest.raises(sq.SllmError) as e:
        sq.model_matmul_quant_into_f32(w, np.zeros(96, np.float32), 1, 96)
    assert e.value.status == 1
    with pytest.raises(sq.SllmError) as e:
        sq.DeviceWeight.from_quant(sq.QuantWeight("q9", raw, 2, 4, 64))
    assert e.value.status == 2


@pytest.mark.parametrize("qtype", ["q8", "q4_1", "q5k1"])
@pytest.mark.parametrize("Ns", [(10001,), (5000, 5001), (17003,), (9000, 4100, 3)])
def test_row_orders_with_partial_and_spare_waves(qtype, Ns):
    # rows per wave = ceil(total rows / 4096 wave slots): 3 (10001 rows) and
    # 5 (17003 rows) take consecutive rows per wave, 4 (13103 rows) strided
    # ones; a partly filled last wave per weight, spare waves that own no row,
    # and several weights sharing one launch (q/k/v-style segments)
    K = 256
    ws, raws = [], []
    for i, N in enumerate(Ns):
        raw = make_raw(qtype, N, K, seed=N + i)
        raws.append(raw)
        ws.append(sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K)))
    x = make_x(1, K, seed=len(Ns))
    outs = sq.model_matmul_multi_quant_into_f32(ws, x, 1, K)
    for N, raw, got in zip(Ns, raws, outs):
        ref = oracle.matmul(qtype, raw, N, x)
        assert_fp32_parity(got.reshape(1, N), ref, term_abs_sum(qtype, raw, N, x), f"{qtype} {Ns} N={N}")
        single, _, _ = sq.model_matmul_quant_into_f32(ws[Ns.index(N)], x, 1, K)
        assert np.array_equal(single.view(np.uint32), got.view(np.uint32))
