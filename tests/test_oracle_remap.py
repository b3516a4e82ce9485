"""Pins the oracle's load-time remaps and requantization (gguf.go:818-934).

The remaps must preserve the represented weights: dequant(remap(w)) equals
dequant(w) up to the f16 truncation of the new per-block scale and min (the
reference's own parity bound is 5e-3 relative, kquant_kernels_test.go:107-114),
and exactly when those products are f16-representable.
"""
import numpy as np
import pytest

import oracle
from sllm_qmm import synth


def test_scale_min_k4_inverts_the_packing():
    rng = np.random.default_rng(0)
    for _ in range(200):
        sc = rng.integers(0, 64, 8).astype(np.uint8)
        m = rng.integers(0, 64, 8).astype(np.uint8)
        q = synth._pack_scale_min_k4(sc[None], m[None])[0]
        for j in range(8):
            assert oracle.scale_min_k4(j, q) == (sc[j], m[j])


def _pow2_kquant(src: np.ndarray, bb: int) -> np.ndarray:
    """Force d, dmin to powers of two so d*sc and dmin*m are exact in f16."""
    b = src.reshape(-1, bb).copy()
    rng = np.random.default_rng(1)
    e = rng.integers(-12, -4, (b.shape[0], 2))
    bits = (e + 15) << 10
    b[:, 0], b[:, 1] = bits[:, 0] & 0xFF, bits[:, 0] >> 8
    b[:, 2], b[:, 3] = bits[:, 1] & 0xFF, bits[:, 1] >> 8
    return b.reshape(-1)


def _bound(a, b, scale):
    return np.abs(a - b).max() <= scale


def test_q4k_to_q41_preserves_weights():
    rows, cols = 24, 1024
    src = synth.q4k_blocks(3, rows, cols)
    out = oracle.convert_q4k_to_q41(src, rows, cols)
    ref = oracle.dequant("q4_k", src, rows * cols)
    got = oracle.dequant("q4_1", out, rows * cols)
    assert np.abs(got - ref).max() <= 2 ** -9 * np.abs(ref).max()
    exact_src = _pow2_kquant(src, 144)
    got = oracle.dequant("q4_1", oracle.convert_q4k_to_q41(exact_src, rows, cols), rows * cols)
    assert np.array_equal(got, oracle.dequant("q4_k", exact_src, rows * cols))


def test_q5k_to_two_q41_preserves_weights():
    rows, cols = 16, 512
    src = synth.q5k_blocks(4, rows, cols)
    out = oracle.convert_q5k_to_two_q41(src, rows, cols)
    half = rows * cols // 32 * 20
    ref = oracle.dequant("q5_k", src, rows * cols)
    got = oracle.dequant("q4_1", out[:half], rows * cols) + oracle.dequant("q4_1", out[half:], rows * cols)
    assert np.abs(got - ref).max() <= 2 ** -8 * np.abs(ref).max()
    # the high half is a Q4_1 tensor with min 0 and 0/1 codes
    hi = out[half:].reshape(-1, 20)
    assert np.all(hi[:, 2:4] == 0) and np.all((hi[:, 4:] & 0xEE) == 0)
    exact_src = _pow2_kquant(src, 176)
    out = oracle.convert_q5k_to_two_q41(exact_src, rows, cols)
    got = oracle.dequant("q4_1", out[:half], rows * cols) + oracle.dequant("q4_1", out[half:], rows * cols)
    assert np.array_equal(got, oracle.dequant("q5_k", exact_src, rows * cols))


def _q6k_dequant_by_element(raw: np.ndarray) -> np.ndarray:
    """Q6_K by the per-element index formula (ggml dequantize_row_q6_K layout)."""
    b = raw.reshape(-1, 210)
    e = np.arange(256)
    n, r = e // 128, e % 128
    k, l = r // 32, r % 32
    ql = b[:, 64 * n + l + 32 * (k & 1)]
    nib = np.where(k < 2, ql & 0x0F, ql >> 4).astype(np.int64)
    hb = ((b[:, 128 + 32 * n + l] >> (2 * k)) & 3).astype(np.int64)
    q = (nib | (hb << 4)) - 32
    sc = b[:, 192 + 8 * n + l // 16 + 2 * k].view(np.int8).astype(np.float64)
    d = b[:, 208:210].copy().view(np.float16).astype(np.float64)
    return (d * sc * q).reshape(-1)


def test_q6k_dequant_layout():
    src = synth.q6k_blocks(5, 8, 512)
    assert np.array_equal(oracle.dequant("q6_k", src, 8 * 512), _q6k_dequant_by_element(src))
    b = np.zeros(210, np.uint8)
    b[192:208] = 1
    b[208:210] = [0x00, 0x3C]                 # d = 1, sc = 1, ql = qh = 0 -> every weight -32
    assert np.all(oracle.dequant("q6_k", b, 256) == -32.0)


def test_iq4nl_codebook():
    # iquants_test.go:13-30
    cb = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]
    b = np.zeros(18, np.uint8)
    b[0:2] = [0x00, 0x40]                     # d = 2.0
    b[2:] = [j | ((15 - j) << 4) for j in range(16)]
    d = oracle.dequant("iq4_nl", b, 32)
    assert d[:16].tolist() == [2.0 * cb[j] for j in range(16)]
    assert d[16:].tolist() == [2.0 * cb[15 - j] for j in range(16)]


@pytest.mark.parametrize("t,kind", [(14, "q6_k"), (20, "iq4_nl")])
def test_requant_to_q8_closed_form(t, kind):
    rows, cols = 8, 512
    src = synth.gguf_tensor(t, 6, rows, cols)
    qt, out = oracle.load_weight(t, src, rows, cols)
    assert qt == "q8"
    v = oracle.dequant(kind, src, rows * cols).reshape(-1, 32)
    o = out.reshape(-1, 34)
    amax = np.abs(v).max(axis=1)
    scale = amax / 127.0
    bits = np.array([oracle.f64_to_f16(s) for s in scale])
    assert np.array_equal(o[:, 0].astype(np.uint16) | (o[:, 1].astype(np.uint16) << 8), bits)
    with np.errstate(divide="ignore", invalid="ignore"):
        val = np.clip(v * (1.0 / scale)[:, None], -128, 127)
    q = np.where(np.isnan(val), 0, np.sign(val) * np.floor(np.abs(np.nan_to_num(val)) + 0.5))
    assert np.array_equal(o[:, 2:].view(np.int8).astype(np.float64), q)


def test_load_weight_type_gate():
    # kquants_test.go:10-33 / gguf.go:818-934: int8 types map to a QType, the rest fall back to dense
    rows, cols = 4, 256
    for t, qt in [(8, "q8"), (2, "q4"), (3, "q4_1"), (6, "q5")]:
        bb = {8: 34, 2: 18, 3: 20, 6: 22}[t]
        raw = synth.random_bytes(t, rows * cols // 32 * bb)
        got = oracle.load_weight(t, raw, rows, cols)
        assert got[0] == qt and np.array_equal(got[1], raw)
    assert oracle.load_weight(12, synth.q4k_blocks(1, rows, cols), rows, cols)[0] == "q4_1"
    assert oracle.load_weight(13, synth.q5k_blocks(1, rows, cols), rows, cols)[0] == "q5k1"
    for t in (0, 1, 7, 10, 11, 16, 99):
        assert oracle.load_weight(t, np.zeros(rows * cols * 4, np.uint8), rows, cols) is None
    assert oracle.load_weight(12, np.zeros(144 * 4, np.uint8), 4, 160) is None  # cols % 256 != 0
