"""Shared test data builders and the fp32 parity criterion."""
from __future__ import annotations

import numpy as np

import oracle
from sllm_qmm import synth

# fp32 outputs may differ from the reference's sequential sum only by the order
# in which per-block terms are added (reassociation). Bound, per output:
#   |got - ref| <= REL_TOL * sum_g |term_g|        (conditioning-aware)
# and, as the reference's own tests measure (q8q8_test.go:77-84), relative to
# the output vector's scale:  max|got - ref| / max|ref| <= REL_TOL.
REL_TOL = 1e-5


def _f16(raw_u16: np.ndarray) -> np.ndarray:
    return raw_u16.astype(np.uint16).view(np.float16).astype(np.float64)


def raw_fields(qtype: str, raw: np.ndarray, N: int, G: int):
    """Decode the per-block scale fields of a QuantWeight.Raw (float64)."""
    bb = oracle.BLOCK_BYTES[qtype]
    if qtype == "q5k1":
        half = raw[: N * G * 20].reshape(N, G, 20)
        high = raw[N * G * 20:].reshape(N, G, 20)
        d = _f16(half[..., 0].astype(np.uint16) | (half[..., 1].astype(np.uint16) << 8))
        m = _f16(half[..., 2].astype(np.uint16) | (half[..., 3].astype(np.uint16) << 8))
        dh = _f16(high[..., 0].astype(np.uint16) | (high[..., 1].astype(np.uint16) << 8))
        return d, m, dh
    b = raw.reshape(N, G, bb)
    d = _f16(b[..., 0].astype(np.uint16) | (b[..., 1].astype(np.uint16) << 8))
    m = None
    if qtype == "q4_1":
        m = _f16(b[..., 2].astype(np.uint16) | (b[..., 3].astype(np.uint16) << 8))
    return d, m, None


def term_abs_sum(qtype: str, raw: np.ndarray, N: int, x: np.ndarray) -> np.ndarray:
    """sum_g |term_g| per (m, n), from the oracle's block dots and the Raw scales."""
    x = np.asarray(x, np.float32).reshape(-1, x.shape[-1])
    K = x.shape[1]
    G = K // 32
    dots = oracle.block_dots(qtype, raw, N, K, x)
    _, xs = oracle.quantize_act_q8(x)
    xs = xs.astype(np.float64)[:, None, :]
    d, m, dh = raw_fields(qtype, raw, N, G)
    if qtype == "q5":
        s = dots.view(np.float32).astype(np.float64)
        return np.abs(d[None] * s).sum(-1)
    if qtype in ("q8", "q4"):
        return np.abs(d[None] * xs * dots).sum(-1)
    xq, _ = oracle.quantize_act_q8(x)
    sx = xq.reshape(x.shape[0], G, 32).astype(np.int64).sum(-1)[:, None, :]
    if qtype == "q4_1":
        return np.abs(xs * (d[None] * dots + m[None] * sx)).sum(-1)
    lo = np.abs(xs * (d[None] * dots[..., 0] + m[None] * sx)).sum(-1)
    hi = np.abs(xs * dh[None] * dots[..., 1]).sum(-1)
    return lo + hi


def assert_fp32_parity(got: np.ndarray, ref: np.ndarray, bound: np.ndarray, what: str = "") -> None:
    got = np.asarray(got, np.float64).reshape(ref.shape)
    ref = np.asarray(ref, np.float64)
    bound = np.asarray(bound, np.float64).reshape(ref.shape)
    # special values must match exactly: NaN where the reference has NaN, the
    # same infinity where it has one (the bound below cannot see either)
    nan_r, nan_g = np.isnan(ref), np.isnan(got)
    assert np.array_equal(nan_r, nan_g), f"{what}: NaN positions differ ({int(nan_r.sum())} ref, {int(nan_g.sum())} got)"
    inf_r = np.isinf(ref)
    assert np.array_equal(got[inf_r], ref[inf_r]) and not np.isinf(got[~inf_r]).any(), f"{what}: infinities differ"
    fin = ~(nan_r | inf_r)
    got, ref, bound = got[fin], ref[fin], bound[fin]
    if got.size == 0:
        return
    err = np.abs(got - ref)
    lim = REL_TOL * bound + 1e-30
    bad = np.flatnonzero(err > lim)
    assert bad.size == 0, (
        f"{what}: {len(bad)} outputs exceed {REL_TOL:g}*sum|terms|; first (finite index {int(bad[0])}): "
        f"got {got[bad[0]]!r} ref {ref[bad[0]]!r} bound {lim[bad[0]]!r}")
    scale = np.abs(ref).max()
    if scale > 0:
        assert err.max() / scale <= REL_TOL, f"{what}: vector-scale error {err.max() / scale:g}"


def make_raw(qtype: str, N: int, K: int, seed: int = 0) -> np.ndarray:
    """Random QuantWeight.Raw of the given QType (N rows, K cols)."""
    if qtype == "q8":
        return oracle.quantize_q8_rows_f32(synth.normal(seed, N * K, 0.02).reshape(N, K))
    if qtype == "q4":
        return synth.quantize_q4_0(synth.normal(seed, N * K, 0.02))
    if qtype == "q4_1":
        return synth.quantize_q4_1(synth.normal(seed, N * K, 0.02))
    if qtype == "q5":
        return synth.quantize_q5_0(synth.normal(seed, N * K, 0.02))
    if qtype == "q5k1":
        assert K % 256 == 0
        return oracle.convert_q5k_to_two_q41(synth.q5k_blocks(seed, N, K), N, K)
    raise ValueError(qtype)


def make_x(M: int, K: int, seed: int = 1) -> np.ndarray:
    return synth.normal(seed, M * K, 1.0).reshape(M, K)
