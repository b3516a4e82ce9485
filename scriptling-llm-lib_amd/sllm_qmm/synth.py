"""Seeded synthetic inputs for the BASELINE configs (this repository's own generator).

One generator for tests and bench: SplitMix64(seed) -> 53-bit uniforms ->
Box-Muller normals. Block synthesis for the k-quant formats draws the block
fields directly (scales, mins, nibbles), as the reference ships no Q4_K / Q5_K /
Q6_K quantizer; Q4_0 / Q4_1 / Q5_0 weights come from fp32 via the usual
ggml-style rounding quantizers defined here. None of this is reference
arithmetic: parity is always on identical packed bytes.
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    """Outputs start .. start + n - 1 of the SplitMix64 stream for `seed`."""
    with np.errstate(over="ignore"):
        z = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z *= _GOLDEN
        z += np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        z ^= z >> np.uint64(30)
        z *= _M1
        z ^= z >> np.uint64(27)
        z *= _M2
        z ^= z >> np.uint64(31)
        return z


def uniform(seed: int, n: int, start: int = 0) -> np.ndarray:
    """n doubles in [0, 1) from the top 53 bits."""
    u = splitmix64(seed, n, start)
    u >>= np.uint64(11)
    f = u.astype(np.float64)
    f *= 1.0 / (1 << 53)
    return f


def normal(seed: int, n: int, std: float = 1.0, chunk: int = 1 << 20) -> np.ndarray:
    """n float32 ~ N(0, std^2) by Box-Muller over consecutive uniform pairs
    (generated in chunks of `chunk` pairs; the values do not depend on it)."""
    m = (n + 1) // 2
    out = np.empty(2 * m, np.float32)
    for p0 in range(0, m, chunk):
        p1 = min(m, p0 + chunk)
        u = uniform(seed, 2 * (p1 - p0), 2 * p0)
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        t = 2.0 * np.pi * u[1::2]
        z = np.empty(2 * (p1 - p0), np.float64)
        z[0::2] = r * np.cos(t)
        z[1::2] = r * np.sin(t)
        z *= std
        out[2 * p0:2 * p1] = z
    return out[:n]


def random_bytes(seed: int, n: int) -> np.ndarray:
    words = splitmix64(seed, (n + 7) // 8)
    return words.view(np.uint8)[:n].copy()


def _f16_bits(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def _put16(dst: np.ndarray, off: int, bits: np.ndarray) -> None:
    dst[:, off] = (bits & 0xFF).astype(np.uint8)
    dst[:, off + 1] = (bits >> 8).astype(np.uint8)


def _pack_scale_min_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of getScaleMinK4 (kquants.go:62-71): 8 six-bit (sc, m) -> 12 bytes."""
    nb = sc.shape[0]
    q = np.zeros((nb, 12), np.uint8)
    q[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    q[:, 4:8] = m[:, 0:4] | ((m[:, 4:8] >> 4) << 6)
    q[:, 8:12] = (sc[:, 4:8] & 0x0F) | ((m[:, 4:8] & 0x0F) << 4)
    return q


def q4k_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """Random Q4_K tensor (144 B / 256): d, dmin ~ U(1e-4, 1e-2), 6-bit sc/m, random nibbles."""
    nb = rows * cols // 256
    out = np.zeros((nb, 144), np.uint8)
    u = uniform(seed, 2 * nb).reshape(nb, 2)
    _put16(out, 0, _f16_bits(1e-4 + u[:, 0] * (1e-2 - 1e-4)))
    _put16(out, 2, _f16_bits(1e-4 + u[:, 1] * (1e-2 - 1e-4)))
    sm = (splitmix64(seed + 1, nb * 16) & np.uint64(63)).astype(np.uint8).reshape(nb, 16)
    out[:, 4:16] = _pack_scale_min_k4(sm[:, :8], sm[:, 8:])
    out[:, 16:144] = random_bytes(seed + 2, nb * 128).reshape(nb, 128)
    return out.reshape(-1)


def q5k_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """Random Q5_K tensor (176 B / 256): as Q4_K plus 32 random high-bit bytes."""
    nb = rows * cols // 256
    out = np.zeros((nb, 176), np.uint8)
    u = uniform(seed, 2 * nb).reshape(nb, 2)
    _put16(out, 0, _f16_bits(1e-4 + u[:, 0] * (1e-2 - 1e-4)))
    _put16(out, 2, _f16_bits(1e-4 + u[:, 1] * (1e-2 - 1e-4)))
    sm = (splitmix64(seed + 1, nb * 16) & np.uint64(63)).astype(np.uint8).reshape(nb, 16)
    out[:, 4:16] = _pack_scale_min_k4(sm[:, :8], sm[:, 8:])
    out[:, 16:176] = random_bytes(seed + 2, nb * 160).reshape(nb, 160)
    return out.reshape(-1)


def q6k_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """Random Q6_K tensor (210 B / 256): random ql/qh, int8 sc ~ U{-128..127}, d ~ U(1e-4, 1e-2)."""
    nb = rows * cols // 256
    out = np.zeros((nb, 210), np.uint8)
    out[:, 0:208] = random_bytes(seed, nb * 208).reshape(nb, 208)
    u = uniform(seed + 1, nb)
    _put16(out, 208, _f16_bits(1e-4 + u * (1e-2 - 1e-4)))
    return out.reshape(-1)


def q2k_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """Random Q2_K tensor (84 B / 256): random scale and code bytes, d ~ U(1e-4, 1e-2),
    dmin ~ U(1e-4, 5e-3)."""
    nb = rows * cols // 256
    out = np.zeros((nb, 84), np.uint8)
    out[:, 0:80] = random_bytes(seed, nb * 80).reshape(nb, 80)
    _put16(out, 80, _f16_bits(1e-4 + uniform(seed + 1, nb) * (1e-2 - 1e-4)))
    _put16(out, 82, _f16_bits(1e-4 + uniform(seed + 2, nb) * (5e-3 - 1e-4)))
    return out.reshape(-1)


def q3k_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """Random Q3_K tensor (110 B / 256): random mask, code and scale bytes, d ~ U(1e-4, 1e-2)."""
    nb = rows * cols // 256
    out = np.zeros((nb, 110), np.uint8)
    out[:, 0:108] = random_bytes(seed, nb * 108).reshape(nb, 108)
    _put16(out, 108, _f16_bits(1e-4 + uniform(seed + 1, nb) * (1e-2 - 1e-4)))
    return out.reshape(-1)


def iq4nl_blocks(seed: int, rows: int, cols: int) -> np.ndarray:
    """Random IQ4_NL tensor (18 B / 32)."""
    nb = rows * cols // 32
    out = np.zeros((nb, 18), np.uint8)
    u = uniform(seed, nb)
    _put16(out, 0, _f16_bits(1e-4 + u * (1e-2 - 1e-4)))
    out[:, 2:] = random_bytes(seed + 1, nb * 16).reshape(nb, 16)
    return out.reshape(-1)


def _nibble_bytes(q: np.ndarray) -> np.ndarray:
    """32 4-bit codes per block -> 16 bytes (byte i = code i | code i+16 << 4)."""
    return (q[:, :16] & 0x0F) | ((q[:, 16:] & 0x0F) << 4)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q4_0 Raw (18 B / 32): d = signed absmax / -8, q = clamp(floor(x/d + 8.5), 0, 15)."""
    b = np.asarray(w, np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.clip(np.floor(b * inv[:, None] + np.float32(8.5)), 0, 15).astype(np.uint8)
    out = np.zeros((b.shape[0], 18), np.uint8)
    _put16(out, 0, _f16_bits(d))
    out[:, 2:] = _nibble_bytes(q)
    return out.reshape(-1)


def quantize_q4_1(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q4_1 Raw (20 B / 32): d = (max - min) / 15, m = min."""
    b = np.asarray(w, np.float32).reshape(-1, 32)
    mn, mx = b.min(axis=1), b.max(axis=1)
    d = ((mx - mn) / np.float32(15.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.clip(np.floor((b - mn[:, None]) * inv[:, None] + np.float32(0.5)), 0, 15).astype(np.uint8)
    out = np.zeros((b.shape[0], 20), np.uint8)
    _put16(out, 0, _f16_bits(d))
    _put16(out, 2, _f16_bits(mn))
    out[:, 4:] = _nibble_bytes(q)
    return out.reshape(-1)


def quantize_q5_0(w: np.ndarray) -> np.ndarray:
    """fp32 -> Q5_0 Raw (22 B / 32): d = signed absmax / -16, q = clamp(floor(x/d + 16.5), 0, 31)."""
    b = np.asarray(w, np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-16.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    q = np.clip(np.floor(b * inv[:, None] + np.float32(16.5)), 0, 31).astype(np.uint32)
    qh = ((q >> 4) << np.arange(32, dtype=np.uint32)).sum(axis=1).astype(np.uint32)
    out = np.zeros((b.shape[0], 22), np.uint8)
    _put16(out, 0, _f16_bits(d))
    out[:, 2:6] = qh.view(np.uint8).reshape(-1, 4)
    out[:, 6:] = _nibble_bytes(q.astype(np.uint8))
    return out.reshape(-1)


# GGUF tensor type ids used by the BASELINE configs.
GGML_Q4_0, GGML_Q4_1, GGML_Q5_0, GGML_Q8_0 = 2, 3, 6, 8
GGML_Q4_K, GGML_Q5_K, GGML_Q6_K, GGML_IQ4_NL = 12, 13, 14, 20
GGML_Q2_K, GGML_Q3_K = 10, 11

BLOCKS = {GGML_Q4_K: q4k_blocks, GGML_Q5_K: q5k_blocks, GGML_Q6_K: q6k_blocks, GGML_IQ4_NL: iq4nl_blocks}


def gguf_tensor(ggml_type: int, seed: int, rows: int, cols: int) -> np.ndarray:
    """Raw GGUF block bytes of a rows x cols tensor of the given type."""
    if ggml_type in BLOCKS:
        return BLOCKS[ggml_type](seed, rows, cols)
    w = normal(seed, rows * cols, 0.02)
    if ggml_type == GGML_Q4_0:
        return quantize_q4_0(w)
    if ggml_type == GGML_Q4_1:
        return quantize_q4_1(w)
    if ggml_type == GGML_Q5_0:
        return quantize_q5_0(w)
    raise ValueError(f"no synthetic generator for GGUF type {ggml_type}")
