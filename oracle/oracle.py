"""ctypes/numpy front-end for the refcpu oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or the timed CPU baseline. The product
library (scriptling-llm-lib_amd/) never imports it.

The shared objects are built by ``build()`` (also called from
``__graft_entry__.build()``): ``liboracle.so`` (the scalar restatement,
refcpu.c) and ``libbaseline.so`` (the threaded AVX2/AVX-VNNI restatement of
the reference's CPU kernels, refcpu_simd.c).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
BASELINE_PATH = os.path.join(HERE, "libbaseline.so")

BLOCK_BYTES = {"q8": 34, "q4": 18, "q4_1": 20, "q5": 22, "q5k1": 40}


def build() -> None:
    """Compile the oracle and the CPU baseline (gcc; no fast-math, no FMA contraction)."""
    flags = ["-O2", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-shared", "-fPIC"]
    subprocess.check_call(["gcc", *flags, os.path.join(HERE, "refcpu.c"), "-o", LIB_PATH, "-lm"])
    subprocess.check_call(["gcc", *flags, "-pthread", "-mavx2", "-mf16c", "-mfma",
                           os.path.join(HERE, "refcpu_simd.c"), os.path.join(HERE, "refcpu.c"),
                           "-o", BASELINE_PATH, "-lm"])


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} missing (run __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        i32, i64 = C.c_int, C.c_int64
        L.ref_f16_to_f32_lut.restype = C.c_float
        L.ref_f16_to_f32_lut.argtypes = [C.c_uint16]
        L.ref_f16_to_f32_cvtph.restype = C.c_float
        L.ref_f16_to_f32_cvtph.argtypes = [C.c_uint16]
        L.ref_f16_to_f64.restype = C.c_double
        L.ref_f16_to_f64.argtypes = [C.c_uint16]
        L.ref_f64_to_f16.restype = C.c_uint16
        L.ref_f64_to_f16.argtypes = [C.c_double]
        L.ref_quantize_act_q8.argtypes = [P, i32, P, P]
        L.ref_quantize_q8_rows_f32.argtypes = [P, i32, i32, P]
        L.ref_quantize_q8_rows_f64.argtypes = [P, i32, i32, P]
        for n in ("q8_0", "q4_0", "q4_1", "q5_0", "q4_k", "q5_k", "q6_k", "iq4_nl", "q2_k", "q3_k"):
            getattr(L, "ref_dequant_" + n).argtypes = [P, i64, P]
        L.ref_convert_q4k_to_q41.argtypes = [P, i32, i32, P]
        L.ref_convert_q5k_to_two_q41.argtypes = [P, i32, i32, P]
        L.ref_load_weight.restype = i64
        L.ref_load_weight.argtypes = [C.c_uint32, P, i32, i32, C.c_char_p, P, i64]
        L.ref_int8_dot.restype = C.c_int32
        L.ref_int8_dot.argtypes = [P, P, i32]
        L.ref_block_dots.argtypes = [C.c_char_p, P, i32, i32, P, P, i32, P]
        L.ref_q8q8_row.restype = C.c_float
        L.ref_q8q8_row.argtypes = [P, P, P, i32]
        L.ref_q4q8_row.restype = C.c_float
        L.ref_q4q8_row.argtypes = [P, P, P, i32]
        L.ref_q41q8_row.restype = C.c_float
        L.ref_q41q8_row.argtypes = [P, P, P, P, i32]
        L.ref_q5_row.restype = C.c_float
        L.ref_q5_row.argtypes = [P, P, i32]
        L.ref_matmul_quant.argtypes = [C.c_char_p, P, i32, i32, P, i32, P]
        L.ref_argmax.argtypes = [P, i32]
        L.ref_scale_min_k4.argtypes = [i32, P, P, P]
        L.ref_block_bytes.argtypes = [C.c_char_p]
        L.ref_swiglu.restype = C.c_float
        L.ref_swiglu.argtypes = [C.c_float, C.c_float]
        L.ref_swiglu_n.argtypes = [P, P, P, i64]
        L.ref_rmsnorm.argtypes = [P, P, C.c_float, i32, i32, P]
        L.ref_rmsnorm_lib.argtypes = [P, P, C.c_float, i32, i32, P]
        L.ref_rope.argtypes = [P, i32, i32, i32, P, i32]
        L.ref_matmul_dense.argtypes = [P, i32, i32, P, i32, P]
        L.ref_dense_block_sums.argtypes = [P, i32, i32, P, i32, P]
        L.ref_attention_head.argtypes = [P, P, P, i32, i32, i32, i32, i32, P, i32]
        L.ref_attention_layer.argtypes = [P, P, P, i32, i32, i32, i32, P, i32, P, i32, P, i32, P, P,
                                          C.c_float, i32, P, i32, i32, P, P, i32, i32, P, P]
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def f16_to_f32_lut(h: int) -> float:
    return lib().ref_f16_to_f32_lut(h)


def f16_to_f32_cvtph(h: int) -> float:
    return lib().ref_f16_to_f32_cvtph(h)


def f16_to_f64(h: int) -> float:
    return lib().ref_f16_to_f64(h)


def f64_to_f16(f: float) -> int:
    return lib().ref_f64_to_f16(f)


def quantize_act_q8(x: np.ndarray):
    """q8q8.go:96-125 over every row of x (M x K or K): returns (xq int8, xs float32)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    assert K % 32 == 0
    G = K // 32
    rows = x.reshape(-1, K)
    xq = np.empty(rows.shape, np.int8)
    xs = np.empty((rows.shape[0], G), np.float32)
    for r in range(rows.shape[0]):
        lib().ref_quantize_act_q8(_p(rows[r]), G, _p(xq[r]), _p(xs[r]))
    return xq.reshape(x.shape), xs.reshape(x.shape[:-1] + (G,))


def quantize_q8_rows_f32(w: np.ndarray) -> bytes:
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    out = np.empty(rows * cols // 32 * 34, np.uint8)
    if lib().ref_quantize_q8_rows_f32(_p(w), rows, cols, _p(out)):
        raise ValueError("cols must be a multiple of 32")
    return out


def quantize_q8_rows_f64(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float64)
    rows, cols = w.shape
    out = np.empty(rows * cols // 32 * 34, np.uint8)
    if lib().ref_quantize_q8_rows_f64(_p(w), rows, cols, _p(out)):
        raise ValueError("cols must be a multiple of 32")
    return out


def dequant(kind: str, raw: np.ndarray, n: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty(n, np.float64)
    getattr(lib(), "ref_dequant_" + kind)(_p(raw), n, _p(out))
    return out


def convert_q4k_to_q41(src: np.ndarray, rows: int, cols: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(rows * cols // 32 * 20, np.uint8)
    lib().ref_convert_q4k_to_q41(_p(src), rows, cols, _p(out))
    return out


def convert_q5k_to_two_q41(src: np.ndarray, rows: int, cols: int) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint8)
    out = np.empty(2 * rows * cols // 32 * 20, np.uint8)
    lib().ref_convert_q5k_to_two_q41(_p(src), rows, cols, _p(out))
    return out


def load_weight(ggml_type: int, raw: np.ndarray, rows: int, cols: int):
    """gguf.go:818-934: returns (qtype, Raw bytes) or None for the dense fallback."""
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    cap = rows * cols // 32 * 40 + 64
    out = np.empty(cap, np.uint8)
    qt = C.create_string_buffer(16)
    n = lib().ref_load_weight(ggml_type, _p(raw), rows, cols, qt, _p(out), cap)
    if n < 0:
        return None
    return qt.value.decode(), out[:n].copy()


def int8_dot(a: np.ndarray, b: np.ndarray) -> int:
    a = np.ascontiguousarray(a, dtype=np.int8)
    b = np.ascontiguousarray(b, dtype=np.int8)
    return lib().ref_int8_dot(_p(a), _p(b), a.size)


def block_dots(qtype: str, raw: np.ndarray, N: int, K: int, x: np.ndarray) -> np.ndarray:
    """Per-(m, n, g) block dots (int32; fp32 bits for q5; [..., 2] for q5k1)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, K)
    M, G = x.shape[0], K // 32
    xq, _ = quantize_act_q8(x)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    shape = (M, N, G, 2) if qtype == "q5k1" else (M, N, G)
    out = np.empty(shape, np.int32)
    if lib().ref_block_dots(qtype.encode(), _p(raw), N, G, _p(xq), _p(x), M, _p(out)):
        raise ValueError(qtype)
    return out


def matmul(qtype: str, raw: np.ndarray, N: int, x: np.ndarray) -> np.ndarray:
    """float32_ops.go:379-460 modelMatmulQuantIntoF32: x (M x K) -> dst (M x N)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    M = x.size // K
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    dst = np.empty((M, N), np.float32)
    if lib().ref_matmul_quant(qtype.encode(), _p(raw), N, K, _p(x), M, _p(dst)):
        raise ValueError(f"unknown qtype {qtype}")
    return dst


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """model_f32.go:486-489 elementwise (libm exp standing in for Go's math.Exp)."""
    g = np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    u = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
    h = np.empty_like(g)
    lib().ref_swiglu_n(_p(g), _p(u), _p(h), g.size)
    return h.reshape(np.shape(gate))


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float, lib_order: bool = False) -> np.ndarray:
    """rmsNormFlatF32 (float32_ops.go:159-172) of every row of x; lib_order: the
    library's association of the sum of squares instead of the reference's."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    rows = x.size // K
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    fn = lib().ref_rmsnorm_lib if lib_order else lib().ref_rmsnorm
    fn(_p(x), _p(w), eps, rows, K, _p(out))
    return out


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return lib().ref_argmax(_p(v), v.size)


def row_q8q8(w, xq, xs):
    return lib().ref_q8q8_row(_p(w), _p(xq), _p(xs), xs.size)


def row_q4q8(w, xq, xs):
    return lib().ref_q4q8_row(_p(w), _p(xq), _p(xs), xs.size)


def row_q41q8(w, xq, xs, sxq):
    return lib().ref_q41q8_row(_p(w), _p(xq), _p(xs), _p(sxq), xs.size)


def row_q5(w, x):
    return lib().ref_q5_row(_p(w), _p(x), x.size // 32)


def scale_min_k4(j: int, q: np.ndarray):
    q = np.ascontiguousarray(q, dtype=np.uint8)
    sc, m = C.c_uint8(), C.c_uint8()
    lib().ref_scale_min_k4(j, _p(q), C.addressof(sc), C.addressof(m))
    return sc.value, m.value


_bl = None


def baseline() -> C.CDLL:
    """The threaded AVX2/AVX-VNNI restatement (refcpu_simd.c): the cpu_baseline leg."""
    global _bl
    if _bl is None:
        if not os.path.exists(BASELINE_PATH):
            raise RuntimeError(f"baseline not built: {BASELINE_PATH} missing")
        B = C.CDLL(BASELINE_PATH)
        B.bl_matmul.argtypes = [C.c_char_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p]
        B.bl_time_matmul.argtypes = [C.c_char_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                                     C.c_int, C.c_int]
        B.bl_time_matmul.restype = C.c_double
        B.bl_set_workers.argtypes = [C.c_int]
        _bl = B
    return _bl


def baseline_matmul(qtype: str, raw: np.ndarray, N: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    M = x.size // K
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    dst = np.empty((M, N), np.float32)
    if baseline().bl_matmul(qtype.encode(), _p(raw), N, K, _p(x), M, _p(dst)):
        raise ValueError(qtype)
    return dst


def baseline_time(qtype: str, raw: np.ndarray, N: int, x: np.ndarray, reps: int, trials: int = 7) -> float:
    """Seconds per matmul: min over `trials` of the mean of `reps` calls (q8q8.go:280-294)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    M = x.size // K
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    dst = np.empty((M, N), np.float32)
    return baseline().bl_time_matmul(qtype.encode(), _p(raw), N, K, _p(x), M, _p(dst), reps, trials)


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _po(a):
    return None if a is None else _p(a)


def rope(data: np.ndarray, start_pos: int, freqs: np.ndarray, half_dim: int) -> np.ndarray:
    """applyRopeInPlaceF32 (float32_ops.go:174-188) on a copy of data (rows x d_k)."""
    out = np.array(data, dtype=np.float32, order="C", copy=True)
    rows, d_k = out.shape
    fr = _f32(freqs)
    lib().ref_rope(_p(out), rows, d_k, start_pos, _p(fr), half_dim)
    return out


def attention_head(q, k, v, causal=True, cache_len=0) -> np.ndarray:
    """fusedAttentionHeadF32 (float32_ops.go:190-235): q (q_rows x d_k) against
    k / v (k_rows x d_k)."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros_like(q)
    lib().ref_attention_head(_p(q), _p(k), _p(v), q.shape[0], q.shape[1], k.shape[0], int(causal), cache_len,
                             _p(out), 0)
    return out


def attention_layer(q, k, v, n_heads, n_kv, d_k, cache_k, cache_v, cache_len, start_pos, freqs, half_dim,
                    q_bias=None, k_bias=None, v_bias=None, q_norm_w=None, k_norm_w=None, eps=1e-5,
                    lib_norm=False, return_q_rot=False):
    """forwardBlock's attention section (model_f32.go:398-466) for one layer.

    q: seq x n_heads*d_k, k / v: seq x n_kv*d_k (matmul outputs); cache_k /
    cache_v: n_kv x cap x d_k holding cache_len rows per head. Returns (out
    seq x n_heads*d_k, new cache_k, new cache_v[, q_rot: the normed, rotated q
    heads, seq x n_heads*d_k]); the inputs are not modified.
    """
    q, k, v = (np.array(a, dtype=np.float32, order="C", copy=True) for a in (q, k, v))
    ck = np.array(cache_k, dtype=np.float32, order="C", copy=True)
    cv = np.array(cache_v, dtype=np.float32, order="C", copy=True)
    seq = q.shape[0]
    cap = ck.shape[1]
    assert cache_len + seq <= cap
    out = np.zeros((seq, n_heads * d_k), np.float32)
    qr = np.zeros((seq, n_heads * d_k), np.float32)
    qb, kb, vb = _f32(q_bias), _f32(k_bias), _f32(v_bias)
    qn, kn, fr = _f32(q_norm_w), _f32(k_norm_w), _f32(freqs)
    lib().ref_attention_layer(_p(q), _p(k), _p(v), seq, n_heads, n_kv, d_k,
                              _po(qb), 0 if qb is None else qb.size, _po(kb), 0 if kb is None else kb.size,
                              _po(vb), 0 if vb is None else vb.size, _po(qn), _po(kn), eps, int(lib_norm),
                              _p(fr), half_dim, start_pos, _p(ck), _p(cv), cap, cache_len, _p(out),
                              _p(qr) if return_q_rot else None)
    return (out, ck, cv, qr) if return_q_rot else (out, ck, cv)


def dense_weights(ggml_type: int, raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The dense float32 weights the reference builds for a type it has no
    quantized kernel for (gguf.go:907-911: f64ToF32(dequantize1D(...)))."""
    kind = {10: "q2_k", 11: "q3_k"}[ggml_type]
    return dequant(kind, raw, rows * cols).astype(np.float32).reshape(rows, cols)


def matmul_dense(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """modelMatmulFloatIntoF32 (float32_ops.go:462-482): x (M x K) -> M x N."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, w.shape[1])
    out = np.empty((x.shape[0], w.shape[0]), np.float32)
    lib().ref_matmul_dense(_p(w), w.shape[0], w.shape[1], _p(x), x.shape[0], _p(out))
    return out


def dense_block_sums(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    """The dense products summed per 32-element block from zero: M x N x K/32."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, w.shape[1])
    out = np.empty((x.shape[0], w.shape[0], w.shape[1] // 32), np.float32)
    lib().ref_dense_block_sums(_p(w), w.shape[0], w.shape[1], _p(x), x.shape[0], _p(out))
    return out
