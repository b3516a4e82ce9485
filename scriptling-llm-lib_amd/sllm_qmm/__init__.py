"""Python host side of the MI355X quantized-matmul path (ctypes over libsllm_qmm.so).

Mirrors the reference's Go interface for this path so callers and tests read
like the reference's own:

=============================================  =======================================
reference (scriptling-llm-lib)                 here
=============================================  =======================================
``QuantWeight`` (gguf.go:73-79)                :class:`QuantWeight` (host Raw) and
                                               :class:`DeviceWeight` (HBM planes)
``loadWeightF32Direct`` (gguf.go:818-934)      :func:`load_weight_f32_direct`
``quantizeQ8RowsF32`` (gguf.go:1136-1186)      :func:`quantize_q8_rows_f32`
``modelMatmulQuantIntoF32`` (float32_ops.go:379)  :func:`model_matmul_quant_into_f32`
``modelMatmulRowQuantIntoF32`` (:620)          :func:`model_matmul_row_quant_into_f32`
``argmaxF32`` (float32_ops.go:812)             :func:`argmax_f32_dev`
=============================================  =======================================

There is no CPU fallback: if the shared library or the GPU is missing every
call raises :class:`SllmError`.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(HERE)
REPO_ROOT = os.path.dirname(PKG_ROOT)
LIB_PATH = os.path.join(PKG_ROOT, "libsllm_qmm.so")
HEADER_PATH = os.path.join(REPO_ROOT, "include", "sllm_qmm.h")

QTYPES = {"q8": 0, "q4": 1, "q4_1": 2, "q5": 3, "q5k1": 4, "q2k": 5, "q3k": 6}
QTYPE_NAMES = {v: k for k, v in QTYPES.items()}
RAW_BLOCK_BYTES = {"q8": 34, "q4": 18, "q4_1": 20, "q5": 22, "q5k1": 40}
# Bytes the device planes hold (and a GEMV streams) per 32-element block.
PLANE_BLOCK_BYTES = {"q8": 34, "q4": 18, "q4_1": 20, "q5": 22, "q5k1": 26, "q2k": 10.5, "q3k": 14.5}

STATUS = {0: "SLLM_OK", 1: "SLLM_ERR_ARG", 2: "SLLM_ERR_QTYPE", 3: "SLLM_ERR_SHAPE",
          4: "SLLM_ERR_DEVICE", 5: "SLLM_ERR_OOM", 6: "SLLM_ERR_FORMAT"}


class SllmError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS.get(status, status)}: {msg}")
        self.status = status


_lib = None


class AttnParams(C.Structure):
    """sllm_attn_params: the model constants of the attention section (device
    pointers to the model's tensors, 0 / None where the model has none)."""
    _fields_ = [("n_heads", C.c_int), ("n_kv_heads", C.c_int), ("d_k", C.c_int), ("rope_half_dim", C.c_int),
                ("rope_freqs", C.c_void_p), ("q_bias", C.c_void_p), ("q_bias_len", C.c_int),
                ("k_bias", C.c_void_p), ("k_bias_len", C.c_int), ("v_bias", C.c_void_p), ("v_bias_len", C.c_int),
                ("q_norm_w", C.c_void_p), ("k_norm_w", C.c_void_p), ("norm_eps", C.c_float)]


def lib() -> C.CDLL:
    """Load libsllm_qmm.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise SllmError(4, f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
    # One HIP runtime per process: torch ships its own libamdhip64.so.7. Loading
    # torch first makes the library bind to that same runtime (same SONAME)
    # instead of bringing up a second one from /opt/rocm next to it.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = C.CDLL(LIB_PATH)
    P, i32, sz = C.c_void_p, C.c_int, C.c_size_t
    W = C.c_void_p
    L.sllm_weight_from_quant.argtypes = [C.c_char_p, P, sz, i32, i32, i32, C.POINTER(W)]
    L.sllm_weight_from_gguf.argtypes = [C.c_uint32, P, sz, i32, i32, C.POINTER(W)]
    L.sllm_weight_from_f32.argtypes = [P, i32, i32, C.POINTER(W)]
    L.sllm_weight_destroy.argtypes = [W]
    L.sllm_weight_info.argtypes = [W, C.POINTER(i32), C.POINTER(i32), C.POINTER(i32), C.POINTER(i32),
                                   C.POINTER(sz)]
    L.sllm_weight_export.argtypes = [W, P, sz]
    L.sllm_matmul_quant_into_f32.argtypes = [W, P, i32, i32, P]
    L.sllm_matmul_row_quant_into_f32.argtypes = [W, P, P]
    L.sllm_matmul_dev.argtypes = [W, P, i32, i32, P, P]
    L.sllm_matmul_multi_quant_into_f32.argtypes = [C.POINTER(W), i32, P, i32, i32, C.POINTER(P)]
    L.sllm_matmul_multi_dev.argtypes = [C.POINTER(W), i32, P, i32, i32, C.POINTER(P), P]
    L.sllm_matmul_swiglu_dev.argtypes = [W, W, P, i32, i32, P, P, P, P]
    L.sllm_matmul_argmax_dev.argtypes = [W, P, i32, P, P, P]
    L.sllm_matmul_argmax.argtypes = [W, P, C.POINTER(i32)]
    f32 = C.c_float
    L.sllm_rmsnorm_matmul_multi_dev.argtypes = [C.POINTER(W), i32, P, P, f32, i32, i32, C.POINTER(P), P]
    L.sllm_rmsnorm_matmul_swiglu_dev.argtypes = [W, W, P, P, f32, i32, i32, P, P]
    L.sllm_rmsnorm_matmul_argmax_dev.argtypes = [W, P, P, f32, i32, P, P, P]
    L.sllm_matmul_swiglu_into_f32.argtypes = [W, W, P, i32, i32, P]
    L.sllm_argmax_dev.argtypes = [P, i32, C.POINTER(i32), P]
    L.sllm_debug_quantize_act.argtypes = [P, i32, i32, P, P, P]
    L.sllm_debug_block_dots.argtypes = [W, P, i32, i32, P]
    L.sllm_debug_gemm_block_dots.argtypes = [W, P, i32, i32, i32, i32, P]
    L.sllm_set_param.argtypes = [C.c_char_p, i32]
    L.sllm_matmul_add_dev.argtypes = [W, P, i32, i32, P, P]
    L.sllm_weight_stream_bytes.argtypes = [W, C.POINTER(sz)]
    L.sllm_weight_q6k_exact_blocks.argtypes = [W, C.POINTER(C.c_int64)]
    L.sllm_weight_q5k1_one_mfma.argtypes = [W, C.POINTER(i32)]
    L.sllm_kv_cache_create.argtypes = [i32, i32, i32, i32, C.POINTER(P)]
    L.sllm_kv_cache_destroy.argtypes = [P]
    L.sllm_kv_cache_length.argtypes = [P, i32, C.POINTER(i32)]
    L.sllm_kv_cache_set_length.argtypes = [P, i32]
    L.sllm_kv_cache_data.argtypes = [P, i32, C.POINTER(P), C.POINTER(P)]
    L.sllm_attention_dev.argtypes = [P, i32, C.POINTER(AttnParams), P, P, P, i32, i32, P, P]
    L.sllm_attention_noalloc_dev.argtypes = [P, i32, C.POINTER(AttnParams), P, P, P, i32, i32, P, P]
    L.sllm_workspace_reserve.argtypes = [P, sz]
    for name in exported_names():  # raises AttributeError if a declared symbol is missing
        f = getattr(L, name)
        if name in ("sllm_last_error", "sllm_kernel_info"):
            f.restype = C.c_char_p
        elif name in ("sllm_weight_destroy", "sllm_kv_cache_destroy"):
            f.restype = None
        else:
            f.restype = i32
    _lib = L
    return L


def exported_names() -> list[str]:
    """Every function the public header declares."""
    with open(HEADER_PATH) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(sllm_[a-z0-9_]+)\s*\(", text)))


def _check(st: int) -> None:
    if st != 0:
        msg = lib().sllm_last_error()
        raise SllmError(st, msg.decode() if msg else "")


def _flat_f32(a) -> np.ndarray:
    """a as a 1-D C-contiguous float32 array (no copy when it already is one)."""
    if type(a) is np.ndarray and a.dtype == np.float32 and a.ndim == 1 and a.flags.c_contiguous:
        return a
    return np.ascontiguousarray(a, dtype=np.float32).reshape(-1)


def _ptr(a: np.ndarray) -> int:
    """Address of a C-contiguous array's data (ctypes.addressof on a buffer view
    costs a third of ndarray.ctypes.data; read-only or empty arrays take the
    latter)."""
    if not a.flags.c_contiguous:
        raise ValueError("array must be C-contiguous")
    try:
        return C.addressof(C.c_char.from_buffer(a))
    except (TypeError, ValueError):
        return a.ctypes.data


def init() -> None:
    _check(lib().sllm_init())


def kernel_info() -> str:
    return lib().sllm_kernel_info().decode()


def set_param(name: str, value: int) -> None:
    _check(lib().sllm_set_param(name.encode(), int(value)))


@dataclass
class QuantWeight:
    """The reference's QuantWeight (gguf.go:73-79): QType, Raw, Groups, Rows, Cols."""
    qtype: str
    raw: np.ndarray
    groups: int
    rows: int
    cols: int


class DeviceWeight:
    """A weight repacked into HBM planes (opaque sllm_weight handle)."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)
        q, g, r, c = C.c_int(), C.c_int(), C.c_int(), C.c_int()
        n = C.c_size_t()
        _check(lib().sllm_weight_info(self._h, C.byref(q), C.byref(g), C.byref(r), C.byref(c), C.byref(n)))
        self.qtype = QTYPE_NAMES[q.value]
        self.groups, self.rows, self.cols, self.raw_bytes = g.value, r.value, c.value, n.value

    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise SllmError(1, "weight already destroyed")
        return self._h

    @property
    def plane_bytes(self) -> int:
        """Bytes one GEMV streams from this weight's planes (sllm_weight_stream_bytes)."""
        n = C.c_size_t()
        _check(lib().sllm_weight_stream_bytes(self.handle, C.byref(n)))
        return n.value

    @property
    def q6k_exact_blocks(self) -> int:
        """Q6_K streamed: blocks the GEMV recomputes in fp64; -1 without the
        streamed planes (sllm_weight_q6k_exact_blocks)."""
        n = C.c_int64()
        _check(lib().sllm_weight_q6k_exact_blocks(self.handle, C.byref(n)))
        return n.value

    @property
    def q5k1_one_mfma(self) -> bool:
        """Q5K1: the prefill GEMM takes one MFMA per block (every block's
        high-block scale is 16 x its low scale; sllm_weight_q5k1_one_mfma)."""
        n = C.c_int()
        _check(lib().sllm_weight_q5k1_one_mfma(self.handle, C.byref(n)))
        return bool(n.value)

    @classmethod
    def from_quant(cls, w: QuantWeight) -> "DeviceWeight":
        raw = np.ascontiguousarray(np.frombuffer(memoryview(w.raw).cast("B"), np.uint8))
        h = C.c_void_p()
        _check(lib().sllm_weight_from_quant(w.qtype.encode(), _ptr(raw), raw.nbytes, w.groups, w.rows, w.cols,
                                            C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_gguf(cls, ggml_type: int, raw, rows: int, cols: int) -> "DeviceWeight":
        raw = np.ascontiguousarray(np.frombuffer(memoryview(raw).cast("B"), np.uint8))
        h = C.c_void_p()
        _check(lib().sllm_weight_from_gguf(int(ggml_type), _ptr(raw), raw.nbytes, rows, cols, C.byref(h)))
        return cls(h.value)

    @classmethod
    def from_f32(cls, w: np.ndarray) -> "DeviceWeight":
        w = np.ascontiguousarray(w, dtype=np.float32)
        rows, cols = w.shape
        h = C.c_void_p()
        _check(lib().sllm_weight_from_f32(_ptr(w), rows, cols, C.byref(h)))
        return cls(h.value)

    def export(self) -> np.ndarray:
        """QuantWeight.Raw bytes rebuilt from the device planes."""
        out = np.empty(self.raw_bytes, np.uint8)
        _check(lib().sllm_weight_export(self.handle, _ptr(out), out.nbytes))
        return out

    def to_quant(self) -> QuantWeight:
        return QuantWeight(self.qtype, self.export(), self.groups, self.rows, self.cols)

    def close(self) -> None:
        if self._h is not None:
            lib().sllm_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def load_weight_f32_direct(ggml_type: int, raw, rows: int, cols: int) -> DeviceWeight:
    """gguf.go:818-934 for the int8-kernel types (8, 2, 3, 6, 12, 13, 14, 20), and Q2_K / Q3_K
    (10, 11) kept native where the reference goes to dense float32 (gguf.go:907-911)."""
    return DeviceWeight.from_gguf(ggml_type, raw, rows, cols)


def quantize_q8_rows_f32(flat: np.ndarray, rows: int, cols: int) -> DeviceWeight:
    """gguf.go:1136-1186 on the GPU (the tied-head path, model_f32.go:150-152)."""
    return DeviceWeight.from_f32(np.asarray(flat, np.float32).reshape(rows, cols))


def model_matmul_quant_into_f32(w: DeviceWeight, x_data: np.ndarray, x_rows: int, x_cols: int,
                                dst: np.ndarray | None = None):
    """float32_ops.go:379-460: returns (dst, xRows, Rows) like the Go function."""
    x = _flat_f32(x_data)
    if x.size < x_rows * x_cols:
        raise SllmError(1, "xData shorter than xRows*xCols")
    n = x_rows * w.rows
    if dst is None or dst.size < n or dst.dtype != np.float32 or not dst.flags["C_CONTIGUOUS"]:
        dst = np.empty(n, np.float32)  # growSlice (float32_ops.go:79-84)
    _check(lib().sllm_matmul_quant_into_f32(w.handle, _ptr(x), x_rows, x_cols, _ptr(dst)))
    return dst[:n], x_rows, w.rows


def model_matmul_row_quant_into_f32(w: DeviceWeight, normed: np.ndarray, dst: np.ndarray | None = None):
    """float32_ops.go:620-707: one activation row."""
    x = _flat_f32(normed)
    if dst is None or dst.size < w.rows:
        dst = np.empty(w.rows, np.float32)
    _check(lib().sllm_matmul_row_quant_into_f32(w.handle, _ptr(x), _ptr(dst)))
    return dst[: w.rows]


def matmul_dev(w: DeviceWeight, x_ptr: int, x_rows: int, x_cols: int, dst_ptr: int, stream: int = 0) -> None:
    """Device-resident matmul: raw device pointers, enqueued on `stream`."""
    _check(lib().sllm_matmul_dev(w.handle, C.c_void_p(x_ptr), x_rows, x_cols, C.c_void_p(dst_ptr),
                                 C.c_void_p(stream)))


def model_matmul_multi_quant_into_f32(ws: list, x_data: np.ndarray, x_rows: int, x_cols: int) -> list:
    """Consecutive modelMatmulIntoF32 calls on one input (forwardBlock's q/k/v,
    model_f32.go:391-396, and gate/up, :479-482) in one call: returns one
    (x_rows * Rows) array per weight, as the single calls would."""
    x = _flat_f32(x_data)
    if x.size < x_rows * x_cols:
        raise SllmError(1, "xData shorter than xRows*xCols")
    outs = [np.empty(x_rows * w.rows, np.float32) for w in ws]
    hs = (C.c_void_p * len(ws))(*[w.handle for w in ws])
    ds = (C.c_void_p * len(ws))(*[_ptr(o) for o in outs])
    _check(lib().sllm_matmul_multi_quant_into_f32(hs, len(ws), _ptr(x), x_rows, x_cols, ds))
    return outs


def matmul_multi_dev(ws: list, x_ptr: int, x_rows: int, x_cols: int, dst_ptrs: list, stream: int = 0) -> None:
    """Device-resident multi-weight matmul on one activation input."""
    hs = (C.c_void_p * len(ws))(*[w.handle for w in ws])
    ds = (C.c_void_p * len(ws))(*[C.c_void_p(p) for p in dst_ptrs])
    _check(lib().sllm_matmul_multi_dev(hs, len(ws), C.c_void_p(x_ptr), x_rows, x_cols, ds, C.c_void_p(stream)))


def model_matmul_swiglu_into_f32(w_gate: DeviceWeight, w_up: DeviceWeight, x_data: np.ndarray, x_rows: int,
                                 x_cols: int) -> np.ndarray:
    """forwardBlock's gate / up matmuls and SwiGLU loop (model_f32.go:479-490) in
    one call: returns h (x_rows * Rows float32)."""
    x = _flat_f32(x_data)
    if x.size < x_rows * x_cols:
        raise SllmError(1, "xData shorter than xRows*xCols")
    h = np.empty(x_rows * w_gate.rows, np.float32)
    _check(lib().sllm_matmul_swiglu_into_f32(w_gate.handle, w_up.handle, _ptr(x), x_rows, x_cols, _ptr(h)))
    return h


def matmul_swiglu_dev(w_gate: DeviceWeight, w_up: DeviceWeight, x_ptr: int, x_rows: int, x_cols: int, h_ptr: int,
                      gate_ptr: int = 0, up_ptr: int = 0, stream: int = 0) -> None:
    """Device-resident gate / up matmuls + SwiGLU (gate / up outputs optional)."""
    _check(lib().sllm_matmul_swiglu_dev(w_gate.handle, w_up.handle, C.c_void_p(x_ptr), x_rows, x_cols,
                                        C.c_void_p(h_ptr), C.c_void_p(gate_ptr or None),
                                        C.c_void_p(up_ptr or None), C.c_void_p(stream)))


def matmul_argmax(w: DeviceWeight, normed: np.ndarray) -> int:
    """outputLogits' head matmul + argmaxF32 (greedy token) in one launch; only
    the index comes back to the host."""
    x = _flat_f32(normed)
    if x.size < w.cols:
        raise SllmError(1, "normed shorter than Cols")
    out = C.c_int()
    _check(lib().sllm_matmul_argmax(w.handle, _ptr(x), C.byref(out)))
    return out.value


def matmul_argmax_dev(w: DeviceWeight, x_ptr: int, argmax_ptr: int, logits_ptr: int = 0, stream: int = 0) -> None:
    """Device-resident head matmul + argmax: *argmax_ptr (device int32) gets the index."""
    _check(lib().sllm_matmul_argmax_dev(w.handle, C.c_void_p(x_ptr), w.cols, C.c_void_p(logits_ptr or None),
                                        C.c_void_p(argmax_ptr), C.c_void_p(stream)))


def rmsnorm_matmul_multi_dev(ws: list, x_ptr: int, norm_w_ptr: int, eps: float, x_rows: int, x_cols: int,
                             dst_ptrs: list, stream: int = 0) -> None:
    """rmsNormFlatF32 + the layer's matmuls on the normed rows, one launch per format (decode)."""
    hs = (C.c_void_p * len(ws))(*[w.handle for w in ws])
    ds = (C.c_void_p * len(ws))(*[C.c_void_p(p) for p in dst_ptrs])
    _check(lib().sllm_rmsnorm_matmul_multi_dev(hs, len(ws), C.c_void_p(x_ptr), C.c_void_p(norm_w_ptr), eps,
                                               x_rows, x_cols, ds, C.c_void_p(stream)))


def rmsnorm_matmul_swiglu_dev(w_gate, w_up, x_ptr: int, norm_w_ptr: int, eps: float, x_rows: int, x_cols: int,
                              h_ptr: int, stream: int = 0) -> None:
    _check(lib().sllm_rmsnorm_matmul_swiglu_dev(w_gate.handle, w_up.handle, C.c_void_p(x_ptr),
                                                C.c_void_p(norm_w_ptr), eps, x_rows, x_cols, C.c_void_p(h_ptr),
                                                C.c_void_p(stream)))


def rmsnorm_matmul_argmax_dev(w, x_ptr: int, norm_w_ptr: int, eps: float, argmax_ptr: int, logits_ptr: int = 0,
                              stream: int = 0) -> None:
    _check(lib().sllm_rmsnorm_matmul_argmax_dev(w.handle, C.c_void_p(x_ptr), C.c_void_p(norm_w_ptr), eps, w.cols,
                                                C.c_void_p(logits_ptr or None), C.c_void_p(argmax_ptr),
                                                C.c_void_p(stream)))


def matmul_add_dev(w: DeviceWeight, x_ptr: int, x_rows: int, x_cols: int, dst_ptr: int, stream: int = 0) -> None:
    """dst += x W^T on device buffers: the o / down matmul with the residual add
    that follows it (model_f32.go:469-474, 492-497)."""
    _check(lib().sllm_matmul_add_dev(w.handle, C.c_void_p(x_ptr), x_rows, x_cols, C.c_void_p(dst_ptr),
                                     C.c_void_p(stream)))


class KVCache:
    """KVCacheF32 (float32_ops.go:11-14) of every layer, resident in device
    memory: n_kv_heads x max_seq x d_k floats of K and of V per layer."""

    def __init__(self, n_layers: int, n_kv_heads: int, d_k: int, max_seq: int):
        h = C.c_void_p()
        _check(lib().sllm_kv_cache_create(n_layers, n_kv_heads, d_k, max_seq, C.byref(h)))
        self.handle = h
        self.n_layers, self.n_kv_heads, self.d_k, self.max_seq = n_layers, n_kv_heads, d_k, max_seq

    def close(self) -> None:
        if self.handle:
            lib().sllm_kv_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def length(self, layer: int) -> int:
        n = C.c_int()
        _check(lib().sllm_kv_cache_length(self.handle, layer, C.byref(n)))
        return n.value

    def set_length(self, n: int) -> None:
        _check(lib().sllm_kv_cache_set_length(self.handle, n))

    def data(self, layer: int) -> tuple[int, int]:
        k, v = C.c_void_p(), C.c_void_p()
        _check(lib().sllm_kv_cache_data(self.handle, layer, C.byref(k), C.byref(v)))
        return k.value, v.value


def attention_dev(kv: KVCache, layer: int, params: AttnParams, q_ptr: int, k_ptr: int, v_ptr: int, seq_len: int,
                  start_pos: int, out_ptr: int, stream: int = 0) -> None:
    """forwardBlock's attention section for one layer (model_f32.go:398-466):
    bias, QK norm, RoPE at start_pos, KV append, causal GQA attention, merged
    heads into out (seq_len x n_heads*d_k)."""
    _check(lib().sllm_attention_dev(kv.handle, layer, C.byref(params), C.c_void_p(q_ptr), C.c_void_p(k_ptr),
                                    C.c_void_p(v_ptr), seq_len, start_pos, C.c_void_p(out_ptr),
                                    C.c_void_p(stream)))


def attention_noalloc_dev(kv: KVCache, layer: int, params: AttnParams, q_ptr: int, k_ptr: int, v_ptr: int,
                          seq_len: int, start_pos: int, out_ptr: int, stream: int = 0) -> None:
    """attention_dev with its scratch in the library's static device array:
    allocates nothing (usable under graph capture without a warm-up call);
    calls that overlap on one GPU race."""
    _check(lib().sllm_attention_noalloc_dev(kv.handle, layer, C.byref(params), C.c_void_p(q_ptr),
                                            C.c_void_p(k_ptr), C.c_void_p(v_ptr), seq_len, start_pos,
                                            C.c_void_p(out_ptr), C.c_void_p(stream)))


def workspace_reserve(stream: int, nbytes: int) -> None:
    """Grow the stream's device workspace to at least nbytes now (before a graph capture)."""
    _check(lib().sllm_workspace_reserve(C.c_void_p(stream), int(nbytes)))


def argmax_f32_dev(v_ptr: int, n: int, stream: int = 0) -> int:
    out = C.c_int()
    _check(lib().sllm_argmax_dev(C.c_void_p(v_ptr), n, C.byref(out), C.c_void_p(stream)))
    return out.value


def debug_quantize_act(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    K = x.shape[-1]
    rows = x.size // K
    xq = np.empty(x.shape, np.int8)
    xs = np.empty(x.shape[:-1] + (K // 32,), np.float32)
    sx = np.empty(x.shape[:-1] + (K // 32,), np.int32)
    _check(lib().sllm_debug_quantize_act(_ptr(x), rows, K, _ptr(xq), _ptr(xs), _ptr(sx)))
    return xq, xs, sx


def debug_block_dots(w: DeviceWeight, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, w.cols)
    M = x.shape[0]
    shape = (M, w.rows, w.groups, 2) if w.qtype == "q5k1" else (M, w.rows, w.groups)
    out = np.empty(shape, np.int32)
    _check(lib().sllm_debug_block_dots(w.handle, _ptr(x), M, w.cols, _ptr(out)))
    return out


def debug_gemm_block_dots(w: DeviceWeight, x: np.ndarray, row0: int = 0, n_rows: int | None = None) -> np.ndarray:
    """The int32 block dots the prefill GEMM's matrix cores produce for weight
    rows [row0, row0 + n_rows): [M][n_rows][groups] (x2 for Q5K1)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, w.cols)
    M = x.shape[0]
    n = w.rows - row0 if n_rows is None else n_rows
    shape = (M, n, w.groups, 2) if w.qtype == "q5k1" else (M, n, w.groups)
    out = np.empty(shape, np.int32)
    _check(lib().sllm_debug_gemm_block_dots(w.handle, _ptr(x), M, w.cols, int(row0), int(n), _ptr(out)))
    return out
