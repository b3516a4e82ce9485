"""The C ABI on the CPU: the library loads, exports every symbol the header
declares, and rejects bad arguments with status codes before touching a GPU."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import sllm_qmm as sq


def test_library_exports_every_declared_symbol():
    names = sq.exported_names()
    assert len(names) >= 15
    lib = sq.lib()
    for n in names:
        assert hasattr(lib, n), n
    # and nothing else under the sllm_ prefix is exported by accident
    out = subprocess.run(["nm", "-D", "--defined-only", sq.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.split() and l.split()[-1].startswith("sllm_")}
    assert exported == set(names)


def test_kernel_info_names_the_target():
    assert "gfx950" in sq.kernel_info()


def _status(fn, *args):
    return fn(*args)


def test_argument_errors_need_no_device():
    lib = sq.lib()
    raw = np.zeros(34 * 4, np.uint8)
    h = C.c_void_p()
    p = raw.ctypes.data
    assert lib.sllm_weight_from_quant(b"q9", p, raw.nbytes, 1, 4, 32, C.byref(h)) == 2      # unknown QType
    assert "q9" in lib.sllm_last_error().decode()
    assert lib.sllm_weight_from_quant(b"q8", p, raw.nbytes, 1, 4, 33, C.byref(h)) == 3      # cols % 32
    assert lib.sllm_weight_from_quant(b"q8", p, raw.nbytes, 2, 4, 32, C.byref(h)) == 1      # groups != cols/32
    assert lib.sllm_weight_from_quant(b"q8", p, 10, 1, 4, 32, C.byref(h)) == 1              # Raw too short
    assert lib.sllm_weight_from_quant(b"q8", None, 10, 1, 4, 32, C.byref(h)) == 1           # null Raw
    assert lib.sllm_weight_from_gguf(7, p, raw.nbytes, 4, 256, C.byref(h)) == 2             # Q5_1: dense in the reference
    assert lib.sllm_weight_from_gguf(10, p, raw.nbytes, 4, 128, C.byref(h)) == 3            # Q2_K needs cols % 256
    assert lib.sllm_weight_from_gguf(11, p, 16, 1, 256, C.byref(h)) == 1                    # Q3_K: too short
    assert lib.sllm_weight_from_gguf(12, p, raw.nbytes, 4, 128, C.byref(h)) == 3            # Q4_K needs cols % 256
    assert lib.sllm_weight_from_gguf(12, p, 16, 1, 256, C.byref(h)) == 1                    # too short
    assert lib.sllm_matmul_quant_into_f32(None, p, 1, 32, p) == 1
    assert lib.sllm_set_param(b"no_such_knob", 3) == 1
    assert lib.sllm_matmul_multi_quant_into_f32(None, 1, p, 1, 32, None) == 1
    hs = (C.c_void_p * 1)(None)
    ds = (C.c_void_p * 1)(p)
    assert lib.sllm_matmul_multi_quant_into_f32(hs, 0, p, 1, 32, ds) == 1                 # count 0
    assert lib.sllm_matmul_multi_dev(hs, 1, p, 1, 32, ds, None) == 1                        # null weight
    assert lib.sllm_matmul_swiglu_dev(None, None, p, 1, 32, p, None, None, None) == 1      # null weights
    assert lib.sllm_matmul_swiglu_into_f32(None, None, p, 1, 32, p) == 1
    assert lib.sllm_matmul_argmax(None, p, C.byref(C.c_int())) == 1
    assert lib.sllm_matmul_argmax_dev(None, p, 32, None, p, None) == 1
    assert lib.sllm_rmsnorm_matmul_argmax_dev(None, p, p, C.c_float(1e-5), 32, None, p, None) == 1
    assert lib.sllm_rmsnorm_matmul_swiglu_dev(None, None, p, p, C.c_float(1e-5), 1, 32, p, None) == 1
    assert lib.sllm_matmul_add_dev(None, p, 1, 32, p, None) == 1
    kv = C.c_void_p()
    assert lib.sllm_kv_cache_create(0, 8, 128, 16, C.byref(kv)) == 1                      # no layers
    assert lib.sllm_kv_cache_create(2, 8, 130, 16, C.byref(kv)) == 3                      # d_k % 4
    assert lib.sllm_kv_cache_create(2, 8, 512, 16, C.byref(kv)) == 3                      # d_k > 256
    assert lib.sllm_kv_cache_create(1, 1, 256, 1 << 22, C.byref(kv)) == 3                  # 4 GiB per kv head
    assert lib.sllm_kv_cache_length(None, 0, C.byref(C.c_int())) == 1
    assert lib.sllm_kv_cache_set_length(None, 0) == 1
    prm = sq.AttnParams(n_heads=32, n_kv_heads=8, d_k=128, rope_half_dim=64)
    assert lib.sllm_attention_dev(None, 0, C.byref(prm), p, p, p, 1, 0, p, None) == 1
    lib.sllm_kv_cache_destroy(None)                                                        # no-op


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="checks the no-GPU error path")
def test_no_gpu_is_a_device_error_not_a_fallback():
    lib = sq.lib()
    assert lib.sllm_init() == 4
    assert "gfx950" in lib.sllm_last_error().decode() or "device" in lib.sllm_last_error().decode()
    raw = np.zeros(34, np.uint8)
    h = C.c_void_p()
    assert lib.sllm_weight_from_quant(b"q8", raw.ctypes.data, 34, 1, 1, 32, C.byref(h)) == 4
    with pytest.raises(sq.SllmError) as e:
        sq.DeviceWeight.from_quant(sq.QuantWeight("q8", raw, 1, 1, 32))
    assert e.value.status == 4


def test_python_host_mirror_names():
    # the Go entry points this path replaces, mirrored by the host module
    for name in ("QuantWeight", "load_weight_f32_direct", "quantize_q8_rows_f32",
                 "model_matmul_quant_into_f32", "model_matmul_row_quant_into_f32", "argmax_f32_dev",
                 "model_matmul_multi_quant_into_f32", "model_matmul_swiglu_into_f32", "matmul_argmax",
                 "KVCache", "attention_dev", "matmul_add_dev"):
        assert hasattr(sq, name)
