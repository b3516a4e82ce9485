"""The host-buffer entry points' transport: outputs of at most 1 MiB per call
are written by the kernels straight into the call context's pinned bounce
buffer, larger ones are staged on the device and downloaded; the call waits
on a pinned completion word. Calls of both kinds alternate here (the bounce
buffer grows between them) and every output must be bit-identical to the
device-resident entry point on the same input."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import sllm_qmm as sq

from _helpers import make_raw, make_x

pytestmark = pytest.mark.gpu


def _dev_matmul(w, x: np.ndarray, M: int, K: int) -> np.ndarray:
    torch.cuda.set_device(0)
    s = torch.cuda.current_stream()
    xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32).reshape(-1)).cuda()
    yd = torch.empty(M * w.rows, device="cuda")
    sq.matmul_dev(w, xd.data_ptr(), M, K, yd.data_ptr(), s.cuda_stream)
    torch.cuda.synchronize()
    return yd.cpu().numpy()


def test_direct_and_staged_outputs_alternate():
    K = 1024
    small = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", make_raw("q4_1", 768, K, seed=5), K // 32, 768, K))
    big = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", make_raw("q8", 6144, K, seed=6), K // 32, 6144, K))
    # (weight, rows): outputs 3 KB, 1.5 MB (GEMM, staged), 9 KB, 24 KB, 1.5 MB again
    calls = [(small, 1), (big, 64), (small, 3), (big, 1), (big, 64), (small, 1)]
    for rnd in range(2):
        for i, (w, M) in enumerate(calls):
            x = make_x(M, K, seed=100 * rnd + i)
            got, rows, cols = sq.model_matmul_quant_into_f32(w, x, M, K)
            assert (rows, cols) == (M, w.rows)
            want = _dev_matmul(w, x, M, K)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"round {rnd} call {i} M={M} N={w.rows}"


def test_host_calls_with_changing_inputs_see_each_call_s_data():
    # one small weight called back to back with a new input each time: every
    # call must return its own input's result (no stale bounce-buffer data)
    K, N = 512, 256
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q4", make_raw("q4", N, K, seed=9), K // 32, N, K))
    xs = [make_x(1, K, seed=s) for s in range(40)]
    wants = [_dev_matmul(w, x, 1, K) for x in xs]
    dst = np.empty(N, np.float32)
    for x, want in zip(xs, wants):
        got = sq.model_matmul_row_quant_into_f32(w, x.reshape(-1), dst)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # the argmax entry point through the same transport
    for x, want in zip(xs[:8], wants[:8]):
        assert sq.matmul_argmax(w, x.reshape(-1)) == int(np.argmax(want))


def test_direct_and_uploaded_inputs_alternate():
    # inputs of at most 64 KiB are read by the kernels from the pinned bounce
    # buffer, larger ones are uploaded first: 16 rows of 1024 floats are the
    # largest direct input, 17 rows go through the upload
    K = 1024
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", make_raw("q8", 256, K, seed=11), K // 32, 256, K))
    for rnd in range(2):
        for i, M in enumerate((16, 17, 1, 17, 16, 2)):
            x = make_x(M, K, seed=1000 + 10 * rnd + i)
            got, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
            want = _dev_matmul(w, x, M, K)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"round {rnd} M={M}"


def test_multi_and_swiglu_host_entries_with_changing_inputs():
    K, N = 1024, 512
    wg = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", make_raw("q4_1", N, K, seed=21), K // 32, N, K))
    wu = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", make_raw("q4_1", N, K, seed=22), K // 32, N, K))
    for s in range(6):
        x = make_x(1, K, seed=200 + s)
        g, u = sq.model_matmul_multi_quant_into_f32([wg, wu], x, 1, K)
        assert np.array_equal(g.view(np.uint32), _dev_matmul(wg, x, 1, K).view(np.uint32))
        assert np.array_equal(u.view(np.uint32), _dev_matmul(wu, x, 1, K).view(np.uint32))
        h = sq.model_matmul_swiglu_into_f32(wg, wu, x, 1, K)
        torch.cuda.set_device(0)
        st = torch.cuda.current_stream()
        xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32).reshape(-1)).cuda()
        hd = torch.empty(N, device="cuda")
        sq.matmul_swiglu_dev(wg, wu, xd.data_ptr(), 1, K, hd.data_ptr(), stream=st.cuda_stream)
        torch.cuda.synchronize()
        assert np.array_equal(h.view(np.uint32), hd.cpu().numpy().view(np.uint32))
