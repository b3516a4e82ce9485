"""GPU tests of the multi-weight entry points (one activation input, several
weights: forwardBlock's q/k/v and gate/up calls, model_f32.go:391-396 and
:479-482). Each weight's output must be bit-identical to its own single call
(same per-row lane split and summation order), and within the fp32 parity
bound of the oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq

from _helpers import assert_fp32_parity, make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu


def _weights(specs, K, seed):
    out = []
    for i, (qtype, N) in enumerate(specs):
        raw = make_raw(qtype, N, K, seed=seed + i)
        out.append((qtype, raw, N, sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))))
    return out


@pytest.mark.parametrize("specs", [
    [("q4_1", 512), ("q4_1", 128), ("q4_1", 128)],            # q/k/v-like, one launch
    [("q4_1", 1792), ("q4_1", 1792)],                         # gate/up-like
    [("q8", 300), ("q4_1", 96), ("q8", 33), ("q4", 64), ("q5", 40), ("q5k1", 70)],   # mixed formats
    [("q8", 64)] * 6,                                         # more than 4 of one format: two launches
])
@pytest.mark.parametrize("M", [1, 3, 64])
def test_multi_equals_single_calls(specs, M):
    K = 512
    ws = _weights(specs, K, seed=11 * M)
    x = make_x(M, K, seed=M)
    outs = sq.model_matmul_multi_quant_into_f32([w for *_, w in ws], x, M, K)
    for (qtype, raw, N, w), got in zip(ws, outs):
        single, _, _ = sq.model_matmul_quant_into_f32(w, x, M, K)
        assert np.array_equal(got.view(np.uint32), single.view(np.uint32)), f"{qtype} N={N} M={M}"
        ref = oracle.matmul(qtype, raw, N, x)
        assert_fp32_parity(got.reshape(M, N), ref, term_abs_sum(qtype, raw, N, x), f"multi {qtype} N={N} M={M}")


def test_multi_dev_llama_qkv_shapes():
    # the 8B q/k/v (Q4_K -> Q4_1) and gate/up shapes through the device entry point
    from sllm_qmm import synth
    H, KV, F = 4096, 1024, 14336
    torch.cuda.set_device(0)
    s = torch.cuda.current_stream()
    x = torch.from_numpy(make_x(1, H, seed=3)).cuda()
    for rows in ([H, KV, KV], [F, F]):
        ws = [sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(40 + i, n, H), n, H)
              for i, n in enumerate(rows)]
        fused = [torch.empty(n, device="cuda") for n in rows]
        sq.matmul_multi_dev(ws, x.data_ptr(), 1, H, [t.data_ptr() for t in fused], s.cuda_stream)
        for w, f in zip(ws, fused):
            one = torch.empty(w.rows, device="cuda")
            sq.matmul_dev(w, x.data_ptr(), 1, H, one.data_ptr(), s.cuda_stream)
            torch.cuda.synchronize()
            assert torch.equal(f.view(torch.int32), one.view(torch.int32)), f"rows {w.rows}"


def test_multi_errors():
    K = 64
    (_, _, _, a), (_, _, _, b) = _weights([("q8", 8), ("q4", 8)], K, seed=1)
    c = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", make_raw("q8", 8, 96, seed=2), 3, 8, 96))
    x = make_x(1, K, seed=1)
    with pytest.raises(sq.SllmError) as e:
        sq.model_matmul_multi_quant_into_f32([a, c], x, 1, K)      # Cols mismatch
    assert e.value.status == 1
    with pytest.raises(sq.SllmError) as e:
        sq.model_matmul_multi_quant_into_f32([], x, 1, K)
    assert e.value.status == 1
