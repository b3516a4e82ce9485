"""GPU tests of the fused head GEMV + greedy argmax (outputLogits' head matmul,
model_f32.go:521, then argmaxF32, float32_ops.go:812-822): the index is the
first maximum of the logits the same launch computes, NaN logits never win,
and a NaN at index 0 gives 0, as in the reference's loop."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq

from _helpers import make_raw, make_x, term_abs_sum

pytestmark = pytest.mark.gpu

N, K = 5000, 512


def first_max(v: np.ndarray) -> int:
    # argmaxF32 restated over the values the GPU produced
    best, bv = 0, v[0]
    for i in range(1, v.size):
        if v[i] > bv:
            best, bv = i, v[i]
    return best


def run(w, x, stream=None):
    s = stream or torch.cuda.current_stream()
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    logits = torch.empty(w.rows, device="cuda")
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    sq.matmul_argmax_dev(w, xd.data_ptr(), idx.data_ptr(), logits.data_ptr(), s.cuda_stream)
    s.synchronize()
    return int(idx.item()), logits.cpu().numpy()


def q8_weight(raw):
    return sq.DeviceWeight.from_quant(sq.QuantWeight("q8", raw, K // 32, N, K))


def test_argmax_is_first_max_of_its_logits_and_matches_oracle():
    raw = make_raw("q8", N, K, seed=11)
    w = q8_weight(raw)
    for seed in range(5):  # repeated launches: the scratch resets itself
        x = make_x(1, K, seed=100 + seed)[0]
        idx, logits = run(w, x)
        single = torch.empty(N, device="cuda")
        xd = torch.from_numpy(x).cuda()
        sq.matmul_dev(w, xd.data_ptr(), 1, K, single.data_ptr())
        torch.cuda.synchronize()
        assert np.array_equal(logits.view(np.uint32), single.cpu().numpy().view(np.uint32))
        assert idx == first_max(logits)
        ref = oracle.matmul("q8", raw, N, x[None])[0].astype(np.float64)
        bound = 1e-5 * term_abs_sum("q8", raw, N, x[None])[0]
        top = np.argsort(-ref)[:2]
        if ref[top[0]] - ref[top[1]] > bound[top[0]] + bound[top[1]]:
            assert idx == oracle.argmax(ref.astype(np.float32))


def _with_rows_copied(raw, src, dsts):
    r = raw.reshape(N, -1).copy()
    for d in dsts:
        r[d] = r[src]
    return r.reshape(-1)


def test_ties_go_to_the_lowest_index():
    raw = make_raw("q8", N, K, seed=12)
    x = make_x(1, K, seed=13)[0]
    _, logits = run(q8_weight(raw), x)
    top = int(np.argmax(logits))
    raw2 = _with_rows_copied(raw, top, [37, 4321])
    idx, logits2 = run(q8_weight(raw2), x)
    assert logits2[37] == logits2[top] == logits2[4321]
    assert idx == min(37, top)


def _set_scale(raw, row, bits):
    r = raw.reshape(N, -1).copy()
    r[row, 0], r[row, 1] = bits & 0xFF, bits >> 8   # first block's f16 d
    return r.reshape(-1)


def test_nan_rules():
    raw = make_raw("q8", N, K, seed=14)
    x = make_x(1, K, seed=15)[0]
    base, logits = run(q8_weight(raw), x)
    # a NaN logit elsewhere never wins
    raw_nan = _set_scale(raw, (base + 7) % N, 0x7E00)
    idx, lg = run(q8_weight(raw_nan), x)
    assert np.isnan(lg[(base + 7) % N]) and idx == base
    # NaN at index 0: nothing compares greater, the answer is 0
    raw_nan0 = _set_scale(raw, 0, 0x7E00)
    idx0, lg0 = run(q8_weight(raw_nan0), x)
    assert np.isnan(lg0[0]) and idx0 == 0


def test_two_streams_and_host_entry():
    raw = make_raw("q8", N, K, seed=16)
    w = q8_weight(raw)
    x1, x2 = make_x(1, K, seed=17)[0], make_x(1, K, seed=18)[0]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    i1, l1 = run(w, x1, s1)
    i2, l2 = run(w, x2, s2)
    assert i1 == first_max(l1) and i2 == first_max(l2)
    assert sq.matmul_argmax(w, x1) == i1


def test_graph_replays_reset_the_scratch():
    raw = make_raw("q8", N, K, seed=19)
    w = q8_weight(raw)
    s = torch.cuda.Stream()
    xd = torch.from_numpy(make_x(1, K, seed=20)).cuda()
    idx = torch.zeros(1, dtype=torch.int32, device="cuda")
    with torch.cuda.stream(s):
        # the first call on a stream allocates its scratch: before capture
        sq.matmul_argmax_dev(w, xd.data_ptr(), idx.data_ptr(), 0, s.cuda_stream)
    s.synchronize()
    want = int(idx.item())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sq.matmul_argmax_dev(w, xd.data_ptr(), idx.data_ptr(), 0, s.cuda_stream)
    for rep in range(4):
        idx.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        assert int(idx.item()) == want, rep
    xd.copy_(torch.from_numpy(make_x(1, K, seed=21)).cuda())
    g.replay()
    torch.cuda.synchronize()
    _, logits = run(w, xd.cpu().numpy()[0])
    assert int(idx.item()) == first_max(logits)
