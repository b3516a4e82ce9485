"""sllm_attention_noalloc_dev: the attention with its scratch in the
library's static device array (no allocation). Its outputs and cache
appends must equal sllm_attention_dev's bit for bit (same kernels), on two
calls in a row with the second smaller than the first; it must capture into
a HIP graph on a stream that was never used before; and a call that needs
more scratch than the array holds is refused before anything runs."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import sllm_qmm as sq

from test_gpu_attention import Model, dev_view

pytestmark = pytest.mark.gpu

H, KV, DK, HALF = 32, 8, 128, 64


def _fill(kv, rng, cap):
    ck = rng.normal(size=(KV, cap, DK)).astype(np.float32)
    cv = rng.normal(size=(KV, cap, DK)).astype(np.float32)
    kp, vp = kv.data(0)
    dev_view(kp, KV * cap * DK).copy_(torch.from_numpy(ck.reshape(-1)))
    dev_view(vp, KV * cap * DK).copy_(torch.from_numpy(cv.reshape(-1)))


def _cache(kv, cap):
    kp, vp = kv.data(0)
    return (dev_view(kp, KV * cap * DK).clone(), dev_view(vp, KV * cap * DK).clone())


def test_noalloc_equals_attention_dev_on_two_calls():
    rng = np.random.default_rng(7)
    m = Model(H, KV, DK, HALF, rng, base=500000.0)
    cap = 600
    a, b = sq.KVCache(1, KV, DK, cap), sq.KVCache(1, KV, DK, cap)
    _fill(a, np.random.default_rng(8), cap)
    _fill(b, np.random.default_rng(8), cap)
    P = lambda t: t.data_ptr()
    # first call: 5 rows against 400 cached positions (several splits); second,
    # smaller: one row against 40
    for seq, start in ((5, 400), (1, 40)):
        a.set_length(start)
        b.set_length(start)
        q = torch.from_numpy(rng.normal(size=(seq, H * DK)).astype(np.float32)).cuda()
        k = torch.from_numpy(rng.normal(size=(seq, KV * DK)).astype(np.float32)).cuda()
        v = torch.from_numpy(rng.normal(size=(seq, KV * DK)).astype(np.float32)).cuda()
        oa = torch.full((seq, H * DK), float("nan"), device="cuda")
        ob = torch.full((seq, H * DK), float("nan"), device="cuda")
        sq.attention_dev(a, 0, m.params, P(q), P(k), P(v), seq, start, P(oa))
        sq.attention_noalloc_dev(b, 0, m.params, P(q), P(k), P(v), seq, start, P(ob))
        torch.cuda.synchronize()
        assert a.length(0) == b.length(0) == start + seq
        assert torch.equal(oa.view(torch.int32), ob.view(torch.int32)), (seq, start)
        for x, y in zip(_cache(a, cap), _cache(b, cap)):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32)), (seq, start)
    a.close()
    b.close()


def test_noalloc_captures_on_a_fresh_stream():
    rng = np.random.default_rng(9)
    m = Model(H, KV, DK, HALF, rng, base=500000.0)
    cap = 300
    kv = sq.KVCache(1, KV, DK, cap)
    _fill(kv, np.random.default_rng(10), cap)
    P = lambda t: t.data_ptr()
    q = torch.from_numpy(rng.normal(size=(1, H * DK)).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.normal(size=(1, KV * DK)).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.normal(size=(1, KV * DK)).astype(np.float32)).cuda()
    out = torch.empty(H * DK, device="cuda")
    ref = torch.empty(H * DK, device="cuda")
    kv.set_length(200)
    sq.attention_dev(kv, 0, m.params, P(q), P(k), P(v), 1, 200, P(ref))  # eager, default stream
    torch.cuda.synchronize()
    s = torch.cuda.Stream()  # never used by the library before the capture
    kv.set_length(200)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        sq.attention_noalloc_dev(kv, 0, m.params, P(q), P(k), P(v), 1, 200, P(out), s.cuda_stream)
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), rep
        # eager work between replays (it appends at 200 again, the same row)
        kv.set_length(200)
        sq.attention_dev(kv, 0, m.params, P(q), P(k), P(v), 1, 200, P(ref))
        torch.cuda.synchronize()
    kv.close()


def test_noalloc_refuses_more_than_the_static_scratch():
    rng = np.random.default_rng(11)
    m = Model(H, KV, DK, HALF, rng)
    seq = 600  # q rows alone: 600 x 32 x 128 x 4 bytes = 9.8 MB > 8 MiB
    kv = sq.KVCache(1, KV, DK, seq + 1)
    x = torch.zeros(seq * H * DK, device="cuda")
    p = x.data_ptr()
    with pytest.raises(sq.SllmError) as e:
        sq.attention_noalloc_dev(kv, 0, m.params, p, p, p, seq, 0, p)
    assert e.value.status == 3 and "static scratch" in str(e.value)
    assert kv.length(0) == 0  # nothing ran
    kv.close()
