"""GEMV launches captured in a HIP graph (torch.cuda.CUDAGraph) replay to the
same bits as the eager launches, replay after replay, with eager work and
input changes in between (the decode loop's use of the library)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

import sllm_qmm as sq

from _helpers import make_raw, make_x

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager():
    torch.cuda.set_device(0)
    K = 1024
    specs = [("q4_1", 512), ("q4_1", 128), ("q4_1", 128), ("q8", 256), ("q5", 96), ("q5k1", 64)]
    ws = [sq.DeviceWeight.from_quant(sq.QuantWeight(q, make_raw(q, n, K, seed=i), K // 32, n, K))
          for i, (q, n) in enumerate(specs)]
    x = torch.from_numpy(make_x(1, K, seed=5)).cuda()
    outs = [torch.empty(w.rows, device="cuda") for w in ws]
    P = lambda t: t.data_ptr()

    def seq(stream):
        sq.matmul_multi_dev(ws[:3], P(x), 1, K, [P(o) for o in outs[:3]], stream)
        for w, o in zip(ws[3:], outs[3:]):
            sq.matmul_dev(w, P(x), 1, K, P(o), stream)

    def eager():
        seq(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        return [o.clone() for o in outs]

    want = eager()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        seq(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for i, (o, w) in enumerate(zip(outs, want)):
            assert torch.equal(o.view(torch.int32), w.view(torch.int32)), f"replay {rep}, weight {i}"
        eager()  # eager work between replays

    # the graph reads x's current contents: new input, same as eager on it
    x.copy_(torch.from_numpy(make_x(1, K, seed=6)).cuda())
    want2 = eager()
    assert not torch.equal(want2[0], want[0])
    g.replay()
    torch.cuda.synchronize()
    for o, w in zip(outs, want2):
        assert torch.equal(o.view(torch.int32), w.view(torch.int32))


def test_workspace_growth_keeps_captured_graphs_valid():
    # A decode step captured on a stream (its attention keeps the rotated q
    # rows in the stream's workspace), then a large prefill on the same
    # stream grows that workspace: the old buffer must stay valid, so the
    # graph still replays to the eager result.
    from test_gpu_attention import Model
    from sllm_qmm import synth
    rng = np.random.default_rng(3)
    H, KV, DK, K = 8, 2, 128, 1024
    m = Model(H, KV, DK, 64, rng, base=500000.0)
    kv = sq.KVCache(1, KV, DK, 256)
    kv.set_length(100)
    q = torch.from_numpy(rng.normal(size=H * DK).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.normal(size=KV * DK).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.normal(size=KV * DK).astype(np.float32)).cuda()
    att = torch.empty(H * DK, device="cuda")
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q4_1", make_raw("q4_1", 512, K, seed=1), K // 32, 512, K))
    y = torch.empty(512, device="cuda")
    P = lambda t: t.data_ptr()
    s = torch.cuda.Stream()

    def step(sp):
        kv.set_length(100)
        sq.attention_dev(kv, 0, m.params, P(q), P(k), P(v), 1, 100, P(att), sp)
        sq.matmul_dev(w, P(att), 1, K, P(y), sp)

    with torch.cuda.stream(s):
        step(s.cuda_stream)  # eager: the workspace is allocated here, before the capture
    s.synchronize()
    want = (att.clone(), y.clone())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        step(s.cuda_stream)
    # prefill on the same stream: M = 512, K = 14336 needs far more workspace
    F = 14336
    big = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(5, 256, F), 256, F)
    xb = torch.from_numpy(make_x(512, F, seed=2)).cuda()
    yb = torch.empty(512 * 256, device="cuda")
    with torch.cuda.stream(s):
        sq.matmul_dev(big, P(xb), 512, F, P(yb), s.cuda_stream)
    s.synchronize()
    for rep in range(3):
        att.fill_(float("nan"))
        y.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(att.view(torch.int32), want[0].view(torch.int32)), rep
        assert torch.equal(y.view(torch.int32), want[1].view(torch.int32)), rep
        with torch.cuda.stream(s):
            sq.matmul_dev(big, P(xb), 512, F, P(yb), s.cuda_stream)  # eager work in between
        s.synchronize()
    kv.close()


def test_workspace_growth_under_capture_is_an_error_and_reserve_avoids_it():
    from sllm_qmm import synth
    F, M = 8192, 256
    big = sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(6, 128, F), 128, F)
    xb = torch.from_numpy(make_x(M, F, seed=3)).cuda()
    yb = torch.empty(M * 128, device="cuda")
    small = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", make_raw("q8", 64, 256, seed=2), 8, 64, 256))
    xs = torch.from_numpy(make_x(1, 256, seed=4)).cuda()
    ys = torch.empty(64, device="cuda")
    P = lambda t: t.data_ptr()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    err = None
    with torch.cuda.graph(g, stream=s):
        sq.matmul_dev(small, P(xs), 1, 256, P(ys), s.cuda_stream)  # no workspace
        try:
            sq.matmul_dev(big, P(xb), M, F, P(yb), s.cuda_stream)  # would allocate: refused
        except sq.SllmError as e:
            err = e
    assert err is not None and err.status == 1 and "sllm_workspace_reserve" in str(err)
    del g
    # reserved before the capture, the same call captures and replays to the eager result
    s2 = torch.cuda.Stream()
    sq.workspace_reserve(s2.cuda_stream, 64 << 20)
    with torch.cuda.stream(s2):
        sq.matmul_dev(big, P(xb), M, F, P(yb), s2.cuda_stream)
    s2.synchronize()
    want = yb.clone()
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s2):
        sq.matmul_dev(big, P(xb), M, F, P(yb), s2.cuda_stream)
    for rep in range(3):
        yb.fill_(float("nan"))
        g2.replay()
        torch.cuda.synchronize()
        assert torch.equal(yb.view(torch.int32), want.view(torch.int32)), rep
