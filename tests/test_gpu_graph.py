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
