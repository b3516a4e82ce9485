"""The HIP path against the committed golden fixtures (tests/golden): no oracle
at run time. Integer results bit-exact; fp32 outputs within the reassociation
bound |got - want| <= 1e-5 * sum_g |term_g| stored with each fixture."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import sllm_qmm as sq

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_activation_quantizer_fixture():
    g = load("act_q8.npz")
    xq, xs, _ = sq.debug_quantize_act(g["x"])
    assert np.array_equal(xq, g["xq"])
    assert np.array_equal(xs.view(np.uint32), g["xs"].view(np.uint32))


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5", "q5k1"])
def test_matmul_fixture(qtype):
    g = load(f"matmul_{qtype}.npz")
    N, K = int(g["N"]), int(g["K"])
    x = g["x"]
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, g["raw"], K // 32, N, K))
    assert np.array_equal(sq.debug_block_dots(w, x), g["dots"])
    got, _, _ = sq.model_matmul_quant_into_f32(w, x, x.shape[0], K)
    err = np.abs(got.reshape(-1, N).astype(np.float64) - g["dst"])
    assert np.all(err <= 1e-5 * g["tabs"] + 1e-30)


@pytest.mark.parametrize("t", [12, 13, 14, 20])
def test_load_fixture(t):
    g = load(f"load_gguf{t}.npz")
    w = sq.load_weight_f32_direct(t, g["src"], int(g["rows"]), int(g["cols"]))
    assert w.qtype == str(g["qtype"])
    assert np.array_equal(w.export(), g["raw"])


def test_f32_and_argmax_fixtures():
    g = load("load_f32.npz")
    w = sq.quantize_q8_rows_f32(g["w"], *g["w"].shape)
    assert np.array_equal(w.export(), g["raw"])
    a = load("argmax.npz")
    v = torch.from_numpy(a["v"]).cuda()
    assert sq.argmax_f32_dev(v.data_ptr(), v.numel()) == int(a["want"])
