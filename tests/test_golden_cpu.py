"""The committed golden fixtures (tests/golden, written by make_golden.py from
the oracle) are reproduced by the oracle today, and the reference's LCG
activation generator is restated correctly."""
from __future__ import annotations

import os
import struct
import sys

import numpy as np
import pytest

import oracle
from sllm_qmm import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)
from make_golden import edge_rows, lcg_activations  # noqa: E402


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_lcg_matches_integer_arithmetic():
    # kquant_kernels_test.go:43-48 with Python integers and IEEE single rounding via struct
    s = 12345
    want = []
    for _ in range(200):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        i32 = s - (1 << 32) if s >= (1 << 31) else s
        f = struct.unpack("<f", struct.pack("<f", float(i32)))[0]     # float32(int32)
        f = struct.unpack("<f", struct.pack("<f", f / float(1 << 31)))[0]
        f = struct.unpack("<f", struct.pack("<f", f - 0.5))[0]
        want.append(f)
    assert np.array_equal(lcg_activations(200), np.array(want, np.float32))


def test_activation_fixture():
    g = load("act_q8.npz")
    xq, xs = oracle.quantize_act_q8(g["x"])
    assert np.array_equal(xq, g["xq"]) and np.array_equal(xs.view(np.uint32), g["xs"].view(np.uint32))


@pytest.mark.parametrize("qtype", ["q8", "q4", "q4_1", "q5", "q5k1"])
def test_matmul_fixture(qtype):
    g = load(f"matmul_{qtype}.npz")
    N, K = int(g["N"]), int(g["K"])
    assert np.array_equal(oracle.block_dots(qtype, g["raw"], N, K, g["x"]), g["dots"])
    assert np.array_equal(oracle.matmul(qtype, g["raw"], N, g["x"]).view(np.uint32), g["dst"].view(np.uint32))


@pytest.mark.parametrize("t", [12, 13, 14, 20])
def test_load_fixture(t):
    g = load(f"load_gguf{t}.npz")
    qtype, raw = oracle.load_weight(t, g["src"], int(g["rows"]), int(g["cols"]))
    assert qtype == str(g["qtype"]) and np.array_equal(raw, g["raw"])
    assert np.array_equal(synth.gguf_tensor(t, {12: 200, 13: 201, 14: 202, 20: 203}[t], 6, 512), g["src"])


def test_f32_and_argmax_fixtures():
    g = load("load_f32.npz")
    assert np.array_equal(np.asarray(oracle.quantize_q8_rows_f32(g["w"])), g["raw"])
    a = load("argmax.npz")
    assert oracle.argmax(a["v"]) == int(a["want"]) == 17


def test_edge_rows_are_the_committed_inputs():
    g = load("act_q8.npz")
    assert np.array_equal(g["x"][3:].view(np.uint32), edge_rows(512).view(np.uint32))
