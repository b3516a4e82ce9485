"""Writes the small golden fixtures in this directory (run from the repository
root: ``python tests/golden/make_golden.py``).

The reference (Go) cannot run here, so the expected outputs come from this
repository's CPU restatement of it (oracle/refcpu.c), which the oracle tests
pin independently (closed forms, brute force, the reference tests' own
vectors). The fixtures freeze those outputs for inputs built the way the
reference's tests build theirs - the LCG activation generator of
kquant_kernels_test.go:43-48 and the pattern rows of q8q8_test.go:24-43 - so
the GPU path can be checked against data that needs no oracle at run time,
and any later change to the oracle shows up as a fixture mismatch.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "scriptling-llm-lib_amd"))


def lcg_activations(n: int, seed: int = 12345) -> np.ndarray:
    """kquant_kernels_test.go:43-48: seed = seed*1664525 + 1013904223 (uint32);
    x = float32(int32(seed)) / float32(1<<31) - 0.5, all in float32."""
    out = np.empty(n, np.float32)
    s = np.uint32(seed)
    with np.errstate(over="ignore"):
        for i in range(n):
            s = np.uint32(s * np.uint32(1664525) + np.uint32(1013904223))
            out[i] = np.float32(np.int32(s.view(np.int32))) / np.float32(1 << 31) - np.float32(0.5)
    return out


def edge_rows(K: int) -> np.ndarray:
    """Rows that exercise the quantizer's special cases."""
    rows = np.zeros((6, K), np.float32)
    rows[1] = lcg_activations(K, 7) * np.float32(1e-39)     # denormal block maxima: 1/scale overflows
    rows[2] = lcg_activations(K, 8) * np.float32(1e30)
    rows[3] = lcg_activations(K, 9)
    rows[3, 5] = np.nan
    rows[3, 40] = np.inf
    rows[3, 77] = -np.inf
    rows[4, ::32] = np.float32(-2.5)                         # one nonzero per block: q = -127
    rows[5] = np.arange(K, dtype=np.float32) - K / 2
    return rows


def main() -> None:
    import oracle
    from sllm_qmm import synth

    sys.path.insert(0, os.path.dirname(HERE))
    from _helpers import term_abs_sum

    oracle.build()
    K, M = 512, 3
    x = lcg_activations(M * K).reshape(M, K)
    xe = edge_rows(K)
    xq, xs = oracle.quantize_act_q8(np.concatenate([x, xe]))
    np.savez_compressed(os.path.join(HERE, "act_q8.npz"), x=np.concatenate([x, xe]), xq=xq, xs=xs)

    specs = {"q8": 40, "q4": 40, "q4_1": 40, "q5": 40, "q5k1": 24}
    for qtype, N in specs.items():
        if qtype == "q8":
            raw = oracle.quantize_q8_rows_f32(synth.normal(100, N * K, 0.02).reshape(N, K))
        elif qtype == "q4":
            raw = synth.quantize_q4_0(synth.normal(101, N * K, 0.02))
        elif qtype == "q4_1":
            raw = synth.quantize_q4_1(synth.normal(102, N * K, 0.02))
        elif qtype == "q5":
            raw = synth.quantize_q5_0(synth.normal(103, N * K, 0.02))
        else:
            raw = oracle.convert_q5k_to_two_q41(synth.q5k_blocks(104, N, K), N, K)
        raw = np.asarray(raw, np.uint8)
        dots = oracle.block_dots(qtype, raw, N, K, x)
        dst = oracle.matmul(qtype, raw, N, x)
        # sum over blocks of |per-block term|: the scale of the fp32 reassociation bound
        tabs = term_abs_sum(qtype, raw, N, x)
        np.savez_compressed(os.path.join(HERE, f"matmul_{qtype}.npz"), raw=raw, N=N, K=K, x=x, dots=dots,
                            dst=dst, tabs=tabs)

    # load-time remaps / requantization: GGUF bytes -> the reference's Raw
    for t, seed in ((12, 200), (13, 201), (14, 202), (20, 203)):
        rows = 6
        src = synth.gguf_tensor(t, seed, rows, K)
        qtype, raw = oracle.load_weight(t, src, rows, K)
        np.savez_compressed(os.path.join(HERE, f"load_gguf{t}.npz"), src=src, rows=rows, cols=K,
                            qtype=np.array(qtype), raw=raw)
    wf = synth.normal(300, 8 * K, 0.02).reshape(8, K)
    wf[0, :32] = 0.0
    wf[1, 3] = np.float32(2.5) * np.abs(wf[1]).max()
    np.savez_compressed(os.path.join(HERE, "load_f32.npz"), w=wf, raw=np.asarray(oracle.quantize_q8_rows_f32(wf)))

    v = lcg_activations(1000, 42)
    v[[17, 400, 999]] = v.max() + np.float32(1.0)       # ties: lowest index wins
    v[[3, 600]] = np.nan                                  # NaN never wins the > compare
    np.savez_compressed(os.path.join(HERE, "argmax.npz"), v=v, want=oracle.argmax(v))
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
