"""BASELINE config C5 (the decode step of a Llama-3-8B-shaped Q4_K_M model)
as a teacher-forced parity harness: two full-width layers and the full Q6_K
head, eight greedy tokens from an empty cache and two at cache positions 2046
and 2047 (the cache pre-filled with 2046 seeded rows, the last position of the
2048 context bench.py's decode step reports), through the device entry points
bench.py's decode step uses (forwardBlock model_f32.go:382-500, outputLogits :502-527, the
greedy loop :643-652). After every launch the GPU's output is compared with
the oracle applied to the GPU's own inputs to that launch (teacher forcing),
so each check carries only that launch's reassociation bound:

* RMSNorm + q/k/v: oracle.rmsnorm (the library's sum-of-squares order, which
  yields the GEMV's normed row bit for bit) then oracle.matmul, 1e-5 of
  sum|terms|;
* attention: oracle.attention_layer on the GPU's q/k/v and the GPU's cache
  rows before the call, the bound of tests/test_gpu_attention.py;
* o + residual, down + residual: x + oracle.matmul(...), 1e-5 of sum|terms|
  plus the rounding of the one float32 add;
* RMSNorm + gate/up + SwiGLU: oracle.swiglu of the oracle's gate / up, the
  bound of tests/test_gpu_swiglu.py;
* RMSNorm + head + argmax: logits 1e-5 of sum|terms|; the token is the first
  maximum of the launch's own logits, and the oracle's argmax wherever the
  top two logits are further apart than their bounds.
The next token's embedding row is the GPU token's (synthetic fp32 table
rows ~N(0, 0.02^2), one per token id)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq
from sllm_qmm import synth

from _helpers import REL_TOL, assert_fp32_parity, term_abs_sum
from test_gpu_attention import dev_view, out_bound

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

H, F, KVH, NH, DK, V = 4096, 14336, 8, 32, 128, 128256
L, T = 2, 8
EPS = 1e-5
U = 2.0 ** -24


class _AttnModel:
    """What out_bound needs of a model (no bias, no QK norm)."""

    def __init__(self):
        self.H, self.KV, self.dk = NH, KVH, DK


def _embed(tok: int) -> np.ndarray:
    return synth.normal(100000 + tok, H, 0.02)


def _load(t, raw, n, k):
    w = sq.load_weight_f32_direct(t, raw, n, k)
    qt, ref = oracle.load_weight(t, raw, n, k)
    assert w.qtype == qt and np.array_equal(w.export(), ref)
    return w, ref


def _close(got, ref, bound, what):
    assert_fp32_parity(np.asarray(got).reshape(ref.shape), ref, bound, what)


def _residual_check(x_in, got, wraw, qtype, n, inp, what):
    """got == x_in + matmul(inp) with one float32 add, within the matmul's
    bound plus that add's rounding."""
    ref = oracle.matmul(qtype, wraw, n, inp[None])[0]
    want = (x_in.astype(np.float32) + ref).astype(np.float64)
    bound = REL_TOL * term_abs_sum(qtype, wraw, n, inp[None])[0] + 2 * U * np.abs(want) + 1e-30
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), (what, float((err / bound).max()))


def _run_c5(start: int, ntok: int) -> None:
    """ntok teacher-forced greedy tokens at cache positions start .. start + ntok - 1;
    rows [0, start) of every layer's cache hold seeded K ~ N(0, 0.5^2), V ~ N(0, 1)."""
    torch.cuda.set_device(0)
    mk = _load
    layers = []
    for li in range(L):
        s = 300 + 10 * li
        layers.append({
            "q": mk(12, synth.q4k_blocks(s, H, H), H, H),
            "k": mk(12, synth.q4k_blocks(s + 1, KVH * DK, H), KVH * DK, H),
            "v": mk(12, synth.q4k_blocks(s + 2, KVH * DK, H), KVH * DK, H),
            "o": mk(12, synth.q4k_blocks(s + 3, H, H), H, H),
            "gate": mk(12, synth.q4k_blocks(s + 4, F, H), F, H),
            "up": mk(12, synth.q4k_blocks(s + 5, F, H), F, H),
            "down": mk(14, synth.q6k_blocks(s + 6, H, F), H, F),
            "n1": (synth.normal(s + 7, H, 0.1) + np.float32(1.0)).astype(np.float32),
            "n2": (synth.normal(s + 8, H, 0.1) + np.float32(1.0)).astype(np.float32),
        })
    head, hraw = mk(14, synth.q6k_blocks(399, V, H), V, H)
    nout = (synth.normal(398, H, 0.1) + np.float32(1.0)).astype(np.float32)
    half = DK // 2
    freqs = np.array([1.0 / math.pow(500000.0, 2.0 * i / DK) for i in range(half)], np.float32)

    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    P = lambda t: t.data_ptr()
    fr = dev(freqs)
    prm = sq.AttnParams(n_heads=NH, n_kv_heads=KVH, d_k=DK, rope_half_dim=half, rope_freqs=P(fr), norm_eps=EPS)
    for lw in layers:
        lw["n1d"], lw["n2d"] = dev(lw["n1"]), dev(lw["n2"])
    noutd = dev(nout)
    cap = start + ntok + 4
    kvc = sq.KVCache(L, KVH, DK, cap)
    if start:
        rng = np.random.default_rng(4242)
        for li in range(L):
            kp, vp = kvc.data(li)
            kc = np.zeros((KVH, cap, DK), np.float32)
            vc = np.zeros((KVH, cap, DK), np.float32)
            kc[:, :start] = rng.normal(0, 0.5, (KVH, start, DK))
            vc[:, :start] = rng.normal(0, 1.0, (KVH, start, DK))
            dev_view(kp, KVH * cap * DK).copy_(torch.from_numpy(kc.reshape(-1)))
            dev_view(vp, KVH * cap * DK).copy_(torch.from_numpy(vc.reshape(-1)))
        torch.cuda.synchronize()
        kvc.set_length(start)
    x = torch.empty(H, device="cuda")
    q, k, v = torch.empty(H, device="cuda"), torch.empty(KVH * DK, device="cuda"), torch.empty(KVH * DK, device="cuda")
    att, h = torch.empty(H, device="cuda"), torch.empty(F, device="cuda")
    logits = torch.empty(V, device="cuda")
    tokd = torch.zeros(1, dtype=torch.int32, device="cuda")
    sp = torch.cuda.current_stream().cuda_stream
    host = lambda t: t.cpu().numpy().copy()

    tok, tokens = 1, []
    for pos in range(start, start + ntok):
        x.copy_(dev(_embed(tok)))
        for li, lw in enumerate(layers):
            (wq, rq), (wk, rk), (wv, rv) = lw["q"], lw["k"], lw["v"]
            x0 = host(x)
            sq.rmsnorm_matmul_multi_dev([wq, wk, wv], P(x), P(lw["n1d"]), EPS, 1, H, [P(q), P(k), P(v)], sp)
            normed = oracle.rmsnorm(x0[None], lw["n1"], EPS, lib_order=True)
            for got, raw, n, name in ((q, rq, H, "q"), (k, rk, KVH * DK, "k"), (v, rv, KVH * DK, "v")):
                _close(host(got)[None], oracle.matmul("q4_1", raw, n, normed), term_abs_sum("q4_1", raw, n, normed),
                       f"pos {pos} layer {li} {name}")
            # attention on the GPU's q / k / v and the GPU's cache before the call
            kp, vp = kvc.data(li)
            ck0 = dev_view(kp, KVH * cap * DK).cpu().numpy().reshape(KVH, cap, DK).copy()
            cv0 = dev_view(vp, KVH * cap * DK).cpu().numpy().reshape(KVH, cap, DK).copy()
            qh, kh, vh = host(q), host(k), host(v)
            sq.attention_dev(kvc, li, prm, P(q), P(k), P(v), 1, pos, P(att), sp)
            want, wk_, wv_, qrot = oracle.attention_layer(qh[None], kh[None], vh[None], NH, KVH, DK, ck0, cv0, pos,
                                                          pos, freqs, half, eps=EPS, lib_norm=True,
                                                          return_q_rot=True)
            got_att = host(att)
            bound = out_bound(_AttnModel(), qrot, wk_, wv_, pos, 1)
            err = np.abs(got_att[None].astype(np.float64) - want)
            assert np.all(err <= bound), (pos, li, "attention", float((err / bound).max()))
            # o + residual
            sq.matmul_add_dev(lw["o"][0], P(att), 1, H, P(x), sp)
            x1 = host(x)
            _residual_check(x0, x1, lw["o"][1], "q4_1", H, got_att, f"pos {pos} layer {li} o + residual")
            # RMSNorm + gate / up + SwiGLU
            sq.rmsnorm_matmul_swiglu_dev(lw["gate"][0], lw["up"][0], P(x), P(lw["n2d"]), EPS, 1, H, P(h), sp)
            n2 = oracle.rmsnorm(x1[None], lw["n2"], EPS, lib_order=True)
            gr = oracle.matmul("q4_1", lw["gate"][1], F, n2)[0].astype(np.float64)
            ur = oracle.matmul("q4_1", lw["up"][1], F, n2)[0].astype(np.float64)
            tg = term_abs_sum("q4_1", lw["gate"][1], F, n2)[0]
            tu = term_abs_sum("q4_1", lw["up"][1], F, n2)[0]
            href = oracle.swiglu(gr.astype(np.float32), ur.astype(np.float32)).astype(np.float64)
            hb = REL_TOL * (1.1 * tg * np.abs(ur) + tu * np.abs(gr)) + 1e-6 * np.abs(href) + 1e-30
            got_h = host(h)
            assert np.all(np.abs(got_h.astype(np.float64) - href) <= hb), (pos, li, "swiglu")
            # down + residual
            sq.matmul_add_dev(lw["down"][0], P(h), 1, F, P(x), sp)
            _residual_check(x1, host(x), lw["down"][1], "q8", H, got_h, f"pos {pos} layer {li} down + residual")
        # output RMSNorm + head + greedy argmax
        xf = host(x)
        sq.rmsnorm_matmul_argmax_dev(head, P(x), P(noutd), EPS, P(tokd), P(logits), sp)
        lg = host(logits)
        t = int(tokd.item())
        assert t == int(np.argmax(lg)), "token is not the first maximum of its logits"
        nf = oracle.rmsnorm(xf[None], nout, EPS, lib_order=True)
        ref = oracle.matmul("q8", hraw, V, nf)[0]
        hbound = term_abs_sum("q8", hraw, V, nf)[0]
        _close(lg[None], ref[None], hbound[None], f"pos {pos} head")
        top = np.argsort(-ref.astype(np.float64))[:2]
        if ref[top[0]] - ref[top[1]] > REL_TOL * (hbound[top[0]] + hbound[top[1]]):
            assert t == oracle.argmax(ref), (pos, t, oracle.argmax(ref))
        tokens.append(t)
        tok = t
        assert kvc.length(0) == kvc.length(L - 1) == pos + 1
    print(f"C5 teacher-forced greedy tokens at positions {start}..{start + ntok - 1}: {tokens}")
    kvc.close()


def test_c5_teacher_forced_decode():
    _run_c5(0, T)


def test_c5_teacher_forced_decode_kv2047():
    # the decode step at the end of the 2048 context (bench.py's
    # decode_full_*_kv2047 lines): attention over 2047 and 2048 cached rows
    _run_c5(2046, 2)
