"""GPU tests of the attention section (sllm_attention_dev: forwardBlock,
model_f32.go:398-466) and of the matmul + residual add (sllm_matmul_add_dev),
against the oracle (oracle.attention_layer, pinned in
tests/test_oracle_attention.py).

What must agree and how closely:
* the cache rows the call appends: v (bias add) bit for bit; k (bias, norm,
  RoPE) bit for bit up to the last bit of the float64 cos / sin (the device's
  vs the C library's), so within 4 ulp-of-|x| per element;
* the attention output: the scores are the reference's sequential float32
  dots, the softmax sums and the weighted sum of values are reassociated
  (split over positions and combined; the weighted sum with fused
  multiply-adds, one rounding per step). Bound per output element, from the
  float64 scores s_k and weights p_k the oracle's rotated q and the cache
  give: sum_k p_k |v_k| (2 ds_k + (2 kv_len + 160) u + 6 u (max s - s_k)),
  u = 2^-24, ds_k = 4 u scale sum_d |q_d k_kd| (rotated inputs that differ in
  a last bit). The reference's own float32 sums carry errors of that order;
  a wrong position, head, mask or split combine changes outputs by O(|v|).
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
import sllm_qmm as sq

from _helpers import make_raw, make_x

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def dev_view(ptr: int, n: int) -> torch.Tensor:
    """A float32 tensor over n floats of device memory the library owns."""
    class _Mem:
        pass
    m = _Mem()
    m.__cuda_array_interface__ = {"shape": (n,), "typestr": "<f4", "data": (ptr, False), "version": 2}
    return torch.as_tensor(m, device="cuda")


def freqs_for(half_dim, base=10000.0):
    rope_dim = 2 * half_dim
    return np.array([1.0 / math.pow(base, 2.0 * i / rope_dim) for i in range(half_dim)], np.float32)


class Model:
    """The attention constants of one layer, on the device."""

    def __init__(self, H, KV, dk, half, rng, bias=False, qk=False, eps=1e-5, base=10000.0):
        self.H, self.KV, self.dk, self.half, self.eps = H, KV, dk, half, eps
        self.freqs = freqs_for(half, base)
        self.qb = self.kb = self.vb = self.qn = self.kn = None
        if bias:
            self.qb = rng.normal(size=H * dk - 5).astype(np.float32)
            self.kb = rng.normal(size=KV * dk + 3).astype(np.float32)
            self.vb = rng.normal(size=KV * dk).astype(np.float32)
        if qk:
            self.qn = rng.normal(1, 0.2, dk).astype(np.float32)
            self.kn = rng.normal(1, 0.2, dk).astype(np.float32)
        self._keep = []

        def d(a):
            if a is None:
                return None, 0
            t = torch.from_numpy(a).cuda()
            self._keep.append(t)
            return t.data_ptr(), a.size

        fp, _ = d(self.freqs)
        qb, qbl = d(self.qb)
        kb, kbl = d(self.kb)
        vb, vbl = d(self.vb)
        qn, _ = d(self.qn)
        kn, _ = d(self.kn)
        self.params = sq.AttnParams(n_heads=H, n_kv_heads=KV, d_k=dk, rope_half_dim=half, rope_freqs=fp,
                                    q_bias=qb, q_bias_len=qbl, k_bias=kb, k_bias_len=kbl, v_bias=vb,
                                    v_bias_len=vbl, q_norm_w=qn, k_norm_w=kn, norm_eps=eps)

    def oracle(self, q, k, v, ck, cv, cache_len, start_pos):
        return oracle.attention_layer(q, k, v, self.H, self.KV, self.dk, ck, cv, cache_len, start_pos, self.freqs,
                                      self.half, self.qb, self.kb, self.vb, self.qn, self.kn, self.eps,
                                      lib_norm=True, return_q_rot=True)


def out_bound(m: Model, q_rot, ck, cv, cache_len, seq):
    dk, rep = m.dk, m.H // m.KV
    scale = 1.0 / math.sqrt(dk)
    b = np.zeros((seq, m.H * dk))
    for qi in range(seq):
        kv = cache_len + qi + 1
        for h in range(m.H):
            g = h // rep
            q = q_rot[qi, h * dk:(h + 1) * dk].astype(np.float64)
            K = ck[g, :kv].astype(np.float64)
            V = np.abs(cv[g, :kv].astype(np.float64))
            s = K @ q * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            ds = 4 * U * scale * (np.abs(K) @ np.abs(q))
            rel = 2 * ds + (2 * kv + 160) * U + 6 * U * (s.max() - s)
            b[qi, h * dk:(h + 1) * dk] = (p * rel) @ V
    return b + 1e-30


def run_case(m: Model, seq, cache_len, rng, layer=1, n_layers=2, cap=None):
    dk, KV = m.dk, m.KV
    cap = cap or cache_len + seq + 5
    kv = sq.KVCache(n_layers, KV, dk, cap)
    # the rows already cached: random (rotated-looking) values written directly
    ck0 = rng.normal(size=(KV, cap, dk)).astype(np.float32)
    cv0 = rng.normal(size=(KV, cap, dk)).astype(np.float32)
    kp, vp = kv.data(layer)
    dev_view(kp, KV * cap * dk).copy_(torch.from_numpy(ck0.reshape(-1)))
    dev_view(vp, KV * cap * dk).copy_(torch.from_numpy(cv0.reshape(-1)))
    kv.set_length(cache_len)
    q = (rng.normal(size=(seq, m.H * dk)) * 1.5).astype(np.float32)
    k = rng.normal(size=(seq, KV * dk)).astype(np.float32)
    v = rng.normal(size=(seq, KV * dk)).astype(np.float32)
    qd, kd, vd = (torch.from_numpy(a).cuda() for a in (q, k, v))
    out = torch.full((seq, m.H * dk), float("nan"), device="cuda")
    sq.attention_dev(kv, layer, m.params, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), seq, cache_len,
                     out.data_ptr())
    torch.cuda.synchronize()
    assert kv.length(layer) == cache_len + seq
    assert kv.length(1 - layer) == cache_len  # the other layer is untouched
    gk = dev_view(kp, KV * cap * dk).cpu().numpy().reshape(KV, cap, dk)
    gv = dev_view(vp, KV * cap * dk).cpu().numpy().reshape(KV, cap, dk)
    want, wk, wv, qrot = m.oracle(q, k, v, ck0, cv0, cache_len, cache_len)
    # appended rows
    new = slice(cache_len, cache_len + seq)
    assert np.array_equal(gv[:, new], wv[:, new])
    assert np.all(np.abs(gk[:, new].astype(np.float64) - wk[:, new]) <= 4 * 2.0 ** -23 * np.abs(wk[:, new]) + 1e-30)
    # rows outside the appended range are untouched
    assert np.array_equal(gk[:, :cache_len], ck0[:, :cache_len])
    assert np.array_equal(gk[:, cache_len + seq:], ck0[:, cache_len + seq:])
    got = out.cpu().numpy()
    bound = out_bound(m, qrot, wk, wv, cache_len, seq)
    err = np.abs(got.astype(np.float64) - want)
    assert np.all(err <= bound), (float(err.max()), float((err / bound).max()))
    kv.close()
    return got, want


@pytest.mark.parametrize("cache_len", [0, 1, 63, 64, 65, 200, 2047])
def test_decode_llama_heads(cache_len):
    rng = np.random.default_rng(cache_len)
    m = Model(8, 2, 128, 64, rng, base=500000.0)
    run_case(m, 1, cache_len, rng)


@pytest.mark.parametrize("groups,target", [(1, 512), (2, 512), (4, 512), (4, 8), (3, 1)])
@pytest.mark.parametrize("cache_len", [0, 63, 130, 300, 1100])
def test_tile_groups_and_splits(groups, target, cache_len):
    # 1-4 tile groups per workgroup, merged in LDS; one split (the workgroup
    # writes the output) or several (the combine launch), including groups
    # whose tiles lie past the causal range
    sq.set_param("attn_tile_groups", groups)
    sq.set_param("attn_target_blocks", target)
    try:
        rng = np.random.default_rng(cache_len + 1000 * groups)
        m = Model(8, 2, 128, 64, rng, base=500000.0)
        run_case(m, 1, cache_len, rng)
        run_case(m, 3, cache_len, rng)
    finally:
        sq.set_param("attn_tile_groups", 4)
        sq.set_param("attn_target_blocks", 512)


@pytest.mark.parametrize("H,KV,dk,half,seq,cache_len", [
    (8, 2, 128, 64, 1, 0), (8, 2, 128, 64, 1, 130), (8, 2, 128, 64, 1, 2047), (8, 2, 128, 64, 3, 70),
    (32, 8, 128, 64, 1, 128), (16, 2, 64, 32, 1, 300), (6, 3, 96, 48, 1, 65), (4, 2, 64, 32, 5, 40)])
def test_head_slices_give_the_same_bits(H, KV, dk, half, seq, cache_len):
    # the q heads of a kv head spread over 1, 2, 4 or 8 workgroups (the
    # planner keeps a divisor of the heads per kv head) or as many as the
    # planner picks: every head's arithmetic is the same, so are the outputs
    outs = []
    try:
        for hs in (1, 2, 4, 8, 0):
            sq.set_param("attn_head_slices", hs)
            rng = np.random.default_rng(H * 1000 + cache_len * 10 + seq)
            m = Model(H, KV, dk, half, rng, base=500000.0)
            got, _ = run_case(m, seq, cache_len, rng)
            outs.append(got)
    finally:
        sq.set_param("attn_head_slices", 0)
    for hs, o in zip((2, 4, 8, 0), outs[1:]):
        assert np.array_equal(o.view(np.uint32), outs[0].view(np.uint32)), hs


def test_first_position_after_a_launch_that_leaves_nan_in_lds():
    # a tile with one row: the value loop must not multiply stale LDS rows
    # (here NaN activations a GEMV staged there) by zero weights
    K, N = 4096, 14336
    raw = make_raw("q8", N, K, seed=3)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight("q8", raw, K // 32, N, K))
    xn = torch.full((K,), float("nan"), device="cuda")
    y = torch.empty(N, device="cuda")
    sq.matmul_dev(w, xn.data_ptr(), 1, K, y.data_ptr())
    torch.cuda.synchronize()
    rng = np.random.default_rng(99)
    m = Model(8, 2, 128, 64, rng)
    got, _ = run_case(m, 1, 0, rng)
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("seq,cache_len", [(37, 0), (5, 70), (70, 3)])
def test_prefill_rows_are_causal(seq, cache_len):
    rng = np.random.default_rng(seq * 7 + cache_len)
    m = Model(4, 2, 64, 32, rng)
    run_case(m, seq, cache_len, rng)


def test_mha_bias_qk_norm_partial_rope():
    rng = np.random.default_rng(11)
    m = Model(4, 4, 64, 16, rng, bias=True, qk=True)
    run_case(m, 3, 40, rng, layer=0)


@pytest.mark.parametrize("H,KV,dk,half", [(16, 2, 256, 128), (6, 3, 96, 48), (8, 8, 32, 16)])
def test_head_shapes(H, KV, dk, half):
    # 8 q heads per kv head (two per wave), K staged in two column chunks;
    # a head size that is not a multiple of 64; a small one
    rng = np.random.default_rng(H * dk)
    m = Model(H, KV, dk, half, rng, qk=dk == 256)
    run_case(m, 1, 150, rng)
    run_case(m, 2, 9, rng)


def test_successive_decode_steps_follow_the_oracle():
    rng = np.random.default_rng(21)
    m = Model(8, 2, 64, 32, rng)
    H, KV, dk, cap = 8, 2, 64, 16
    kv = sq.KVCache(1, KV, dk, cap)
    ck = np.zeros((KV, cap, dk), np.float32)
    cv = np.zeros((KV, cap, dk), np.float32)
    out = torch.empty(H * dk, device="cuda")
    for pos in range(5):
        q = rng.normal(size=(1, H * dk)).astype(np.float32)
        k = rng.normal(size=(1, KV * dk)).astype(np.float32)
        v = rng.normal(size=(1, KV * dk)).astype(np.float32)
        qd, kd, vd = (torch.from_numpy(a).cuda() for a in (q, k, v))
        sq.attention_dev(kv, 0, m.params, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 1, pos, out.data_ptr())
        want, ck, cv, qrot = m.oracle(q, k, v, ck, cv, pos, pos)
        got = out.cpu().numpy()[None]
        assert np.all(np.abs(got - want) <= out_bound(m, qrot, ck, cv, pos, 1))
    assert kv.length(0) == 5
    # a full cache is an error, not an overwrite
    kv.set_length(cap)
    with pytest.raises(sq.SllmError) as e:
        sq.attention_dev(kv, 0, m.params, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 1, cap, out.data_ptr())
    assert e.value.status == 3
    kv.close()


def test_argument_errors():
    rng = np.random.default_rng(1)
    m = Model(8, 2, 64, 32, rng)
    kv = sq.KVCache(2, 4, 64, 8)  # 4 kv heads: differs from the params' 2
    x = torch.zeros(8 * 64, device="cuda")
    p = x.data_ptr()
    with pytest.raises(sq.SllmError):
        sq.attention_dev(kv, 0, m.params, p, p, p, 1, 0, p)
    with pytest.raises(sq.SllmError):
        sq.attention_dev(kv, 2, m.params, p, p, p, 1, 0, p)  # layer out of range
    kv.close()


@pytest.mark.parametrize("qtype,M", [("q4_1", 1), ("q8", 3), ("q4_1", 64), ("q5", 64)])
def test_matmul_add_is_matmul_then_one_add(qtype, M):
    N, K = 300, 512
    raw = make_raw(qtype, N, K, seed=5)
    w = sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))
    x = torch.from_numpy(make_x(M, K, seed=6)).cuda()
    base = np.random.default_rng(7).normal(size=(M, N)).astype(np.float32)
    dst = torch.from_numpy(base).cuda()
    sq.matmul_add_dev(w, x.data_ptr(), M, K, dst.data_ptr())
    plain = torch.empty(M, N, device="cuda")
    sq.matmul_dev(w, x.data_ptr(), M, K, plain.data_ptr())
    torch.cuda.synchronize()
    want = base + plain.cpu().numpy()  # one float32 add per element
    assert np.array_equal(dst.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.slow
def test_prefill_rows_beyond_the_grid_limit():
    # seq_len x n_kv_heads above 65535 (the split kernel's grid y): the rows
    # run in chunks, each against the whole cache the prep kernel filled
    rng = np.random.default_rng(5)
    m = Model(64, 64, 8, 4, rng)
    run_case(m, 1030, 0, rng, layer=0, n_layers=2)
