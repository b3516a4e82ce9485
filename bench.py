"""Benchmark of the MI355X quantized-matmul path (one JSON line on stdout).

Workload (the one the metric is quoted on): one Llama-3-8B
layer's decode GEMVs at M = 1 token -
    gate, up : Q4_K 14336 x 4096, remapped at load to Q4_1 (20 B / 32 weights)
    down     : Q6_K 4096 x 14336, requantized at load to Q8_0 (34 B / 32)
A step is those three matmuls over one layer's weights: gate and up share
their input and run as one launch (sllm_matmul_multi_dev), down as another.
Steps rotate over enough layer copies (> 1 GiB) that no step finds its
weights in the 256 MB MALL. Inputs are synthetic, already resident in HBM;
the remaps run once at load.

value        = algorithmic bytes per step x steps / elapsed   (GB/s, whole job);
               per GEMV: plane bytes + 4 K (fp32 x) + 4 N (fp32 out)
roofline     = dominant kernel (the fused gate+up Q4_1 GEMV, 54 % of the step's
               bytes): its algorithmic bytes per launch / its mean duration (HIP
               events around back-to-back launches on the launch stream)
cpu_baseline = the reference's CPU kernels restated with AVX2/AVX-VNNI intrinsics
               and its worker pool (oracle/refcpu_simd.c), on a bounded sample
extra        = per-kernel times; every other BASELINE config's kernels (C1, C2,
               C4 GEMV and GEMM); decode tok/s over all linears of a 32-layer
               Q4_K_M 8B-shaped model + Q6_K head (weights only; attention etc.
               are not part of this path)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "scriptling-llm-lib_amd"))

HBM_PEAK_GBS = 8000.0
INT8_MFMA_PEAK_TOPS = 5000.0
BF16_MFMA_PEAK_TOPS = 2500.0  # MI355X dense bf16 matrix peak (TFLOP/s)
METRIC = "quant GEMV GB/s (% of 8 TB/s HBM); Q4_K_M 8B-shape decode tok/s"
TRAFFIC_JSON = os.path.join(ROOT, "profiles", "traffic_gemv_q4_1_gate_up_c3.json")
ROTATE_BYTES = 1 << 30  # weight copies per timed kernel: > 4x the 256 MB MALL


def algo_bytes(ws, m_rows: int = 1) -> int:
    """Weight plane bytes + fp32 activations in (once per launch) + fp32 outputs."""
    ws = ws if isinstance(ws, (list, tuple)) else [ws]
    return sum(w.plane_bytes + 4 * w.rows * m_rows for w in ws) + 4 * ws[0].cols * m_rows


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--layers", type=int, default=8, help="layer copies rotated over (>1 GiB)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1/C2/C4 kernel table")
    ap.add_argument("--decode-tokens", type=int, default=20)
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only launch the dominant GEMV and a 256 MiB copy (for rocprofv3 --pmc runs)")
    ap.add_argument("--gemm-probe", action="store_true",
                    help="only launch the prefill GEMMs (C3 / C4 shapes, M = 64 and 512) for rocprofv3 runs")
    ap.add_argument("--valu-probe", action="store_true",
                    help="only print the VALU issue rate of the instruction kinds the GEMV kernels use")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "Each GPU would own a slice of the weight rows (its dst rows) and read the whole activation row.",
              file=sys.stderr)
        return 2

    import torch

    import sllm_qmm as sq
    from sllm_qmm import synth

    torch.cuda.set_device(0)
    sq.init()
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    H, F = 4096, 14336
    if args.traffic_probe:
        return traffic_probe(sq, synth, torch, stream, args.layers)
    if args.gemm_probe:
        return gemm_probe(sq, synth, torch, stream)
    if args.valu_probe:
        print(json.dumps({"valu_issue_rates": valu_rates()}), flush=True)
        return 0
    print(f"[bench] building {args.layers} layer copies of C3 weights", file=sys.stderr, flush=True)
    gate_raw = synth.q4k_blocks(100, F, H)
    up_raw = synth.q4k_blocks(101, F, H)
    down_raw = synth.q6k_blocks(102, H, F)
    layers = []
    for _ in range(args.layers):
        layers.append((sq.load_weight_f32_direct(synth.GGML_Q4_K, gate_raw, F, H),
                       sq.load_weight_f32_direct(synth.GGML_Q4_K, up_raw, F, H),
                       sq.load_weight_f32_direct(synth.GGML_Q6_K, down_raw, H, F)))
    g0, u0, d0 = layers[0]
    x = torch.from_numpy(synth.normal(1, H)).cuda()
    h = torch.from_numpy(synth.normal(2, F)).cuda()
    yg = torch.empty(F, device="cuda")
    yu = torch.empty(F, device="cuda")
    yd = torch.empty(H, device="cuda")
    step_bytes = algo_bytes(g0) + algo_bytes(u0) + algo_bytes(d0)

    def gate_up(i):
        g, u, _ = layers[i % len(layers)]
        sq.matmul_multi_dev([g, u], x.data_ptr(), 1, H, [yg.data_ptr(), yu.data_ptr()], sp)

    def down(i):
        d = layers[i % len(layers)][2]
        sq.matmul_dev(d, h.data_ptr(), 1, F, yd.data_ptr(), sp)

    def gate_only(i):
        g = layers[i % len(layers)][0]
        sq.matmul_dev(g, x.data_ptr(), 1, H, yg.data_ptr(), sp)

    def step(i):
        gate_up(i)
        down(i)

    # correctness before timing: one step's outputs against the restated
    # reference CPU path on the same bytes (the cpu_baseline leg)
    parity = None
    if not args.no_cpu_baseline:
        step(0)
        torch.cuda.synchronize()
        pre = (yg.cpu().numpy().copy(), yu.cpu().numpy().copy(), yd.cpu().numpy().copy())
        parity = cpu_parity(g0, u0, d0, x.cpu().numpy(), h.cpu().numpy(), pre)
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for i in range(args.steps):
        step(i)
    t1.record(stream)
    torch.cuda.synchronize()
    elapsed_ms = t0.elapsed_time(t1)
    ms_per_step = elapsed_ms / args.steps
    value = step_bytes * args.steps / (elapsed_ms * 1e-3) / 1e9

    # the timed launches' outputs: every step computes the same values (the
    # layer copies hold the same bytes), so they must equal the checked step's
    if parity is not None:
        post = (yg.cpu().numpy(), yu.cpu().numpy(), yd.cpu().numpy())
        parity["timed_outputs_equal_checked_step"] = all(
            bool((a.view("u4") == b.view("u4")).all()) for a, b in zip(pre, post))

    n_roof = max(args.steps, 100)
    gu = time_launches(torch, stream, gate_up, n_roof, trials=7)
    gu_us = gu["mean"]
    gu_bytes = algo_bytes([g0, u0])
    achieved = gu_bytes / (gu_us * 1e-6) / 1e9
    dn = time_launches(torch, stream, down, n_roof, trials=7)
    ga = time_launches(torch, stream, gate_only, n_roof, trials=7)
    r3 = lambda d: {k: (round(v, 3) if isinstance(v, float) else v) for k, v in d.items()}

    extra = {
        "gate_up_fused_q4_1_gemv_us": r3(gu),
        "gate_up_fused_bytes": gu_bytes,
        "gate_up_fused_GBps_median": round(gu_bytes / (gu["median"] * 1e-6) / 1e9, 1),
        "gate_up_fused_GBps_min_time": round(gu_bytes / (gu["min"] * 1e-6) / 1e9, 1),
        "down_q8_0_gemv_us": r3(dn),
        "down_q8_0_gemv_GBps": round(algo_bytes(d0) / (dn["mean"] * 1e-6) / 1e9, 1),
        "gate_q4_1_gemv_alone_us": r3(ga),
        "gate_q4_1_gemv_alone_GBps": round(algo_bytes(g0) / (ga["mean"] * 1e-6) / 1e9, 1),
        "kernel_info": sq.kernel_info(),
    }
    if parity is not None:
        extra["parity_vs_cpu_reference"] = parity
    peaks = mfma_peaks()
    if peaks:
        extra["int8_mfma_peak_tops_measured"] = peaks
    del layers

    if not args.no_configs:
        extra["configs"] = config_table(sq, synth, torch, stream, peaks)
    if not args.no_decode:
        extra.update(decode_tok_s(sq, synth, torch, stream, args.decode_tokens))

    tr = load_traffic()
    traffic_bytes = tr["traffic_bytes_per_launch"] if tr else None
    if tr:
        extra["traffic_source"] = tr["source"]

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(sq, synth, gate_raw, up_raw, down_raw, args.layers, step_bytes)

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "C3: Llama-3-8B Q4_K_M layer decode GEMVs, M=1: Q4_K gate+up 14336x4096 -> Q4_1 "
                        "(one fused launch), Q6_K down 4096x14336 -> Q8_0",
            "bytes_per_step": step_bytes,
            "rotating_layer_copies": args.layers,
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "gemv_kernel<Q4_1>, gate+up fused (2 x Q4_K->Q4_1 14336x4096, one launch)",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_bytes,
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


def time_launches(torch, stream, launch, n: int, warm: int = 10, trials: int = 1):
    """Mean duration (us) of `launch(i)` over n back-to-back calls between two HIP
    events on the launch stream. Consecutive launches on one stream run with no
    measurable gap, so this is the kernel time rocprofv3 --kernel-trace reports
    for the same launches. trials > 1: that measurement repeated, returning
    {"mean": over every launch, "median" / "min": of the trials' means} (the
    reference's micro-benchmark keeps the min of 7 trials, q8q8.go:280-294)."""
    for i in range(warm):
        launch(i)
    means = []
    k = 0
    for _ in range(trials):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(n):
            launch(k)
            k += 1
        b.record(stream)
        torch.cuda.synchronize()
        means.append(a.elapsed_time(b) / n * 1e3)
    if trials == 1:
        return means[0]
    srt = sorted(means)
    return {"mean": sum(means) / len(means), "median": srt[len(srt) // 2], "min": srt[0], "trials": trials,
            "launches_per_trial": n}


def graph_launch_us(torch, stream, launch, n: int, replays: int = 10) -> float:
    """Per-launch time (us) of n calls launch(i, stream) captured into one HIP
    graph on a side stream and replayed on `stream` (median of `replays`)."""
    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        for i in range(2):
            launch(i, cs.cuda_stream)
    cs.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        for i in range(n):
            launch(i, cs.cuda_stream)
    g.replay()
    torch.cuda.synchronize()
    ts = []
    for _ in range(replays):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        g.replay()
        b.record(stream)
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b) / n * 1e3)
    del g
    return sorted(ts)[len(ts) // 2]


def config_table(sq, synth, torch, stream, peaks=None) -> dict:
    """The kernels of BASELINE configs C1, C2, C4 (and C3 at prefill sizes).

    Each entry rotates over copies of its weight totalling >= 1 GiB (at most
    512 copies, so C1's 0.9 MB weight can stay in the MALL: C1 is launch-bound
    at any rate). GEMV lines give GB/s of algorithmic bytes; GEMM lines (M >=
    8 or 16) also give TOPS (2 M N K per call) against the published 5.0 POPS
    dense int8 MFMA peak, or for Q5_0 (fp32 activations split into three exact
    bf16 parts, so the bf16 matrix cores execute 3 x 2 M N K) against the 2.5
    PFLOP/s dense bf16 peak. Q5_K rows stream 26 B / 32 weights (the two Q4_1 halves of
    convertQ5KToTwoQ41 without the high half's zero mins and 4-bit codes).
    M = 1 lines also give us_graph: the per-launch time of 100 of the same
    calls replayed from one HIP graph (C1-sized GEMVs are launch-bound)."""
    import numpy as np
    H, F, KV = 4096, 14336, 1024
    sp = stream.cuda_stream
    print("[bench] config table (C1, C2, C4 and C3 prefill)", file=sys.stderr, flush=True)

    def copies(make_one):
        w0 = make_one()
        n = int(min(512, max(2, -(-ROTATE_BYTES // w0.plane_bytes))))
        raw = w0.export()
        if w0.qtype in ("q2k", "q3k"):  # native k-quants: rebuilt from their GGUF blocks
            t = {"q2k": synth.GGML_Q2_K, "q3k": synth.GGML_Q3_K}[w0.qtype]
            return [w0] + [sq.load_weight_f32_direct(t, raw, w0.rows, w0.cols) for _ in range(n - 1)]
        q = sq.QuantWeight(w0.qtype, raw, w0.groups, w0.rows, w0.cols)
        return [w0] + [sq.DeviceWeight.from_quant(q) for _ in range(n - 1)]

    def run(ws, M, reps):
        K, N = ws[0].cols, ws[0].rows
        xin = torch.from_numpy(synth.normal(7, M * K)).cuda()
        out = torch.empty(M * N, device="cuda")
        st = time_launches(torch, stream, lambda i: sq.matmul_dev(ws[i % len(ws)], xin.data_ptr(), M, K,
                                                                   out.data_ptr(), sp), max(reps // 5, 20), trials=5)
        us = st["mean"]
        nbytes = algo_bytes(ws[0], M)
        r = {"us": round(us, 2), "us_median": round(st["median"], 2), "us_min": round(st["min"], 2),
             "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        if M == 1:
            # launch-bound shapes: the same calls replayed from one HIP graph
            # (n launches, rotating copies), the per-launch cost without the
            # host's enqueue path
            r["us_graph"] = round(graph_launch_us(torch, stream, lambda i, s_: sq.matmul_dev(
                ws[i % len(ws)], xin.data_ptr(), M, K, out.data_ptr(), s_), 100), 2)
        if M >= 64:
            tops = 2.0 * M * N * K / (us * 1e-6) / 1e12
            if ws[0].qtype == "q5":
                # fp32 activations as three exact bf16 parts: 3 x 2 M N K on the bf16 matrix cores
                r.update({"TOPS": round(tops, 1), "frac_bf16_mfma": round(3 * tops / BF16_MFMA_PEAK_TOPS, 4),
                          "path": "bf16 MFMA GEMM (Q5_0 keeps fp32 activations, split into three bf16 parts)"})
            else:
                r.update({"TOPS": round(tops, 1), "frac_int8_mfma": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                          "path": "int8 MFMA GEMM"})
        return r

    def q_from_f32(qtype, seed, N, K):
        wf = synth.normal(seed, N * K, 0.02).reshape(N, K)
        raw = {"q4": synth.quantize_q4_0, "q4_1": synth.quantize_q4_1, "q5": synth.quantize_q5_0}[qtype](wf)
        return lambda: sq.DeviceWeight.from_quant(sq.QuantWeight(qtype, raw, K // 32, N, K))

    table = {}
    c1 = copies(lambda: sq.quantize_q8_rows_f32(synth.normal(0, 1536 * 576, 0.02), 1536, 576))
    table["C1 q8 1536x576 M=1"] = run(c1, 1, 400)
    del c1
    for qtype in ("q4", "q4_1"):
        for N, K in ((8192, 2048), (2048, 8192)):
            ws = copies(q_from_f32(qtype, 10 + N // 1024, N, K))
            table[f"C2 {qtype} {N}x{K} M=1"] = run(ws, 1, 200)
            del ws
    for N in (H, KV, F):
        ws = copies(lambda: sq.load_weight_f32_direct(synth.GGML_Q5_K, synth.q5k_blocks(20 + N // 1024, N, H), N, H))
        for M in (1, 64, 512):
            table[f"C4 q5k1 {N}x{H} M={M}"] = run(ws, M, 200 if M == 1 else 100)
        del ws
        ws = copies(q_from_f32("q5", 30 + N // 1024, N, H))
        for M in (1, 64, 512):
            table[f"C4 q5 {N}x{H} M={M}"] = run(ws, M, 200 if M == 1 else 100)
        del ws
    g = copies(lambda: sq.load_weight_f32_direct(synth.GGML_Q4_K, synth.q4k_blocks(100, F, H), F, H))
    for M in (64, 512):
        table[f"C3 q4_1 gate {F}x{H} M={M}"] = run(g, M, 100)
    del g
    d = copies(lambda: sq.load_weight_f32_direct(synth.GGML_Q6_K, synth.q6k_blocks(102, H, F), H, F))
    for M in (64, 512):
        table[f"C3 q8 down {H}x{F} M={M}"] = run(d, M, 100)
    del d
    # native Q2_K / Q3_K (the reference's dense-fp32 types): GEMV over the
    # native blocks; dense_fp32_equiv_GBps counts the 4 B / weight the
    # reference's dense layout would stream in the same time
    for t, name, make in ((synth.GGML_Q2_K, "q2k", synth.q2k_blocks), (synth.GGML_Q3_K, "q3k", synth.q3k_blocks)):
        for N, K in ((F, H), (H, F)):
            ws = copies(lambda: sq.load_weight_f32_direct(t, make(40 + t, N, K), N, K))
            r = run(ws, 1, 200)
            r["dense_fp32_equiv_GBps"] = round(4.0 * N * K / (r["us"] * 1e-6) / 1e9, 1)
            table[f"{name} native {N}x{K} M=1"] = r
            del ws
    # Q6_K streamed from its 6-bit codes (opt-in: load option gemv_q6k_stream):
    # the C3 down and the output head, the same blocks timed streamed and from
    # weights loaded without the option (us_q8_planes)
    for N, K, seed in ((H, F, 102), (128256, H, 204)):
        raw = synth.q6k_blocks(seed, N, K)
        sq.set_param("gemv_q6k_stream", 1)
        try:
            w0 = sq.load_weight_f32_direct(synth.GGML_Q6_K, raw, N, K)
            n = int(min(64, max(2, -(-ROTATE_BYTES // w0.plane_bytes))))
            ws = [w0] + [sq.load_weight_f32_direct(synth.GGML_Q6_K, raw, N, K) for _ in range(n - 1)]
        finally:
            sq.set_param("gemv_q6k_stream", 0)
        r = run(ws, 1, 100)
        r["fp64_blocks"] = ws[0].q6k_exact_blocks
        del ws
        wq = copies(lambda: sq.load_weight_f32_direct(synth.GGML_Q6_K, raw, N, K))
        r["us_q8_planes"] = run(wq, 1, 100)["us"]
        del wq
        table[f"q6k streamed {N}x{K} M=1 (opt-in)"] = r
    torch.cuda.empty_cache()
    return table


COPY_BYTES = 256 << 20


def traffic_probe(sq, synth, torch, stream, copies: int) -> int:
    """Launches for the counter runs: 20 fused gate+up GEMVs (rotating copies),
    then 5 device copies of COPY_BYTES (the calibration kernel of known traffic)."""
    H, F = 4096, 14336
    gr, ur = synth.q4k_blocks(100, F, H), synth.q4k_blocks(101, F, H)
    pairs = [(sq.load_weight_f32_direct(synth.GGML_Q4_K, gr, F, H),
              sq.load_weight_f32_direct(synth.GGML_Q4_K, ur, F, H)) for _ in range(copies)]
    x = torch.from_numpy(synth.normal(1, H)).cuda()
    yg = torch.empty(F, device="cuda")
    yu = torch.empty(F, device="cuda")
    for i in range(20):
        g, u = pairs[i % len(pairs)]
        sq.matmul_multi_dev([g, u], x.data_ptr(), 1, H, [yg.data_ptr(), yu.data_ptr()], stream.cuda_stream)
    a = torch.empty(COPY_BYTES // 4, device="cuda")
    b = torch.empty(COPY_BYTES // 4, device="cuda")
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"traffic probe done: gate+up algorithmic bytes {algo_bytes(list(pairs[0]))}, copy {COPY_BYTES} B",
          flush=True)
    return 0


def gemm_probe(sq, synth, torch, stream) -> int:
    """Launches for the GEMM profiles: each C3 / C4 prefill shape at M = 64 and
    512, 10 calls each over 4 rotating weight copies, in a fixed order."""
    H, F, KV = 4096, 14336, 1024
    mk = sq.load_weight_f32_direct
    shapes = [("q4_1 gate", lambda: mk(synth.GGML_Q4_K, synth.q4k_blocks(100, F, H), F, H)),
              ("q8 down", lambda: mk(synth.GGML_Q6_K, synth.q6k_blocks(102, H, F), H, F)),
              ("q5k1 q/o", lambda: mk(synth.GGML_Q5_K, synth.q5k_blocks(21, H, H), H, H)),
              ("q5k1 ffn", lambda: mk(synth.GGML_Q5_K, synth.q5k_blocks(22, F, H), F, H))]
    q5raw = synth.quantize_q5_0(synth.normal(30, H * H, 0.02).reshape(H, H))
    shapes.append(("q5 q/o", lambda: sq.DeviceWeight.from_quant(sq.QuantWeight("q5", q5raw, H // 32, H, H))))
    q5raw_f = synth.quantize_q5_0(synth.normal(31, F * H, 0.02).reshape(F, H))
    shapes.append(("q5 ffn", lambda: sq.DeviceWeight.from_quant(sq.QuantWeight("q5", q5raw_f, H // 32, F, H))))
    xs = {c: torch.from_numpy(synth.normal(7, 512 * c)).cuda() for c in (H, F)}
    y = torch.empty(512 * F, device="cuda")
    for name, make in shapes:
        ws = [make() for _ in range(4)]
        K = ws[0].cols
        for M in (64, 512):
            for i in range(10):
                sq.matmul_dev(ws[i % 4], xs[K].data_ptr(), M, K, y.data_ptr(), stream.cuda_stream)
            torch.cuda.synchronize()
            print(f"gemm probe: {name} {ws[0].rows}x{K} M={M} done", flush=True)
        del ws
    return 0


def load_traffic() -> dict | None:
    """HBM bytes per launch of the dominant kernel from the committed counter runs."""
    try:
        with open(TRAFFIC_JSON) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def decode_tok_s(sq, synth, torch, stream, tokens: int) -> dict:
    """All linears of one decode token of a 32-layer Q4_K_M Llama-3-8B shape + Q6_K head,
    with the RMSNorms, the SwiGLU and the greedy argmax fused into them.

    Per layer: RMSNorm + q/k/v (one launch: they share their input), o,
    RMSNorm + gate/up + SwiGLU (one launch), down on h; then the final
    RMSNorm + head + argmax: 32 x 4 + 1 = 129 launches per token."""
    import numpy as np
    H, F, KV, V, L = 4096, 14336, 1024, 128256, 32
    print("[bench] building the 32-layer decode weight set", file=sys.stderr, flush=True)
    q4k_hh = synth.q4k_blocks(200, H, H)
    q4k_kv = synth.q4k_blocks(201, KV, H)
    q4k_fh = synth.q4k_blocks(202, F, H)
    q6k_hf = synth.q6k_blocks(203, H, F)
    q6k_head = synth.q6k_blocks(204, V, H)
    mk = sq.load_weight_f32_direct
    layer_ws = []
    for _ in range(L):
        layer_ws.append([mk(12, q4k_hh, H, H), mk(12, q4k_kv, KV, H), mk(12, q4k_kv, KV, H),
                         mk(12, q4k_hh, H, H), mk(12, q4k_fh, F, H), mk(12, q4k_fh, F, H),
                         mk(14, q6k_hf, H, F)])
    head = mk(14, q6k_head, V, H)
    tok_bytes = sum(w.plane_bytes for ws in layer_ws for w in ws) + head.plane_bytes
    xh = torch.from_numpy(synth.normal(3, H)).cuda()
    q, k, v = (torch.empty(n, device="cuda") for n in (H, KV, KV))
    o, dn = (torch.empty(n, device="cuda") for n in (H, H))
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    P = lambda t: t.data_ptr()

    h = torch.empty(F, device="cuda")
    nw = torch.from_numpy(synth.normal(5, H, 0.1) + np.float32(1.0)).cuda()  # RMSNorm weight vectors
    eps = 1e-5

    def token(sp, norms=True):
        # per layer: RMSNorm + q/k/v in one launch, o, RMSNorm + gate/up + SwiGLU
        # in one launch (h), down on h; then the final RMSNorm + head + greedy
        # argmax in one launch. Attention and the residual adds are not part
        # of this path (they read q/k/v and write the next x). norms=False: the
        # same launches without the fused RMSNorm prologues.
        for wq, wk, wv, wo, wg, wu, wd in layer_ws:
            if norms:
                sq.rmsnorm_matmul_multi_dev([wq, wk, wv], P(xh), P(nw), eps, 1, H, [P(q), P(k), P(v)], sp)
            else:
                sq.matmul_multi_dev([wq, wk, wv], P(xh), 1, H, [P(q), P(k), P(v)], sp)
            sq.matmul_dev(wo, P(xh), 1, H, P(o), sp)
            if norms:
                sq.rmsnorm_matmul_swiglu_dev(wg, wu, P(xh), P(nw), eps, 1, H, P(h), sp)
            else:
                sq.matmul_swiglu_dev(wg, wu, P(xh), 1, H, P(h), 0, 0, sp)
            sq.matmul_dev(wd, P(h), 1, F, P(dn), sp)
        if norms:
            sq.rmsnorm_matmul_argmax_dev(head, P(xh), P(nw), eps, P(tok), 0, sp)
        else:
            sq.matmul_argmax_dev(head, P(xh), P(tok), 0, sp)

    def timed(run) -> float:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(tokens):
            run()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / tokens

    for _ in range(3):
        token(stream.cuda_stream)
    torch.cuda.synchronize()
    ms = timed(lambda: token(stream.cuda_stream))
    token(stream.cuda_stream, norms=False)
    torch.cuda.synchronize()
    ms_plain = timed(lambda: token(stream.cuda_stream, norms=False))
    # The same 129 launches captured once in a HIP graph and replayed: the
    # GEMV path allocates nothing and issues no memset, so it captures as is.
    token(stream.cuda_stream)  # the captured token's own eager outputs are the reference
    torch.cuda.synchronize()
    ref = (tok.clone(), dn.clone(), h.clone())
    cs = torch.cuda.Stream()
    with torch.cuda.stream(cs):
        token(cs.cuda_stream)  # first use of cs allocates its argmax scratch: before capture
    cs.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cs):
        token(cs.cuda_stream)
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    same = all(bool(torch.equal(a.view(torch.int32), b.view(torch.int32))) for a, b in zip((tok, dn, h), ref))
    ms_graph = timed(g.replay)
    del g

    full = decode_full_step(sq, torch, stream, layer_ws, head, nw, eps, xh, tokens)

    # the per-token head launch alone (RMSNorm + head + greedy argmax; its
    # 558 MB do not fit the MALL, so back-to-back launches read HBM)
    sp = stream.cuda_stream
    hst = time_launches(torch, stream, lambda i: sq.rmsnorm_matmul_argmax_dev(head, P(xh), P(nw), eps, P(tok), 0, sp),
                        20, trials=5)
    head_us = {k: round(hst[k], 2) for k in ("mean", "median", "min")}

    # The drop-in path as the Go binding would drive it: host buffers in and
    # out of every call (x uploaded, dst downloaded, synchronous), with the
    # host-side multi-weight and SwiGLU entries: 129 calls per token.
    xh_h = xh.cpu().numpy()

    def token_host():
        for wq, wk, wv, wo, wg, wu, wd in layer_ws:
            sq.model_matmul_multi_quant_into_f32([wq, wk, wv], xh_h, 1, H)
            sq.model_matmul_row_quant_into_f32(wo, xh_h)
            hh = sq.model_matmul_swiglu_into_f32(wg, wu, xh_h, 1, H)
            sq.model_matmul_row_quant_into_f32(wd, hh)
        return sq.matmul_argmax(head, xh_h)

    token_host()
    t0 = time.time()
    nh = 0
    while nh < 3 or (time.time() - t0 < 3.0 and nh < tokens):
        token_host()
        nh += 1
    ms_host = (time.time() - t0) / nh * 1e3
    del layer_ws, head
    torch.cuda.empty_cache()
    return {**full, "rmsnorm_head_argmax_us": head_us,
            "decode_gemv_tok_s": round(1e3 / ms, 1), "decode_gemv_ms_per_token": round(ms, 4),
            "decode_gemv_tok_s_without_norms": round(1e3 / ms_plain, 1),
            "decode_gemv_tok_s_graph": round(1e3 / ms_graph, 1),
            "decode_gemv_ms_per_token_graph": round(ms_graph, 4),
            "decode_graph_replay_matches_eager": same,
            "decode_weight_bytes_per_token": tok_bytes,
            "decode_gemv_GBps": round(tok_bytes / (ms * 1e-3) / 1e9, 1),
            "decode_gemv_GBps_graph": round(tok_bytes / (ms_graph * 1e-3) / 1e9, 1),
            "decode_host_entry_tok_s": round(1e3 / ms_host, 1),
            "decode_note": "129 launches per token (32 layers x [RMSNorm+qkv, o, RMSNorm+gate/up+SwiGLU, down] + "
                           "final RMSNorm+head+greedy argmax), device-resident, eager on one stream and replayed "
                           "from one HIP graph; _without_norms: the same launches without the RMSNorm "
                           "prologues; decode_host_entry_"
                           "tok_s: the same 129 calls through the host-buffer entry points (x in, dst out, "
                           "synchronous, from Python); attention and norms not included"}


def decode_full_step(sq, torch, stream, layer_ws, head, nw, eps, xh, tokens: int) -> dict:
    """The whole decode step on the device at stated KV positions: per layer
    RMSNorm + q/k/v, the attention section (bias / norm / RoPE / KV append /
    causal GQA attention over the cache), o + residual add, RMSNorm + gate/up
    + SwiGLU, down + residual add; then RMSNorm + head + greedy argmax
    (forwardBlock model_f32.go:382-500, outputLogits :502-527). x starts from
    the same embedding row every token (a device copy); the cache is set back
    to `pos` rows before each token, so every timed token runs at position pos."""
    import numpy as np
    H, F, L, NH, NKV, DK = 4096, 14336, 32, 32, 8, 128
    P = lambda t: t.data_ptr()
    half = DK // 2
    freqs = torch.from_numpy(np.array([1.0 / 500000.0 ** (2.0 * i / DK) for i in range(half)], np.float32)).cuda()
    prm = sq.AttnParams(n_heads=NH, n_kv_heads=NKV, d_k=DK, rope_half_dim=half, rope_freqs=P(freqs), norm_eps=eps)
    kvc = sq.KVCache(L, NKV, DK, 2048 + 16)
    x = torch.empty(H, device="cuda")
    q, k, v = (torch.empty(n, device="cuda") for n in (H, NKV * DK, NKV * DK))
    att = torch.empty(H, device="cuda")
    h = torch.empty(F, device="cuda")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda")
    sp = stream.cuda_stream

    def token(pos, sp):
        kvc.set_length(pos)
        x.copy_(xh)
        for li, (wq, wk, wv, wo, wg, wu, wd) in enumerate(layer_ws):
            sq.rmsnorm_matmul_multi_dev([wq, wk, wv], P(x), P(nw), eps, 1, H, [P(q), P(k), P(v)], sp)
            sq.attention_dev(kvc, li, prm, P(q), P(k), P(v), 1, pos, P(att), sp)
            sq.matmul_add_dev(wo, P(att), 1, H, P(x), sp)
            sq.rmsnorm_matmul_swiglu_dev(wg, wu, P(x), P(nw), eps, 1, H, P(h), sp)
            sq.matmul_add_dev(wd, P(h), 1, F, P(x), sp)
        sq.rmsnorm_matmul_argmax_dev(head, P(x), P(nw), eps, P(tok), 0, sp)

    def attention_only(pos, sp):
        kvc.set_length(pos)
        for li in range(L):
            sq.attention_dev(kvc, li, prm, P(q), P(k), P(v), 1, pos, P(att), sp)

    def timed(run, n, st) -> float:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(st)
        for _ in range(n):
            run()
        b.record(st)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / n

    def graph_of(fn, pos, cs):
        # eager uses on cs first: its workspace, counters and argmax scratch
        # are allocated before the capture
        with torch.cuda.stream(cs):
            fn(pos, cs.cuda_stream)
            fn(pos, cs.cuda_stream)
        cs.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cs):
            fn(pos, cs.cuda_stream)
        return g

    res = {}
    cs = torch.cuda.Stream()
    for pos in (128, 2047):
        # eager, driven from Python (host-bound: five ctypes calls per layer)
        for _ in range(2):
            token(pos, stream.cuda_stream)
        torch.cuda.synchronize()
        ms_eager = timed(lambda: token(pos, stream.cuda_stream), tokens, stream)
        want = int(tok.item())
        # the same launches replayed from a HIP graph: the GPU-side cost
        g = graph_of(token, pos, cs)
        tok.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        same = int(tok.item()) == want
        ms = timed(g.replay, tokens, stream)  # replay() runs on the current stream
        del g
        ga = graph_of(attention_only, pos, cs)
        ms_att = timed(ga.replay, max(tokens, 20), stream)
        del ga
        att_us = ms_att * 1e3 / L
        kv_bytes = 2 * NKV * (pos + 1) * DK * 4  # K and V rows read per layer
        res[f"decode_full_tok_s_kv{pos}"] = round(1e3 / ms, 1)
        res[f"decode_full_ms_per_token_kv{pos}"] = round(ms, 4)
        res[f"decode_full_eager_tok_s_kv{pos}"] = round(1e3 / ms_eager, 1)
        res[f"decode_full_graph_matches_eager_kv{pos}"] = same
        res[f"attention_us_per_layer_kv{pos}"] = round(att_us, 2)
        res[f"attention_kv_GBps_kv{pos}"] = round(kv_bytes / (att_us * 1e-6) / 1e9, 1)
    res["decode_full_note"] = ("whole step on the device: 32 x [RMSNorm+qkv, attention (split kernel with the "
                               "q/k preparation and the cache append, + a combine launch when the positions "
                               "are split over workgroups: at KV 2047, not at KV 128), o + residual, "
                               "RMSNorm+gate/up+SwiGLU, down + residual] + RMSNorm+head+argmax, + one "
                               "embedding-row copy: 161 launches per token at KV 128, 193 at KV 2047 "
                               "(Llama-3-8B shape: 32 q heads, 8 kv heads, d_k 128, RoPE base 500000), replayed "
                               "from a HIP graph (the GPU-side cost); _eager: the same calls issued from Python "
                               "(host-bound). attention_us_per_layer: the attention launches of one layer "
                               "(graph of the 32 layers' calls); attention_kv_GBps: K and V bytes read per layer "
                               "over that time")
    kvc.close()
    return res


def cpu_baseline(sq, synth, gate_raw, up_raw, down_raw, copies: int, step_bytes: int,
                 budget_s: float = 12.0) -> dict:
    """Restated reference CPU path (AVX2/AVX-VNNI kernels, parallel.go pool) on C3 steps.

    The weights are the same remapped bytes the GPU streams (exported from the
    device planes). Steps rotate over `copies` layer copies (> 1 GiB), so the
    host's caches do not hold the weights either; runs for ~budget_s seconds.
    """
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes as C
    import numpy as np
    import oracle  # the cpu_baseline leg is the one part of bench.py allowed to use oracle/

    H, F = 4096, 14336
    B = oracle.baseline()
    workers = B.bl_workers()
    one = [sq.load_weight_f32_direct(synth.GGML_Q4_K, gate_raw, F, H),
           sq.load_weight_f32_direct(synth.GGML_Q4_K, up_raw, F, H),
           sq.load_weight_f32_direct(synth.GGML_Q6_K, down_raw, H, F)]
    base = [w.export() for w in one]
    host = [tuple(b.copy() for b in base) for _ in range(copies)]
    x = synth.normal(1, H).reshape(1, -1)
    hx = synth.normal(2, F).reshape(1, -1)
    yg = np.empty(F, np.float32)
    yd = np.empty(H, np.float32)
    P = lambda a: C.c_void_p(a.ctypes.data)

    def step(i):
        gr, ur, dr = host[i % len(host)]
        B.bl_matmul(b"q4_1", P(gr), F, H, P(x), 1, P(yg))
        B.bl_matmul(b"q4_1", P(ur), F, H, P(x), 1, P(yg))
        B.bl_matmul(b"q8", P(dr), H, F, P(hx), 1, P(yd))

    for i in range(len(host)):
        step(i)
    t0 = time.time()
    n = 0
    while n < len(host) or time.time() - t0 < budget_s:
        step(n)
        n += 1
    sec = (time.time() - t0) / n
    isa = "VNNI" if B.bl_has_vnni() else "AVX2"
    model = cpu_model()
    return {
        "value": round(step_bytes / sec / 1e9, 2),
        "unit": "GB/s",
        "cores": workers,
        "kind": "port",
        "sample": f"{n} C3 steps rotating over {len(host)} layer copies (gate+up Q4_1 {isa}, down Q8_0 {isa}), "
                  f"{sec * 1e3:.2f} ms/step over {n * sec:.1f} s; {workers} worker threads (parallel.go rule) "
                  f"on {os.cpu_count()} visible CPUs, {model}",
    }


def cpu_model() -> str:
    """The host CPU's model name (lscpu's "Model name", from /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown CPU"


def mfma_peaks() -> dict | None:
    """Sustained int8 MFMA rate of the box, TOPS, from libsllm_probe.so: the
    K = 32 form the prefill GEMM issues (one Q8_0 block per result) and the
    K = 64 form the published 5.0 POPS figure refers to."""
    import ctypes as C
    path = os.path.join(ROOT, "scriptling-llm-lib_amd", "libsllm_probe.so")
    if not os.path.exists(path):
        return None
    L = C.CDLL(path)
    L.sllm_probe_mfma_tops.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
    out = {}
    for form, name in ((0, "v_mfma_i32_16x16x32_i8"), (1, "v_mfma_i32_16x16x64_i8"), (2, "v_mfma_i32_32x32x32_i8")):
        for blocks in (1024, 4096):
            t = C.c_double()
            if L.sllm_probe_mfma_tops(form, blocks, 2048, 5, C.byref(t)) == 0:
                out[f"{name} x{blocks}"] = round(t.value, 1)
    out["note"] = ("1024 or 4096 workgroups x 4 waves (1 or 4 waves per SIMD), 8 independent MFMA chains per wave "
                   "(4 for the 32x32 form), register operands only; the fastest of 5 launches. The GEMM lines' "
                   "frac_int8_mfma is against the published 5.0 POPS dense figure, not against these.")
    return out


VALU_KINDS = ["v_fma_f32", "v_mul_f32", "v_add_u32", "v_lshrrev_b32", "v_cvt_f32_ubyte1", "v_cvt_i32_f32",
              "v_perm_b32", "v_dot4_i32_i8", "v_bfe_u32", "v_and_or_b32", "v_mad_i32_i24"]


def valu_rates() -> dict | None:
    """VALU issue rate, T lane-instructions per second, of each instruction kind
    in VALU_KINDS on the box, from libsllm_probe.so (eight independent chains
    per lane on register operands, 2048 workgroups x 4 waves, fastest of 5)."""
    import ctypes as C
    path = os.path.join(ROOT, "scriptling-llm-lib_amd", "libsllm_probe.so")
    if not os.path.exists(path):
        return None
    L = C.CDLL(path)
    L.sllm_probe_valu_rate.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.POINTER(C.c_double)]
    out = {}
    for op, name in enumerate(VALU_KINDS):
        t = C.c_double()
        if L.sllm_probe_valu_rate(op, 2048, 1024, 5, C.byref(t)) == 0:
            out[name] = round(t.value, 1)
    return out


def cpu_parity(g0, u0, d0, x, h, got) -> dict:
    """The C3 step's outputs (gate, up, down) against the restated reference
    CPU path (oracle/refcpu_simd.c, the cpu_baseline kernels) on the same
    remapped bytes: the vector-scale relative error the reference's own tests
    use (q8q8_test.go:77-84, max|got - ref| / max|ref|; north star: 1e-5) and
    the argmax of each output."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np
    import oracle  # part of the cpu_baseline leg
    H, F = 4096, 14336
    res, ok = {}, True
    for name, w, xin, qt, n, y in (("gate", g0, x, "q4_1", F, got[0]), ("up", u0, x, "q4_1", F, got[1]),
                                   ("down", d0, h, "q8", H, got[2])):
        ref = oracle.baseline_matmul(qt, w.export(), n, xin.reshape(1, -1))[0].astype(np.float64)
        err = float(np.abs(y.astype(np.float64) - ref).max() / np.abs(ref).max())
        same = int(np.argmax(y)) == int(np.argmax(ref))
        res[name] = {"max_rel_err": err, "argmax_equal": same}
        ok = ok and err <= 1e-5 and same
    res["ok"] = ok
    res["reference"] = "oracle/refcpu_simd.c (AVX2/AVX-VNNI restatement, the cpu_baseline kernels)"
    return res


if __name__ == "__main__":
    sys.exit(main())
