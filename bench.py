"""Benchmark: Q4_K decode GEMV weight GB/s on one MI355X, plus the prefill GEMM.

Default workload (the config the headline metric is quoted on): one decode step
of Llama-3.2-3B's Q4_K linear layers at M=1 — 28 layers x (q, k, v, o, gate, up,
down) + lm_head = 197 GEMVs over 1,807,073,280 weight bytes (synthetic weights with
the benchmark distribution, fp16 N(0,1) activations, fp32 output).  The weight set
is 7x the 256 MB Infinity Cache, so every launch streams its weights from HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-prefill] [--no-configs]
                    [--decode-only [--eager]] [--configs-only] [--copy-calibration]
    python bench.py --prefill-only [--eager] [--gemm-opts N]

Prints ONE JSON line.  The step's 197 launches are captured once in a HIP graph (the decode loop is
launch-bound otherwise); ``value`` = total weight bytes x K / elapsed time of K
graph replays (HIP events on the replay stream, synchronized on both sides).
``roofline`` is for the dominant kernel (the Q4_K v_dot2 GEMV, every launch of the
step): algorithmic bytes per launch / the timed region's average launch duration (time
per step / 197); ``per_shape`` adds each weight shape's average launch duration from a
graph of launches over distinct weights of that shape totalling >= 512 MB (HBM-cold),
timed the same way (``--roofline-only`` runs the step and these graphs, for the
profiler).  ``cpu_baseline`` times the CPU restatement
(NumPy dequant + PyTorch-CPU fp32 matmul) on one layer and on configs 1, 3, 4 and 5.
``prefill_gemm`` reports the Q4_K MFMA GEMM at M = 512, 2048, 4096 on the three config-4
shapes, ``prefill_gemm_other_formats`` the other formats' GEMM at M = 2048;
``other_configs`` the remaining BASELINE configurations (1, 3 and 5) with their weight
GB/s, each timed over rotating weight copies of >= 512 MB.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2516.6

LAYERS = 28
# (name, K, N) per transformer layer, then lm_head
LLAMA32_3B = [("q", 3072, 3072), ("k", 3072, 1024), ("v", 3072, 1024), ("o", 3072, 3072),
              ("gate", 3072, 8192), ("up", 3072, 8192), ("down", 8192, 3072)]
LM_HEAD = ("lm_head", 3072, 128256)
PREFILL = [(4096, 4096), (4096, 14336), (14336, 4096)]   # (K, N)


def q4k_bytes(K, N):
    return (K // 256) * 144 * N


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def build_decode_step(dev):
    import torch
    from alloy_amd import synth

    mats = []
    seed = 1000
    for layer in range(LAYERS):
        for name, K, N in LLAMA32_3B:
            mats.append((f"{name}{layer}", K, N, synth.torch_blocks("q4_k", N, K, seed, dev)))
            seed += 1
    name, K, N = LM_HEAD
    mats.append((name, K, N, synth.torch_blocks("q4_k", N, K, seed, dev)))
    xs = {K: synth.torch_x(1, K, 7 + K, dev) for K in (3072, 8192)}
    ys = {N: torch.empty((1, N), dtype=torch.float32, device=dev) for N in {m[2] for m in mats}}
    return mats, xs, ys


def run_step(mats, xs, ys, qmm):
    for _, K, N, w in mats:
        qmm("q4_k", xs[K], w, out=ys[N])


def run_batched_step(mats, xs):
    """The same weights through the reference's batched projections (its trace-time
    rewrite, packages/alloy-torch/src/alloy_torch/rewrites/dequant.py:394-436):
    per layer batched(q, k, v), o, batched(gate, up), down; then lm_head."""
    import torch

    op = torch.ops.alloy.batched_gguf_q4_k_mm
    per = len(LLAMA32_3B)
    for layer in range(LAYERS):
        q, k, v, o, g, u, d = mats[layer * per:(layer + 1) * per]
        op(xs[3072], [q[3], k[3], v[3]])
        op(xs[3072], [o[3]])
        op(xs[3072], [g[3], u[3]])
        op(xs[8192], [d[3]])
    op(xs[3072], [mats[-1][3]])


def capture(fn, dev):
    """Capture fn's launches (on torch's capture stream) into a HIP graph."""
    import torch

    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        fn()                                    # warm: first launches outside capture
    torch.cuda.current_stream(dev).wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def time_replays(g, steps, warmup, stream):
    import torch

    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1000.0


MIN_ROTATE_BYTES = 512_000_000   # 2x the 256 MB Infinity Cache: every launch reads its weights from HBM


def per_shape_times(mats, xs, ys, qmm, dev, reps=5):
    """Average launch duration per weight shape: a graph of launches over distinct
    weights totalling >= 512 MB (the step's own matrices of that shape, plus copies),
    replayed `reps` times, divided by launches (HBM-cold, inter-kernel gaps included)."""
    import torch

    from alloy_amd import synth

    stream = torch.cuda.current_stream(dev)
    out = {}
    for key in sorted({(K, N) for _, K, N, _ in mats}):
        K, N = key
        sel = [m for m in mats if (m[1], m[2]) == key]
        need = max(len(sel), -(-MIN_ROTATE_BYTES // q4k_bytes(K, N)))
        seq = sel + [(f"copy{i}", K, N, synth.torch_blocks("q4_k", N, K, 4242 + i, dev))
                     for i in range(need - len(sel))]
        g = capture(lambda: [qmm("q4_k", xs[K], w, out=ys[N]) for _, K, N, w in seq], dev)
        t = time_replays(g, reps, 2, stream)
        out[key] = t / (reps * len(seq))
        del g, seq
    return out


def _median_time(fn, budget_s, max_reps=20, min_reps=3):
    fn()                                              # warm-up
    times, t_all = [], time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - t_all < budget_s and len(times) < max_reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], len(times)


def roofline(mats, xs, ys, qmm, dev, total_bytes, step_s):
    """Roofline of the dominant kernel (the Q4_K M=1 GEMV, every launch of the step):
    algorithmic bytes per launch = the step's N*K/256*144 weight bytes / its launches;
    average launch duration = the timed region's time per step (HIP events on the replay
    stream) / launches.  per_shape: each weight shape's average launch duration from its
    own graph over >= 512 MB of distinct weights (per_shape_times), and the step fraction
    those give when weighted by the shapes' launches (per_shape_frac)."""
    per = per_shape_times(mats, xs, ys, qmm, dev)
    counts = {}
    for _, K, N, _ in mats:
        counts[(K, N)] = counts.get((K, N), 0) + 1
    tot_t = sum(per[k] * c for k, c in counts.items())
    launches = len(mats)
    achieved = total_bytes / step_s / 1e9
    shapes = {f"{K}x{N}": {"us": round(v * 1e6, 2), "GBps": round(q4k_bytes(K, N) / v / 1e9, 1),
                           "launches_per_step": counts[(K, N)]}
              for (K, N), v in per.items()}
    return {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic_from_profiles(),
            "kernel": "k_gemv_w1<FQ4K> (Q4_K M=1 wave-row GEMV, single-matrix entry)",
            "bytes_per_launch": round(total_bytes / launches),
            "avg_launch_us": round(step_s / launches * 1e6, 3), "per_shape": shapes,
            "per_shape_frac": round(total_bytes / tot_t / 1e9 / HBM_PEAK_GBS, 4),
            "per_shape_avg_launch_us": round(tot_t / launches * 1e6, 3)}


def cpu_baseline():
    """The reference path's CPU restatement, timed on this host: NumPy decode of the wire
    blocks (the oracle's formulas) + PyTorch-CPU fp32 matmul, per call, and the matmul
    alone on pre-decoded weights.  Headline row: one Llama-3.2-3B layer (config 2, M=1);
    further rows: config 1, config 3 (one Q6_K and one Q5_0 shape, M=1), config 4
    (M=512, one shape), config 5 (MLX MoE, T=1)."""
    import numpy as np
    import torch

    from alloy_amd import synth
    from oracle import moe as om
    from oracle import quant as oq

    torch.set_num_threads(os.cpu_count() or 1)
    rng = np.random.default_rng(0)
    rows = []

    def dense_row(name, fmt, K, N, M, budget):
        blob = synth.numpy_blocks(fmt, N, K, rng)
        x = torch.from_numpy(synth.numpy_x(M, K, rng)).float()
        W = torch.from_numpy(oq.dequant(fmt, blob, K))
        t_full, n_full = _median_time(lambda: torch.matmul(x, torch.from_numpy(oq.dequant(fmt, blob, K)).T), budget)
        t_mm, n_mm = _median_time(lambda: torch.matmul(x, W.T), budget / 4)
        nbytes = blob.nbytes
        rows.append({"config": name, "format": fmt, "M": M, "K": K, "N": N, "weight_bytes": nbytes,
                     "dequant_matmul_ms": round(t_full * 1e3, 3), "matmul_only_ms": round(t_mm * 1e3, 3),
                     "weight_GBps": round(nbytes / t_full / 1e9, 4), "TFLOPs": round(2 * M * N * K / t_full / 1e12, 5),
                     "reps": [n_full, n_mm]})

    # headline: config 2, one transformer layer (7 matrices), M = 1
    layer = [(K, N, synth.numpy_blocks("q4_k", N, K, rng)) for _, K, N in LLAMA32_3B]
    xs = {K: torch.from_numpy(synth.numpy_x(1, K, rng)).float() for K in (3072, 8192)}
    Ws = [torch.from_numpy(oq.dequant_q4_k(b, K)) for K, _, b in layer]
    nbytes = sum(q4k_bytes(K, N) for K, N, _ in layer)
    t_layer, n_layer = _median_time(lambda: [torch.matmul(xs[K], torch.from_numpy(oq.dequant_q4_k(b, K)).T)
                                             for K, _, b in layer], 5.0)
    t_layer_mm, _ = _median_time(lambda: [torch.matmul(xs[K], W.T) for (K, _, _), W in zip(layer, Ws)], 1.5)
    del Ws
    rows.append({"config": "config2 Llama-3.2-3B layer (7 matrices)", "format": "q4_k", "M": 1, "weight_bytes": nbytes,
                 "dequant_matmul_ms": round(t_layer * 1e3, 3), "matmul_only_ms": round(t_layer_mm * 1e3, 3),
                 "weight_GBps": round(nbytes / t_layer / 1e9, 4), "reps": [n_layer]})
    dense_row("config1", "q8_0", 4096, 4096, 1, 2.0)
    dense_row("config3", "q6_k", 4096, 4096, 1, 2.0)
    dense_row("config3", "q5_0", 4096, 4096, 1, 2.0)
    dense_row("config4", "q4_k", 4096, 4096, 512, 3.0)
    # config 5: MLX MoE, T = 1 (router + the 8 routed experts' gate/up and down)
    E, k, H, I, gs = 128, 8, 2048, 768, 64
    gu = [synth.numpy_mlx(2 * I, H, gs, rng) for _ in range(E)]
    dn = [synth.numpy_mlx(H, I, gs, rng) for _ in range(E)]
    x5 = synth.numpy_x(1, H, rng).astype(np.float32)
    lg = rng.standard_normal((1, E)).astype(np.float32)

    def moe(decoded=None):
        idx, w = om.router_topk(lg, k)
        y = torch.zeros(H)
        xt = torch.from_numpy(x5[0])
        for s_ in range(k):
            e = int(idx[0, s_])
            G, D = decoded[e] if decoded else (torch.from_numpy(oq.dequant_mlx_q4(*gu[e], gs)),
                                               torch.from_numpy(oq.dequant_mlx_q4(*dn[e], gs)))
            a = G @ xt
            h = torch.nn.functional.silu(a[:I]) * a[I:]
            y += float(w[0, s_]) * (D @ h)
        return y

    t_moe, n_moe = _median_time(moe, 2.0)
    used = {int(e) for e in om.router_topk(lg, k)[0][0]}
    dec = {e: (torch.from_numpy(oq.dequant_mlx_q4(*gu[e], gs)), torch.from_numpy(oq.dequant_mlx_q4(*dn[e], gs)))
           for e in used}
    t_moe_mm, _ = _median_time(lambda: moe(dec), 0.5)
    moe_bytes = len(used) * (2 * I * (H // 2 + 4 * H // gs) + H * (I // 2 + 4 * I // gs))
    rows.append({"config": "config5 MLX MoE", "format": "mlx_q4", "T": 1, "weight_bytes": moe_bytes,
                 "dequant_matmul_ms": round(t_moe * 1e3, 3), "matmul_only_ms": round(t_moe_mm * 1e3, 3),
                 "weight_GBps": round(moe_bytes / t_moe / 1e9, 4), "reps": [n_moe]})
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": rows[0]["weight_GBps"],
        "unit": "weight GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"one Llama-3.2-3B layer (7 Q4_K matrices, {nbytes} weight bytes), M=1, NumPy dequant + torch "
                  f"fp32 matmul per call, median of {n_layer} reps; further rows: configs 1, 3 (4096x4096), 4 (M=512, 4096x4096), "
                  f"5 (T=1), each also timed as matmul only on pre-decoded weights",
        "ms_per_call": rows[0]["dequant_matmul_ms"],
        "cpu_model": model,
        "os_cpu_count": os.cpu_count(),
        "torch_threads": torch.get_num_threads(),
        "rows": rows,
    }


def prefill_gemm(dev, qmm, Ms=(512, 2048, 4096), reps=10, opts=0, eager=False):
    """Q4_K GEMM on the config-4 shapes; opts: forced tile / split (bits 36-39, 40-43);
    eager: direct launches timed by events (counter runs) instead of graph replays."""
    import torch

    from alloy_amd import synth

    out = []
    for M, (K, N) in [(M, kn) for M in Ms for kn in PREFILL]:
        w = synth.torch_blocks("q4_k", N, K, 77 + N, dev)
        x = synth.torch_x(M, K, 78 + K, dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        stream = torch.cuda.current_stream(dev)
        fn = lambda: qmm("q4_k", x, w, out=y, path="gemm", opts=opts)  # noqa: E731
        if eager:
            fn()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(reps):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            t = e0.elapsed_time(e1) / 1000.0 / reps
        else:
            g = capture(fn, dev)
            t = time_replays(g, reps, 2, stream) / reps
        tf = 2.0 * M * N * K / t / 1e12
        out.append({"M": M, "K": K, "N": N, "us": round(t * 1e6, 1), "tflops": round(tf, 2),
                    "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)})
        del w, x, y
    return out


def prefill_gemm_other_formats(dev, qmm, M=2048, reps=5):
    """The prefill GEMM of the other formats (generic double-buffered kernel) on config-4
    shapes at M = 2048, graph replays, fp32 output."""
    import torch

    from alloy_amd import synth

    out = []
    for fmt in ("q8_0", "q5_0", "q6_k", "mlx_q4"):
        for K, N in [(4096, 4096), (4096, 14336)]:
            if fmt == "mlx_q4":
                q, sc, bi = synth.torch_mlx(N, K, 64, 90 + N, dev)
                fn_w = lambda xx, yy: qmm("mlx_q4", xx, q, scales=sc, biases=bi, group_size=64, out=yy,  # noqa: E731
                                          path="gemm")
            else:
                w = synth.torch_blocks(fmt, N, K, 90 + N, dev)
                fn_w = lambda xx, yy, w=w, fmt=fmt: qmm(fmt, xx, w, out=yy, path="gemm")  # noqa: E731
            x = synth.torch_x(M, K, 91 + K, dev)
            y = torch.empty((M, N), dtype=torch.float32, device=dev)
            g = capture(lambda: fn_w(x, y), dev)
            t = time_replays(g, reps, 2, torch.cuda.current_stream(dev)) / reps
            tf = 2.0 * M * N * K / t / 1e12
            out.append({"format": fmt, "M": M, "K": K, "N": N, "us": round(t * 1e6, 1), "tflops": round(tf, 2),
                        "frac_fp16_peak": round(tf / FP16_PEAK_TFLOPS, 4)})
            del g, x, y
    return out


def _rotating_time(dev, fn_for, copies, reps=5, eager=False):
    """Average seconds per call of fn_for(copy) over a graph that cycles through
    `copies` (together larger than the 256 MB Infinity Cache, so weights come from HBM);
    eager: the same calls launched directly (counter runs)."""
    import torch

    seq = copies * max(1, 24 // len(copies))
    stream = torch.cuda.current_stream(dev)
    if eager:
        for c in seq:
            fn_for(c)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(reps):
            for c in seq:
                fn_for(c)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / 1000.0 / (reps * len(seq))
    g = capture(lambda: [fn_for(c) for c in seq], dev)
    t = time_replays(g, reps, 2, stream) / (reps * len(seq))
    del g
    return t


def other_configs(dev, qmm, eager=False):
    """The other BASELINE configurations, on the GPU: config 1 (Q8_0 4096x4096, M=1,
    fp32 out), config 3 (Q6_K and Q5_0 at Llama-3-8B shapes, M=1 and M=8) and config 5
    (MLX 4-bit MoE, 128 experts, top-8, H=2048, I=768, T in {1, 16, 256}); config 2 is
    repeated at M=4 and M=16 (its distinct shapes)."""
    import torch

    from alloy_amd import formats, synth

    out = {}

    def gemv_case(fmt, K, N, M, seed):
        nbytes = formats.row_bytes(fmt, K) * N
        ncopy = max(2, -(-MIN_ROTATE_BYTES // nbytes))
        ws = [synth.torch_blocks(fmt, N, K, seed + i, dev) for i in range(ncopy)]
        x = synth.torch_x(M, K, seed, dev)
        y = torch.empty((M, N), dtype=torch.float32, device=dev)
        t = _rotating_time(dev, lambda w: qmm(fmt, x, w, out=y), ws, eager=eager)
        del ws
        return {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                "frac_hbm_peak": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}

    out["config1_q8_0_4096x4096_M1"] = gemv_case("q8_0", 4096, 4096, 1, 300)
    # the same weights in the layout the reference's gguf_q8_0_mm takes (int8 quants and
    # fp16 scales in separate arrays, same bytes): its drop-in call
    nbytes = formats.row_bytes("q8_0", 4096) * 4096
    ws = [synth.torch_q8_0_split(4096, 4096, 310 + i, dev) for i in range(max(2, -(-MIN_ROTATE_BYTES // nbytes)))]
    x1 = synth.torch_x(1, 4096, 300, dev)
    y1 = torch.empty((1, 4096), dtype=torch.float32, device=dev)
    t = _rotating_time(dev, lambda w: qmm("q8_0_split", x1, w[0], scales=w[1], N=4096, out=y1), ws, eager=eager)
    del ws
    out["config1_q8_0_split_4096x4096_M1"] = {"us": round(t * 1e6, 2), "GBps": round(nbytes / t / 1e9, 1),
                                              "frac_hbm_peak": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4),
                                              "layout": "split (the reference op's qweight + scales)"}
    for M in (4, 16):
        out[f"config2_q4_k_M{M}"] = {f"{K}x{N}": gemv_case("q4_k", K, N, M, 350 + K + N)
                                     for _, K, N in LLAMA32_3B[:2] + LLAMA32_3B[4:5] + LLAMA32_3B[6:] + [LM_HEAD]}
    for fmt in ("q6_k", "q5_0"):
        for M in (1, 8):
            out[f"config3_{fmt}_M{M}"] = {f"{K}x{N}": gemv_case(fmt, K, N, M, 400 + K + N)
                                           for K, N in [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]}
    # config 5: MLX MoE
    E, k, H, I, gs = 128, 8, 2048, 768, 64
    experts = []
    for c in range(2):                       # 2 x 340 MB rotate past the Infinity Cache
        gq, gsc, gbi = synth.torch_mlx(E * 2 * I, H, gs, 500 + c, dev)   # scales |N(0,1)|*0.01, biases N(0, 0.01)
        dq, dsc, dbi = synth.torch_mlx(E * H, I, gs, 600 + c, dev)
        experts.append((gq.view(E, 2 * I, H // 2), gsc.view(E, 2 * I, H // gs), gbi.view(E, 2 * I, H // gs),
                        dq.view(E, H, I // 2), dsc.view(E, H, I // gs), dbi.view(E, H, I // gs)))
    per_expert = sum(t.numel() * t.element_size() for t in experts[0]) // E
    moe = {}
    for T in (1, 16, 256):
        x = synth.torch_x(T, H, 600 + T, dev)
        lg = torch.randn((T, E), device=dev, generator=torch.Generator(device=dev).manual_seed(T))
        t = _rotating_time(dev, lambda c: torch.ops.alloy.mlx_moe_routed(x, lg, *c, E, k, I), experts, eager=eager)
        touched = int(torch.unique(torch.topk(lg, k, dim=1).indices).numel())
        moe[f"T{T}"] = {"us": round(t * 1e6, 1), "experts_touched": touched,
                        "GBps_touched_weights": round(touched * per_expert / t / 1e9, 1)}
    out["config5_mlx_moe"] = moe
    del experts
    return out


def traffic_from_profiles():
    """HBM bytes per launch of the dominant kernel, from the committed PMC summary
    (a line ``traffic_bytes_per_launch = N`` in profiles/q4k_gemv_decode_pmc.md)."""
    import re

    p = ROOT / "profiles" / "q4k_gemv_decode_pmc.md"
    try:
        m = re.search(r"^traffic_bytes_per_launch = (\d+)", p.read_text(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def copy_calibration(dev, mib=256, reps=5):
    """A plain device copy of known size (torch's copy kernel), for scaling the
    FETCH_SIZE / WRITE_SIZE counters: each launch reads and writes mib MiB."""
    import torch

    a = torch.empty(mib << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    a.fill_(1)
    torch.cuda.synchronize()
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": mib << 20, "launches": reps}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other BASELINE configurations")
    ap.add_argument("--decode-only", action="store_true",
                    help="time the decode step only (no per-shape, prefill or CPU legs)")
    ap.add_argument("--eager", action="store_true",
                    help="launch eagerly instead of replaying HIP graphs (counter runs; decode step or configs)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="time only the per-shape graphs the roofline is computed from (profiler runs)")
    ap.add_argument("--cpu-only", action="store_true",
                    help="run only the CPU baseline (no GPU needed) and print it")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 256 MiB device copy (counter calibration) and exit")
    ap.add_argument("--configs-only", action="store_true",
                    help="time only the other BASELINE configurations (profiler runs of their kernels)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time only the config-4 prefill GEMMs (with --eager: direct launches)")
    ap.add_argument("--gemm-opts", type=int, default=0,
                    help="alloy_qmm opts for --prefill-only: forced Q4_K tile (bits 36-39) and K splits (40-43)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    if args.cpu_only:
        print(json.dumps({"cpu_baseline": cpu_baseline()}))
        return
    import torch

    import alloy_amd
    from alloy_amd import qmm

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        copy_calibration(dev)
        return
    alloy_amd.lib()
    if args.configs_only:
        print(json.dumps({"other_configs": other_configs(dev, qmm, eager=args.eager), "eager": args.eager}))
        return
    if args.prefill_only:
        print(json.dumps({"prefill_gemm": prefill_gemm(dev, qmm, opts=args.gemm_opts, eager=args.eager),
                          "gemm_opts": args.gemm_opts, "eager": args.eager}))
        return
    log("building decode step weights ...")
    mats, xs, ys = build_decode_step(dev)
    total_bytes = sum(q4k_bytes(K, N) for _, K, N, _ in mats)
    if args.roofline_only:
        g = capture(lambda: run_step(mats, xs, ys, qmm), dev)
        t = time_replays(g, args.steps, args.warmup, torch.cuda.current_stream(dev))
        del g
        print(json.dumps({"roofline": roofline(mats, xs, ys, qmm, dev, total_bytes, t / args.steps)}))
        return
    stream = torch.cuda.current_stream(dev)
    if args.eager:
        log(f"{len(mats)} GEMVs, {total_bytes} weight bytes; eager launches")
        for _ in range(args.warmup):
            run_step(mats, xs, ys, qmm)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            run_step(mats, xs, ys, qmm)
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
    else:
        log(f"{len(mats)} GEMVs, {total_bytes} weight bytes; capturing the step as a HIP graph")
        graph = capture(lambda: run_step(mats, xs, ys, qmm), dev)
        t = time_replays(graph, args.steps, args.warmup, stream)
    ms = t / args.steps * 1e3
    value = total_bytes * args.steps / t / 1e9
    if args.decode_only:
        print(json.dumps({"decode_step_ms": round(ms, 4), "weight_GBps": round(value, 2),
                          "eager": args.eager, "steps": args.steps}))
        return

    xs16 = {K: v for K, v in xs.items()}
    gb = capture(lambda: run_batched_step(mats, xs16), dev)
    tb = time_replays(gb, args.steps, args.warmup, stream)
    del gb
    batched = {"ms_per_step": round(tb / args.steps * 1e3, 4),
               "weight_GBps": round(total_bytes * args.steps / tb / 1e9, 2),
               "launches_per_step": LAYERS * 4 + 1,
               "note": "same weights and bytes; q/k/v and gate/up each as one batched_gguf_q4_k_mm "
                       "(one launch serving several matrices), fp16 outputs"}
    log(json.dumps({"batched_step": batched}))

    roof = roofline(mats, xs, ys, qmm, dev, total_bytes, t / args.steps)
    log(json.dumps(roof["per_shape"]))

    prefill = None if args.no_prefill else prefill_gemm(dev, qmm)
    if prefill:
        log(json.dumps(prefill))
    prefill_other = None if args.no_prefill else prefill_gemm_other_formats(dev, qmm)
    if prefill_other:
        log(json.dumps({"prefill_gemm_other_formats": prefill_other}))
    cpu = None if args.no_cpu else cpu_baseline()
    configs = None if args.no_configs else other_configs(dev, qmm)
    if configs:
        log(json.dumps(configs))

    rec = {
        "metric": "Q4_K decode GEMV weight GB/s (% HBM peak); Q4_K prefill GEMM TFLOP/s",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_k weights x fp16 activations, fp32 accumulate",
        "data": "synthetic (BASELINE config 2 distributions), weights resident in HBM",
        "config": {"workload": "Llama-3.2-3B Q4_K decode step, M=1: 28 layers x (q,k,v,o,gate,up,down) + lm_head",
                   "launches_per_step": len(mats), "weight_bytes_per_step": total_bytes,
                   "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roof,
        "cpu_baseline": cpu,
        "prefill_gemm": prefill,
        "prefill_gemm_other_formats": prefill_other,
        "batched_step": batched,
        "other_configs": configs,
    }
    print(json.dumps(rec))


if __name__ == "__main__":
    main()
