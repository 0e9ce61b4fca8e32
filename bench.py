#!/usr/bin/env python3
"""Benchmark of the quantized linear-layer path on one MI355X.

Headline workload (the `value`): the Q4_K decode GEMV set of one
Qwen2-0.5B-shaped layer at batch 1 -- q/o 896x896, k/v 128x896, gate/up
4864x896, down 896x4864, f32 activations and outputs.  One step is one decode
token through R distinct device copies of that layer (R*7 GEMV launches,
R*8.48 MB >= 1 GB so the 256 MB Infinity Cache cannot hold the weights),
captured once as a HIP graph and replayed.  value = algorithmic bytes per step
(GGUF block bytes + activation bytes + output bytes) / time per step.

The same JSON line carries the roofline of the dominant kernel (the gate/up
projection GEMV, timed in its own graph of R launches), a CPU baseline (the
oracle's runtimed-gguf dequant + f32 GEMV on this host's cores) and, under
"extra", the other workloads: the decode set with fused weights, the Q8_0
GEMV, the streaming-shape Q4_K GEMV, the small-M verify sweep (bf16 and f32
activations), the M=512 prefill GEMMs, the FP8 e4m3 GEMM, the Marlin INT4
GEMV, the paged-KV quantizer, the GGUF upload and a vendor-BLAS reference
point.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP8_PEAK_TFLOPS = 5000.0

# (name, n, k) of the Qwen2-0.5B layer, y = x W^T with W [n, k]
LAYER = [("q", 896, 896), ("k", 128, 896), ("v", 128, 896), ("o", 896, 896),
         ("gate", 4864, 896), ("up", 4864, 896), ("down", 896, 4864)]
Q4K_BLOCK = 144


def layer_bytes(act_bytes=4, out_bytes=4, m=1):
    w = sum(n * k // 256 * Q4K_BLOCK for _, n, k in LAYER)
    x = sum(m * k * act_bytes for _, n, k in LAYER)
    y = sum(m * n * out_bytes for _, n, k in LAYER)
    return w + x + y


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


class Timer:
    """HIP-event timing of graph replays on the current stream."""

    def __init__(self, torch):
        self.torch = torch

    def replay(self, graph, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            graph.replay()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            graph.replay()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps  # ms per replay


def capture(torch, fn):
    """fn's launches in a HIP graph, captured on the stream that ran fn once
    eagerly just before (its library workspace already has the size fn
    needs, so the graph holds no allocations)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        fn()
    torch.cuda.synchronize()
    return g


def decode_workload(torch, rq, synth, layers, steps, warmup, dev):
    """The headline: R layers x 7 Q4_K GEMVs, one token, f32 in and out."""
    blocks = {name: synth.q4_k_blocks(100 + i, n * k // 256) for i, (name, n, k) in enumerate(LAYER)}
    W = [{name: rq.QWeight(rq.Q4_K, blocks[name], n, k) for name, n, k in LAYER} for _ in range(layers)]
    x896 = torch.from_numpy(synth.activations(1, 1, 896)).to(dev)
    x4864 = torch.from_numpy(synth.activations(2, 1, 4864)).to(dev)
    ys = {name: torch.empty((1, n), dtype=torch.float32, device=dev) for name, n, k in LAYER}

    def token():
        for lw in W:
            for name, n, k in LAYER:
                lw[name].forward(x4864 if k == 4864 else x896, out=ys[name])

    timer = Timer(torch)
    g = capture(torch, token)
    ms = timer.replay(g, steps, warmup)
    del g
    return W, ms


def extra_decode_fused(torch, rq, synth, layers, steps, warmup, dev):
    """The same layer set with the usual load-time weight fusion: q/k/v
    concatenated into one 1152x896 weight and gate/up into one 9728x896 (the
    GGUF streams concatenate exactly: every matrix holds a whole number of
    Q4_K blocks), so a token is 4 GEMVs per layer over the same bytes."""
    blocks = {name: synth.q4_k_blocks(100 + i, n * k // 256) for i, (name, n, k) in enumerate(LAYER)}
    qkv = np.concatenate([blocks["q"], blocks["k"], blocks["v"]])
    gu = np.concatenate([blocks["gate"], blocks["up"]])
    fused = [("qkv", qkv, 1152, 896), ("o", blocks["o"], 896, 896), ("gate_up", gu, 9728, 896),
             ("down", blocks["down"], 896, 4864)]
    W = [[(rq.QWeight(rq.Q4_K, b, n, k), n, k) for _, b, n, k in fused] for _ in range(layers)]
    x896 = torch.from_numpy(synth.activations(1, 1, 896)).to(dev)
    x4864 = torch.from_numpy(synth.activations(2, 1, 4864)).to(dev)
    ys = {n: torch.empty((1, n), dtype=torch.float32, device=dev) for _, _, n, _ in fused}

    def token():
        for lw in W:
            for w, n, k in lw:
                w.forward(x4864 if k == 4864 else x896, out=ys[n])

    g = capture(torch, token)
    ms = Timer(torch).replay(g, steps, warmup)
    del g, W
    value = layer_bytes() * layers / (ms * 1e-3) / 1e9
    return {"workload": "decode layer set with fused q/k/v and gate/up weights (4 GEMVs per layer, same bytes)",
            "GB/s": round(value, 1), "frac_hbm": round(value / HBM_PEAK_GBS, 4),
            "us_per_layer": round(ms * 1e3 / layers, 2)}


def extra_decode_multi(torch, rq, W, steps, warmup, dev):
    """The headline's 7 GEMVs per layer on the same 128 weight copies, issued
    as the reference's layer issues them: q/k/v and gate/up each share their
    input (qwen2.rs:99-125), so each triple / pair is one rq_linear_multi
    call (one launch, separate weights and outputs), o and down one call
    each: 4 launches per layer, same bytes."""
    x896 = torch.from_numpy(synth_act(1, 896)).to(dev)
    x4864 = torch.from_numpy(synth_act(2, 4864)).to(dev)
    ys = {name: torch.empty((1, n), dtype=torch.float32, device=dev) for name, n, k in LAYER}
    sets = [([lw["q"], lw["k"], lw["v"]], [lw["o"]], [lw["gate"], lw["up"]], [lw["down"]]) for lw in W]
    outs = ([ys["q"], ys["k"], ys["v"]], [ys["o"]], [ys["gate"], ys["up"]], [ys["down"]])

    def token():
        for layer in sets:
            for ws, yl, x in zip(layer, outs, (x896, x896, x896, x4864)):
                rq.linear_multi_into(ws, x, yl)

    g = capture(torch, token)
    ms = Timer(torch).replay(g, steps, warmup)
    del g
    value = layer_bytes() * len(W) / (ms * 1e-3) / 1e9
    return {"workload": "decode layer set, q/k/v and gate/up through rq_linear_multi (4 launches per layer, "
                        "same 7 weights and outputs)",
            "GB/s": round(value, 1), "frac_hbm": round(value / HBM_PEAK_GBS, 4),
            "us_per_layer": round(ms * 1e3 / len(W), 2)}


def synth_act(seed, k):
    from runtimed_amd import synth

    return synth.activations(seed, 1, k)


def host_cpu():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1


def cpu_baseline(oracle, synth, budget_s):
    """Oracle dequant (load time) + f32 GEMV over the dequantized layer."""
    threads = cpu_threads()
    blocks = {name: synth.q4_k_blocks(100 + i, n * k // 256) for i, (name, n, k) in enumerate(LAYER)}
    t0 = time.perf_counter()
    dense = {}
    for name, n, k in LAYER:
        rc, wf = oracle.dequant_tensor(12, blocks[name], n * k)
        dense[name] = wf.reshape(n, k)
    deq_1t = time.perf_counter() - t0
    t0 = time.perf_counter()
    for name, n, k in LAYER:
        oracle.dequant_tensor(12, blocks[name], n * k, threads=threads)
    deq_mt = time.perf_counter() - t0
    copies = 16  # 16 x 33.5 MB of f32 weights: larger than a CPU last-level cache slice
    layers = [{nm: w.copy() for nm, w in dense.items()} for _ in range(copies)]
    x896 = synth.activations(1, 1, 896)
    x4864 = synth.activations(2, 1, 4864)
    passes, t0 = 0, time.perf_counter()
    while True:
        for lw in layers:
            for name, n, k in LAYER:
                oracle.linear_f32(x4864 if k == 4864 else x896, lw[name], threads=threads)
        passes += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per_layer = el / (passes * copies)
    gbs = layer_bytes() / per_layer / 1e9
    w_bytes = sum(n * k // 256 * Q4K_BLOCK for _, n, k in LAYER)
    model, nproc = host_cpu()
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "cpu_model": model, "nproc": nproc,
        "sample": f"{passes} passes over {copies} Qwen2-0.5B Q4_K layers (7 f32 GEMVs each on "
                  f"oracle-dequantized weights, blocked OpenMP SGEMV, {threads} threads); "
                  f"{el:.1f} s",
        "ms_per_layer": round(per_layer * 1e3, 4),
        "dequant_load_gbs_1thread": round(w_bytes / deq_1t / 1e9, 3),
        f"dequant_load_gbs_{threads}threads": round(w_bytes / deq_mt / 1e9, 3),
    }


def extra_q8_gemv(torch, rq, synth, dev, steps, warmup):
    n, k = 4864, 896
    blocks = synth.q8_0_blocks(5, n * k // 32)
    copies = 224  # 224 x 4.63 MB > 1 GB
    W = [rq.QWeight(rq.Q8_0, blocks, n, k) for _ in range(copies)]
    x = torch.from_numpy(synth.activations(3, 1, k)).to(dev)
    y = torch.empty((1, n), device=dev)
    g = capture(torch, lambda: [w.forward(x, out=y) for w in W])
    ms = Timer(torch).replay(g, steps, warmup) / copies
    b = n * k // 32 * 34 + k * 4 + n * 4
    return {"workload": "Q8_0 GEMV 4864x896 f32, M=1", "us_per_gemv": round(ms * 1e3, 3),
            "GB/s": round(b / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def extra_large_gemv(torch, rq, synth, dev, steps, warmup):
    """The M=1 GEMV kernel where the launch cost is small next to the bytes:
    Q4_K 14336x4096 (33 MB, a Llama-3-8B FFN shape), 16 copies (528 MB, more
    than the 256 MB Infinity Cache) replayed in a HIP graph."""
    n, k = 14336, 4096
    blocks = synth.q4_k_blocks(9, n * k // 256)
    copies = 16
    W = [rq.QWeight(rq.Q4_K, blocks, n, k) for _ in range(copies)]
    x = torch.from_numpy(synth.activations(4, 1, k)).to(dev)
    y = torch.empty((1, n), device=dev)
    g = capture(torch, lambda: [w.forward(x, out=y) for w in W])
    ms = Timer(torch).replay(g, steps, warmup) / copies
    b = n * k // 256 * Q4K_BLOCK + k * 4 + n * 4
    return {"workload": "Q4_K GEMV 14336x4096 f32, M=1 (streaming shape)", "us_per_gemv": round(ms * 1e3, 3),
            "GB/s": round(b / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def extra_head_gemv(torch, rq, synth, dev, steps, warmup):
    """The decode step's largest GEMV in the Q4_K_M model of the prefill
    workload: the output projection 262144x2048 at M=1 (f32 activations), as
    Q6_K (the Q4_K_M head) and as Q4_K, 3-4 distinct copies (> 1 GB) replayed
    in a HIP graph."""
    n, k = 262144, 2048
    res = []
    for name, qt, copies in (("Q6_K", rq.Q6_K, 3), ("Q4_K", rq.Q4_K, 4)):
        blocks = synth.weight_blocks(qt, 11, n, k)
        W = [rq.QWeight(qt, blocks, n, k) for _ in range(copies)]
        x = torch.from_numpy(synth.activations(12, 1, k)).to(dev)
        y = torch.empty((1, n), device=dev)
        g = capture(torch, lambda: [w.forward(x, out=y) for w in W])
        ms = Timer(torch).replay(g, max(2, steps // 4), 1) / copies
        b = len(blocks) + k * 4 + n * 4
        res.append({"format": name, "us_per_gemv": round(ms * 1e3, 2), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        del g, W
        torch.cuda.empty_cache()
    return {"workload": "decode output projection 262144x2048 f32, M=1", "formats": res}


def extra_verify(torch, rq, W, dev, steps, warmup, dtype=None, ms_list=(1, 2, 4, 8, 16, 64), multi=False):
    """The verify sweep over all layer copies: 7 rq_linear calls per layer,
    or (multi) q/k/v and gate/up each through one rq_linear_multi call."""
    dt = dtype if dtype is not None else torch.bfloat16
    eb = 4 if dt == torch.float32 else 2
    out = []
    for m in ms_list:
        xs = {k: torch.randn((m, k), device=dev).to(dt) for k in (896, 4864)}
        ys = {name: torch.empty((m, n), dtype=dt, device=dev) for name, n, k in LAYER}
        groups = (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))

        def tok():
            for lw in W:
                if multi:
                    for grp in groups:
                        k = lw[grp[0]].k
                        rq.linear_multi_into([lw[nm] for nm in grp], xs[k], [ys[nm] for nm in grp])
                    continue
                for name, n, k in LAYER:
                    lw[name].forward(xs[k], out=ys[name])

        g = capture(torch, tok)
        ms = Timer(torch).replay(g, max(2, steps // 4), 1)
        b = layer_bytes(eb, eb, m) * len(W)  # 128 layer copies: >= 1.08 GB a replay
        fl = 2.0 * m * sum(n * k for _, n, k in LAYER) * len(W)
        out.append({"m": m, "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                    "TFLOP/s": round(fl / (ms * 1e-3) / 1e12, 3),
                    "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        del g
    name = "bf16" if dt == torch.bfloat16 else "f32 (the reference's compute type)"
    how = "q/k/v and gate/up through rq_linear_multi (4 launches a layer)" if multi else "7 launches a layer"
    return {"workload": f"verify sweep, Qwen2-0.5B Q4_K layer, {name} activations, {len(W)} layer copies, {how}",
            "sweep": out}


def extra_prefill(torch, rq, synth, dev, steps, warmup, f32=False):
    m = 512
    shapes = [("q/k/o Q4_K", rq.Q4_K, 2048, 2048), ("v Q6_K", rq.Q6_K, 2048, 2048),
              ("gate/up Q4_K", rq.Q4_K, 8192, 2048), ("down Q6_K", rq.Q6_K, 2048, 8192),
              ("lm_head Q6_K", rq.Q6_K, 262144, 2048)]
    dt = torch.float32 if f32 else torch.bfloat16
    res = []
    for name, qt, n, k in shapes:
        w = rq.QWeight(qt, synth.weight_blocks(qt, 7, n, k), n, k)
        x = torch.randn((m, k), device=dev).to(dt)
        y = torch.empty((m, n), dtype=dt, device=dev)
        w.forward(x, out=y)
        torch.cuda.synchronize()
        # launches captured in one graph (the split-K shapes allocate their
        # partials stream-ordered inside it), timed over replays
        reps = 3 if n * k > 1e8 else 10

        def launches():
            for _ in range(reps):
                w.forward(x, out=y)

        g = capture(torch, launches)
        ms = Timer(torch).replay(g, 2 if n * k > 1e8 else max(2, steps // 4), 1) / reps
        del g
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        # f32 activations run on the bf16 matrix cores too (three MFMAs a
        # product): the fraction is of the bf16 peak either way
        res.append({"shape": f"{name} {n}x{k}", "ms": round(ms, 4), "TFLOP/s": round(tf, 2),
                    "frac_mfma_bf16": round(tf / BF16_PEAK_TFLOPS, 4)})
        del w
        torch.cuda.empty_cache()
    if f32:
        return {"workload": "prefill M=512, f32 activations and outputs (the reference's compute type), "
                            "bf16 matrix cores on two bf16 limbs per operand (exact weights)", "shapes": res}
    return {"workload": "prefill M=512, bf16 activations and outputs, f32 accumulation", "shapes": res}


def extra_fp8(torch, rq, synth, dev, steps, warmup):
    m, n, k = 2048, 14336, 4096
    wv = torch.from_numpy(synth.fp8_weight_values(11, n, k)).to(dev)
    wq, _ = rq.fp8_quantize(wv, rq.FP8_UNSCALED)
    del wv
    ws = torch.from_numpy(synth.fp8_row_scales(11, n)).to(dev)
    x = torch.from_numpy(synth.activations(12, m, k)).to(dev).to(torch.bfloat16)
    xq = torch.empty((m, k), dtype=torch.uint8, device=dev)
    xs = torch.empty(m, dtype=torch.float32, device=dev)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)

    def quant():
        rq.check(rq.lib().rq_fp8_quantize(rq._ptr(x), rq.BF16, m, k, rq.FP8_PER_TOKEN, rq._ptr(xq),
                                          rq._ptr(xs), rq._stream(dev)))

    def gemm():
        rq.fp8_gemm_q(xq, xs, wq, ws, y)

    def both():
        rq.fp8_gemm(x, wq, ws, mode=rq.FP8_PER_TOKEN, out=y)

    # four calls per graph, timed over replays (a one-node graph's replay
    # adds several microseconds of its own).  The three graphs are timed in
    # turn over five rounds, each round starting with the next of them, and
    # each figure is the median of its five: timed one after the other once,
    # whichever ran later ran on a warmer, faster-clocked GPU.
    reps = 4
    t = Timer(torch)
    fns = {"quant": quant, "gemm": gemm, "both": both}
    graphs = {nm: capture(torch, lambda fn=fn: [fn() for _ in range(reps)]) for nm, fn in fns.items()}
    samples = {nm: [] for nm in fns}
    order = list(fns)
    for r in range(5):
        for nm in order[r % 3:] + order[:r % 3]:
            samples[nm].append(t.replay(graphs[nm], max(2, steps // 2), warmup if r == 0 else 1) / reps)
    del graphs
    ms_q, ms_g, ms_b = (statistics.median(samples[nm]) for nm in ("quant", "gemm", "both"))
    tf = 2.0 * m * n * k / (ms_b * 1e-3) / 1e12
    tf_g = 2.0 * m * n * k / (ms_g * 1e-3) / 1e12
    return {"workload": "FP8 e4m3 GEMM 2048x14336x4096, per-token activation quantize + GEMM, bf16 out",
            "ms": round(ms_b, 4), "TFLOP/s": round(tf, 1), "frac_mfma_fp8": round(tf / FP8_PEAK_TFLOPS, 4),
            "gemm_only_ms": round(ms_g, 4), "gemm_only_TFLOP/s": round(tf_g, 1),
            "quantize_ms": round(ms_q, 4)}


def extra_marlin(torch, rq, dev, steps, warmup):
    """Marlin INT4 GEMV, M=1, f32: the Qwen2-0.5B up-projection shape and the
    streaming shape, enough distinct copies to exceed the Infinity Cache."""
    res = []
    for n, k, copies in ((4864, 896, 480), (14336, 4096, 32)):
        kc = (k + 31) // 32
        words = torch.randint(-2**31, 2**31 - 1, (kc, n, 4), dtype=torch.int32, device=dev)
        scales = torch.rand(n, device=dev) * 0.02 + 0.001
        W = [(words.clone(), scales.clone()) for _ in range(copies)]
        x = torch.randn((1, k), device=dev)
        y = torch.empty((1, n), device=dev)

        def run():
            st = rq._stream(dev)
            for p, sc in W:
                rq.check(rq.lib().rq_marlin_linear(rq._ptr(p), rq._ptr(sc), n, k, rq._ptr(x), rq.F32, 1,
                                                   rq._ptr(y), rq.F32, st))

        g = capture(torch, run)
        ms = Timer(torch).replay(g, steps, warmup) / copies
        b = kc * n * 16 + n * 4 + k * 4 + n * 4
        res.append({"shape": f"{n}x{k}", "us_per_gemv": round(ms * 1e3, 3), "GB/s": round(b / (ms * 1e-3) / 1e9, 1),
                    "frac_hbm": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        del W, g
        torch.cuda.empty_cache()
    return {"workload": "Marlin INT4 GEMV, M=1, f32 activations", "shapes": res}


def extra_kv(torch, rq, dev, steps, warmup):
    """Paged-KV quantizer: one layer's K for a 4096-token prompt with 8 KV
    heads of 128 ([1, 8, 4096, 128] bf16, 8 MB), 64 distinct inputs; bytes
    counted once each way (input read, codes and scales written).  The 64
    calls are captured in one graph (the quantizer's partial maxima are
    allocated stream-ordered inside it) and timed over replays."""
    shape = (1, 8, 4096, 128)
    copies = 64
    ins = [torch.randn(shape, device=dev).to(torch.bfloat16) for _ in range(copies)]
    q = torch.empty(shape, dtype=torch.uint8, device=dev)
    s = torch.empty(8, device=dev)
    out = torch.empty(shape, dtype=torch.bfloat16, device=dev)
    b, h, sd = 1, 8, 4096 * 128
    res = {}
    for mode, name in ((rq.KV_FP8, "fp8"), (rq.KV_INT8, "int8")):
        def quant():
            st = rq._stream(dev)
            for t in ins:
                rq.check(rq.lib().rq_kv_quantize(rq._ptr(t), rq.BF16, b, h, sd, mode, rq._ptr(q), rq._ptr(s), st))

        def deq():
            st = rq._stream(dev)
            for _ in range(copies):
                rq.check(rq.lib().rq_kv_dequantize(rq._ptr(q), mode, rq._ptr(s), b, h, sd, rq._ptr(out), rq.BF16, st))

        for label, fn, nbytes in (("quantize", quant, b * h * sd * 3 + h * 4), ("dequantize", deq, b * h * sd * 3)):
            g = capture(torch, fn)
            ms = Timer(torch).replay(g, max(2, steps // 4), warmup) / copies
            del g
            res[f"{name}_{label}"] = {"us": round(ms * 1e3, 3), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                      "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
    return {"workload": "KV block quantizer [1, 8, 4096, 128] bf16 <-> fp8 / int8 codes, per-head scales", **res}


def extra_upload(torch, rq, synth, dev):
    """GGUF upload: the tensors of 8 Q4_K_M layers of the prefill model
    (hidden 2048, FFN 8192; q/k/o/gate/up Q4_K, v/down Q6_K) and its Q6_K
    262144x2048 output head, written back to back into a file, memory-mapped
    (pages populated), and turned into device handles with rq_weight_create
    (pinned double-buffered DMA, Q6_K split on the device).  The file is in the page cache (just written), as after a warm
    start; disk read time is not part of the figure."""
    import mmap
    import tempfile
    import time

    import numpy as np

    layer = [(rq.Q4_K, 2048, 2048)] * 3 + [(rq.Q6_K, 2048, 2048), (rq.Q4_K, 8192, 2048),
                                           (rq.Q4_K, 8192, 2048), (rq.Q6_K, 2048, 8192)]
    tensors = layer * 8 + [(rq.Q6_K, 262144, 2048)]
    tmpdir = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    fd, path = tempfile.mkstemp(suffix=".gguf.bin", dir=tmpdir)
    try:
        offs, total = [], 0
        cache = {}
        with os.fdopen(fd, "wb") as f:
            for qt, n, k in tensors:
                key = (qt, n, k)
                if key not in cache:
                    cache[key] = synth.weight_blocks(qt, 21, n, k)
                f.write(cache[key].tobytes())
                offs.append(total)
                total += cache[key].nbytes
        del cache
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        # mapped read-only with populated pages, as GgufFile::open maps a model
        with open(path, "rb") as f:
            mapping = mmap.mmap(f.fileno(), 0, flags=mmap.MAP_PRIVATE | mmap.MAP_POPULATE, prot=mmap.PROT_READ)
        mm = np.frombuffer(mapping, dtype=np.uint8)
        W = [rq.QWeight(qt, mm[o:o + n * k // rq.GEOMETRY[qt][0] * rq.GEOMETRY[qt][1]], n, k)
             for (qt, n, k), o in zip(tensors, offs)]
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        del W, mm
        mapping.close()
    finally:
        os.unlink(path)
    return {"workload": "GGUF upload, 8 Q4_K_M layers (2048/8192) + Q6_K 262144x2048 head, page-cache file",
            "bytes": total, "tensors": len(tensors), "s": round(dt, 4), "GB/s": round(total / dt / 1e9, 2)}


def extra_library(torch, dev, steps):
    """Context, not a result of this library: the vendor BLAS (hipBLASLt via
    torch) on the same problem sizes with the weights already dense -- bf16
    GEMMs for the M=512 prefill shapes, and the FP8 workload through
    torch._scaled_mm with per-row / per-column scales."""
    def timed(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        reps = max(5, steps)
        t0.record()
        for _ in range(reps):
            fn()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / reps

    out = []
    for name, n, k in (("q/k/o 2048x2048", 2048, 2048), ("gate/up 8192x2048", 8192, 2048),
                       ("down 2048x8192", 2048, 8192), ("lm_head 262144x2048", 262144, 2048)):
        a = torch.randn((512, k), device=dev).to(torch.bfloat16)
        w = torch.randn((n, k), device=dev).to(torch.bfloat16)
        ms = timed(lambda: a @ w.t())
        out.append({"shape": f"bf16 M=512 {name}", "ms": round(ms, 4), "TFLOP/s": round(2 * 512 * n * k / ms / 1e9, 1)})
        del a, w
        torch.cuda.empty_cache()
    m, n, k = 2048, 14336, 4096
    a = torch.randn((m, k), device=dev).to(torch.float8_e4m3fn)
    w = torch.randn((n, k), device=dev).to(torch.float8_e4m3fn)
    sa = torch.ones((m, 1), device=dev)
    sw = torch.ones((1, n), device=dev)
    ms = timed(lambda: torch._scaled_mm(a, w.t(), scale_a=sa, scale_b=sw, out_dtype=torch.bfloat16))
    out.append({"shape": "fp8 e4m3 2048x14336x4096, row/column scales", "ms": round(ms, 4),
                "TFLOP/s": round(2 * m * n * k / ms / 1e9, 1)})
    return {"workload": "vendor BLAS on dense weights (reference point)", "shapes": out}


GATE_COPIES = 512  # 512 x 2.45 MB = 1.25 GB: more than the 256 MB Infinity Cache


def gate_weights(rq, synth):
    n, k = 4864, 896
    blocks = synth.q4_k_blocks(104, n * k // 256)
    return [rq.QWeight(rq.Q4_K, blocks, n, k) for _ in range(GATE_COPIES)], n, k


def gate_timing(torch, rq, synth, dev, steps, warmup):
    """The dominant kernel alone: GATE_COPIES distinct 4864x896 Q4_K gate
    weights, one GEMV each, captured in one HIP graph; microseconds per
    launch (gaps included) from HIP events around the replays."""
    W, n, k = gate_weights(rq, synth)
    x = torch.from_numpy(synth.activations(1, 1, k)).to(dev)
    y = torch.empty((1, n), device=dev)
    g = capture(torch, lambda: [w.forward(x, out=y) for w in W])
    ms = Timer(torch).replay(g, steps, warmup) / len(W)
    del g, W
    return ms * 1e3, n * k // 256 * Q4K_BLOCK + k * 4 + n * 4


def mode_gate(torch, rq, synth, dev, steps, warmup, eager=False):
    """Only the dominant kernel (gate_timing), or the same launches without a
    HIP graph for counter collection."""
    if eager:
        W, n, k = gate_weights(rq, synth)
        x = torch.from_numpy(synth.activations(1, 1, k)).to(dev)
        y = torch.empty((1, n), device=dev)
        for _ in range(steps):
            for w in W:
                w.forward(x, out=y)
        torch.cuda.synchronize()
        b = n * k // 256 * Q4K_BLOCK + k * 4 + n * 4
        print(json.dumps({"mode": "gate-eager", "launches": len(W) * steps, "bytes_per_launch": b}), flush=True)
        return
    us, b = gate_timing(torch, rq, synth, dev, steps, warmup)
    print(json.dumps({"mode": "gate", "launches": GATE_COPIES * (steps + warmup + 2), "us_per_launch": round(us, 3),
                      "GB/s": round(b / (us * 1e-6) / 1e9, 1)}), flush=True)


def mode_prefill(torch, rq, synth, dev, steps):
    """The four M=512 layer GEMMs of the prefill workload (q/k/o, v,
    gate/up, down), eager launches (for traces and counters)."""
    m = 512
    for qt, n, k in ((rq.Q4_K, 2048, 2048), (rq.Q6_K, 2048, 2048), (rq.Q4_K, 8192, 2048), (rq.Q6_K, 2048, 8192)):
        w = rq.QWeight(qt, synth.weight_blocks(qt, 7, n, k), n, k)
        x = torch.randn((m, k), device=dev).to(torch.bfloat16)
        y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
        for _ in range(steps):
            w.forward(x, out=y)
        torch.cuda.synchronize()
        del w
    print(json.dumps({"mode": "prefill", "launches": 4 * steps}), flush=True)


def mode_gemv_large(torch, rq, synth, dev, steps):
    """Only the Q4_K 14336x4096 M=1 GEMV over 16 distinct copies (eager, for
    counters)."""
    n, k, copies = 14336, 4096, 16
    blocks = synth.q4_k_blocks(9, n * k // 256)
    W = [rq.QWeight(rq.Q4_K, blocks, n, k) for _ in range(copies)]
    x = torch.from_numpy(synth.activations(4, 1, k)).to(dev)
    y = torch.empty((1, n), device=dev)
    for _ in range(steps):
        for w in W:
            w.forward(x, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "gemv-large", "launches": steps * copies}), flush=True)


def mode_copy(torch, dev, steps):
    """A plain device copy of 512 MiB: the calibration kernel for HBM byte
    counters (FETCH_SIZE / WRITE_SIZE per dispatch vs. 512 MiB moved)."""
    nbytes = 512 << 20
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(steps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "copy", "bytes_read_per_copy": nbytes, "bytes_written_per_copy": nbytes,
                      "copies": steps}), flush=True)


def mode_fp8(torch, rq, synth, dev, steps):
    """Only the FP8 GEMM 2048x14336x4096 (eager launches, for counters)."""
    r = extra_fp8(torch, rq, synth, dev, steps, 1)
    print(json.dumps({"mode": "fp8", **r}), flush=True)


def mode_prefill_head(torch, rq, synth, dev, steps):
    """Only the Q6_K 262144x2048 head GEMM at M=512 (eager, for counters)."""
    m, n, k = 512, 262144, 2048
    w = rq.QWeight(rq.Q6_K, synth.weight_blocks(rq.Q6_K, 7, n, k), n, k)
    x = torch.randn((m, k), device=dev).to(torch.bfloat16)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    for _ in range(steps):
        w.forward(x, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"mode": "prefill-head", "launches": steps}), flush=True)


def mode_gemv_head(torch, rq, synth, dev, steps):
    """Only the M=1 output projection 262144x2048 (Q6_K, then Q4_K), three
    distinct copies each, eager launches (for traces and counters)."""
    n, k = 262144, 2048
    for qt in (rq.Q6_K, rq.Q4_K):
        blocks = synth.weight_blocks(qt, 11, n, k)
        W = [rq.QWeight(qt, blocks, n, k) for _ in range(3)]
        x = torch.from_numpy(synth.activations(12, 1, k)).to(dev)
        y = torch.empty((1, n), device=dev)
        for _ in range(steps):
            for w in W:
                w.forward(x, out=y)
        torch.cuda.synchronize()
        del W
        torch.cuda.empty_cache()
    print(json.dumps({"mode": "gemv-head", "launches": 6 * steps}), flush=True)


def mode_verify(torch, rq, synth, dev, steps, m, layers=128, xdt="bf16", multi=False):
    """Only the verify sweep at one M: the 7 GEMMs of `layers` layer copies
    (q/k/v and gate/up through rq_linear_multi with multi), eager launches
    (for traces and counters)."""
    blocks = {name: synth.q4_k_blocks(100 + i, n * k // 256) for i, (name, n, k) in enumerate(LAYER)}
    W = [{name: rq.QWeight(rq.Q4_K, blocks[name], n, k) for name, n, k in LAYER} for _ in range(layers)]
    dt = torch.bfloat16 if xdt == "bf16" else torch.float32
    xs = {k: torch.randn((m, k), device=dev).to(dt) for k in (896, 4864)}
    ys = {name: torch.empty((m, n), dtype=dt, device=dev) for name, n, k in LAYER}
    groups = (("q", "k", "v"), ("o",), ("gate", "up"), ("down",))
    for _ in range(steps):
        for lw in W:
            if multi:
                for grp in groups:
                    rq.linear_multi_into([lw[nm] for nm in grp], xs[lw[grp[0]].k], [ys[nm] for nm in grp])
                continue
            for name, n, k in LAYER:
                lw[name].forward(xs[k], out=ys[name])
    torch.cuda.synchronize()
    print(json.dumps({"mode": "verify", "m": m, "multi": multi, "launches": steps * layers * (4 if multi else 7)}),
          flush=True)


def traffic_from_profile():
    p = ROOT / "profiles" / "traffic_q4k_gate_gemv.json"
    if p.exists():
        try:
            return json.loads(p.read_text()).get("hbm_bytes_per_launch")
        except Exception:
            return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=128)
    ap.add_argument("--no-extras", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--m", type=int, default=16, help="activation rows of --mode verify")
    ap.add_argument("--multi", action="store_true", help="--mode verify through rq_linear_multi")
    ap.add_argument("--xdt", choices=["bf16", "f32"], default="bf16", help="activation type of --mode verify")
    ap.add_argument("--mode", choices=["full", "gate", "copy", "fp8", "prefill", "prefill-head", "gemv-large",
                                       "gemv-head", "verify"],
                    default="full",
                    help="gate: only the dominant GEMV; copy: counter calibration copy")
    ap.add_argument("--eager", action="store_true", help="gate mode without a HIP graph")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the quantized linear path runs on a single MI355X "
              "(no tensor parallelism, no collectives); run it with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import runtimed_amd  # noqa: F401
    from runtimed_amd import rq, synth

    rq.lib()
    dev = torch.device("cuda", 0)
    if args.mode == "gate":
        return mode_gate(torch, rq, synth, dev, args.steps, args.warmup, args.eager)
    if args.mode == "copy":
        return mode_copy(torch, dev, args.steps)
    if args.mode == "fp8":
        return mode_fp8(torch, rq, synth, dev, args.steps)
    if args.mode == "prefill":
        return mode_prefill(torch, rq, synth, dev, args.steps)
    if args.mode == "prefill-head":
        return mode_prefill_head(torch, rq, synth, dev, args.steps)
    if args.mode == "gemv-head":
        return mode_gemv_head(torch, rq, synth, dev, args.steps)
    if args.mode == "gemv-large":
        return mode_gemv_large(torch, rq, synth, dev, args.steps)
    if args.mode == "verify":
        return mode_verify(torch, rq, synth, dev, args.steps, args.m, xdt=args.xdt, multi=args.multi)
    log(f"decode workload: {args.layers} layer copies, steps={args.steps} warmup={args.warmup}")
    W, ms = decode_workload(torch, rq, synth, args.layers, args.steps, args.warmup, dev)
    step_bytes = layer_bytes() * args.layers
    value = step_bytes / (ms * 1e-3) / 1e9
    gate_us, gate_bytes = gate_timing(torch, rq, synth, dev, max(args.steps, 20), args.warmup)
    gate_gbs = gate_bytes / (gate_us * 1e-6) / 1e9
    log(f"decode: {ms:.4f} ms/step, {value:.1f} GB/s; gate GEMV {gate_us:.3f} us, {gate_gbs:.1f} GB/s")

    extra = {}
    if not args.no_extras:
        for name, fn in (("decode_fused_weights", lambda: extra_decode_fused(torch, rq, synth, args.layers, args.steps,
                                                                               args.warmup, dev)),
                         ("q8_0_gemv", lambda: extra_q8_gemv(torch, rq, synth, dev, args.steps, args.warmup)),
                         ("q4_k_gemv_large", lambda: extra_large_gemv(torch, rq, synth, dev, args.steps, args.warmup)),
                         ("head_gemv_m1", lambda: extra_head_gemv(torch, rq, synth, dev, args.steps, args.warmup)),
                         ("decode_multi", lambda: extra_decode_multi(torch, rq, W, args.steps, args.warmup, dev)),
                         ("verify", lambda: extra_verify(torch, rq, W, dev, args.steps, args.warmup)),
                         ("verify_multi", lambda: extra_verify(torch, rq, W, dev, args.steps, args.warmup,
                                                               multi=True)),
                         ("verify_f32", lambda: extra_verify(torch, rq, W, dev, args.steps, args.warmup,
                                                             torch.float32, (2, 4, 16, 64))),
                         ("verify_f32_multi", lambda: extra_verify(torch, rq, W, dev, args.steps, args.warmup,
                                                                   torch.float32, (4, 16, 64), multi=True)),
                         ("prefill_f32", lambda: extra_prefill(torch, rq, synth, dev, args.steps, args.warmup,
                                                               f32=True)),
                         ("prefill", lambda: extra_prefill(torch, rq, synth, dev, args.steps, args.warmup)),
                         ("fp8_gemm", lambda: extra_fp8(torch, rq, synth, dev, args.steps, args.warmup)),
                         ("marlin_int4_gemv", lambda: extra_marlin(torch, rq, dev, args.steps, args.warmup)),
                         ("kv_quantizer", lambda: extra_kv(torch, rq, dev, args.steps, args.warmup)),
                         ("gguf_upload", lambda: extra_upload(torch, rq, synth, dev)),
                         ("library_reference", lambda: extra_library(torch, dev, args.steps))):
            log(f"extra: {name}")
            try:
                extra[name] = fn()
                log(f"  {json.dumps(extra[name])}")
            except Exception as e:  # report, keep the headline line
                extra[name] = {"error": f"{type(e).__name__}: {e}"}
                log(f"  failed: {e}")
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
    del W

    cpu = None
    if not args.no_cpu:
        import oracle

        log("cpu baseline (oracle on host cores)")
        cpu = cpu_baseline(oracle, synth, args.cpu_seconds)
        log(f"  {json.dumps(cpu)}")

    line = {
        "metric": "Q4_K decode GEMV GB/s (% HBM peak); prefill dequant-GEMM TFLOPS (% MFMA)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded splitmix64 GGUF Q4_K blocks, N(0,1) activations)",
        "config": {"workload": "Q4_K decode GEMV set, one Qwen2-0.5B layer (q/o 896x896, k/v 128x896, "
                               "gate/up 4864x896, down 896x4864), M=1, f32 activations",
                   "layer_copies": args.layers, "bytes_per_step": step_bytes,
                   "frac_hbm": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gate_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gate_gbs / HBM_PEAK_GBS, 4), "traffic": traffic_from_profile(),
                     "traffic_source": "stored: profiles/traffic_q4k_gate_gemv.json (rocprofv3 --pmc FETCH_SIZE "
                                       "and WRITE_SIZE runs of bench.py --mode gate --eager, scaled by the same "
                                       "counters on a 512 MiB copy)",
                     "timing": f"HIP events around graph replays of {GATE_COPIES} launches on {GATE_COPIES} "
                               "distinct weights (1.25 GB) on the replay stream, gaps included: the figure "
                               "bench.py --mode gate prints (profiles/gemv_q4k_gate_4864x896.md)",
                     "kernel": "k_gemv_m1<FmtQ4K,1,1,true> (gate/up 4864x896; the plain f32 form, non-temporal weight loads)",
                     "bytes_per_launch": gate_bytes, "us_per_launch": round(gate_us, 3)},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
