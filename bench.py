#!/usr/bin/env python3
"""Benchmark of the MXFP4 MoE expert hot path on one MI355X.

Workload (the benchmark definition config 2, the metric's "GPT-OSS-120B MXFP4 MoE layer,
batch 1"): 36 MoE layers x 128 GPT-OSS-120B experts (hidden 2880,
intermediate 2880, gate/up interleaved, bf16 biases in the .gwt stride layout),
all resident in HBM (61.2 GB), decode batch 1, top-4 routing from per-layer
logits ~ N(0,1) that change every token.  One step = one token through the 36
MoE blocks: route -> fused gate_up + SwiGLU -> fused down + weighted combine,
each layer's bf16 output feeding the next layer (the trunk between MoE
blocks is outside the timed path).  Weights are seeded synthetic MXFP4
(nibbles U{0..15}, scales U{119..127}, biases N(0, 0.02)).

Prints ONE JSON line (the driver's contract).  `value` is whole-job algorithmic
HBM throughput in GB/s: every selected expert's packed nibbles, scales and bf16
biases, plus the logits, activations and outputs, per token, divided by the
wall time per token of the median timing round.  The timed steps run as the
reference's protocol does (DequantGEMVBenchmark.swift:290-322): 7 rounds of
--steps tokens each, every round bracketed by a device synchronisation, the
median round reported beside the min and max.  Each round's tokens are one
captured graph (36 layer launches a token, each layer reading its token's
logits where they lie in HBM), replayed once; `us_per_token_graph_per_token`
is the same tokens run as one graph per token behind a copy of its logits.
The `roofline` object covers
the dominant kernel (decode_layer_kernel, the one-kernel MoE layer) timed
with hipEvents on the library's stream; `sync_errors` counts the layer
kernel's failed exchange waits (the run fails if there is any);
`cpu_baseline` is the CPU oracle (a scalar port of the reference's CPU path)
on a bounded sample of the same workload, one thread, with the same port's
GEMV rows split over the host's cores beside it (`all_cores`).

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0       # MI355X HBM3E, 8 TB/s

H = F = 2880                # GPT-OSS hidden / intermediate
E, K, L = 128, 4, 36        # experts, top-k, MoE layers (GPT-OSS-120B)
METRIC = "HBM GB/s (% of peak) + µs/token, GPT-OSS-120B MXFP4 MoE layer, batch 1"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def expert_bytes(lay) -> int:
    """Algorithmic bytes of one selected expert: both projections' packed
    nibbles and scales, and the two bf16 bias vectors."""
    return sum(lay.sizes[s] for s in lay.sizes)


def gate_up_bytes(lay) -> int:
    """Algorithmic bytes of one gate_up launch (one layer): k experts' gate_up
    nibbles, scales and bias, the bf16 input read and the fp16 activations written."""
    per = lay.sizes["gate_up_blocks"] + lay.sizes["gate_up_scales"] + lay.sizes["gate_up_bias"]
    return K * per + H * 2 + K * F * 2


COUNTER_LAYERS = L
# Measured HBM bytes per launch of a roofline kernel: rocprofv3 FETCH_SIZE and
# WRITE_SIZE per dispatch (separate --pmc runs), each scaled by what the
# counter reads for a 256 MiB device-to-device copy.  Each figure is tied to
# the SHA-256 (first 16 hex digits) of the kernel source it was measured on:
# a run whose source differs reports `traffic: null` rather than a stale
# number.
#   gate_up_kernel, GPT-OSS-120B layer, batch 1 (profiles/decode_gate_up_down_traffic.md)
GATE_UP_TRAFFIC = (35_944_526, "gw_kernels.hip", None)
#   prefill gate_up GEMM, 512 tokens, seed 1 (profiles/prefill_gemm_gptoss_512.md)
PREFILL_GATE_UP_TRAFFIC = (1_248_605_362, "gw_prefill.hip", "38f5ec0c68d728b2")
#   decode_layer_kernel (the one-kernel layer), GPT-OSS-120B, batch 1, over the
#   whole 36-layer stack (profiles/decode_layer_traffic.md)
DECODE_LAYER_TRAFFIC = (54_469_014, "gw_decode.hip", "723e1fa7217756e3")


def source_sha16(name: str) -> str:
    import hashlib
    with open(os.path.join(ROOT, "godwit_amd", "csrc", name), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def measured_traffic(entry) -> dict:
    """The `traffic` figure for the roofline object and where it came from:
    the bytes when the kernel source is the one they were measured on."""
    nbytes, src, sha = entry
    cur = source_sha16(src)
    if sha is not None and cur == sha:
        return {"traffic": nbytes, "traffic_source": f"{src} {sha}"}
    return {"traffic": None,
            "traffic_source": f"not measured on this {src} ({cur}); see profiles/"}


def build_model(ctx, gw, lay, seed: int):
    """36 layer files of 128 expert strides each, filled on the device."""
    return build_model_layers(ctx, gw, lay, seed, L)


def fill_layer(ctx, gw, buf, lay, n_experts: int, s: int, biases: bool = True) -> None:
    """One layer file of synthetic experts in five launches: every packed byte
    U{0..255} (nibbles U{0..15}), then each section over all experts at once
    (rows of the expert stride): scales U{119..127}, biases N(0, 0.02) bf16 or
    zeros."""
    o, sz = lay.offsets, lay.sizes
    ctx.fill_uniform_u8(buf, 0, 255, s)
    for sec, k in (("gate_up_scales", 1), ("down_scales", 2)):
        ctx.fill_uniform_u8(buf, 119, 127, s * 131 + k, offset=o[sec], count=sz[sec],
                            rows=n_experts, row_stride=lay.stride)
    for sec, k in (("gate_up_bias", 3), ("down_bias", 4)):
        if biases:
            ctx.fill_normal(buf, gw.BF16, sz[sec] // 2, 0.0, 0.02, s * 131 + k, offset=o[sec],
                            rows=n_experts, row_stride=lay.stride)
        else:
            ctx.fill_uniform_u8(buf, 0, 0, 0, offset=o[sec], count=sz[sec], rows=n_experts,
                                row_stride=lay.stride)


def build_model_layers(ctx, gw, lay, seed: int, n_layers: int):
    bufs = []
    for l in range(n_layers):
        buf = ctx.empty(lay.layer_file_size)
        fill_layer(ctx, gw, buf, lay, E, seed * 1000003 + l * 7919)
        bufs.append(buf)
    ctx.synchronize()
    return bufs


def counter_pass(gw, args) -> int:
    """The run rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE profiles for the decode
    kernels: the benchmark's own 36-layer GPT-OSS-120B stack (five fill
    launches per layer), --warmup + --steps tokens through it eagerly with
    fresh N(0,1) logits per layer and token, then three device-to-device
    copies of --counter-pass MiB, whose known bytes scale the counters."""
    ctx = gw.Context(0)
    lay = gw.ExpertLayout(H, F, E)
    runner = gw.ExpertRunner(ctx, H, F, "gptOssClampedGLU", 7.0, 1.702)
    layers = build_model_layers(ctx, gw, lay, args.seed, COUNTER_LAYERS)
    n_tok = args.warmup + args.steps
    logits = ctx.empty(n_tok * COUNTER_LAYERS * E * 4)
    ctx.fill_normal(logits, gw.F32, n_tok * COUNTER_LAYERS * E, 0.0, 1.0, args.seed * 31 + 7)
    xs = [ctx.empty(H * 2) for _ in range(COUNTER_LAYERS + 1)]
    ctx.fill_normal(xs[0], gw.BF16, H, 0.0, 1.0, args.seed * 31 + 9)
    out = ctx.empty(H * 4)
    for i in range(n_tok):
        for l in range(COUNTER_LAYERS):
            runner.layer_forward(layers[l].ptr, lay.stride, E, K, xs[l].ptr, gw.BF16, 1, out.ptr,
                                 logits=logits.address(((i * COUNTER_LAYERS) + l) * E * 4),
                                 out_bf16=xs[l + 1].ptr)
    nb = args.counter_pass << 20
    src, dst = ctx.empty(nb), ctx.empty(nb)
    ctx.fill_uniform_u8(src, 0, 255, 3)
    for _ in range(3):
        ctx.copy_async(dst.ptr, src.ptr, nb)
    ctx.synchronize()
    log(f"counter pass: {n_tok} eager tokens x {COUNTER_LAYERS} layers, then 3 copies of "
        f"{nb} B (__amd_rocclr_copyBuffer: {nb} B read + {nb} B written each)")
    runner.close()
    ctx.close()
    return 0


def gemv_bench(gw, args) -> int:
    """Benchmark config 0: one MXFP4 GEMV at the GPT-OSS-120B gate_up shape, y =
    dequant(W) x + b, W 5760 x 2880 (nibbles U{0..15}, scales U{119..127}), x fp32
    N(0,1), b fp32 N(0, 0.02).  128 distinct weight copies (1.13 GB) are cycled
    so no launch finds its weights in the 256 MB MALL.  Reports GB/s of the
    launch's algorithmic bytes (8,870,400: packed + scales + x + bias + y) and
    the oracle's scalar GEMV timed on the host beside it."""
    rows, cols, ncopy = 2 * F, H, 128
    pbytes, sbytes = rows * cols // 2, rows * cols // 32
    ctx = gw.Context(0)
    wbuf = ctx.empty(ncopy * (pbytes + sbytes))
    ctx.fill_uniform_u8(wbuf, 0, 255, args.seed * 7 + 1, offset=0, count=ncopy * pbytes)
    ctx.fill_uniform_u8(wbuf, 119, 127, args.seed * 7 + 2, offset=ncopy * pbytes,
                        count=ncopy * sbytes)
    xb, bb, yb = ctx.empty(cols * 4), ctx.empty(rows * 4), ctx.empty(rows * 4)
    ctx.fill_normal(xb, gw.F32, cols, 0.0, 1.0, args.seed * 7 + 3)
    ctx.fill_normal(bb, gw.F32, rows, 0.0, 0.02, args.seed * 7 + 4)
    ctx.synchronize()

    class View:   # a copy's packed / scales sections as DeviceBuffer-like views
        def __init__(self, ptr):
            self.ptr = ptr

    def launch(i):
        k = i % ncopy
        gw.mxfp4_gemv_bias(ctx, View(wbuf.address(k * pbytes)),
                           View(wbuf.address(ncopy * pbytes + k * sbytes)), bb, gw.F32, xb,
                           gw.F32, yb, rows, cols)

    for i in range(args.warmup):
        launch(i)
    ctx.synchronize()
    # Back to back: one graph of ncopy launches (every copy once), replayed
    # `steps` times per round, 7 rounds (the host's launch cost is not in it).
    graph = gw.Graph.capture(ctx, lambda: [launch(i) for i in range(ncopy)])
    graph.launch()
    per_step, _ = timed_rounds(args.steps, lambda j: graph.launch(), ctx.synchronize)
    dt = round_stats(per_step, 1e6 / ncopy)["median"] * 1e-6
    n = TIMING_ROUNDS * args.steps * ncopy
    # Kernel duration: HIP events around eager launches, enqueued behind a graph
    # replay so that the device is still busy when each launch's start event
    # reaches it (a host slower than the kernel would otherwise put its own
    # enqueue time between the two events).
    ctx.set_profiling(True)
    ctx.profile_reset()
    prof_n = 0
    for c in range(8):
        graph.launch()
        for i in range(64):
            launch(c * 64 + i)
            prof_n += 1
    ctx.synchronize()
    ms, cnt = ctx.profile("gemv")
    ctx.set_profiling(False)
    assert cnt == prof_n, (cnt, prof_n)
    graph.destroy()
    k_us = ms / cnt * 1e3
    nbytes = pbytes + sbytes + cols * 4 + rows * 4 + rows * 4
    value = nbytes / (k_us * 1e-6) / 1e9
    log(f"gemv {rows}x{cols}: {k_us:.2f} us per launch (HIP events), {dt * 1e6:.2f} us "
        f"per launch back to back, {value:.0f} GB/s ({value / PEAK_HBM_GBS * 100:.1f}% of "
        f"{PEAK_HBM_GBS:.0f})")
    cpu = None
    if args.cpu_seconds > 0:
        import oracle
        r = np.random.default_rng(5)
        packed = r.integers(0, 256, pbytes, dtype=np.uint8)
        scales = r.integers(119, 128, sbytes, dtype=np.uint8)
        x = r.standard_normal(cols).astype(np.float32)
        bias = (r.standard_normal(rows) * 0.02).astype(np.float32)
        calls, c0 = 0, time.perf_counter()
        while time.perf_counter() - c0 < args.cpu_seconds:
            oracle.gemv_bias(packed, scales, bias, x, rows, cols)
            calls += 1
        c_us = (time.perf_counter() - c0) / calls * 1e6
        cpu = {"value": round(nbytes / (c_us * 1e-6) / 1e9, 4), "unit": "GB/s",
               "us_per_gemv": round(c_us, 1), "cores": 1, "kind": "port",
               "sample": f"{calls} GEMVs of the same shape (one weight set), scalar C oracle "
                         f"(referenceMXFP4 + bias), 1 thread"}
        log(f"cpu baseline: {c_us:.0f} us per GEMV")
    print(json.dumps({
        "metric": "HBM GB/s (% of peak), MXFP4 GEMV at the GPT-OSS-120B gate_up shape",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": n,
        "warmup": args.warmup, "ms_per_step": round(k_us * 1e-3, 5),
        "us_per_gemv_back_to_back": round(dt * 1e6, 3),
        "back_to_back": f"graph of {ncopy} launches, {args.steps} replays per round, "
                        f"median of {TIMING_ROUNDS} rounds",
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "compute": "e2m1 weights (MXFP4, exact) x fp32 x, fp32 products and sums",
        "data": "synthetic (seeded MXFP4 nibbles U{0..15}, scales U{119..127}, x N(0,1), "
                "bias N(0,0.02) fp32; 128 weight copies cycled)",
        "config": {"workload": "gptoss-gate_up-gemv", "rows": rows, "cols": cols,
                   "weight_copies": ncopy, "parallelism": "single-gpu"},
        "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": PEAK_HBM_GBS,
                     "unit": "GB/s", "frac": round(value / PEAK_HBM_GBS, 4), "traffic": None,
                     "kernel": "gemv_kernel (MXFP4 GEMV + bias)", "bytes_per_launch": nbytes,
                     "avg_launch_us": round(k_us, 3)},
        "cpu_baseline": cpu}), flush=True)
    ctx.close()
    return 0


def gptoss20b_bench(gw, args) -> int:
    """Benchmark config 1: one GPT-OSS-20B-shaped MoE layer at batch 1 with its fp32
    router on the device: 32 experts (hidden 2880), router weights fp32 [32 x 2880]
    N(0, 0.02), x bf16 N(0,1), top-4, softmax over the 4, SwiGLU (1.702, 7.0),
    weighted sum.  Four copies of the layer (1.7 GB) run in turn, each layer's
    output feeding the next layer's input, so no copy stays in the MALL; one
    replayed graph holds 24 layer launches (GPT-OSS-20B's depth: six passes over
    the copies), so a replay's own launch cost is spread as over a token's
    layers.  Reports us per layer and GB/s of algorithmic bytes (4 experts +
    router + x + out), and, for comparison, us per layer from a graph of the four
    copies alone."""
    E20, ncopy = 32, 4
    ctx = gw.Context(0)
    lay = gw.ExpertLayout(H, F, E20)
    runner = gw.ExpertRunner(ctx, H, F, "gptOssClampedGLU", 7.0, 1.702)
    layers, routers = [], []
    for l in range(ncopy):
        buf = ctx.empty(lay.layer_file_size)
        sd = args.seed * 1000003 + l * 7919
        fill_layer(ctx, gw, buf, lay, E20, sd)
        rw = ctx.empty(E20 * H * 4)
        ctx.fill_normal(rw, gw.F32, E20 * H, 0.0, 0.02, sd * 17 + 5)
        layers.append(buf)
        routers.append(rw)
    xs = [ctx.empty(H * 2) for _ in range(ncopy + 1)]
    ctx.fill_normal(xs[0], gw.BF16, H, 0.0, 1.0, args.seed * 31 + 9)
    out = ctx.empty(H * 4)
    ctx.synchronize()

    depth = 24

    def layers_of(n):
        def run():
            for i in range(n):
                l = i % ncopy
                runner.layer_forward(layers[l].ptr, lay.stride, E20, K, xs[l].ptr, gw.BF16, 1,
                                     out.ptr, router_weight=routers[l].ptr,
                                     router_weight_dtype=gw.F32,
                                     out_bf16=xs[(l + 1) % ncopy].ptr)
        return run

    def timed(n):
        g = gw.Graph.capture(ctx, layers_of(n))
        for _ in range(args.warmup):
            g.launch()
        ctx.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            g.launch()
        ctx.synchronize()
        g.destroy()
        return (time.perf_counter() - t0) / (args.steps * n)

    dt4 = timed(ncopy)
    dt = timed(depth)
    step = layers_of(ncopy)
    kernels = {}
    if not args.no_profile_pass:
        ctx.set_profiling(True)
        ctx.profile_reset()
        for _ in range(args.steps):
            step()
        ctx.synchronize()
        for name in ("router", "moe_layer", "gate_up", "down"):
            ms, n = ctx.profile(name)
            if n:
                kernels[name] = {"launches": n, "avg_us": ms / n * 1e3}
        ctx.set_profiling(False)
        log("kernels: " + ", ".join(f"{k} {v['avg_us']:.2f} us" for k, v in kernels.items()))
    sync_err = runner.sync_errors()
    nbytes = K * expert_bytes(lay) + E20 * H * 4 + H * 2 + H * 4 + H * 2
    value = nbytes / dt / 1e9
    log(f"gpt-oss-20b layer: {dt * 1e6:.2f} us per layer in a graph of {depth} "
        f"({dt4 * 1e6:.2f} in a graph of {ncopy}), {value:.0f} GB/s "
        f"({value / PEAK_HBM_GBS * 100:.1f}% of {PEAK_HBM_GBS:.0f})")
    roof = None
    if "moe_layer" in kernels:
        lb = K * expert_bytes(lay) + E20 * 4 + H * 2 + H * 4 + H * 2
        ach = lb / (kernels["moe_layer"]["avg_us"] * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
                "kernel": "decode_layer_kernel (route + gate_up + SwiGLU + down + combine)",
                "bytes_per_launch": lb, "avg_launch_us": round(kernels["moe_layer"]["avg_us"], 3)}
    elif "gate_up" in kernels:
        ach = gate_up_bytes(lay) / (kernels["gate_up"]["avg_us"] * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
                "kernel": "gate_up_kernel (fused MXFP4 gate_up GEMV + bias + SwiGLU)",
                "bytes_per_launch": gate_up_bytes(lay),
                "avg_launch_us": round(kernels["gate_up"]["avg_us"], 3)}
    print(json.dumps({
        "metric": "HBM GB/s (% of peak) + us/layer, GPT-OSS-20B MXFP4 MoE layer with its "
                  "router, batch 1",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * depth * 1e3, 4),
        "us_per_layer": round(dt * 1e6, 2), "layers_per_graph": depth,
        "us_per_layer_graph_of_4": round(dt4 * 1e6, 2), "sync_errors": sync_err,
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "compute": "e2m1 weights (MXFP4, exact) x bf16 activations, fp32 products and sums; "
                   "fp32 router",
        "data": "synthetic (seeded MXFP4, biases N(0,0.02) bf16, router fp32 N(0,0.02), "
                "x N(0,1) bf16)",
        "config": {"workload": "gptoss20b-moe-layer-decode", "experts": E20, "top_k": K,
                   "hidden": H, "intermediate": F, "layer_copies": ncopy,
                   "parallelism": "single-gpu"},
        "kernels": kernels, "roofline": roof, "cpu_baseline": None}), flush=True)
    runner.close()
    ctx.close()
    return 0


def host_cpus() -> dict:
    """The host's CPU counts: all logical CPUs, the ones this process may run
    on (affinity), and OMP_NUM_THREADS when set."""
    omp = os.environ.get("OMP_NUM_THREADS")
    return {"os_cpu_count": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "omp_num_threads": int(omp) if omp and omp.isdigit() else None}


def host_threads() -> int:
    """Host threads for the all-core CPU baseline: every CPU this process may
    run on (its affinity mask)."""
    return max(1, len(os.sched_getaffinity(0)))


def cpu_baseline(seconds: float, threads: int = 1) -> dict:
    """The oracle (scalar C port of the reference CPU path: referenceMXFP4 + bias,
    gptoss activation with fp16 rounding, Router.select, sequential combine) on
    whole tokens of the same workload until `seconds` have elapsed: per layer,
    top-4 of 128 N(0,1) logits, as on the GPU.  The 128 expert slots of a layer
    point into a pool of 32 distinct synthetic experts (425 MB; slot e of layer l
    is pool entry (e + 5 l) mod 32), so no selected expert's 13 MB stays in the
    host caches from one layer to the next.  threads > 1 splits each GEMV's rows
    over that many OpenMP threads (same results)."""
    import oracle
    oracle.set_threads(threads)
    r = np.random.default_rng(77)
    pool = []
    for _ in range(32):
        pool.append(oracle.Expert(
            r.integers(0, 256, 2 * F * H // 2, dtype=np.uint8),
            r.integers(119, 128, 2 * F * H // 32, dtype=np.uint8),
            r.integers(0, 256, H * F // 2, dtype=np.uint8),
            r.integers(119, 128, H * F // 32, dtype=np.uint8),
            oracle.round_to_bf16((r.standard_normal(2 * F) * 0.02).astype(np.float32)),
            oracle.round_to_bf16((r.standard_normal(H) * 0.02).astype(np.float32))))
    slots = [[pool[(e + 5 * l) % 32] for e in range(E)] for l in range(L)]
    x = oracle.round_to_bf16(r.standard_normal(H).astype(np.float32))
    tokens = 0
    t0 = time.perf_counter()
    while True:
        for l in range(L):
            logits = r.standard_normal((1, E)).astype(np.float32)
            out, _, _ = oracle.moe_layer(slots[l], K, logits, x, H, F)
            x = oracle.round_to_bf16(out[0])
        tokens += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    oracle.set_threads(1)
    return {"tokens": tokens, "seconds": dt, "us_per_token": dt / tokens * 1e6,
            "threads": threads}


TIMING_ROUNDS = 7   # DequantGEMVBenchmark.timingRounds


def timed_rounds(steps: int, run_step, sync, rounds: int = TIMING_ROUNDS):
    """The reference's timing protocol (DequantGEMVBenchmark.swift:290-322):
    `rounds` consecutive rounds of `steps` steps each (step indices run on
    across rounds), each bracketed by a device synchronisation.  Returns
    (per-step seconds of each round, total seconds)."""
    per_step = []
    sync()
    t0 = time.perf_counter()
    for i in range(rounds):
        tr = time.perf_counter()
        for j in range(i * steps, (i + 1) * steps):
            run_step(j)
        sync()
        per_step.append((time.perf_counter() - tr) / steps)
    return per_step, time.perf_counter() - t0


def round_graphs(gw, ctx, args, run_tokens, rounds: int = TIMING_ROUNDS):
    """timed_rounds with each round's `args.steps` tokens captured as one graph
    (run_tokens(first, n) enqueues tokens first .. first+n-1) and replayed
    once, so the per-token cost holds no graph launch or input copy: warm-up
    tokens 0 .. warmup-1 first (one graph) and one untimed replay of every
    round's graph, then `rounds` timed rounds of args.steps tokens, each
    bracketed by a device synchronisation.  Returns (per-token seconds of each
    round, total seconds)."""
    if args.warmup:
        warm = gw.Graph.capture(ctx, run_tokens(0, args.warmup))
        warm.launch()
        ctx.synchronize()
        warm.destroy()
    graphs = [gw.Graph.capture(ctx, run_tokens(args.warmup + r * args.steps, args.steps))
              for r in range(rounds)]
    # every graph replayed once before timing (its first launch also moves it
    # to the device); the replay recomputes everything, weights included
    for g in graphs:
        g.launch()
    per_step = []
    ctx.synchronize()
    t0 = time.perf_counter()
    for g in graphs:
        tr = time.perf_counter()
        g.launch()
        ctx.synchronize()
        per_step.append((time.perf_counter() - tr) / args.steps)
    total = time.perf_counter() - t0
    for g in graphs:
        g.destroy()
    return per_step, total


def round_stats(per_step, scale: float) -> dict:
    """rounds / median / min / max of the per-step times, times `scale`."""
    v = sorted(x * scale for x in per_step)
    return {"rounds": len(v), "median": round(v[len(v) // 2], 3), "min": round(v[0], 3),
            "max": round(v[-1], 3)}


def prefill_cpu_baseline(seconds: float, logits: np.ndarray) -> dict:
    """The oracle's MoE layer (as in cpu_baseline) on the first tokens of the
    prefill workload, one at a time, until `seconds` have elapsed: the tokens'
    own Zipf-routed top-4 of 128 experts, whose slots point into a pool of 32
    distinct synthetic experts (slot e is pool entry e mod 32)."""
    import oracle
    r = np.random.default_rng(78)
    pool = []
    for _ in range(32):
        pool.append(oracle.Expert(
            r.integers(0, 256, 2 * F * H // 2, dtype=np.uint8),
            r.integers(119, 128, 2 * F * H // 32, dtype=np.uint8),
            r.integers(0, 256, H * F // 2, dtype=np.uint8),
            r.integers(119, 128, H * F // 32, dtype=np.uint8),
            oracle.round_to_bf16((r.standard_normal(2 * F) * 0.02).astype(np.float32)),
            oracle.round_to_bf16((r.standard_normal(H) * 0.02).astype(np.float32))))
    slots = [pool[e % 32] for e in range(E)]
    tokens, t0 = 0, time.perf_counter()
    while True:
        x = oracle.round_to_bf16(r.standard_normal((1, H)).astype(np.float32))
        oracle.moe_layer(slots, K, logits[tokens % len(logits)][None, :], x, H, F)
        tokens += 1
        dt = time.perf_counter() - t0
        if dt >= seconds:
            break
    return {"tokens": tokens, "seconds": dt, "tokens_per_s": tokens / dt}


PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 matrix peak
PEAK_FP4_TFLOPS = 10100.0    # MI355X dense FP4 matrix cores (block-scaled MXFP4 MFMA)
PREFILL_T = 512


def zipf_logits(T: int, seed: int, s_exp: float = 1.1) -> np.ndarray:
    """Logits whose top-4 per token is a Zipf(s)-popular draw of 4 distinct experts
    (benchmark config 4), ranked by decreasing logit."""
    r = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, E + 1) ** s_exp
    p /= p.sum()
    logits = (r.standard_normal((T, E)) - 10.0).astype(np.float32)
    for t in range(T):
        chosen = r.choice(E, size=K, replace=False, p=p)
        logits[t, chosen] = (5.0 - np.arange(K) + r.uniform(0, 0.5, K)).astype(np.float32)
    return logits


def prefill_bench(gw, args) -> int:
    """Benchmark config 4: one GPT-OSS-120B MoE layer (128 experts, 1.70 GB resident),
    batched prefill of 512 tokens with Zipf(1.1)-popular top-4 routing, bf16 x.
    Reports µs per layer, HBM GB/s over the distinct experts touched, and matrix-core
    use: algorithmic flops (2 x tokens x 4 x (5760 x 2880 + 2880 x 2880)) against the
    dense bf16 peak, plus the flops the matrix cores execute (the same here: bf16 x
    enters gate_up as one plane and the fp16 activation enters the down projection
    as itself, on the fp16 matrix cores)."""
    ctx = gw.Context(0)
    lay = gw.ExpertLayout(H, F, E)
    runner = gw.ExpertRunner(ctx, H, F, "gptOssClampedGLU", 7.0, 1.702)
    T = PREFILL_T
    layers = build_model_layers(ctx, gw, lay, args.seed, 2)
    logits = zipf_logits(T, args.seed)
    lb = ctx.buffer(logits)
    x = ctx.empty(T * H * 2)
    ctx.fill_normal(x, gw.BF16, T * H, 0.0, 1.0, args.seed * 31 + 9)
    out = ctx.empty(T * H * 4)
    runner.reserve_prefill(T, K, E)
    ctx.synchronize()

    def call(i: int):
        runner.prefill_forward(layers[i % len(layers)].ptr, lay.stride, E, K, x.ptr, gw.BF16, T,
                               out.ptr, logits=lb.ptr)

    # The layers run back to back as one captured graph (as the decode
    # workloads are timed): 36 layer launches (GPT-OSS-120B's depth, the two
    # copies in turn), replayed until --steps layers have run; a graph of the
    # two copies alone is timed the same way for comparison.  The per-kernel
    # event pass below runs eagerly.
    def timed(depth: int):
        graph = gw.Graph.capture(ctx, lambda: [call(i) for i in range(depth)])
        for i in range(max(1, args.warmup // depth)):
            graph.launch()
        ctx.synchronize()
        reps = max(1, args.steps // depth)
        t0 = time.perf_counter()
        for i in range(reps):
            graph.launch()
        ctx.synchronize()
        graph.destroy()
        return (time.perf_counter() - t0) / (reps * depth), reps * depth

    depth = 36
    dt2, _ = timed(len(layers))
    dt, n_timed = timed(depth)
    touched = len(set(np.argsort(-logits, axis=1)[:, :K].ravel().tolist()))
    nbytes = touched * expert_bytes(lay) + T * H * 2 + T * H * 4
    flops = 2.0 * T * K * (2 * F * H + H * F)
    mfma_flops = 2.0 * T * K * (2 * F * H + H * F)
    kernels = {}
    if not args.no_profile_pass:
        ctx.set_profiling(True)
        ctx.profile_reset()
        for i in range(args.steps):
            call(i)
        ctx.synchronize()
        for name in ("prefill_route", "prefill_group", "prefill_gate_up", "prefill_down",
                     "prefill_combine"):
            ms, n = ctx.profile(name)
            if n:
                kernels[name] = {"launches": n, "avg_us": ms / n * 1e3}
        ctx.set_profiling(False)
    value = T / dt
    log(f"prefill {T} tokens: {dt * 1e6:.1f} us/layer in a graph of {depth} "
        f"({dt2 * 1e6:.1f} in a graph of the {len(layers)} copies), {value:.0f} tokens/s, "
        f"{nbytes / dt / 1e9:.0f} GB/s over {touched} experts, "
        f"{flops / dt / 1e12:.1f} TFLOP/s algorithmic")
    if kernels:
        log("kernels: " + ", ".join(f"{k} {v['avg_us']:.2f} us" for k, v in kernels.items()))
    cpu = None
    if args.cpu_seconds > 0:
        c = prefill_cpu_baseline(args.cpu_seconds, logits)
        cpu = {"value": round(c["tokens_per_s"], 3), "unit": "tokens/s", "cores": 1, "kind": "port",
               "sample": f"the first {c['tokens']} of the {T} tokens, one at a time through the "
                         f"scalar C oracle's MoE layer (their own top-4 of 128, experts drawn "
                         f"from a pool of 32 synthetic ones), 1 thread, {c['seconds']:.1f} s"}
        log(f"cpu baseline: {c['tokens_per_s']:.2f} tokens/s")
    # The grouped GEMMs sit below the bf16 ridge (about 60 flop per weight byte
    # against 2500 TFLOP/s / 8 TB/s = 312), so the roofline is HBM: the gate_up
    # launch moves the gate_up sections of every touched expert once.
    gu = kernels.get("prefill_gate_up", {}).get("avg_us")
    roof = None
    if gu:
        gu_bytes = touched * sum(lay.sizes[k] for k in ("gate_up_blocks", "gate_up_scales",
                                                         "gate_up_bias")) + T * H * 2
        ach = gu_bytes / (gu * 1e-6) / 1e9
        gu_tflops = 2.0 * T * K * 2 * F * H / (gu * 1e-6) / 1e12
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), **measured_traffic(PREFILL_GATE_UP_TRAFFIC),
                "kernel": "prefill_gemm_kernel (gate_up grouped GEMM)",
                "avg_launch_us": round(gu, 3), "algorithmic_bytes": gu_bytes,
                "mfma_tflops": round(gu_tflops, 1),
                # algorithmic flops against both dense peaks: the bf16 one the
                # kernel runs on, and the FP4 one of the block-scaled MXFP4 MFMA
                "mfma_frac": round(gu_tflops / PEAK_BF16_TFLOPS, 4),
                "mfma_frac_bf16_peak": round(gu_tflops / PEAK_BF16_TFLOPS, 4),
                "mfma_frac_fp4_peak": round(gu_tflops / PEAK_FP4_TFLOPS, 4)}
    print(json.dumps({
        "metric": "prefill tokens/s, GPT-OSS-120B MXFP4 MoE layer, 512 tokens",
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": n_timed,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "us_per_layer": round(dt * 1e6, 2), "layers_per_graph": depth,
        "us_per_layer_graph_of_2": round(dt2 * 1e6, 2), "hbm_gbs": round(nbytes / dt / 1e9, 1),
        "tflops_algorithmic": round(flops / dt / 1e12, 2),
        "tflops_matrix_core": round(mfma_flops / dt / 1e12, 2),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "compute": "e2m1 weights widened exactly (scale folded) to bf16 for gate_up x bf16 x "
                   "and to fp16 for down x fp16 activations, fp32 MFMA accumulation",
        "data": "synthetic (seeded MXFP4, Zipf(1.1) top-4 routing, x N(0,1) bf16)",
        "config": {"workload": "gptoss120b-moe-layer-prefill-512", "tokens": T, "experts": E,
                   "experts_touched": touched, "top_k": K, "hidden": H, "intermediate": F,
                   "parallelism": "single-gpu"},
        "kernels": kernels, "roofline": roof, "cpu_baseline": cpu}), flush=True)
    runner.close()
    ctx.close()
    return 0


QWEN3 = dict(H=2048, F=768, E=128, K=8, L=48)


def qwen3_bench(gw, args, batch: int) -> int:
    """Benchmark config 3: Qwen3 MoE stack, 48 layers x 128 experts (hidden 2048,
    expert intermediate 768, gate/up interleaved row-wise, zero bias sections as
    the reference's install writes them, SiLU-GLU), top-8, bf16 x; `batch` tokens
    per step (1 or 8) with independent N(0,1) logits per token and layer.  Bytes per
    step: every distinct selected expert of every layer once (the packed nibbles,
    scales and zero bias sections), plus logits, activations and outputs."""
    q = QWEN3
    Hq, Fq, Eq, Kq, Lq = q["H"], q["F"], q["E"], q["K"], q["L"]
    ctx = gw.Context(0)
    lay = gw.ExpertLayout(Hq, Fq, Eq)
    runner = gw.ExpertRunner(ctx, Hq, Fq, "silu")
    # A batch may take the grouped GEMMs (GODWIT_PREFILL_ABOVE below the
    # batch): their scratch has to exist before the step is captured.
    runner.reserve_prefill(batch, Kq, Eq)
    layers = []
    for l in range(Lq):
        buf = ctx.empty(lay.layer_file_size)
        fill_layer(ctx, gw, buf, lay, Eq, args.seed * 1000003 + l * 7919, biases=False)
        layers.append(buf)
    ctx.synchronize()
    log(f"resident experts: {Lq} x {Eq} x {lay.stride} B = {Lq * lay.layer_file_size / 1e9:.2f} GB")
    timed = TIMING_ROUNDS * args.steps
    total = args.warmup + timed
    step_logits = Lq * batch * Eq * 4
    logits_all = ctx.empty(total * step_logits)
    ctx.fill_normal(logits_all, gw.F32, total * Lq * batch * Eq, 0.0, 1.0, args.seed * 31 + 7)
    cur = ctx.empty(step_logits)
    xs = [ctx.empty(batch * Hq * 2) for _ in range(Lq + 1)]
    ctx.fill_normal(xs[0], gw.BF16, batch * Hq, 0.0, 1.0, args.seed * 31 + 9)
    outs = [ctx.empty(batch * Hq * 4) for _ in range(Lq)]
    ids = ctx.empty(Lq * batch * Kq * 4)
    ctx.synchronize()

    def token():
        for l in range(Lq):
            runner.layer_forward(layers[l].ptr, lay.stride, Eq, Kq, xs[l].ptr, gw.BF16, batch,
                                 outs[l].ptr, logits=cur.address(l * batch * Eq * 4),
                                 out_bf16=xs[l + 1].ptr,
                                 routing_ids=ids.address(l * batch * Kq * 4))

    def run_tokens(first: int, n: int):
        # steps first .. first+n-1, each layer reading its own logits in place
        def run():
            for i in range(first, first + n):
                for l in range(Lq):
                    runner.layer_forward(layers[l].ptr, lay.stride, Eq, Kq, xs[l].ptr, gw.BF16,
                                         batch, outs[l].ptr,
                                         logits=logits_all.address(i * step_logits +
                                                                   l * batch * Eq * 4),
                                         out_bf16=xs[l + 1].ptr,
                                         routing_ids=ids.address(l * batch * Kq * 4))
        return run

    uniq = []
    # one graph a round (as the GPT-OSS stack); then one graph a step behind a
    # logits copy, reported beside it
    if not (args.token_graphs or args.eager):
        per_step, elapsed = round_graphs(gw, ctx, args, run_tokens)
    graph = None if args.eager else gw.Graph.capture(ctx, token)

    def step(i):
        ctx.copy_async(cur.ptr, logits_all.address(i * step_logits), step_logits)
        if args.eager:
            token()
        else:
            graph.launch()

    for i in range(args.warmup):
        step(i)
    per_step_tok, elapsed_tok = timed_rounds(args.steps, lambda j: step(args.warmup + j),
                                             ctx.synchronize)
    stats_tok = round_stats(per_step_tok, 1e6 / batch)
    if args.token_graphs or args.eager:
        per_step, elapsed = per_step_tok, elapsed_tok
    stats = round_stats(per_step, 1e6 / batch)
    dt = stats["median"] * 1e-6 * batch
    # distinct experts per layer, from the routing of the steps just timed
    lg = logits_all.download(np.float32, total * Lq * batch * Eq).reshape(total, Lq, batch, Eq)
    for i in range(args.warmup, total):
        top = np.argsort(-lg[i], axis=-1)[..., :Kq]
        uniq.append(sum(len(set(top[l].ravel().tolist())) for l in range(Lq)))
    per_expert = sum(lay.sizes[k] for k in lay.sizes)
    nbytes = float(np.mean(uniq)) * per_expert + Lq * batch * (Eq * 4 + Hq * 2 + Hq * 4 + Hq * 2)
    value = nbytes / dt / 1e9
    log(f"qwen3 batch {batch}: {dt * 1e6:.1f} us/step ({dt * 1e6 / batch:.1f} us/token), "
        f"{value:.0f} GB/s ({value / PEAK_HBM_GBS * 100:.1f}% of {PEAK_HBM_GBS:.0f}), "
        f"{np.mean(uniq) / Lq:.1f} distinct experts per layer")
    kernels = {}
    if not args.no_profile_pass:
        ctx.set_profiling(True)
        ctx.profile_reset()
        for i in range(args.steps):
            ctx.copy_async(cur.ptr, logits_all.address((args.warmup + i) * step_logits),
                           step_logits)
            token()
        ctx.synchronize()
        for name in ("moe_layer", "gate_up", "down", "prefill_route", "prefill_group",
                     "prefill_gate_up", "prefill_down", "prefill_combine"):
            ms, n = ctx.profile(name)
            if n:
                kernels[name] = {"launches": n, "avg_us": ms / n * 1e3}
        ctx.set_profiling(False)
        log("kernels: " + ", ".join(f"{k} {v['avg_us']:.2f} us x{v['launches']}"
                                    for k, v in kernels.items()))
    sync_err = runner.sync_errors()
    roof = None
    gu = "gate_up" if "gate_up" in kernels else "prefill_gate_up"
    if "moe_layer" in kernels:
        lb = (float(np.mean(uniq)) / Lq) * per_expert + batch * (Eq * 4 + Hq * 2 + Hq * 4 + Hq * 2)
        ach = lb / (kernels["moe_layer"]["avg_us"] * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
                "kernel": "decode_layer_kernel (route + gate_up + SiLU-GLU + down + combine)",
                "bytes_per_launch": int(lb),
                "avg_launch_us": round(kernels["moe_layer"]["avg_us"], 3)}
    elif gu in kernels:
        gu_bytes = (float(np.mean(uniq)) / Lq) * (lay.sizes["gate_up_blocks"] +
                                                  lay.sizes["gate_up_scales"] +
                                                  lay.sizes["gate_up_bias"])
        ach = gu_bytes / (kernels[gu]["avg_us"] * 1e-6) / 1e9
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": None,
                "kernel": ("gate_up_kernel (fused MXFP4 gate_up GEMV + SiLU-GLU)" if gu == "gate_up"
                           else "prefill_gemm_kernel gate_up (grouped MXFP4 GEMM + SiLU-GLU)"),
                "bytes_per_launch": int(gu_bytes),
                "avg_launch_us": round(kernels[gu]["avg_us"], 3)}
    print(json.dumps({
        "metric": f"HBM GB/s (% of peak) + µs/token, Qwen3 MXFP4 MoE stack, batch {batch}",
        "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": timed,
        "steps_per_round": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "us_per_token": round(dt * 1e6 / batch, 2), "hbm_frac_of_peak": round(value / PEAK_HBM_GBS, 4),
        "us_per_token_graph_per_token": stats_tok["median"],
        "timing": ("eager launches" if args.eager else "one graph per step" if args.token_graphs
                   else "one graph per round"),
        "us_per_token_mean": round(elapsed / timed * 1e6 / batch, 2), "sync_errors": sync_err,
        **stats, "rounds_unit": "us/token",
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "compute": "e2m1 weights (MXFP4, exact) x bf16 activations, fp32 products and sums",
        "data": "synthetic (seeded MXFP4, zero bias sections, logits N(0,1) per token and layer)",
        "config": {"workload": f"qwen3-moe-stack-decode-b{batch}", "layers": Lq, "experts": Eq,
                   "top_k": Kq, "hidden": Hq, "intermediate": Fq, "batch": batch,
                   "parallelism": "single-gpu"},
        "kernels": kernels, "roofline": roof, "cpu_baseline": None}), flush=True)
    runner.close()
    ctx.close()
    if sync_err:
        log(f"FAILED: {sync_err} exchange wait(s) gave up; the timed outputs are invalid")
        return 1
    return 0


def sign_test_p(ratios) -> float:
    """Two-sided sign-test p-value of B beating A (ratio > 1), normal
    approximation; NaN below 8 pairs (ABResult.signTestP,
    DequantGEMVBenchmark.swift:237-248)."""
    n = len(ratios)
    if n < 8:
        return float("nan")
    wins = sum(1 for r in ratios if r > 1)
    z = abs(wins - n / 2) / (math.sqrt(n) / 2)
    return math.erfc(z / math.sqrt(2.0))


def interleaved_ab(sample_a, sample_b, pairs: int) -> dict:
    """compareInterleaved (DequantGEMVBenchmark.swift:250-286): `pairs` pairs of
    one timed sample of each side, the side that runs first alternating, so a
    pair's two samples are milliseconds apart.  A sample returns seconds per
    step; a pair's ratio is B's throughput over A's."""
    ratios, ta_all, tb_all = [], [], []
    for i in range(pairs):
        if i % 2 == 0:
            ta = sample_a(i)
            tb = sample_b(i)
        else:
            tb = sample_b(i)
            ta = sample_a(i)
        ratios.append(ta / tb)
        ta_all.append(ta)
        tb_all.append(tb)
    s = sorted(ratios)
    n = len(s)
    med = s[n // 2] if n % 2 else (s[n // 2 - 1] + s[n // 2]) / 2
    return {"pairs": n, "median_ratio": round(med, 4),
            "b_wins": sum(1 for r in ratios if r > 1), "sign_test_p": sign_test_p(ratios),
            "a_median_us": round(sorted(ta_all)[n // 2] * 1e6, 2),
            "b_median_us": round(sorted(tb_all)[n // 2] * 1e6, 2),
            "ratios": [round(r, 4) for r in ratios]}


def stack_sampler(gw, ctx, runner, layers, lay, n_layers: int, n_experts: int, top_k: int,
                  batch: int, logits_all, n_tokens: int, iters: int, seed: int):
    """One side of an A/B over a decode stack: its own activations, outputs and
    logits slot on `ctx`, the shared resident layers, the token captured as one
    graph.  Returns sample(i): `iters` tokens (logits i*iters.. of the shared
    pool, so both sides route alike), timed between two synchronisations,
    seconds per token."""
    H_, step_logits = lay.hidden_size, n_layers * batch * n_experts * 4
    cur = ctx.empty(step_logits)
    xs = [ctx.empty(batch * H_ * 2) for _ in range(n_layers + 1)]
    ctx.fill_normal(xs[0], gw.BF16, batch * H_, 0.0, 1.0, seed * 31 + 9)
    outs = [ctx.empty(batch * H_ * 4) for _ in range(n_layers)]
    ctx.synchronize()

    def token():
        for l in range(n_layers):
            runner.layer_forward(layers[l].ptr, lay.stride, n_experts, top_k, xs[l].ptr, gw.BF16,
                                 batch, outs[l].ptr, logits=cur.address(l * batch * n_experts * 4),
                                 out_bf16=xs[l + 1].ptr)

    graph = gw.Graph.capture(ctx, token)

    def step(t: int):
        ctx.copy_async(cur.ptr, logits_all.address((t % n_tokens) * step_logits), step_logits)
        graph.launch()

    for t in range(iters):   # warm-up
        step(t)
    ctx.synchronize()

    def sample(i: int) -> float:
        ctx.synchronize()
        t0 = time.perf_counter()
        for t in range(i * iters, (i + 1) * iters):
            step(t)
        ctx.synchronize()
        return (time.perf_counter() - t0) / iters / batch

    return sample


def parse_ab(spec: str) -> dict:
    env = {}
    for item in spec.split(","):
        name, sep, val = item.strip().partition("=")
        if not sep or not name.startswith("GODWIT_"):
            raise SystemExit(f"--ab takes GODWIT_NAME=VALUE[,GODWIT_NAME=VALUE...], got {item!r}")
        env[name] = val
    return env


def ab_bench(gw, args) -> int:
    """The reference's interleaved A/B (DequantGEMVBenchmark.swift:220-286) over
    the library's runtime switches: A is a context and runner made with the
    environment as it is, B one made with the `--ab` variables set (they are
    read at context and runner creation), both in this process over the same
    resident layers.  Workloads: decode (config 2's 36-layer GPT-OSS-120B
    stack) and qwen3 / qwen3-b8 (config 3).  Prints one JSON line with the
    pairs' B/A throughput ratios, their median, B's wins and the sign test."""
    b_env = parse_ab(args.ab)
    if args.workload == "decode":
        Hs, Fs, Es, Ks, Ls, act, batch, biases = H, F, E, K, L, ("gptOssClampedGLU", 7.0, 1.702), 1, True
    elif args.workload in ("qwen3", "qwen3-b8"):
        q = QWEN3
        Hs, Fs, Es, Ks, Ls = q["H"], q["F"], q["E"], q["K"], q["L"]
        act, biases = ("silu",), False
        batch = args.batch or (8 if args.workload == "qwen3-b8" else 1)
    else:
        raise SystemExit("--ab runs the decode, qwen3 and qwen3-b8 workloads")
    lay = gw.ExpertLayout(Hs, Fs, Es)

    def side(env: dict):
        saved = {k: os.environ.get(k) for k in env}
        os.environ.update(env)
        try:
            ctx = gw.Context(0)
            runner = gw.ExpertRunner(ctx, Hs, Fs, *act)
            runner.reserve_prefill(batch, Ks, Es)
        finally:
            for k, v in saved.items():
                if v is None:
                    os.environ.pop(k, None)
                else:
                    os.environ[k] = v
        return ctx, runner

    ctx_a, run_a = side({})
    ctx_b, run_b = side(b_env)
    layers = []
    for l in range(Ls):
        buf = ctx_a.empty(lay.layer_file_size)
        fill_layer(ctx_a, gw, buf, lay, Es, args.seed * 1000003 + l * 7919, biases=biases)
        layers.append(buf)
    n_tokens = 64
    logits_all = ctx_a.empty(n_tokens * Ls * batch * Es * 4)
    ctx_a.fill_normal(logits_all, gw.F32, n_tokens * Ls * batch * Es, 0.0, 1.0, args.seed * 31 + 7)
    ctx_a.synchronize()
    log(f"A/B on {args.workload} (batch {batch}): A = the environment as given, "
        f"B = {', '.join(f'{k}={v}' for k, v in b_env.items())}; {args.ab_pairs} pairs of "
        f"{args.ab_iters} tokens")
    sample_a = stack_sampler(gw, ctx_a, run_a, layers, lay, Ls, Es, Ks, batch, logits_all,
                             n_tokens, args.ab_iters, args.seed)
    sample_b = stack_sampler(gw, ctx_b, run_b, layers, lay, Ls, Es, Ks, batch, logits_all,
                             n_tokens, args.ab_iters, args.seed)
    res = interleaved_ab(sample_a, sample_b, args.ab_pairs)
    errs = run_a.sync_errors() + run_b.sync_errors()
    log(f"median B/A {res['median_ratio']:.4f}, B wins {res['b_wins']} of {res['pairs']}, "
        f"sign test p = {res['sign_test_p']:.3g}; A {res['a_median_us']} us/token, "
        f"B {res['b_median_us']} us/token; exchange waits that gave up: {errs}")
    print(json.dumps({"ab": {"workload": args.workload, "batch": batch, "a": "environment as given",
                             "b": b_env, "iterations_per_sample": args.ab_iters, **res,
                             "unit": "us/token", "sync_errors": errs}}), flush=True)
    for r in (run_a, run_b):
        r.close()
    for c in (ctx_a, ctx_b):
        c.close()
    return 1 if errs else 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawTextHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20,
                    help="timed steps per round; 7 rounds run (the median round is reported)")
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--seed", type=int, default=1)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="bounded CPU-baseline sample (0 disables it)")
    ap.add_argument("--no-profile-pass", action="store_true")
    ap.add_argument("--token-graphs", action="store_true",
                    help="decode stacks: time one captured graph per token (behind a copy of "
                         "its logits) instead of one graph per timing round")
    ap.add_argument("--eager", action="store_true",
                    help="decode stacks: as --token-graphs but each token's launches enqueued "
                         "directly, no graph (for profiler runs: rocprofv3's kernel trace has "
                         "crashed on the host inside graph launches of the batch-8 stack)")
    ap.add_argument("--counter-pass", type=int, default=0, metavar="MIB",
                    help="decode only: run --steps tokens eagerly (no graph, no events), then a "
                         "device-to-device copy of MIB MiB three times, and exit; the run "
                         "that rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE profiles (the copy "
                         "scales the counters to bytes)")
    ap.add_argument("--batch", type=int, default=None,
                    help="tokens per step for the qwen3 workloads (default 1, or 8 for qwen3-b8)")
    ap.add_argument("--workload", choices=["decode", "prefill", "qwen3", "qwen3-b8", "gemv",
                                           "gptoss20b"],
                    default="decode",
                    help="decode: benchmark config 2 (the headline line, default); prefill: "
                         "config 4, one GPT-OSS-120B layer, 512 Zipf-routed tokens; qwen3 / "
                         "qwen3-b8: config 3, the Qwen3 stack at batch 1 / 8; gemv: config 0, "
                         "one gate_up-shaped GEMV; gptoss20b: config 1, a 20B layer with its "
                         "router")
    ap.add_argument("--ab", default=None, metavar="GODWIT_NAME=VALUE[,...]",
                    help="interleaved A/B instead of the benchmark line: A = a context and runner "
                         "made with the environment as given, B = made with these variables set; "
                         "decode / qwen3 / qwen3-b8 workloads; prints the B/A ratios, their "
                         "median and a sign test")
    ap.add_argument("--ab-pairs", type=int, default=40)
    ap.add_argument("--ab-iters", type=int, default=12, help="tokens per A/B sample")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported by this "
              "build (the whole model fits one MI355X's HBM and every kernel here runs on a "
              "single GPU; sharding across GPUs is a design note, not code)", file=sys.stderr)
        return 2

    import godwit_amd as gw

    if args.ab:
        return ab_bench(gw, args)
    if args.counter_pass:
        return counter_pass(gw, args)
    if args.workload == "prefill":
        return prefill_bench(gw, args)
    if args.workload == "gemv":
        return gemv_bench(gw, args)
    if args.workload == "gptoss20b":
        return gptoss20b_bench(gw, args)
    if args.workload in ("qwen3", "qwen3-b8"):
        batch = args.batch or (8 if args.workload == "qwen3-b8" else 1)
        return qwen3_bench(gw, args, batch)

    ctx = gw.Context(0)
    lay = gw.ExpertLayout(H, F, E)
    runner = gw.ExpertRunner(ctx, H, F, "gptOssClampedGLU", 7.0, 1.702)
    t0 = time.perf_counter()
    layers = build_model(ctx, gw, lay, args.seed)
    log(f"resident experts: {L} x {E} x {lay.stride} B = {L * lay.layer_file_size / 1e9:.2f} GB "
        f"(filled in {time.perf_counter() - t0:.1f}s); {ctx.cu_count} CUs")

    timed = TIMING_ROUNDS * args.steps
    total_steps = args.warmup + timed
    logits_all = ctx.empty(total_steps * L * E * 4)
    ctx.fill_normal(logits_all, gw.F32, total_steps * L * E, 0.0, 1.0, args.seed * 31 + 7)
    cur_logits = ctx.empty(L * E * 4)
    xs = [ctx.empty(H * 2) for _ in range(L + 1)]
    ctx.fill_normal(xs[0], gw.BF16, H, 0.0, 1.0, args.seed * 31 + 9)
    outs = [ctx.empty(H * 4) for _ in range(L)]
    ids = ctx.empty(L * K * 4)
    ctx.synchronize()

    def token():
        for l in range(L):
            runner.layer_forward(layers[l].ptr, lay.stride, E, K, xs[l].ptr, gw.BF16, 1,
                                 outs[l].ptr, logits=cur_logits.address(l * E * 4),
                                 out_bf16=xs[l + 1].ptr, routing_ids=ids.address(l * K * 4))

    step_logits = L * E * 4

    def run_tokens(first: int, n: int):
        # tokens first .. first+n-1, each layer reading its own logits in place
        def run():
            for i in range(first, first + n):
                for l in range(L):
                    runner.layer_forward(layers[l].ptr, lay.stride, E, K, xs[l].ptr, gw.BF16, 1,
                                         outs[l].ptr,
                                         logits=logits_all.address(i * step_logits + l * E * 4),
                                         out_bf16=xs[l + 1].ptr,
                                         routing_ids=ids.address(l * K * 4))
        return run

    # The timed rounds: each round's tokens captured as one graph (36 layer
    # launches a token), replayed once per round (--token-graphs: one graph
    # per token, below, is the timing).
    if not (args.token_graphs or args.eager):
        per_step, elapsed = round_graphs(gw, ctx, args, run_tokens)
    # The same tokens as one graph per token, each behind a copy of its
    # logits into a fixed buffer (how a serving loop without per-round
    # capture would run them): reported beside the main figure.
    graph = None if args.eager else gw.Graph.capture(ctx, token)

    def step(i: int):
        ctx.copy_async(cur_logits.ptr, logits_all.address(i * step_logits), step_logits)
        if args.eager:
            token()
        else:
            graph.launch()

    for i in range(args.warmup):
        step(i)
    per_step_tok, elapsed_tok = timed_rounds(args.steps, lambda j: step(args.warmup + j),
                                             ctx.synchronize)
    stats_tok = round_stats(per_step_tok, 1e6)
    if args.token_graphs or args.eager:
        per_step, elapsed = per_step_tok, elapsed_tok
    stats = round_stats(per_step, 1e6)
    s_per_token = stats["median"] * 1e-6

    # routing sanity: the last token's experts are distinct and in range
    last = ids.download(np.int32, L * K).reshape(L, K)
    assert np.all((last >= 0) & (last < E)) and all(len(set(r)) == K for r in last)

    bytes_token = L * (K * expert_bytes(lay) + E * 4 + H * 2 + H * 4 + H * 2)
    value = bytes_token / s_per_token / 1e9
    log(f"{timed} tokens in {elapsed * 1e3:.2f} ms ({stats['rounds']} rounds, one graph a "
        f"{'token' if args.token_graphs or args.eager else 'round'}): median {stats['median']:.1f} us/token "
        f"(min {stats['min']:.1f}, max "
        f"{stats['max']:.1f}), {value:.0f} GB/s ({value / PEAK_HBM_GBS * 100:.1f}% of "
        f"{PEAK_HBM_GBS:.0f}); one graph a token behind a logits copy: "
        f"{stats_tok['median']:.1f} us/token")

    roofline = None
    kernels = {}
    if not args.no_profile_pass:
        # Same steps again, eagerly, with every launch bracketed by hipEvents.
        ctx.set_profiling(True)
        ctx.profile_reset()
        for i in range(args.steps):
            ctx.copy_async(cur_logits.ptr, logits_all.address((args.warmup + i) * step_logits),
                           step_logits)
            token()
        ctx.synchronize()
        for name in ("moe_layer", "route", "gate_up", "down"):
            ms, n = ctx.profile(name)
            if n:
                kernels[name] = {"launches": n, "avg_us": ms / n * 1e3}
        ctx.set_profiling(False)
        if "moe_layer" in kernels:
            dom, nbytes = "moe_layer", bytes_token // L
            desc = ("decode_layer_kernel (one launch per layer: route + MXFP4 gate_up GEMV + "
                    "SwiGLU + down GEMV + weighted combine)")
        else:
            dom, nbytes = "gate_up", gate_up_bytes(lay)
            desc = "gate_up_kernel (fused MXFP4 gate_up GEMV + bias + SwiGLU)"
        k_us = kernels[dom]["avg_us"]
        achieved = nbytes / (k_us * 1e-6) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS,
                    "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                    **measured_traffic(GATE_UP_TRAFFIC if dom == "gate_up" else DECODE_LAYER_TRAFFIC),
                    "kernel": desc, "bytes_per_launch": nbytes, "avg_launch_us": round(k_us, 3)}
        log("kernels: " + ", ".join(f"{k} {v['avg_us']:.2f} us x{v['launches']}"
                                    for k, v in kernels.items()))
    # every wave of every one-kernel layer found its exchange words (a wait
    # that gave up would have left wrong outputs in the timed steps)
    sync_err = runner.sync_errors()

    cpu = None
    if args.cpu_seconds > 0:
        c = cpu_baseline(args.cpu_seconds)
        cpu = {"value": round(bytes_token / (c["us_per_token"] * 1e-6) / 1e9, 4), "unit": "GB/s",
               "us_per_token": round(c["us_per_token"], 1), "cores": 1, "kind": "port",
               "sample": f"{c['tokens']} token(s) x {L} GPT-OSS-120B-shaped MoE layers (top-4 "
                         f"of 128 N(0,1) logits, 2880x2880 experts drawn from a pool of 32 "
                         f"synthetic ones), scalar C oracle, 1 thread, {c['seconds']:.1f} s",
               "cpu": platform.processor() or platform.machine()}
        try:
            with open("/proc/cpuinfo") as f:
                for ln in f:
                    if ln.startswith("model name"):
                        cpu["cpu"] = ln.split(":", 1)[1].strip()
                        break
        except OSError:
            pass
        log(f"cpu baseline: {c['us_per_token']:.0f} us/token ({cpu['value']:.3f} GB/s)")
        # The same port with each GEMV's rows split over the host's cores.
        ca = cpu_baseline(args.cpu_seconds / 2, host_threads())
        cpu["all_cores"] = {
            "value": round(bytes_token / (ca["us_per_token"] * 1e-6) / 1e9, 4), "unit": "GB/s",
            "us_per_token": round(ca["us_per_token"], 1), "cores": ca["threads"],
            "host_cpus": host_cpus(),
            "sample": f"{ca['tokens']} token(s), same workload, GEMV rows over "
                      f"{ca['threads']} OpenMP threads (every CPU of the process's affinity "
                      f"mask), {ca['seconds']:.1f} s"}
        log(f"cpu baseline, {ca['threads']} threads: {ca['us_per_token']:.0f} us/token "
            f"({cpu['all_cores']['value']:.3f} GB/s)")

    result = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": timed,
        "steps_per_round": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(s_per_token * 1e3, 4),
        "us_per_token": round(s_per_token * 1e6, 2),
        "us_per_token_mean": round(elapsed / timed * 1e6, 2),
        "us_per_token_graph_per_token": stats_tok["median"],
        "timing": ("eager launches" if args.eager else "one graph per token" if args.token_graphs
                   else "one graph per round"),
        "sync_errors": sync_err,
        **stats, "rounds_unit": "us/token",
        "hbm_frac_of_peak": round(value / PEAK_HBM_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "compute": "e2m1 weights (MXFP4, exact) x bf16 activations, fp32 products and sums",
        "data": "synthetic (seeded MXFP4 nibbles U{0..15}, scales U{119..127}, "
                "biases N(0,0.02) bf16, logits N(0,1) per token)",
        "config": {"workload": "gptoss120b-moe-stack-decode", "layers": L, "experts": E,
                   "top_k": K, "hidden": H, "intermediate": F, "tokens_per_step": 1,
                   "parallelism": "single-gpu",
                   "bytes_per_token": bytes_token, "resident_bytes": L * lay.layer_file_size},
        "kernels": kernels,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)
    if graph is not None:
        graph.destroy()
    runner.close()
    ctx.close()
    if sync_err:
        log(f"FAILED: {sync_err} exchange wait(s) gave up; the timed outputs are invalid")
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
