"""Phase timeline of the one-token layer kernel (decode_layer_kernel).

    python godwit_amd/build.py --trace          # once, on the build host
    python godwit_amd/decode_timeline.py gptoss [layers]
    python godwit_amd/decode_timeline.py qwen3 [layers]

Loads libgodwit_hip_trace.so (the library built with -DGW_DECODE_TRACE),
whose layer kernel stores wall_clock64() (100 MHz) from lane 0 of every wave
at 13 phase boundaries.  A stack of `layers` layers (default 12) with fresh
synthetic experts (nibbles U{0..15}, scales U{119..127}, GPT-OSS biases
N(0, 0.02)) and logits N(0, 1) is captured as one graph of one-token layers,
each layer's bf16 output the next one's input, as in bench.py's decode
stack, and replayed; 8 samples are taken of the last layer of a replay.
For every phase it prints, over the samples, the median of the median and
of the maximum over workgroups, in microseconds from the grid's first start,
for the gate_up waves (0-3) and the DMA waves (4-7) separately; then the
device gap between consecutive layers and each sample's span.  The stamps
cost a store each, so spans run a little longer than the plain kernel's.
"""
import ctypes
import os
import sys

os.environ["GODWIT_TRACE_LIB"] = "1"
sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import numpy as np  # noqa: E402

import godwit_amd as gw  # noqa: E402
from godwit_amd._lib import lib  # noqa: E402

PHASES = ["start", "routed", "stream queued/flagged", "exchange phase", "own pieces + publish",
          "exchange reads out", "down widened", "exchange complete", "products issued",
          "combine start", "end", "first word check", "partials written"]
SHAPES = {"gptoss": (2880, 2880, 128, 4, "gptOssClampedGLU", True),
          "qwen3": (2048, 768, 128, 8, "silu", False)}
LAUNCH_SLOTS, MAX_GRID, WAVES, STAMPS = 4, 256, 8, 16


def fill(ctx, buf, lay, n_experts, seed, biases):
    o, sz = lay.offsets, lay.sizes
    ctx.fill_uniform_u8(buf, 0, 255, seed)
    for sec, k in (("gate_up_scales", 1), ("down_scales", 2)):
        ctx.fill_uniform_u8(buf, 119, 127, seed * 131 + k, offset=o[sec], count=sz[sec],
                            rows=n_experts, row_stride=lay.stride)
    for sec, k in (("gate_up_bias", 3), ("down_bias", 4)):
        if biases:
            ctx.fill_normal(buf, gw.BF16, sz[sec] // 2, 0.0, 0.02, seed * 131 + k,
                            offset=o[sec], rows=n_experts, row_stride=lay.stride)
        else:
            ctx.fill_uniform_u8(buf, 0, 0, 0, offset=o[sec], count=sz[sec], rows=n_experts,
                                row_stride=lay.stride)


def main():
    name = sys.argv[1] if len(sys.argv) > 1 else "gptoss"
    nl = int(sys.argv[2]) if len(sys.argv) > 2 else 12
    H, F, E, K, act, biases = SHAPES[name]
    read = getattr(lib, "gw_debug_decode_trace", None)
    if read is None:
        sys.exit("the loaded library has no phase stamps: build it with build.py --trace")
    read.restype = ctypes.c_int
    read.argtypes = [ctypes.c_void_p]
    ctx = gw.Context(0)
    lay = gw.ExpertLayout(H, F, E)
    runner = gw.ExpertRunner(ctx, H, F, act)
    bufs = []
    for l in range(nl):
        bufs.append(ctx.empty(lay.layer_file_size))
        fill(ctx, bufs[-1], lay, E, 1000003 + l * 7919, biases)
    logits = ctx.empty(nl * E * 4)
    ctx.fill_normal(logits, gw.F32, nl * E, 0.0, 1.0, 7)
    xs = [ctx.empty(H * 2) for _ in range(nl + 1)]
    ctx.fill_normal(xs[0], gw.BF16, H, 0.0, 1.0, 9)
    out = ctx.empty(H * 4)
    ctx.synchronize()

    def token():
        for l in range(nl):
            runner.layer_forward(bufs[l].ptr, lay.stride, E, K, xs[l].ptr, gw.BF16, 1, out.ptr,
                                 logits=logits.address(l * E * 4), out_bf16=xs[l + 1].ptr)

    graph = gw.Graph.capture(ctx, token)
    for _ in range(20):
        graph.launch()
    ctx.synchronize()
    raw = np.zeros(LAUNCH_SLOTS * MAX_GRID * WAVES * STAMPS, np.uint64)
    grid = ctx.cu_count
    samples, gaps = [], []
    for _ in range(8):
        for _ in range(3):
            graph.launch()
        ctx.synchronize()
        if read(raw.ctypes.data) != 0:
            sys.exit("reading the phase stamps failed")
        t = raw.reshape(LAUNCH_SLOTS, MAX_GRID, WAVES, STAMPS)[:, :grid].astype(np.int64)
        # the last four layers of the replay, in launch order
        order = np.argsort([t[e, :, :, 0].min() for e in range(LAUNCH_SLOTS)])
        gaps += [(t[order[i + 1], :, :, 0].min() - t[order[i], :, :, 10].max()) * 0.01
                 for i in range(LAUNCH_SLOTS - 1)]
        samples.append(t[order[-1]])
    print(f"{name}: {nl} layers, grid {grid}, exchange waits that gave up: {runner.sync_errors()}")
    print(f"device gap, one layer's last end to the next one's first start: "
          f"median {np.median(gaps):.2f} us")
    for kind, waves in (("gate_up waves 0-3", range(0, 4)), ("DMA waves 4-7", range(4, 8))):
        print(f"== {kind}: us from the grid's first start, median over samples of the "
              f"[median, max] over workgroups")
        for p, label in enumerate(PHASES):
            med, mx = [], []
            for t in samples:
                v = (t[:, list(waves), p] - t[:, :, 0].min()) * 0.01
                med.append(np.median(v))
                mx.append(v.max())
            print(f"  {p:2d} {label:22s} median {np.median(med):6.2f}  max {np.median(mx):6.2f}")
    print("== per wave: median over samples of the median over workgroups (us)")
    print("  " + " " * 25 + " ".join(f"  w{w}  " for w in range(WAVES)))
    for p, label in enumerate(PHASES):
        row = []
        for w in range(WAVES):
            row.append(np.median([np.median((t[:, w, p] - t[:, :, 0].min()) * 0.01) for t in samples]))
        print(f"  {p:2d} {label:22s}" + " ".join(f"{v:6.2f}" for v in row))
    print("== within a workgroup: median over samples and workgroups of the latest wave minus the "
          "workgroup's median wave (us)")
    for p in (6, 11, 7, 8, 12):
        d = [np.median((t[:, :, p].max(axis=1) - np.median(t[:, :, p], axis=1)) * 0.01) for t in samples]
        print(f"  {p:2d} {PHASES[p]:22s} {np.median(d):5.2f}")
    spans = [(t[:, :, 10].max() - t[:, :, 0].min()) * 0.01 for t in samples]
    print("span, first start to last end, per sample (us):", " ".join(f"{v:.2f}" for v in spans))
    graph.destroy()
    runner.close()
    ctx.close()


if __name__ == "__main__":
    main()
