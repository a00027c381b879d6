"""Batched prefill (grouped GEMMs on the matrix cores) against the CPU oracle and
against the decode path.

The oracle is the reference's layer: route each token (Router.select), run
every selected expert (referenceMXFP4 GEMVs + activation with fp16 rounding)
and combine in router order.  Tolerance: the reference's expert metric
max|d|/mean|ref| per token (GodwitCLI/main.swift:518-532) below 1e-3, see
_close_batch; routing ids exact, weights to 1e-6.  Shapes cover one, two and three bf16
activation planes (bf16, fp16, fp32 x), partial feature tiles, K dimensions
that are not a multiple of the 256-element staging chunk, experts with no
tokens and experts with several 32-token tiles.
"""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from godwit_amd._lib import check, lib
from helpers import ExpertData, expert_metric, layer_check, normal_bf16, rng
from test_gpu_expert import GPTOSS, QWEN3, SMALL, _make_layer

pytestmark = pytest.mark.gpu


def _close_batch(got, ref):
    """Per-token expert metric (GodwitCLI/main.swift:518-532) below 1e-3, the
    north-star tolerance, and the median token below 1e-4.  A gate_up sum whose
    last fp32 bits differ from the oracle's can round its fp16 activation one ulp
    the other way (the reference rounds the activation to fp16, expert.metal:101);
    test_gpu_config4 takes the 512-token layer apart stage by stage and finds
    exactly such flips, plus fp32 summation differences within their bound."""
    m = np.array([expert_metric(got[t], ref[t]) for t in range(len(ref))])
    assert m.max() < 1e-3, (m.max(), np.argmax(m))
    assert np.median(m) < 1e-4, np.median(m)


def _zipf_logits(r, T, E, K, s=1.1):
    """Logits whose top-k per token is a Zipf(s)-popular draw of K distinct experts
    (benchmark config 4's assignment), ranked by decreasing logit."""
    p = 1.0 / np.arange(1, E + 1) ** s
    p /= p.sum()
    logits = (r.standard_normal((T, E)) - 10.0).astype(np.float32)
    for t in range(T):
        chosen = r.choice(E, size=K, replace=False, p=p)
        logits[t, chosen] = (5.0 - np.arange(K) + r.uniform(0, 0.5, K)).astype(np.float32)
    return logits


def _x(ctx, r, T, H, x_dtype):
    xbits, xw = normal_bf16(r, T * H)
    if x_dtype == gw.BF16:
        return ctx.buffer(xbits), xw
    if x_dtype == gw.F16:
        x = xw.astype(np.float16)
        return ctx.buffer(x), x.astype(np.float32)
    return ctx.buffer(xw.astype(np.float32)), xw.astype(np.float32)


def _run(ctx, runner, layout, buf, E, K, xb, x_dtype, lb, T, H, fn="prefill_forward"):
    out, out16 = ctx.empty(T * H * 4), ctx.empty(T * H * 2)
    ids_b, w_b = ctx.empty(T * K * 4), ctx.empty(T * K * 4)
    getattr(runner, fn)(buf.ptr, layout.stride, E, K, xb.ptr, x_dtype, T, out.ptr,
                        logits=lb.ptr, out_bf16=out16.ptr, routing_ids=ids_b.ptr,
                        routing_weights=w_b.ptr)
    ctx.synchronize()
    res = (out.download(np.float32, T * H).reshape(T, H), out16.download(np.uint16, T * H),
           ids_b.download(np.int32, T * K).reshape(T, K),
           w_b.download(np.float32, T * K).reshape(T, K))
    for b in (out, out16, ids_b, w_b):
        b.free()
    return res


@pytest.mark.parametrize("shape,E,K,T,x_dtype,seed", [
    (SMALL, 16, 4, 72, gw.BF16, 1),      # experts with 2-3 tiles, partial feature tiles
    (QWEN3, 32, 8, 24, gw.F16, 2),       # two activation planes, no biases, SiLU-GLU
    (GPTOSS, 12, 4, 20, gw.F32, 3),      # three planes, 2880-wide K (11.25 chunks)
    (SMALL, 200, 4, 32, gw.BF16, 4),     # 200 experts, 32 tokens routed in the group kernel
    (SMALL, 256, 8, 40, gw.BF16, 5),     # route kernel, then a scan over 256 experts
    (SMALL, 8, 2, 2048, gw.BF16, 6),     # ~16 tiles per expert: many units per XCD eighth
], ids=["small-bf16", "qwen3-f16", "gptoss-f32", "small-e200-t32", "small-e256-t40",
        "small-e8-t2048"])
def test_prefill_matches_oracle(ctx, shape, E, K, T, x_dtype, seed):
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2000 + seed)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2100 + seed)
    xb, xw = _x(ctx, r, T, H, x_dtype)
    logits = _zipf_logits(r, T, E, K)
    lb = ctx.buffer(logits)
    got, got16, ids, wts = _run(ctx, runner, layout, buf, E, K, xb, x_dtype, lb, T, H)
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                     shape["oact"])
    assert np.array_equal(ids, rids)
    assert np.allclose(wts, rw, rtol=1e-6, atol=1e-7)
    _close_batch(got, ref)
    rel_rms, worst, bound, ok = layer_check(got, ref)       # check-layer's acceptance
    assert ok, (rel_rms, worst, bound)
    assert np.array_equal(got16, oracle.f32_to_bf16_bits(got.ravel()))
    for b in (xb, lb, buf):
        b.free()
    runner.close()


def test_prefill_agrees_with_decode_path(ctx, monkeypatch):
    """The same 8 tokens through the grouped-GEMM prefill and the decode kernels
    (GODWIT_PREFILL_ABOVE=8 keeps layer_forward's 8-token batch on the latter)."""
    shape, E, K, T = GPTOSS, 8, 4, 8
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2200)
    monkeypatch.setenv("GODWIT_PREFILL_ABOVE", "8")
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2201)
    xb, xw = _x(ctx, r, T, H, gw.BF16)
    logits = r.standard_normal((T, E)).astype(np.float32)
    lb = ctx.buffer(logits)
    pre = _run(ctx, runner, layout, buf, E, K, xb, gw.BF16, lb, T, H, "prefill_forward")
    dec = _run(ctx, runner, layout, buf, E, K, xb, gw.BF16, lb, T, H, "layer_forward")
    assert np.array_equal(pre[2], dec[2])
    assert np.array_equal(pre[3], dec[3])
    _close_batch(pre[0], dec[0])
    for b in (xb, lb, buf):
        b.free()
    runner.close()


def test_layer_forward_sends_large_batches_to_prefill(ctx):
    """TransformerLayer.forward's batch entry: more than 8 tokens run the grouped GEMMs."""
    shape, E, K, T = SMALL, 8, 2, 40
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2300)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2301)
    xb, xw = _x(ctx, r, T, H, gw.BF16)
    logits = r.standard_normal((T, E)).astype(np.float32)
    lb = ctx.buffer(logits)
    ctx.set_profiling(True)
    ctx.profile_reset()
    got = _run(ctx, runner, layout, buf, E, K, xb, gw.BF16, lb, T, H, "layer_forward")
    n_gemm = ctx.profile("prefill_gate_up")[1] + ctx.profile("prefill_down")[1]
    ctx.set_profiling(False)
    assert n_gemm == 2
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                 shape["oact"])
    _close_batch(got[0], ref)
    for b in (xb, lb, buf):
        b.free()
    runner.close()


def test_prefill_router_and_graph_replay(ctx):
    """Device router logits feeding prefill, captured once (scratch reserved first) and
    replayed: every replay equals the eager result."""
    shape, E, K, T = SMALL, 16, 4, 48
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2400)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    runner.reserve_prefill(T, K, E)
    r = rng(2401)
    xb, xw = _x(ctx, r, T, H, gw.BF16)
    W = (r.standard_normal(E * H) * 0.02).astype(np.float32)
    wb = ctx.buffer(W)
    out = ctx.empty(T * H * 4)

    def body():
        runner.prefill_forward(buf.ptr, layout.stride, E, K, xb.ptr, gw.BF16, T, out.ptr,
                               router_weight=wb.ptr, router_weight_dtype=gw.F32)

    body()
    ctx.synchronize()
    eager = out.download(np.float32, T * H)
    logits = np.stack([oracle.router_logits(W, None, xw[t * H:(t + 1) * H], E, H)
                       for t in range(T)])
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                 shape["oact"])
    _close_batch(eager.reshape(T, H), ref)
    graph = gw.Graph.capture(ctx, body)
    for _ in range(3):
        out.zero()
        graph.launch()
        ctx.synchronize()
        assert np.array_equal(out.download(np.float32, T * H), eager)
    graph.destroy()
    for b in (xb, wb, out, buf):
        b.free()
    runner.close()


@pytest.mark.parametrize("shape,E,K,T,x_dtype,seed", [
    (QWEN3, 128, 8, 8, gw.BF16, 1),      # benchmark config 3's batch
    (SMALL, 8, 2, 32, gw.BF16, 2),       # many entries per expert (a full 32-entry tile)
    (SMALL, 256, 8, 32, gw.F16, 3),      # 256 experts, 256 entries, 8192 staged logits
    (GPTOSS, 12, 4, 20, gw.F32, 4),      # three planes, 2880-wide K
    (SMALL, 64, 4, 2, gw.BF16, 5),       # the smallest grouped batch
    (SMALL, 1, 1, 5, gw.BF16, 6),        # one expert: a one-bit mask, every entry in one tile
    (SMALL, 256, 8, 16, gw.F16, 7),      # 16 tokens over 256 experts
], ids=["qwen3-t8", "small-e8-t32", "small-e256-t32", "gptoss-f32-t20", "small-t2",
        "small-e1-t5", "small-e256-t16"])
def test_self_grouped_equals_tile_list(ctx, monkeypatch, shape, E, K, T, x_dtype, seed):
    """Batches of at most 32 tokens are routed and grouped inside the grouped
    GEMMs (every expert holds at most one 32-entry tile); GODWIT_SELF_GROUP_TOKENS=0
    sends them through the group kernel's tile list instead.  Both equal the
    oracle, and each other bit for bit (an entry's outputs depend only on its own
    column of the tile), routing included; a captured self-grouped layer replays
    to the same bytes."""
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2500 + seed)
    r = rng(2600 + seed)
    xb, xw = _x(ctx, r, T, H, x_dtype)
    logits = _zipf_logits(r, T, E, K) if seed % 2 else r.standard_normal((T, E)).astype(np.float32)
    lb = ctx.buffer(logits)
    runs = {}
    for mode in ("self", "list"):
        monkeypatch.setenv("GODWIT_SELF_GROUP_TOKENS", "32" if mode == "self" else "0")
        runner = gw.ExpertRunner(ctx, H, F, shape["act"])
        ctx.set_profiling(True)
        ctx.profile_reset()
        runs[mode] = _run(ctx, runner, layout, buf, E, K, xb, x_dtype, lb, T, H,
                          "prefill_forward")
        n_group = ctx.profile("prefill_group")[1]
        ctx.set_profiling(False)
        assert n_group == (0 if mode == "self" else 1), (mode, n_group)
        if mode == "self":
            runner.reserve_prefill(T, K, E)
            out = ctx.empty(T * H * 4)

            def body():
                runner.prefill_forward(buf.ptr, layout.stride, E, K, xb.ptr, x_dtype, T, out.ptr,
                                       logits=lb.ptr)

            graph = gw.Graph.capture(ctx, body)
            for _ in range(3):
                out.zero()
                graph.launch()
                ctx.synchronize()
                assert np.array_equal(out.download(np.float32, T * H), runs["self"][0].ravel())
            graph.destroy()
            out.free()
        runner.close()
    for i in range(4):
        assert np.array_equal(runs["self"][i], runs["list"][i]), i
    got, _, ids, wts = runs["self"]
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                     shape["oact"])
    assert np.array_equal(ids, rids)
    assert np.allclose(wts, rw, rtol=1e-6, atol=1e-7)
    _close_batch(got, ref)
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound)
    for b in (xb, lb, buf):
        b.free()


@pytest.mark.parametrize("shape,E,K,T,x_dtype,seed", [
    (QWEN3, 128, 8, 8, gw.BF16, 1),      # config 3's batch: one plane in, two for down
    (SMALL, 16, 4, 72, gw.F16, 2),       # two planes in, several tiles per expert (tile list)
    (GPTOSS, 12, 4, 20, gw.F32, 3),      # three planes: 2-deep rings only
    (SMALL, 256, 8, 32, gw.BF16, 4),     # 32 KB of logits: past the 8x2 ring, read in place
], ids=["qwen3-t8", "small-f16-t72", "gptoss-f32-t20", "small-e256-t32"])
def test_gemm_shapes_bit_identical(ctx, monkeypatch, shape, E, K, T, x_dtype, seed):
    """The grouped GEMMs run 8 waves with a 4-deep ring, 12 waves (4-deep; gate_up
    only, the down GEMM takes 8x4 instead), 8 waves with a 2-deep ring held to
    128 VGPRs so that two workgroups share a CU, or 4 waves with a 2-deep ring
    (gate_up with bf16 x only; three workgroups per CU); the launcher picks one
    per launch and GODWIT_PREFILL_SHAPE forces one at runner creation.  Every
    shape gives the same bytes (each output keeps its chunk and MFMA order),
    and the chosen one equals the oracle."""
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2700 + seed)
    r = rng(2800 + seed)
    xb, xw = _x(ctx, r, T, H, x_dtype)
    logits = _zipf_logits(r, T, E, K)
    lb = ctx.buffer(logits)
    runs = {}
    for forced in ("", "8x4", "12x4", "8x2", "4x2"):
        monkeypatch.setenv("GODWIT_PREFILL_SHAPE", forced)
        runner = gw.ExpertRunner(ctx, H, F, shape["act"])
        runs[forced] = _run(ctx, runner, layout, buf, E, K, xb, x_dtype, lb, T, H,
                            "prefill_forward")
        runner.close()
    for forced in ("8x4", "12x4", "8x2", "4x2"):
        for i in range(4):
            assert np.array_equal(runs[forced][i], runs[""][i]), (forced, i)
    got, _, ids, wts = runs[""]
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                     shape["oact"])
    assert np.array_equal(ids, rids)
    _close_batch(got, ref)
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound)
    for b in (xb, lb, buf):
        b.free()


@pytest.mark.parametrize("shape,E,K,T,x_dtype,seed", [
    (QWEN3, 128, 8, 8, gw.BF16, 1),      # self-grouped, 8x2 down GEMM, 8 counts per tile
    (SMALL, 16, 4, 72, gw.F16, 2),       # tile list, several tiles per expert
    (GPTOSS, 12, 4, 20, gw.F32, 3),      # 2880 rows: a partial last feature tile
    (SMALL, 8, 1, 40, gw.BF16, 4),       # top-1: every count completes at once
], ids=["qwen3-t8", "small-f16-t72", "gptoss-f32-t20", "small-top1-t40"])
def test_fused_combine_equals_kernel(ctx, monkeypatch, shape, E, K, T, x_dtype, seed):
    """The down GEMM combines in its epilogue: each entry counts itself on its
    (token, feature tile) and the workgroup whose count completes the tile sums
    it in router order (y stored and read device-coherent).  By default batches
    of up to 32 tokens do so; GODWIT_FUSED_COMBINE_TOKENS sets the bound (0: the
    separate combine kernel always).  Bit-identical to the combine kernel, on
    three calls in a row (the counters return to zero), and equal to the oracle."""
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2900 + seed)
    r = rng(3000 + seed)
    xb, xw = _x(ctx, r, T, H, x_dtype)
    logits = _zipf_logits(r, T, E, K) if K > 1 else r.standard_normal((T, E)).astype(np.float32)
    lb = ctx.buffer(logits)
    runs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("GODWIT_FUSED_COMBINE_TOKENS", "0" if mode == "0" else "100000")
        runner = gw.ExpertRunner(ctx, H, F, shape["act"])
        ctx.set_profiling(True)
        ctx.profile_reset()
        runs[mode] = [_run(ctx, runner, layout, buf, E, K, xb, x_dtype, lb, T, H,
                           "prefill_forward") for _ in range(3)]
        n_comb = ctx.profile("prefill_combine")[1]
        ctx.set_profiling(False)
        assert n_comb == (0 if mode == "1" else 3), (mode, n_comb)
        runner.close()
    for call in range(3):
        for i in range(4):
            assert np.array_equal(runs["1"][call][i], runs["0"][0][i]), (call, i)
    got, _, ids, wts = runs["1"][0]
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                     shape["oact"])
    assert np.array_equal(ids, rids)
    _close_batch(got, ref)
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound)
    for b in (xb, lb, buf):
        b.free()


# Down-projection scale bytes by output row: rows 0..191 take EDGE[r % 6] in
# every block (a 255 row holds one NaN block among 127s), rows 192.. mix the
# six bytes at random.
EDGE = (0, 1, 127, 253, 254, 255)


def _edge_scale_layer(ctx, E, seed):
    """A 256 x 128 GPT-OSS-activation layer without biases whose down scales are
    the e8m0 edge bytes.  Gate_up scales 2^-14 .. 2^-12 keep the activations near
    3e-3 (fp16 normal), so every down block partial stays below 0.2 and a row
    of 253 / 254 blocks sums to under 2^128: finite in the oracle.  Rows with
    codes 8 (-0) only in block 0 every seventh row."""
    shape = dict(hidden=256, inter=128, act="gptOssClampedGLU", oact=oracle.ACT_GPTOSS,
                 bias=False)
    H, F = shape["hidden"], shape["inter"]
    layout = gw.ExpertLayout(H, F, E)
    r = rng(seed)
    experts = []
    nbr = F // 32
    for _ in range(E):
        e = ExpertData(r, H, F, layout.offsets, layout.stride, with_bias=False)
        e.gu_scales[:] = r.integers(113, 116, size=e.gu_scales.size, dtype=np.uint8)
        sc = e.dn_scales.reshape(H, nbr)
        for row in range(H):
            if row < 192:
                b = EDGE[row % 6]
                sc[row] = 127 if b == 255 else b
                if b == 255:
                    sc[row, (row // 6) % nbr] = 255
            else:
                sc[row] = r.choice(EDGE, size=nbr)
        dn = e.dn_packed.reshape(H, F // 2)
        dn[::7, :16] = 0x88
        for name, arr in (("gate_up_scales", e.gu_scales), ("down_scales", e.dn_scales),
                          ("down_blocks", e.dn_packed)):
            off = layout.offsets[name]
            e.blob[off:off + arr.nbytes] = arr.view(np.uint8)
        experts.append(e)
    buf = ctx.buffer(np.concatenate([e.blob for e in experts]))
    return shape, layout, experts, buf


@pytest.mark.parametrize("forced", ["4x2", "8x2"])
@pytest.mark.parametrize("fn", ["prefill_forward", "prefill_forward_static"])
def test_fused_combine_narrow_feature_tiles(ctx, monkeypatch, forced, fn):
    """Batches of up to 32 tokens combine inside the down GEMM, which counts
    each token's arrivals per feature tile; the 4-wave shape cuts 2880 output
    rows into 23 tiles, the 8-wave ones into 12.  At GPT-OSS width, with a
    shape forced, the layer equals the oracle and the default shape bit for
    bit, from the runner's scratch and from the static array (which clears
    the counters itself)."""
    shape, E, K, T = GPTOSS, 16, 4, 24
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 3500)
    r = rng(3600)
    xb, xw = _x(ctx, r, T, H, gw.BF16)
    logits = _zipf_logits(r, T, E, K)
    lb = ctx.buffer(logits)
    runs = {}
    for tag in ("", forced):
        monkeypatch.setenv("GODWIT_PREFILL_SHAPE", tag)
        runner = gw.ExpertRunner(ctx, H, F, shape["act"])
        for rep in range(2):     # the second call finds the counters left at zero
            runs[(tag, rep)] = _run(ctx, runner, layout, buf, E, K, xb, gw.BF16, lb, T, H, fn)
        runner.close()
    for key, res in runs.items():
        for i in range(4):
            assert np.array_equal(res[i], runs[("", 0)][i]), (key, i)
    got, _, ids, wts = runs[(forced, 1)]
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                     shape["oact"])
    assert np.array_equal(ids, rids)
    _close_batch(got, ref)
    for b in (xb, lb, buf):
        b.free()


def _download(ctx, addr, dtype, count):
    out = np.empty(count, dtype)
    check(lib.gw_memcpy_dtoh(ctx.handle, out.ctypes.data, addr, out.nbytes))
    return out


def _fp16_range_layer(ctx, E, seed):
    """A 512 x 256 GPT-OSS-activation layer without biases whose down scale
    bytes sit at the ends of the range where e2m1 * 2^(b-127) is exact in fp16
    (104: 2^-24, the smallest fp16 subnormal, for code 1; 140: 6 * 2^13 for code
    7).  Rows come in classes of 32 (one wave of a workgroup): 139/140 only,
    104/105 only, and two mixed classes in which one row of the 32 holds a 141
    or a 103 block, which sends that wave to the split bf16 body.  Gate_up
    scales 2^-22 .. 2^-20 put most activations among the fp16 subnormals."""
    shape = dict(hidden=512, inter=256, act="gptOssClampedGLU", oact=oracle.ACT_GPTOSS,
                 bias=False)
    H, F = shape["hidden"], shape["inter"]
    layout = gw.ExpertLayout(H, F, E)
    r = rng(seed)
    experts = []
    nbr = F // 32
    for _ in range(E):
        e = ExpertData(r, H, F, layout.offsets, layout.stride, with_bias=False)
        e.gu_scales[:] = r.integers(105, 108, size=e.gu_scales.size, dtype=np.uint8)
        sc = e.dn_scales.reshape(H, nbr)
        for row in range(H):
            cls = (row // 32) % 4
            if cls == 0:
                sc[row] = r.choice([139, 140], size=nbr)
            elif cls == 1:
                sc[row] = r.choice([104, 105], size=nbr)
            else:
                sc[row] = r.choice([104, 105, 120, 139, 140], size=nbr)
                if row % 32 == (7 if cls == 2 else 19):
                    sc[row, row % nbr] = 141 if cls == 2 else 103
        for name, arr in (("gate_up_scales", e.gu_scales), ("down_scales", e.dn_scales)):
            off = layout.offsets[name]
            e.blob[off:off + arr.nbytes] = arr.view(np.uint8)
        experts.append(e)
    buf = ctx.buffer(np.concatenate([e.blob for e in experts]))
    return shape, layout, experts, buf


@pytest.mark.parametrize("T,forced", [(8, "8x2"), (8, "8x4"), (40, "8x2"), (40, "8x4")],
                         ids=["self-grouped-t8-8x2", "self-grouped-t8-8x4", "tile-list-t40-8x2",
                              "tile-list-t40-8x4"])
def test_prefill_down_fp16_range(ctx, monkeypatch, T, forced):
    """The down GEMM multiplies fp16 activations by weights widened to fp16 when
    a wave's scale bytes all lie in [104, 140], and splits each activation into
    two bf16 values otherwise.  Both are exact products summed in fp32: every
    expert output row (the runner's prefill scratch) is within the fp32
    summation bound 2^-16 * sum |terms| of an fp64 evaluation on the GPU's own
    fp16 activations (expert.metal:101 rounds them to fp16), subnormal
    activations and 2^-24 weights included, and the layer output matches
    oracle.moe_layer per feature row (rows span 2^-24 .. 2^13 in scale)."""
    E, K = 4, 2
    monkeypatch.setenv("GODWIT_PREFILL_SHAPE", forced)
    shape, layout, experts, buf = _fp16_range_layer(ctx, E, 3300 + T)
    H, F = shape["hidden"], shape["inter"]
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(3400 + T)
    xb, xw = _x(ctx, r, T, H, gw.BF16)
    logits = r.standard_normal((T, E)).astype(np.float32)
    lb = ctx.buffer(logits)
    got, got16, ids, wts = _run(ctx, runner, layout, buf, E, K, xb, gw.BF16, lb, T, H)
    view = runner.prefill_view()
    N = T * K
    assert view["activation_plane"] == 0
    act = _download(ctx, view["activations"], np.uint16, N * F).reshape(N, F)
    y = _download(ctx, view["expert_outputs"], np.float32, N * H).reshape(N, H)
    a32 = act.view(np.float16).astype(np.float32)
    sub = (a32 != 0) & (np.abs(a32) < 2.0 ** -14)
    assert sub.mean() > 0.5, sub.mean()             # mostly fp16 subnormals
    xw = xw.reshape(T, H)
    for t in range(T):
        for k in range(K):
            j = t * K + k
            o = experts[int(ids[t, k])].oracle_expert().arrays
            wd = oracle.decode(o[2], o[3], H * F // 32).reshape(H, F).astype(np.float64)
            y64 = wd @ a32[j].astype(np.float64)
            bound = (np.abs(wd) @ np.abs(a32[j].astype(np.float64))) * 2.0 ** -16 + 1e-45
            err = np.abs(y[j] - y64) / bound
            assert err.max() <= 1.0, (t, k, int(np.argmax(err)), err.max())
    ref, rids, _ = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                    shape["oact"])
    assert np.array_equal(ids, rids)
    for row in range(H):
        want = ref[:, row].astype(np.float64)
        d = np.abs(got[:, row].astype(np.float64) - want)
        assert d.max() <= 1e-3 * np.abs(want).mean(), (row, d.max(), np.abs(want).mean())
    assert np.array_equal(got16, oracle.f32_to_bf16_bits(got.ravel()))
    for b in (xb, lb, buf):
        b.free()
    runner.close()


@pytest.mark.parametrize("T", [8, 40], ids=["self-grouped-t8", "tile-list-t40"])
def test_prefill_edge_scales(ctx, T):
    """Every e8m0 edge byte through the grouped GEMMs against referenceMXFP4
    (DequantGEMVBenchmark.swift:106-116), which multiplies each finite block
    partial by its scale (MXFP4.decodeScale, MXFP4.swift:37-40): bytes 0 and 1
    (subnormal scales), 127, 253 and 254 (e2m1 * 2^126 and 2^127 pass the bf16
    maximum for |code| >= 4 and >= 2), 255 (NaN), and code 8 (-0).  NaN outputs
    sit exactly where the oracle's are, no output is infinite, and every finite
    output of feature row r is within 1e-3 of the mean |oracle| of that row
    over the batch (rows span 2^-127 .. 2^127, so the bound is per row)."""
    E, K = 4, 2
    shape, layout, experts, buf = _edge_scale_layer(ctx, E, 3100 + T)
    H, F = shape["hidden"], shape["inter"]
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(3200 + T)
    xb, xw = _x(ctx, r, T, H, gw.BF16)
    logits = r.standard_normal((T, E)).astype(np.float32)
    lb = ctx.buffer(logits)
    got, got16, ids, _ = _run(ctx, runner, layout, buf, E, K, xb, gw.BF16, lb, T, H)
    ref, rids, _ = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits, xw, H, F,
                                    shape["oact"])
    assert np.array_equal(ids, rids)
    nan_ref = np.isnan(ref)
    assert nan_ref[:, 5:192:6].all() and not nan_ref[:, :192][:, np.arange(192) % 6 != 5].any()
    assert np.array_equal(np.isnan(got), nan_ref)
    assert not np.isinf(ref).any() and not np.isinf(got).any()
    # Row classes reach the range ends: 2^127-scaled rows near 1e37, 2^-127 near 1e-39.
    assert np.abs(ref[:, 4:192:6]).max() > 1e36 and 0 < np.abs(ref[:, 0:192:6]).max() < 1e-37
    for row in range(H):
        fin = ~nan_ref[:, row]      # a mixed row is NaN only for tokens of its NaN experts
        if not fin.any():
            continue
        want = ref[fin, row].astype(np.float64)
        d = np.abs(got[fin, row].astype(np.float64) - want)
        assert d.max() <= 1e-3 * np.abs(want).mean(), (row, d.max(), np.abs(want).mean())
    assert np.array_equal(got16, oracle.f32_to_bf16_bits(got.ravel()))
    for b in (xb, lb, buf):
        b.free()
    runner.close()
