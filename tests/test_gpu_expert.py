"""GPU parity of ExpertRunner (apply / applyBatch / applyAssignments) and the
device-routed MoE layer against the CPU oracle.

Tolerances: the north star's rel. 1e-3 under both reference metrics — the GEMV
metric max|d|/max(|ref|,1) (DequantGEMVBenchmark.swift:338-349) and the expert
metric max|d|/mean|ref| (GodwitCLI/main.swift:518-532).  Routing is exact.
"""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from helpers import ExpertData, expert_metric, gemv_metric, layer_check, normal_bf16, rng

pytestmark = pytest.mark.gpu

GPTOSS = dict(hidden=2880, inter=2880, act="gptOssClampedGLU", oact=oracle.ACT_GPTOSS, bias=True)
QWEN3 = dict(hidden=2048, inter=768, act="silu", oact=oracle.ACT_SWIGLU, bias=False)
SMALL = dict(hidden=256, inter=128, act="gptOssClampedGLU", oact=oracle.ACT_GPTOSS, bias=True)


def _close(got, ref, tol=1e-3):
    """Composed outputs use the expert metric max|d|/mean|ref| (runExpertCheck,
    GodwitCLI/main.swift:518-532).  The per-element GEMV metric does not apply
    to them: the activation is rounded to fp16 (expert.metal:101), so a gate_up
    sum that differs from the oracle's in its last fp32 bits can round one fp16
    ulp the other way, and that ulp moves every down output by ~0.1 absolute —
    large next to outputs that happen to be near zero.  Each stage is checked
    with the strict GEMV metric in test_expert_stages_decomposed."""
    assert expert_metric(got, ref) < tol, expert_metric(got, ref)


def _make_layer(ctx, shape, n_experts, seed):
    layout = gw.ExpertLayout(shape["hidden"], shape["inter"], n_experts)
    r = rng(seed)
    experts = [ExpertData(r, shape["hidden"], shape["inter"], layout.offsets, layout.stride,
                          with_bias=shape["bias"]) for _ in range(n_experts)]
    buf = ctx.buffer(np.concatenate([e.blob for e in experts]))
    return layout, experts, buf


@pytest.mark.parametrize("shape", [GPTOSS, QWEN3, SMALL], ids=["gptoss", "qwen3", "small"])
@pytest.mark.parametrize("x_dtype", [gw.F16, gw.BF16, gw.F32])
def test_expert_apply(ctx, shape, x_dtype):
    """ExpertRunner.apply (ExpertRunner.swift:275-331) vs the oracle's expert."""
    layout, experts, buf = _make_layer(ctx, shape, 1, 100 + x_dtype)
    runner = gw.ExpertRunner(ctx, shape["hidden"], shape["inter"], shape["act"])
    r = rng(200 + x_dtype)
    if x_dtype == gw.BF16:
        x, xw = normal_bf16(r, shape["hidden"])
    elif x_dtype == gw.F16:
        x = r.standard_normal(shape["hidden"]).astype(np.float16)
        xw = x.astype(np.float32)
    else:
        x = xw = r.standard_normal(shape["hidden"]).astype(np.float32)
    got = runner.apply(x, gw.Weights(buf, runner.section_offsets), dtype=x_dtype)
    ref = oracle.expert_apply(experts[0].oracle_expert(), xw, shape["hidden"], shape["inter"],
                              shape["oact"])
    _close(got, ref)
    runner.close()
    buf.free()


def test_section_offsets_match_layout(ctx):
    runner = gw.ExpertRunner(ctx, 2880, 2880)
    layout = gw.ExpertLayout(2880, 2880, 128)
    assert runner.section_offsets == layout.offsets
    runner.close()


@pytest.mark.parametrize("shape", [GPTOSS, QWEN3], ids=["gptoss", "qwen3"])
def test_expert_stages_decomposed(ctx, shape):
    """The expert's three stages through the kernel-level entry points, each against
    the oracle on the GPU's own input to that stage: gate_up GEMV + bias (GEMV metric
    < 1e-3), activation (fp16 equal up to one ulp), down GEMV + bias on the GPU's fp16
    activation (GEMV metric < 1e-3).  Then the fused runner must agree with this
    unfused chain."""
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, 1, 150)
    e = experts[0]
    r = rng(151)
    xbits, xw = normal_bf16(r, H)
    xb = ctx.buffer(xbits)
    gu = ctx.empty(2 * F * 4)
    act = ctx.empty(F * 2)
    out = ctx.empty(H * 4)
    sec = layout.offsets
    pk = lambda name: buf.address(sec[name])
    import ctypes
    from godwit_amd._lib import check, lib
    check(lib.gw_mxfp4_gemv_bias(ctx.handle, pk("gate_up_blocks"), pk("gate_up_scales"),
                                 pk("gate_up_bias"), gw.BF16, xb.ptr, gw.BF16, gu.ptr, 2 * F, H))
    ctx.synchronize()
    gu_gpu = gu.download(np.float32, 2 * F)
    gu_ref = oracle.gemv_bias(e.gu_packed, e.gu_scales, e.gu_bias, xw, 2 * F, H)
    assert gemv_metric(gu_gpu, gu_ref) < 1e-3
    gw.expert_activation(ctx, shape["act"], gu, act, F)
    act_gpu = act.download(np.float16, F)
    act_ref = oracle.activation(shape["oact"], gu_gpu)
    a, b = act_gpu.astype(np.float32), act_ref.astype(np.float32)
    assert np.all(np.abs(a - b) <= np.spacing(np.abs(b).astype(np.float16)).astype(np.float32))
    check(lib.gw_mxfp4_gemv_bias(ctx.handle, pk("down_blocks"), pk("down_scales"),
                                 pk("down_bias"), gw.BF16, act.ptr, gw.F16, out.ptr, H, F))
    ctx.synchronize()
    dn_gpu = out.download(np.float32, H)
    dn_ref = oracle.gemv_bias(e.dn_packed, e.dn_scales, e.dn_bias, act_gpu.astype(np.float32),
                              H, F)
    assert gemv_metric(dn_gpu, dn_ref) < 1e-3
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    fused = runner.apply(xbits, gw.Weights(buf, runner.section_offsets), dtype=gw.BF16)
    assert expert_metric(fused, dn_gpu) < 1e-3
    runner.close()
    for b_ in (xb, gu, act, out, buf):
        b_.free()


@pytest.mark.parametrize("shape", [GPTOSS, QWEN3], ids=["gptoss", "qwen3"])
def test_apply_batch_is_weighted_sum(ctx, shape):
    """ExpertRunner.applyBatch (:191-269) vs the oracle, and linearity:
    combined == sum_i w_i * apply_i."""
    n = 4 if shape is GPTOSS else 8
    layout, experts, buf = _make_layer(ctx, shape, n, 300)
    runner = gw.ExpertRunner(ctx, shape["hidden"], shape["inter"], shape["act"])
    r = rng(301)
    x = r.standard_normal(shape["hidden"]).astype(np.float16)
    w = r.dirichlet(np.ones(n)).astype(np.float32)
    ws = [gw.Weights(buf.address(i * layout.stride), runner.section_offsets) for i in range(n)]
    got = runner.apply_batch(x, list(zip(ws, w)))
    ref = oracle.expert_apply_batch([e.oracle_expert() for e in experts], w,
                                    x.astype(np.float32), shape["hidden"], shape["inter"],
                                    shape["oact"])
    _close(got, ref)
    singles = np.stack([runner.apply(x, wi) for wi in ws]).astype(np.float64)
    lin = (singles * w[:, None].astype(np.float64)).sum(0)
    assert expert_metric(got, lin) < 1e-6
    runner.close()
    buf.free()


def test_apply_batch_empty_returns_zeros(ctx):
    runner = gw.ExpertRunner(ctx, 256, 128)
    got = runner.apply_batch(np.ones(256, np.float16), [])
    assert np.array_equal(got, np.zeros(256, np.float32))
    runner.close()


def test_apply_assignments_accumulates_expert_major(ctx):
    """ExpertRunner.applyAssignments (:108-182): outputs[token] += w * expert(x), in
    place, with experts shared across tokens read once per plan."""
    shape = GPTOSS
    n_experts, tokens = 6, 5
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 400)
    runner = gw.ExpertRunner(ctx, shape["hidden"], shape["inter"], shape["act"])
    r = rng(401)
    x = r.standard_normal((tokens, shape["hidden"])).astype(np.float16)
    prior = r.standard_normal((tokens, shape["hidden"])).astype(np.float32)
    assigns = []
    for t in range(tokens):
        for e, wt in zip(r.choice(n_experts, 3, replace=False), r.dirichlet(np.ones(3))):
            assigns.append((int(e), t, float(wt)))
    r.shuffle(assigns)
    xb, ob = ctx.buffer(x), ctx.buffer(prior)
    offs = runner.section_offsets
    runner.apply_assignments(
        xb, [gw.Assignment(gw.Weights(buf.address(e * layout.stride), offs), t, wt)
             for e, t, wt in assigns], ob, dtype=gw.F16)
    got = ob.download(np.float32, tokens * shape["hidden"]).reshape(tokens, -1)
    ref = oracle.apply_assignments([e.oracle_expert() for e in experts], assigns,
                                   x.astype(np.float32), prior, shape["hidden"], shape["inter"],
                                   shape["oact"])
    for t in range(tokens):
        _close(got[t], ref[t])
    xb.free()
    ob.free()
    runner.close()
    buf.free()


def test_apply_assignments_many_chunks(ctx):
    """More tokens and assignments than one plan holds (8 tokens, 64 slots): the runner
    splits them and keeps accumulating."""
    shape = SMALL
    n_experts, tokens = 10, 20
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 500)
    runner = gw.ExpertRunner(ctx, shape["hidden"], shape["inter"], shape["act"])
    r = rng(501)
    x = r.standard_normal((tokens, shape["hidden"])).astype(np.float16)
    assigns = [(int(e), t, float(w)) for t in range(tokens)
               for e, w in zip(r.choice(n_experts, 4, replace=False), r.dirichlet(np.ones(4)))]
    xb = ctx.buffer(x)
    ob = ctx.buffer(np.zeros((tokens, shape["hidden"]), np.float32))
    offs = runner.section_offsets
    runner.apply_assignments(
        xb, [gw.Assignment(gw.Weights(buf.address(e * layout.stride), offs), t, w)
             for e, t, w in assigns], ob, dtype=gw.F16)
    got = ob.download(np.float32).reshape(tokens, -1)
    ref = oracle.apply_assignments([e.oracle_expert() for e in experts], assigns,
                                   x.astype(np.float32), np.zeros((tokens, shape["hidden"])),
                                   shape["hidden"], shape["inter"], shape["oact"])
    for t in range(tokens):
        _close(got[t], ref[t])
    xb.free()
    ob.free()
    runner.close()
    buf.free()


def _layer_case(ctx, shape, n_experts, top_k, tokens, seed, router):
    layout, experts, buf = _make_layer(ctx, shape, n_experts, seed)
    runner = gw.ExpertRunner(ctx, shape["hidden"], shape["inter"], shape["act"])
    r = rng(seed + 1)
    H = shape["hidden"]
    xbits, xw = normal_bf16(r, tokens * H)
    xb = ctx.buffer(xbits)
    out = ctx.empty(tokens * H * 4)
    out16 = ctx.empty(tokens * H * 2)
    ids_b, w_b = ctx.empty(tokens * top_k * 4), ctx.empty(tokens * top_k * 4)
    kw = {}
    extra = []
    if router:
        W = (r.standard_normal(n_experts * H) * 0.02).astype(np.float32)
        wbuf = ctx.buffer(W)
        extra.append(wbuf)
        kw = dict(router_weight=wbuf.ptr, router_weight_dtype=gw.F32)
        logits = np.stack([oracle.router_logits(W, None, xw[t * H:(t + 1) * H], n_experts, H)
                           for t in range(tokens)])
    else:
        logits = r.standard_normal((tokens, n_experts)).astype(np.float32)
        lb = ctx.buffer(logits)
        extra.append(lb)
        kw = dict(logits=lb.ptr)
    runner.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xb.ptr, gw.BF16, tokens,
                         out.ptr, out_bf16=out16.ptr, routing_ids=ids_b.ptr,
                         routing_weights=w_b.ptr, **kw)
    ctx.synchronize()
    got = out.download(np.float32, tokens * H).reshape(tokens, H)
    got16 = out16.download(np.uint16, tokens * H)
    ids = ids_b.download(np.int32, tokens * top_k).reshape(tokens, top_k)
    wts = w_b.download(np.float32, tokens * top_k).reshape(tokens, top_k)
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], top_k, logits, xw, H,
                                     shape["inter"], shape["oact"])
    for b in [xb, out, out16, ids_b, w_b, buf] + extra:
        b.free()
    runner.close()
    return got, got16, ids, wts, ref, rids, rw


def test_layer_config1_gptoss20b_router(ctx):
    """Benchmark config 1 shape: 32 GPT-OSS experts, fp32 router N(0, 0.02), top-4,
    bf16 x, batch 1."""
    got, got16, ids, wts, ref, rids, rw = _layer_case(ctx, GPTOSS, 32, 4, 1, 600, router=True)
    assert np.array_equal(ids, rids)
    # the device's router logits differ from the oracle's in their last bits
    # (summation order), which moves the softmax weights by ~1e-6 relative
    assert np.allclose(wts, rw, rtol=1e-5, atol=1e-6)
    _close(got[0], ref[0])
    assert np.array_equal(got16, oracle.f32_to_bf16_bits(got.ravel()))


def test_layer_given_logits_128_experts(ctx):
    """Benchmark config 2 layer: 128 experts, logits ~ N(0,1), top-4.  Also the
    reference's own layer acceptance (check-layer: routing exact, relative RMS
    < 2e-3, max error < 4 fp16 ulps of the peak)."""
    got, _, ids, wts, ref, rids, rw = _layer_case(ctx, GPTOSS, 128, 4, 1, 700, router=False)
    assert np.array_equal(ids, rids)
    assert np.allclose(wts, rw, rtol=1e-6, atol=1e-7)
    _close(got[0], ref[0])
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound)


@pytest.mark.parametrize("tokens,path", [(1, "stream"), (3, "stream"), (8, "stream"),
                                         (3, "grouped"), (8, "grouped"), (8, "listed")])
def test_layer_qwen3_decode(ctx, monkeypatch, tokens, path):
    """Benchmark config 3 layer: Qwen3 shape, top-8 of 128, no biases, SiLU-GLU, batch 1/8.
    A batch of 2..8 tokens takes the grouped GEMMs by default, which group it
    themselves; GODWIT_SELF_GROUP_TOKENS=0 gives them the group kernel's tile list
    ("listed") and GODWIT_PREFILL_ABOVE=8 keeps the batch on the streaming decode
    kernels (both read at runner creation)."""
    monkeypatch.setenv("GODWIT_PREFILL_ABOVE", "8" if path == "stream" else "2")
    monkeypatch.setenv("GODWIT_SELF_GROUP_TOKENS", "0" if path == "listed" else "32")
    got, _, ids, wts, ref, rids, rw = _layer_case(ctx, QWEN3, 128, 8, tokens, 800 + tokens,
                                                  router=False)
    assert np.array_equal(ids, rids)
    for t in range(tokens):
        _close(got[t], ref[t])
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound)


@pytest.mark.parametrize("shape,experts,top_k,tokens", [(GPTOSS, 16, 4, 3), (QWEN3, 128, 8, 5),
                                                      (QWEN3, 128, 8, 8)],
                         ids=["gptoss-gate_up-12-waves", "qwen3-down-12-waves",
                              "qwen3-gate_up-12-waves"])
def test_grouped_gemm_wide_workgroups(ctx, shape, experts, top_k, tokens):
    """Small batches whose grouped GEMMs run 12-wave (384-feature) workgroups,
    chosen when that takes one round of workgroups fewer: GPT-OSS gate_up at
    12 entries, Qwen3 down at 40 entries, Qwen3 gate_up at 64 entries."""
    got, _, ids, wts, ref, rids, rw = _layer_case(ctx, shape, experts, top_k, tokens,
                                                  1500 + tokens, router=False)
    assert np.array_equal(ids, rids)
    for t in range(tokens):
        _close(got[t], ref[t])
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound)


@pytest.mark.parametrize("experts,top_k,tokens,path", [(128, 8, 8, "stream"), (64, 4, 3, "stream"),
                                                        (300, 4, 2, "stream"),
                                                        (128, 8, 8, "grouped")])
def test_layer_routing_ties_exact(ctx, monkeypatch, experts, top_k, tokens, path):
    """Device routing reproduces Router.select's partial selection sort exactly, ties
    included: logits drawn from 6 distinct values, so most top-k picks are ties
    broken by the sort's swap history.  300 experts exercises the standalone route
    kernel, the other streaming cases the routing fused into the gate_up kernel, the
    grouped case the routing inside the self-grouped gate_up GEMM."""
    monkeypatch.setenv("GODWIT_PREFILL_ABOVE", "8" if path == "stream" else "2")
    shape = SMALL
    H = shape["hidden"]
    layout, experts_d, buf = _make_layer(ctx, shape, experts, 1000 + experts)
    runner = gw.ExpertRunner(ctx, H, shape["inter"], shape["act"])
    r = rng(1001)
    logits = r.choice(np.array([-1.0, 0.0, 0.5, 1.0, 2.0, 3.0], np.float32),
                      size=(tokens, experts)).astype(np.float32)
    xbits, xw = normal_bf16(r, tokens * H)
    lb, xb = ctx.buffer(logits), ctx.buffer(xbits)
    out = ctx.empty(tokens * H * 4)
    ids_b, w_b = ctx.empty(tokens * top_k * 4), ctx.empty(tokens * top_k * 4)
    runner.layer_forward(buf.ptr, layout.stride, experts, top_k, xb.ptr, gw.BF16, tokens,
                         out.ptr, logits=lb.ptr, routing_ids=ids_b.ptr, routing_weights=w_b.ptr)
    ctx.synchronize()
    ids = ids_b.download(np.int32, tokens * top_k).reshape(tokens, top_k)
    wts = w_b.download(np.float32, tokens * top_k).reshape(tokens, top_k)
    got = out.download(np.float32, tokens * H).reshape(tokens, H)
    for t in range(tokens):
        rid, rw = oracle.router_select(logits[t], top_k)
        assert list(ids[t]) == list(rid), (t, list(ids[t]), list(rid))
        assert np.allclose(wts[t], rw, rtol=1e-6, atol=1e-7)
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts_d], top_k, logits, xw, H,
                                 shape["inter"], shape["oact"])
    for t in range(tokens):
        _close(got[t], ref[t])
    for b in (lb, xb, out, ids_b, w_b, buf):
        b.free()
    runner.close()


def _routing_logits(case, tokens, experts):
    """Logits for the two device selection paths: distinct values (the fast
    path), ties only below the top k (still fast), a tie inside the top k,
    -0.0 against +0.0 at the top, a NaN among the rest, a NaN as the first
    element (the reference's scan keeps it: nothing compares greater)."""
    r = rng(1100 + len(case) + tokens)
    lg = r.standard_normal((tokens, experts)).astype(np.float32)
    for t in range(tokens):
        order = np.argsort(-lg[t])
        if case == "ties_below":
            lg[t, order[6:]] = lg[t, order[6]]
        elif case == "tie_inside":
            lg[t, order[1]] = lg[t, order[0]]
        elif case == "signed_zero":
            lg[t] = -np.abs(lg[t]) - 1.0
            lg[t, 5], lg[t, 9] = np.float32(-0.0), np.float32(0.0)
        elif case == "nan_rest":
            lg[t, order[-1]] = np.nan
        elif case == "nan_first":
            lg[t, 0] = np.nan
    return lg


@pytest.mark.parametrize("case", ["distinct", "ties_below", "tie_inside", "signed_zero",
                                  "nan_rest", "nan_first"])
@pytest.mark.parametrize("tokens,path", [(1, "stream"), (2, "stream"), (3, "grouped"),
                                         (32, "grouped"), (3, "listed"), (40, "grouped")])
def test_routing_selection_paths(ctx, monkeypatch, case, tokens, path):
    """Device routing equals Router.select (the oracle) for inputs that take the
    fast selection and for those that fall back to the exact sort: decode
    (fused into gate_up, one and two tokens), the self-grouped GEMMs (3 and 32
    tokens, selecting from logits staged in LDS), the grouping kernel (3 tokens
    with GODWIT_SELF_GROUP_TOKENS=0) and the prefill route kernel (40 tokens)."""
    shape = SMALL
    H, E, K = shape["hidden"], 64, 4
    layout, experts_d, buf = _make_layer(ctx, shape, E, 1200)
    monkeypatch.setenv("GODWIT_PREFILL_ABOVE", "8" if path == "stream" else "1")
    monkeypatch.setenv("GODWIT_SELF_GROUP_TOKENS", "0" if path == "listed" else "32")
    runner = gw.ExpertRunner(ctx, H, shape["inter"], shape["act"])
    logits = _routing_logits(case, tokens, E)
    xbits, _ = normal_bf16(rng(1201), tokens * H)
    lb, xb = ctx.buffer(logits), ctx.buffer(xbits)
    out = ctx.empty(tokens * H * 4)
    ids_b, w_b = ctx.empty(tokens * K * 4), ctx.empty(tokens * K * 4)
    runner.layer_forward(buf.ptr, layout.stride, E, K, xb.ptr, gw.BF16, tokens, out.ptr,
                         logits=lb.ptr, routing_ids=ids_b.ptr, routing_weights=w_b.ptr)
    ctx.synchronize()
    ids = ids_b.download(np.int32, tokens * K).reshape(tokens, K)
    wts = w_b.download(np.float32, tokens * K).reshape(tokens, K)
    for t in range(tokens):
        rid, rw = oracle.router_select(logits[t], K)
        assert list(ids[t]) == list(rid), (case, t, list(ids[t]), list(rid))
        assert np.allclose(wts[t], rw, rtol=1e-6, atol=1e-7, equal_nan=True), (case, t)
    for b in (lb, xb, out, ids_b, w_b, buf):
        b.free()
    runner.close()


def test_layer_graph_replay_matches_eager(ctx):
    """A captured 3-layer chain replayed several times equals the eager result each time."""
    shape = SMALL
    n_experts, layers, H = 16, 3, shape["hidden"]
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 900)
    runner = gw.ExpertRunner(ctx, H, shape["inter"], shape["act"])
    r = rng(901)
    xbits, _ = normal_bf16(r, H)
    logits = r.standard_normal((layers, n_experts)).astype(np.float32)
    lb = ctx.buffer(logits)
    xs = [ctx.buffer(xbits)] + [ctx.empty(H * 2) for _ in range(layers)]
    outs = [ctx.empty(H * 4) for _ in range(layers)]

    def chain():
        for l in range(layers):
            runner.layer_forward(buf.ptr, layout.stride, n_experts, 4, xs[l].ptr, gw.BF16, 1,
                                 outs[l].ptr, logits=lb.address(l * n_experts * 4),
                                 out_bf16=xs[l + 1].ptr)

    chain()
    ctx.synchronize()
    eager = outs[-1].download(np.float32, H)
    graph = gw.Graph.capture(ctx, chain)
    for _ in range(4):
        outs[-1].zero()
        graph.launch()
        ctx.synchronize()
        assert np.array_equal(outs[-1].download(np.float32, H), eager)
    graph.destroy()
    for b in xs + outs + [lb, buf]:
        b.free()
    runner.close()


def _random_config(seed):
    r = rng(5000 + seed)
    H = int(r.choice([128, 160, 256, 384, 512]))
    F = int(r.choice([128, 192, 256, 320]))
    act, oact = (("gptOssClampedGLU", oracle.ACT_GPTOSS) if r.random() < 0.5
                 else ("silu", oracle.ACT_SWIGLU))
    E = int(r.integers(1, 40))
    K = int(r.integers(1, min(8, E) + 1))
    T = int(r.choice([1, 1, 2, 3, 5, 8, 13, 33]))
    return dict(hidden=H, inter=F, act=act, oact=oact, bias=bool(r.random() < 0.7)), E, K, T


@pytest.mark.parametrize("seed", range(12))
def test_layer_random_configurations(ctx, seed):
    """Seeded random shapes (hidden and intermediate multiples of 32 from 128 to
    512, 1..39 experts, top-1..8, 1..33 tokens, either activation, with or
    without biases) through gw_moe_layer_forward — the streaming kernels for one
    token, the grouped GEMMs otherwise — against the oracle: routing exact,
    outputs under the expert metric and the reference's layer acceptance."""
    shape, E, K, T = _random_config(seed)
    got, _, ids, wts, ref, rids, rw = _layer_case(ctx, shape, E, K, T, 5100 + seed,
                                                  router=False)
    assert np.array_equal(ids, rids), (shape["hidden"], shape["inter"], E, K, T)
    assert np.allclose(wts, rw, rtol=1e-6, atol=1e-7)
    for t in range(T):
        _close(got[t], ref[t])
    rel_rms, worst, bound, ok = layer_check(got, ref)
    assert ok, (rel_rms, worst, bound, shape["hidden"], shape["inter"], E, K, T)
