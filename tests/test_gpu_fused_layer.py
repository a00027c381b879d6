"""The one-token layer kernel (route -> gate_up + down stream into LDS ->
in-kernel activation exchange -> down + combine, one launch) against the
two-kernel form of the same layer (GODWIT_DECODE_LAYER=0) and against the CPU
oracle.

Both forms compute the gate_up rows with the same lane mapping and order, so
their activations are the same bytes.  The one-kernel form sums the down rows
on the matrix cores (16x16x32 fp16 products accumulated in fp32) where the
two-kernel form sums them lane by lane on the VALU, so the fp32 row sums may
round differently: the forms are required to agree to 1e-5 of the output's
peak.  Routing is exact in both.  The oracle check uses the reference's
expert metric, max|d|/mean|ref| < 1e-3 (GodwitCLI/main.swift:518-532).  Every
test also requires the kernel's bounded waits to have all succeeded, except
the one that makes them give up on purpose (from the host: every kernel
still exits normally).  The one-kernel form takes 16-bit x; fp32 x stays on
the two kernels.
"""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from helpers import normal_bf16, rng
from test_gpu_expert import GPTOSS, QWEN3, _close, _make_layer

pytestmark = pytest.mark.gpu


def _inputs(ctx, r, H, x_dtype):
    xbits, xw = normal_bf16(r, H)
    if x_dtype == gw.BF16:
        return ctx.buffer(xbits), xw
    if x_dtype == gw.F16:
        x = xw.astype(np.float16)
        return ctx.buffer(x), x.astype(np.float32)
    return ctx.buffer(xw.astype(np.float32)), xw.astype(np.float32)


def _forward(ctx, runner, layout, buf, n_experts, top_k, xb, x_dtype, lb, H):
    out, out16 = ctx.empty(H * 4), ctx.empty(H * 2)
    ids_b, w_b = ctx.empty(top_k * 4), ctx.empty(top_k * 4)
    runner.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xb.ptr, x_dtype, 1, out.ptr,
                         logits=lb.ptr, out_bf16=out16.ptr, routing_ids=ids_b.ptr,
                         routing_weights=w_b.ptr)
    ctx.synchronize()
    res = (out.download(np.float32, H), out16.download(np.uint16, H),
           ids_b.download(np.int32, top_k), w_b.download(np.float32, top_k))
    for b in (out, out16, ids_b, w_b):
        b.free()
    return res


def _kernel_counts(ctx, fn, names=("moe_layer", "gate_up", "down")):
    ctx.set_profiling(True)
    ctx.profile_reset()
    fn()
    counts = {k: ctx.profile(k)[1] for k in names}
    ctx.set_profiling(False)
    return counts


def _router(r, n_experts, H, w_dt, with_bias):
    """Router weights N(0, 0.02) in w_dt (and the same values as fp32), and an
    optional bf16 bias N(0, 0.1)."""
    W = (r.standard_normal(n_experts * H) * 0.02).astype(np.float32)
    if w_dt == gw.BF16:
        dev = oracle.f32_to_bf16_bits(W)
        W = oracle.bf16_bits_to_f32(dev)
    elif w_dt == gw.F16:
        dev = W.astype(np.float16)
        W = dev.astype(np.float32)
    else:
        dev = W
    bias_bits = bias = None
    if with_bias:
        bias_bits = oracle.f32_to_bf16_bits((r.standard_normal(n_experts) * 0.1).astype(np.float32))
        bias = oracle.bf16_bits_to_f32(bias_bits)
    return dev, W, bias_bits, bias


@pytest.mark.parametrize("shape,n_experts,top_k,w_dt,with_bias",
                         [(GPTOSS, 32, 4, gw.F32, False), (GPTOSS, 128, 4, gw.BF16, True),
                          (GPTOSS, 64, 4, gw.F16, True), (QWEN3, 128, 8, gw.BF16, False)],
                         ids=["gptoss20b-f32", "gptoss120b-bf16-bias", "gptoss-64-f16-bias",
                              "qwen3-bf16"])
def test_fused_layer_in_kernel_router(ctx, monkeypatch, shape, n_experts, top_k, w_dt, with_bias):
    """Router weights and one 16-bit token: the one-kernel layer computes the
    logits itself (each workgroup one slice of one logit, the partials
    exchanged across the grid), so the layer is one launch with no router
    kernel.  The two-kernel form's router adds the same slices in the same
    order: the routing ids and weights are the same bits and the outputs agree
    to 1e-5 of the peak.  Against the oracle (router_logits then moe_layer,
    its own summation order): ids equal, weights to 1e-5, the expert metric."""
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 1900 + n_experts)
    r = rng(1901 + n_experts)
    xb, xw = _inputs(ctx, r, H, gw.BF16)
    wdev, W, bias_bits, bias = _router(r, n_experts, H, w_dt, with_bias)
    wb = ctx.buffer(wdev)
    bb = ctx.buffer(bias_bits) if with_bias else None
    kw = dict(router_weight=wb.ptr, router_weight_dtype=w_dt)
    if with_bias:
        kw.update(router_bias=bb.ptr, router_bias_dtype=gw.BF16)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    fused = gw.ExpertRunner(ctx, H, F, shape["act"])
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "0")
    split = gw.ExpertRunner(ctx, H, F, shape["act"])
    got, counts = {}, {}
    for name, runner in (("fused", fused), ("split", split)):
        out, ids_b, w_b = ctx.empty(H * 4), ctx.empty(top_k * 4), ctx.empty(top_k * 4)

        def run():
            runner.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xb.ptr, gw.BF16, 1,
                                 out.ptr, routing_ids=ids_b.ptr, routing_weights=w_b.ptr, **kw)
            ctx.synchronize()

        counts[name] = _kernel_counts(ctx, run, ("moe_layer", "router", "gate_up", "down"))
        got[name] = (out.download(np.float32, H), ids_b.download(np.int32, top_k),
                     w_b.download(np.float32, top_k))
        for b in (out, ids_b, w_b):
            b.free()
    assert counts["fused"] == {"moe_layer": 1, "router": 0, "gate_up": 0, "down": 0}, counts
    assert counts["split"] == {"moe_layer": 0, "router": 1, "gate_up": 1, "down": 1}, counts
    f_out, f_ids, f_w = got["fused"]
    s_out, s_ids, s_w = got["split"]
    assert np.array_equal(f_ids, s_ids)
    assert np.array_equal(f_w.view(np.uint32), s_w.view(np.uint32))
    assert np.max(np.abs(f_out - s_out)) <= 1e-5 * np.max(np.abs(s_out))
    assert fused.sync_errors() == 0
    logits = oracle.router_logits(W, bias, xw, n_experts, H)
    ref, rids, rw = oracle.moe_layer([e.oracle_expert() for e in experts], top_k, logits[None, :],
                                     xw, H, F, shape["oact"])
    assert list(f_ids) == list(rids[0])
    assert np.allclose(f_w, rw[0], rtol=1e-5, atol=1e-6)
    _close(f_out, ref[0])
    for b in [xb, wb, buf] + ([bb] if with_bias else []):
        b.free()
    fused.close()
    split.close()


@pytest.mark.parametrize("shape,n_experts,top_k", [(GPTOSS, 32, 4), (QWEN3, 128, 8)],
                         ids=["gptoss", "qwen3"])
@pytest.mark.parametrize("x_dtype", [gw.BF16, gw.F16, gw.F32], ids=["bf16", "f16", "f32"])
def test_fused_layer_equals_two_kernel_form(ctx, monkeypatch, shape, n_experts, top_k, x_dtype):
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 1200 + n_experts)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    fused = gw.ExpertRunner(ctx, H, F, shape["act"])
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "0")
    split = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(1300 + x_dtype)
    xb, xw = _inputs(ctx, r, H, x_dtype)
    logits = r.standard_normal(n_experts).astype(np.float32)
    lb = ctx.buffer(logits)

    got = {}
    counts = {}
    for name, runner in (("fused", fused), ("split", split)):
        counts[name] = _kernel_counts(ctx, lambda: got.__setitem__(
            name, _forward(ctx, runner, layout, buf, n_experts, top_k, xb, x_dtype, lb, H)))
    one = {"moe_layer": 1, "gate_up": 0, "down": 0}
    two = {"moe_layer": 0, "gate_up": 1, "down": 1}
    assert counts["fused"] == (two if x_dtype == gw.F32 else one), counts
    assert counts["split"] == two, counts
    f_out, f16, f_ids, f_w = got["fused"]
    s_out, s16, s_ids, s_w = got["split"]
    assert np.array_equal(f_ids, s_ids) and np.array_equal(f_w, s_w)
    if x_dtype == gw.F32:   # both runners use the two kernels
        assert np.array_equal(f_out, s_out) and np.array_equal(f16, s16)
    else:
        # the one-kernel layer sums the down rows on the matrix cores, in
        # another order than the two-kernel form's lanes: fp32 rounding only
        assert np.max(np.abs(f_out - s_out)) <= 1e-5 * np.max(np.abs(s_out))
    assert np.array_equal(f16, oracle.f32_to_bf16_bits(f_out))
    assert fused.sync_errors() == 0

    rid, rw = oracle.router_select(logits, top_k)
    assert list(got["fused"][2]) == list(rid)
    assert np.allclose(got["fused"][3], rw, rtol=1e-6, atol=1e-7)
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], top_k, logits[None, :],
                                 xw, H, F, shape["oact"])
    _close(got["fused"][0], ref[0])
    assert np.array_equal(got["fused"][1], oracle.f32_to_bf16_bits(got["fused"][0]))
    for b in (xb, lb, buf):
        b.free()
    fused.close()
    split.close()


@pytest.mark.parametrize("shape,n_experts,top_k", [(GPTOSS, 16, 1), (GPTOSS, 16, 2), (GPTOSS, 16, 3),
                                                   (QWEN3, 32, 1), (QWEN3, 32, 3), (QWEN3, 32, 6)],
                         ids=["gptoss-k1", "gptoss-k2", "gptoss-k3", "qwen3-k1", "qwen3-k3",
                              "qwen3-k6"])
def test_fused_layer_smaller_top_k(ctx, monkeypatch, shape, n_experts, top_k):
    """Every top-k the one-kernel layer accepts below the models' own (GPT-OSS
    1-3 of its 4, Qwen3 below 8): fewer down rows per workgroup, so whole
    tiles, down pieces and exchange reads fall past the rows and read zeros.
    One launch per layer; the two-kernel form to 1e-5 of the peak, the oracle
    to the expert metric, routing exact; and three graph replays equal to
    the eager launch."""
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 2100 + 10 * top_k)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    fused = gw.ExpertRunner(ctx, H, F, shape["act"])
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "0")
    split = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2200 + top_k)
    xb, xw = _inputs(ctx, r, H, gw.BF16)
    logits = r.standard_normal(n_experts).astype(np.float32)
    lb = ctx.buffer(logits)
    got = {}
    counts = _kernel_counts(ctx, lambda: got.__setitem__(
        "fused", _forward(ctx, fused, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)))
    assert counts == {"moe_layer": 1, "gate_up": 0, "down": 0}, counts
    got["split"] = _forward(ctx, split, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)
    f_out, f16, f_ids, f_w = got["fused"]
    s_out, _, s_ids, s_w = got["split"]
    assert np.array_equal(f_ids, s_ids) and np.array_equal(f_w, s_w)
    assert np.max(np.abs(f_out - s_out)) <= 1e-5 * np.max(np.abs(s_out))
    assert np.array_equal(f16, oracle.f32_to_bf16_bits(f_out))
    rid, rw = oracle.router_select(logits, top_k)
    assert list(f_ids) == list(rid)
    assert np.allclose(f_w, rw, rtol=1e-6, atol=1e-7)
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], top_k, logits[None, :],
                                 xw, H, F, shape["oact"])
    _close(f_out, ref[0])
    out = ctx.empty(H * 4)
    _replay_equals_eager(
        ctx, lambda: fused.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xb.ptr,
                                         gw.BF16, 1, out.ptr, logits=lb.ptr),
        lambda: None, [out], [f_out], replays=3)
    assert fused.sync_errors() == 0
    for b in (xb, lb, buf, out):
        b.free()
    fused.close()
    split.close()


def _oracle_token(buf, layout, n_experts, top_k, logits, xw, shape):
    """oracle.moe_layer for one token, downloading only the experts the router
    selects (the other entries of the list repeat one of them; the oracle's
    own routing never reads them)."""
    from helpers import expert_from_blob
    ids, _ = oracle.router_select(logits, top_k)
    sel = {int(e): expert_from_blob(buf.download(np.uint8, layout.stride, offset=int(e) * layout.stride),
                                    layout) for e in ids}
    first = sel[int(ids[0])]
    experts = [sel.get(i, first) for i in range(n_experts)]
    out, oids, _ = oracle.moe_layer(experts, top_k, logits[None, :], xw, shape["hidden"],
                                    shape["inter"], shape["oact"])
    assert list(oids[0]) == list(ids)
    return out[0]


def _chain_weights(ctx, shape, n_experts, layers, seed):
    from helpers import fill_layer_device
    layout = gw.ExpertLayout(shape["hidden"], shape["inter"], n_experts)
    bufs = []
    for l in range(layers):
        bufs.append(ctx.empty(layout.stride * n_experts))
        fill_layer_device(ctx, bufs[-1], layout, n_experts, seed + 7 * l, biases=shape["bias"])
    return layout, bufs


def _replay_equals_eager(ctx, chain, reset, outputs, eager, replays=4):
    graph = gw.Graph.capture(ctx, chain)
    for _ in range(replays):
        reset()
        graph.launch()
        ctx.synchronize()
        for l, (o, want) in enumerate(zip(outputs, eager)):
            assert np.array_equal(o.download(want.dtype, want.size), want), l
    graph.destroy()


@pytest.mark.parametrize("shape,n_experts,top_k,layers",
                         [(GPTOSS, 128, 4, 8), (GPTOSS, 16, 4, 12)], ids=["gptoss120b-8", "gptoss-16x12"])
def test_fused_layer_chain_per_layer(ctx, monkeypatch, shape, n_experts, top_k, layers):
    """A chain of one-token layers with their own weights, each layer's bf16
    output the next one's input (GPT-OSS's clamped activation keeps the values
    bounded without the norm between layers): every layer's output matches
    the oracle run on that layer's own GPU bf16 input, and its bf16 copy is
    the next input.  The chain is then captured and replayed 4 times: every
    replay equals the eager chain at every layer, and no exchange ever gave
    up.  The replays advance the kernel's launch epochs well past their first
    values."""
    H, F = shape["hidden"], shape["inter"]
    layout, bufs = _chain_weights(ctx, shape, n_experts, layers, 1400)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(1401 + n_experts)
    xbits, _ = normal_bf16(r, H)
    logits = r.standard_normal((layers, n_experts)).astype(np.float32)
    lb = ctx.buffer(logits)
    xs = [ctx.buffer(xbits)] + [ctx.empty(H * 2) for _ in range(layers)]
    outs = [ctx.empty(H * 4) for _ in range(layers)]

    def chain():
        for l in range(layers):
            runner.layer_forward(bufs[l].ptr, layout.stride, n_experts, top_k, xs[l].ptr, gw.BF16,
                                 1, outs[l].ptr, logits=lb.address(l * n_experts * 4),
                                 out_bf16=xs[l + 1].ptr)

    counts = _kernel_counts(ctx, chain)
    assert counts == {"moe_layer": layers, "gate_up": 0, "down": 0}, counts
    eager = [o.download(np.float32, H) for o in outs]
    inputs = [x.download(np.uint16, H) for x in xs]
    for l in range(layers):
        assert np.all(np.isfinite(eager[l])), l
        assert np.array_equal(inputs[l + 1], oracle.f32_to_bf16_bits(eager[l])), l
        ref = _oracle_token(bufs[l], layout, n_experts, top_k, logits[l],
                            oracle.bf16_bits_to_f32(inputs[l]), shape)
        _close(eager[l], ref)

    def reset():
        for o in outs:
            o.zero()

    _replay_equals_eager(ctx, chain, reset, outs, eager)
    assert runner.sync_errors() == 0
    for b in xs + outs + bufs + [lb]:
        b.free()
    runner.close()


@pytest.mark.parametrize("shape,n_experts,top_k,layers,eps",
                         [(QWEN3, 128, 8, 8, 1e-6), (GPTOSS, 128, 4, 8, 1e-5)],
                         ids=["qwen3-8", "gptoss120b-8"])
def test_fused_block_chain_per_layer(ctx, monkeypatch, shape, n_experts, top_k, layers, eps):
    """The decode step's MoE half over a stack of layers with their own weights
    and norm weights (TransformerLayer.swift:140-143, 232-238): stream +=
    MoE(RMSNorm(stream)), each layer's MoE one launch.  Every layer is run
    eagerly and checked against the oracle composition on that layer's own GPU
    input stream (oracle.rmsnorm_f16, the oracle layer, the fp32 residual add):
    the change the layer made to the stream to the expert metric, the routing
    exact.  The stack is then captured and replayed 4 times from the same
    starting stream: every layer's bf16 copy of the stream equals the eager
    one.  (Qwen3's SwiGLU has no clamp: bare layers chained without the norm
    overflow fp16 within a few layers, so this is the form its chain takes.)"""
    H, F = shape["hidden"], shape["inter"]
    layout, bufs = _chain_weights(ctx, shape, n_experts, layers, 1700)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(1701 + n_experts)
    stream0 = r.standard_normal(H).astype(np.float32)
    wbits = [oracle.f32_to_bf16_bits((1.0 + 0.1 * r.standard_normal(H)).astype(np.float32))
             for _ in range(layers)]
    logits = r.standard_normal((layers, n_experts)).astype(np.float32)
    lb = ctx.buffer(logits)
    wb = [ctx.buffer(w) for w in wbits]
    sb = ctx.buffer(stream0)
    copies = [ctx.empty(H * 2) for _ in range(layers)]
    ids = [ctx.empty(top_k * 4) for _ in range(layers)]

    def layer(l):
        runner.block_forward(bufs[l].ptr, layout.stride, n_experts, top_k, 1, sb.ptr, wb[l].ptr,
                             eps, logits=lb.address(l * n_experts * 4), out_bf16=copies[l].ptr,
                             routing_ids=ids[l].ptr)

    ctx.set_profiling(True)
    ctx.profile_reset()
    stream = stream0
    for l in range(layers):
        layer(l)
        ctx.synchronize()
        after = sb.download(np.float32, H)
        normed = oracle.rmsnorm_f16(stream, wbits[l], eps).view(np.float16).astype(np.float32)
        ref = _oracle_token(bufs[l], layout, n_experts, top_k, logits[l], normed[0], shape)
        rid, _ = oracle.router_select(logits[l], top_k)
        assert list(ids[l].download(np.int32, top_k)) == list(rid), l
        assert np.all(np.isfinite(after)), l
        _close(after - stream, ref)
        assert np.array_equal(copies[l].download(np.uint16, H), oracle.f32_to_bf16_bits(after)), l
        stream = after
    assert ctx.profile("moe_layer")[1] == layers
    assert ctx.profile("gate_up")[1] == 0
    ctx.set_profiling(False)
    eager = [c.download(np.uint16, H) for c in copies]
    _replay_equals_eager(ctx, lambda: [layer(l) for l in range(layers)],
                         lambda: sb.upload(stream0), copies, eager)
    assert runner.sync_errors() == 0
    for b in copies + ids + wb + bufs + [sb, lb]:
        b.free()
    runner.close()


def test_in_kernel_router_interleaved_with_logits(ctx, monkeypatch):
    """One-token layers that alternate given logits and router weights (each
    launch clears the next launch's router-partial words whether it routes
    from weights or not), eagerly and replayed from a graph: every layer's
    routing and output equal the two-kernel form's."""
    shape, n_experts, top_k = GPTOSS, 32, 4
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 2000)
    r = rng(2001)
    pattern = ["router", "logits", "router", "router", "logits", "logits", "router"]
    xs, srcs, keep = [], [], []
    for i, kind in enumerate(pattern):
        xb, _ = _inputs(ctx, r, H, gw.BF16)
        xs.append(xb)
        if kind == "router":
            wdev, _, _, _ = _router(r, n_experts, H, gw.F32, False)
            wb = ctx.buffer(wdev)
            srcs.append(dict(router_weight=wb.ptr, router_weight_dtype=gw.F32))
            keep.append(wb)
        else:
            lb = ctx.buffer(r.standard_normal(n_experts).astype(np.float32))
            srcs.append(dict(logits=lb.ptr))
            keep.append(lb)
    res = {}
    for mode in ("1", "0"):
        monkeypatch.setenv("GODWIT_DECODE_LAYER", mode)
        runner = gw.ExpertRunner(ctx, H, F, shape["act"])
        outs = [ctx.empty(H * 4) for _ in pattern]
        ids = [ctx.empty(top_k * 4) for _ in pattern]

        def seq():
            for i in range(len(pattern)):
                runner.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xs[i].ptr, gw.BF16,
                                     1, outs[i].ptr, routing_ids=ids[i].ptr, **srcs[i])

        seq()
        ctx.synchronize()
        eager = [(o.download(np.float32, H), d.download(np.int32, top_k)) for o, d in zip(outs, ids)]
        if mode == "1":
            graph = gw.Graph.capture(ctx, seq)
            for _ in range(3):
                for o in outs:
                    o.zero()
                graph.launch()
                ctx.synchronize()
                for i, o in enumerate(outs):
                    assert np.array_equal(o.download(np.float32, H), eager[i][0]), i
            graph.destroy()
            assert runner.sync_errors() == 0
        res[mode] = eager
        for b in outs + ids:
            b.free()
        runner.close()
    for i in range(len(pattern)):
        f_out, f_ids = res["1"][i]
        s_out, s_ids = res["0"][i]
        assert np.array_equal(f_ids, s_ids), (i, pattern[i])
        assert np.max(np.abs(f_out - s_out)) <= 1e-5 * np.max(np.abs(s_out)), (i, pattern[i])
    for b in xs + keep + [buf]:
        b.free()


@pytest.mark.parametrize("router", [False, True], ids=["logits", "router"])
def test_exchange_give_up_is_reported_and_falls_back(ctx, monkeypatch, router):
    """The bounded exchange wait made to give up from the host: the one-token
    layer reads a slot no launch writes (the activations', and with router
    weights the router partials' too), with a 64-poll limit.  Every kernel
    exits, the runner counts the waves that gave up, the next synchronize
    reports GW_ERR_EXCHANGE once, and the runner's later one-token layers run
    as two kernels and match the oracle."""
    from godwit_amd._lib import GW_ERR_EXCHANGE
    shape, n_experts, top_k = QWEN3, 32, 8
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 1500)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(1501)
    xb, xw = _inputs(ctx, r, H, gw.BF16)
    if router:
        wdev, W, _, _ = _router(r, n_experts, H, gw.F32, False)
        lb = ctx.buffer(wdev)
        src = dict(router_weight=lb.ptr, router_weight_dtype=gw.F32)
        logits = oracle.router_logits(W, None, xw, n_experts, H)
    else:
        logits = r.standard_normal(n_experts).astype(np.float32)
        lb = ctx.buffer(logits)
        src = dict(logits=lb.ptr)
    out = ctx.empty(H * 4)
    runner.set_wait_limit(64)
    runner.inject_exchange_fault(True)
    counts = _kernel_counts(ctx, lambda: runner.layer_forward(
        buf.ptr, layout.stride, n_experts, top_k, xb.ptr, gw.BF16, 1, out.ptr, **src))
    assert counts == {"moe_layer": 1, "gate_up": 0, "down": 0}, counts
    with pytest.raises(gw.GodwitError) as err:
        ctx.synchronize()
    assert err.value.status == GW_ERR_EXCHANGE, err.value
    gave_up = runner.sync_errors()
    assert gave_up > 0
    ctx.synchronize()   # reported once
    runner.inject_exchange_fault(False)
    runner.set_wait_limit(0)
    got = {}
    if router:
        def fwd():
            runner.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xb.ptr, gw.BF16, 1,
                                 out.ptr, **src)
            ctx.synchronize()
            got["x"] = (out.download(np.float32, H),)
    else:
        def fwd():
            got["x"] = _forward(ctx, runner, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)
    counts = _kernel_counts(ctx, fwd)
    assert counts == {"moe_layer": 0, "gate_up": 1, "down": 1}, counts
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], top_k, logits[None, :], xw,
                                 H, F, shape["oact"])
    _close(got["x"][0], ref[0])
    assert runner.sync_errors() == gave_up
    for b in (xb, lb, out, buf):
        b.free()
    runner.close()


def test_fused_layer_f32_bias_qwen3(ctx, monkeypatch):
    """fp32 bias sections (set_bias_dtype(GW_F32)) on the one-token layer at
    Qwen3's shape: one launch, the oracle fed the same fp32 biases, the
    two-kernel form to 1e-5 of the peak, and no exchange gave up."""
    from test_gpu_boundary import _f32_bias_layer
    shape, n_experts, top_k = QWEN3, 32, 8
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _f32_bias_layer(ctx, shape, n_experts, 1600)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    fused = gw.ExpertRunner(ctx, H, F, shape["act"], bias_dtype=gw.F32)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "0")
    split = gw.ExpertRunner(ctx, H, F, shape["act"], bias_dtype=gw.F32)
    r = rng(1601)
    xb, xw = _inputs(ctx, r, H, gw.BF16)
    logits = r.standard_normal(n_experts).astype(np.float32)
    lb = ctx.buffer(logits)
    got = {}
    counts = _kernel_counts(ctx, lambda: got.__setitem__(
        "fused", _forward(ctx, fused, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)))
    assert counts == {"moe_layer": 1, "gate_up": 0, "down": 0}, counts
    got["split"] = _forward(ctx, split, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)
    f_out, s_out = got["fused"][0], got["split"][0]
    assert np.max(np.abs(f_out - s_out)) <= 1e-5 * np.max(np.abs(s_out))
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], top_k, logits[None, :], xw,
                                 H, F, shape["oact"])
    _close(f_out, ref[0])
    assert fused.sync_errors() == 0
    for b in (xb, lb, buf):
        b.free()
    fused.close()
    split.close()


@pytest.mark.parametrize("shape,n_experts,top_k", [(GPTOSS, 32, 4), (GPTOSS, 128, 4),
                                                   (GPTOSS, 144, 4), (QWEN3, 128, 8),
                                                   (QWEN3, 60, 8)],
                         ids=["gptoss-32", "gptoss-128", "gptoss-144", "qwen3-128", "qwen3-60"])
@pytest.mark.parametrize("case", ["distinct", "ties_below", "tie_inside", "signed_zero",
                                  "nan_rest", "nan_first", "all_equal"])
def test_fused_layer_routing_exact(ctx, monkeypatch, shape, n_experts, top_k, case):
    """The one-kernel layer's routing equals Router.select (Router.swift:78-98)
    on every selection path: up to 128 experts the rank count over all
    threads (distinct keys, ties below the top k), its hand-over to the exact
    selection sort (a tie inside the top k, -0 against +0, a NaN anywhere, all
    logits equal), and above 128 experts the one-wave selection.  Weights are
    the same bits as the two-kernel form's, and so is the layer's output to
    the two-kernel form's tolerance."""
    from helpers import fill_layer_device
    from test_gpu_expert import _routing_logits
    H, F = shape["hidden"], shape["inter"]
    layout = gw.ExpertLayout(H, F, n_experts)
    buf = ctx.empty(layout.stride * n_experts)
    fill_layer_device(ctx, buf, layout, n_experts, 17 + n_experts, biases=shape["bias"])
    if case == "all_equal":
        logits = np.full((1, n_experts), 0.25, np.float32)
    else:
        logits = _routing_logits(case, 1, n_experts)
    lb = ctx.buffer(logits)
    xb, _ = _inputs(ctx, rng(1400 + n_experts), H, gw.BF16)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    fused = gw.ExpertRunner(ctx, H, F, shape["act"])
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "0")
    split = gw.ExpertRunner(ctx, H, F, shape["act"])
    got = {}
    counts = _kernel_counts(ctx, lambda: got.__setitem__(
        "fused", _forward(ctx, fused, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)))
    assert counts == {"moe_layer": 1, "gate_up": 0, "down": 0}, counts
    got["split"] = _forward(ctx, split, layout, buf, n_experts, top_k, xb, gw.BF16, lb, H)
    f_out, _, f_ids, f_w = got["fused"]
    s_out, _, s_ids, s_w = got["split"]
    rid, rw = oracle.router_select(logits[0], top_k)
    assert list(f_ids) == list(rid), (case, list(f_ids), list(rid))
    assert np.allclose(f_w, rw, rtol=1e-6, atol=1e-7, equal_nan=True), (case, f_w, rw)
    assert np.array_equal(f_ids, s_ids)
    assert np.array_equal(f_w.view(np.uint32), s_w.view(np.uint32))
    if np.all(np.isfinite(s_out)):
        assert np.max(np.abs(f_out - s_out)) <= 1e-5 * np.max(np.abs(s_out))
    else:
        assert np.array_equal(np.isnan(f_out), np.isnan(s_out))
    assert fused.sync_errors() == 0
    for b in (xb, lb, buf):
        b.free()
    fused.close()
    split.close()


def test_fused_layer_cooperative_launch(monkeypatch):
    """GODWIT_DECODE_COOP=1 at context creation launches the one-token layer
    through hipLaunchCooperativeKernel (the runtime then refuses a grid that
    cannot be resident at once).  Eager and graph-replayed layers equal the
    ordinary launch's bit for bit."""
    shape, n_experts, top_k = GPTOSS, 32, 4
    H, F = shape["hidden"], shape["inter"]
    outs = {}
    for coop in ("0", "1"):
        monkeypatch.setenv("GODWIT_DECODE_COOP", coop)
        monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
        c = gw.Context(0)
        layout, experts, buf = _make_layer(c, shape, n_experts, 1800)
        runner = gw.ExpertRunner(c, H, F, shape["act"])
        r = rng(1801)
        xb, _ = _inputs(c, r, H, gw.BF16)
        lb = c.buffer(r.standard_normal(n_experts).astype(np.float32))
        out = c.empty(H * 4)

        def one():
            runner.layer_forward(buf.ptr, layout.stride, n_experts, top_k, xb.ptr, gw.BF16, 1,
                                 out.ptr, logits=lb.ptr)

        one()
        c.synchronize()
        eager = out.download(np.float32, H)
        graph = gw.Graph.capture(c, one)
        out.zero()
        for _ in range(3):
            graph.launch()
        c.synchronize()
        assert np.array_equal(out.download(np.float32, H), eager)
        assert runner.sync_errors() == 0
        outs[coop] = eager
        graph.destroy()
        for b in (xb, lb, out, buf):
            b.free()
        runner.close()
        c.close()
    assert np.array_equal(outs["0"], outs["1"])
