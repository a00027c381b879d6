"""The one-token layer kernel (route -> gate_up + down stream into LDS ->
in-kernel activation exchange -> down + combine, one launch) against the
two-kernel form of the same layer (GODWIT_DECODE_LAYER=0) and against the CPU
oracle.

Both forms compute the gate_up rows with the same lane mapping and order, so
their activations are the same bytes.  The one-kernel form splits a GPT-OSS
down row over 32 lanes (3 blocks each) where the two-kernel form uses 16 (6
each), so the fp32 row sums may round differently: the forms are required to
agree to 1e-5 of the output's peak there, and bit for bit for Qwen3 (same down
lane mapping in both).  Routing is exact in both.  The oracle check uses the
reference's expert metric, max|d|/mean|ref| < 1e-3 (GodwitCLI/main.swift:518-532).
Every test also requires the kernel's bounded waits to have all succeeded.  The
one-kernel form takes 16-bit x; fp32 x stays on the two kernels.
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


def _kernel_counts(ctx, fn):
    ctx.set_profiling(True)
    ctx.profile_reset()
    fn()
    counts = {k: ctx.profile(k)[1] for k in ("moe_layer", "gate_up", "down")}
    ctx.set_profiling(False)
    return counts


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


def test_fused_layer_graph_chain_replays(ctx, monkeypatch):
    """A captured chain of 12 one-token layers (each layer's bf16 output is the next
    one's input), replayed 6 times: every replay equals the eager chain, the first
    layer matches the oracle, and no exchange ever gave up.  The replays advance the
    kernel's launch epochs well past their first values."""
    shape = GPTOSS
    H, F, n_experts, layers = shape["hidden"], shape["inter"], 16, 12
    layout, experts, buf = _make_layer(ctx, shape, n_experts, 1400)
    monkeypatch.setenv("GODWIT_DECODE_LAYER", "1")
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(1401)
    xbits, xw = normal_bf16(r, H)
    logits = r.standard_normal((layers, n_experts)).astype(np.float32)
    lb = ctx.buffer(logits)
    xs = [ctx.buffer(xbits)] + [ctx.empty(H * 2) for _ in range(layers)]
    outs = [ctx.empty(H * 4) for _ in range(layers)]

    def chain():
        for l in range(layers):
            runner.layer_forward(buf.ptr, layout.stride, n_experts, 4, xs[l].ptr, gw.BF16, 1,
                                 outs[l].ptr, logits=lb.address(l * n_experts * 4),
                                 out_bf16=xs[l + 1].ptr)

    counts = _kernel_counts(ctx, chain)
    assert counts["moe_layer"] == layers, counts
    first = outs[0].download(np.float32, H)
    eager = outs[-1].download(np.float32, H)
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], 4, logits[:1], xw, H, F,
                                 shape["oact"])
    _close(first, ref[0])
    graph = gw.Graph.capture(ctx, chain)
    for _ in range(6):
        outs[-1].zero()
        graph.launch()
        ctx.synchronize()
        assert np.array_equal(outs[-1].download(np.float32, H), eager)
    assert runner.sync_errors() == 0
    graph.destroy()
    for b in xs + outs + [lb, buf]:
        b.free()
    runner.close()


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
