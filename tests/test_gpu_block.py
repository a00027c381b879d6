"""The MoE block with its surroundings (TransformerLayer.swift:140-143, 232-238):
stream += MoE(RMSNorm(stream)), on the device, against the CPU oracle's
composition: oracle.rmsnorm_f16 (TransformerLayer.normalise, :265-285), the
oracle layer on those fp16 rows, then the fp32 residual add.

Tolerance: the expert metric max|d|/mean|moe| < 1e-3 (GodwitCLI/main.swift:
518-532) on the change the block makes to the stream (prefill: every token
below 1e-3, the median below 1e-4, as in the prefill tests); routing ids
exact.  The GPU's
sum of squares is a tree, so a normalised value can differ from the oracle's by
one fp16 ulp, well inside that bound.
"""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from helpers import expert_metric, rng
from test_gpu_expert import GPTOSS, QWEN3, SMALL, _make_layer

pytestmark = pytest.mark.gpu


def _norm_weight(r, H):
    return oracle.f32_to_bf16_bits((1.0 + 0.1 * r.standard_normal(H)).astype(np.float32))


def _oracle_block(experts, shape, K, logits, stream, wbits, eps):
    H, F = shape["hidden"], shape["inter"]
    normed = oracle.rmsnorm_f16(stream, wbits, eps)
    xs = normed.view(np.float16).astype(np.float32)
    moe, ids, _ = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits,
                                   xs.ravel(), H, F, shape["oact"])
    return oracle.residual_add(stream, moe), moe, ids, xs


def _run(ctx, runner, layout, buf, E, K, T, stream, wbits, eps, logits=None, router=None):
    H = stream.shape[1]
    sb, wb = ctx.buffer(stream.astype(np.float32)), ctx.buffer(wbits)
    ids = ctx.empty(T * K * 4)
    extra = {}
    lb = None
    if logits is not None:
        lb = ctx.buffer(logits.astype(np.float32))
        extra["logits"] = lb.ptr
    else:
        extra.update(router_weight=router.ptr, router_weight_dtype=gw.F32)
    runner.block_forward(buf.ptr, layout.stride, E, K, T, sb.ptr, wb.ptr, eps,
                         routing_ids=ids.ptr, **extra)
    ctx.synchronize()
    got = sb.download(np.float32, T * H).reshape(T, H)
    gid = ids.download(np.int32, T * K).reshape(T, K)
    for b in (sb, wb, ids) + ((lb,) if lb is not None else ()):
        b.free()
    return got, gid


@pytest.mark.parametrize("shape,E,K,T,eps", [(GPTOSS, 32, 4, 1, 1e-5), (QWEN3, 64, 8, 4, 1e-6)],
                         ids=["gptoss-1", "qwen3-4"])
def test_block_decode_matches_oracle(ctx, shape, E, K, T, eps):
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2600 + T)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2610 + T)
    stream = (r.standard_normal((T, H)) * 2.0).astype(np.float32)
    wbits = _norm_weight(r, H)
    logits = r.standard_normal((T, E)).astype(np.float32)
    got, gid = _run(ctx, runner, layout, buf, E, K, T, stream, wbits, eps, logits=logits)
    ref, moe, rid, _ = _oracle_block(experts, shape, K, logits, stream, wbits, eps)
    assert np.array_equal(gid, rid.reshape(T, K))
    for t in range(T):
        assert expert_metric(got[t] - stream[t], moe[t]) < 1e-3
        assert expert_metric(got[t], ref[t]) < 1e-3
    for b in (buf,):
        b.free()
    runner.close()


def test_block_router_sees_normalised_rows(ctx):
    """Without logits the router GEMV runs on RMSNorm(stream), not on the raw stream."""
    shape, E, K, T, eps = GPTOSS, 16, 4, 2, 1e-5
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2700)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2701)
    stream = (r.standard_normal((T, H)) * 3.0 + 0.5).astype(np.float32)
    wbits = _norm_weight(r, H)
    W = (r.standard_normal(E * H) * 0.02).astype(np.float32)
    wrt = ctx.buffer(W)
    got, gid = _run(ctx, runner, layout, buf, E, K, T, stream, wbits, eps, router=wrt)
    normed = oracle.rmsnorm_f16(stream, wbits, eps).view(np.float16).astype(np.float32)
    logits = np.stack([oracle.router_logits(W, None, normed[t], E, H) for t in range(T)])
    ref, moe, rid, _ = _oracle_block(experts, shape, K, logits, stream, wbits, eps)
    assert np.array_equal(gid, rid.reshape(T, K))
    for t in range(T):
        assert expert_metric(got[t] - stream[t], moe[t]) < 1e-3
    wrt.free()
    buf.free()
    runner.close()


@pytest.mark.parametrize("T", [40, 24], ids=["t40-combine-kernel", "t24-fused-combine"])
def test_block_prefill_matches_oracle(ctx, T):
    """More than 8 tokens: RMSNorm rows into the prefill scratch, grouped GEMMs, and
    the residual add folded into the combine — the combine kernel at 40 tokens, the
    down GEMM's own combine at 24 (tile list, up to 32 tokens)."""
    shape, E, K, eps = SMALL, 16, 4, 1e-5
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2800)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2801)
    stream = r.standard_normal((T, H)).astype(np.float32)
    wbits = _norm_weight(r, H)
    logits = r.standard_normal((T, E)).astype(np.float32)
    got, gid = _run(ctx, runner, layout, buf, E, K, T, stream, wbits, eps, logits=logits)
    ref, moe, rid, _ = _oracle_block(experts, shape, K, logits, stream, wbits, eps)
    assert np.array_equal(gid, rid.reshape(T, K))
    m = np.array([expert_metric(got[t] - stream[t], moe[t]) for t in range(T)])
    assert m.max() < 1e-3 and np.median(m) < 1e-4, (m.max(), np.median(m))
    buf.free()
    runner.close()


def test_block_graph_replay(ctx):
    """A captured block updates the stream in place on every replay: replaying it n
    times equals n eager calls."""
    shape, E, K, eps = GPTOSS, 16, 4, 1e-5
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 2900)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(2901)
    stream0 = r.standard_normal((1, H)).astype(np.float32)
    wbits = _norm_weight(r, H)
    logits = r.standard_normal((1, E)).astype(np.float32)
    sb, wb, lb = ctx.buffer(stream0), ctx.buffer(wbits), ctx.buffer(logits)

    def body():
        runner.block_forward(buf.ptr, layout.stride, E, K, 1, sb.ptr, wb.ptr, eps, logits=lb.ptr)

    for _ in range(3):
        body()
    ctx.synchronize()
    eager = sb.download(np.float32, H)
    sb.upload(stream0)
    ctx.synchronize()
    graph = gw.Graph.capture(ctx, body)
    for _ in range(3):
        graph.launch()
    ctx.synchronize()
    assert np.array_equal(sb.download(np.float32, H), eager)
    graph.destroy()
    for b in (sb, wb, lb, buf):
        b.free()
    runner.close()
