"""Edges of the C ABI: fp32 bias sections (ExpertRunner's bias dtype) through
every path against the oracle, the layouts where fp32 biases cannot fit,
out-of-memory reporting, and the calls that graph capture refuses or
records."""
import ctypes

import numpy as np
import pytest

import godwit_amd as gw
import oracle
from godwit_amd._lib import GW_ERR_ARG, GW_ERR_OOM, GW_ERR_SHAPE, check, lib
from helpers import ExpertData, expert_metric, normal_bf16, rng
from test_gpu_expert import GPTOSS, SMALL
from test_gpu_prefill import _close_batch

pytestmark = pytest.mark.gpu


def _f32_bias_layer(ctx, shape, E, seed):
    """Experts whose bias sections hold fp32 values (not bf16-representable)."""
    H, F = shape["hidden"], shape["inter"]
    layout = gw.ExpertLayout(H, F, E)
    r = rng(seed)
    experts = []
    for _ in range(E):
        e = ExpertData(r, H, F, layout.offsets, layout.stride, with_bias=False)
        e.gu_bias = (r.standard_normal(2 * F) * 0.02).astype(np.float32)
        e.dn_bias = (r.standard_normal(H) * 0.02).astype(np.float32)
        for name, arr in (("gate_up_bias", e.gu_bias), ("down_bias", e.dn_bias)):
            off = layout.offsets[name]
            e.blob[off:off + arr.nbytes] = arr.view(np.uint8)
        experts.append(e)
    return layout, experts, ctx.buffer(np.concatenate([e.blob for e in experts]))


WIDE = dict(hidden=2880, inter=1024, act="gptOssClampedGLU", oact=oracle.ACT_GPTOSS, bias=True)


@pytest.mark.parametrize("shape", [SMALL, WIDE], ids=["small", "h2880-f1024"])
def test_f32_bias_through_every_path(ctx, shape):
    """set_bias_dtype(GW_F32): apply (ExpertRunner.apply), the one-token layer, a
    4-token decode batch and a 40-token grouped prefill all read fp32 biases and
    match the oracle fed the same fp32 values; also at GPT-OSS's 2880 width with
    an intermediate size whose fp32 gate_up bias still fits its page."""
    E, K = 8, 2
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _f32_bias_layer(ctx, shape, E, 5100)
    runner = gw.ExpertRunner(ctx, H, F, shape["act"], bias_dtype=gw.F32)
    oexp = [e.oracle_expert() for e in experts]
    r = rng(5101)
    x1, x1w = normal_bf16(r, H)
    got = runner.apply(x1, gw.Weights(buf, runner.section_offsets), dtype=gw.BF16)
    ref = oracle.expert_apply(oexp[0], x1w, H, F, shape["oact"])
    assert expert_metric(got, ref) < 1e-3
    for T in (1, 4, 40):
        xbits, xw = normal_bf16(r, T * H)
        logits = r.standard_normal((T, E)).astype(np.float32)
        xb, lb = ctx.buffer(xbits), ctx.buffer(logits)
        out = ctx.empty(T * H * 4)
        fn = runner.prefill_forward if T == 40 else runner.layer_forward
        fn(buf.ptr, layout.stride, E, K, xb.ptr, gw.BF16, T, out.ptr, logits=lb.ptr)
        ctx.synchronize()
        got = out.download(np.float32, T * H).reshape(T, H)
        ref, _, _ = oracle.moe_layer(oexp, K, logits, xw, H, F, shape["oact"])
        _close_batch(got, ref)
        for b in (xb, lb, out):
            b.free()
    buf.free()
    runner.close()


def test_f32_bias_refused_where_it_overflows(ctx):
    """GPT-OSS's gate_up bias section holds 5760 bf16 values in its 16 KiB page;
    5760 fp32 values (23,040 B) would run into the down bias, so the runner
    refuses the dtype rather than read the neighbouring section."""
    with pytest.raises(gw.GodwitError) as err:
        gw.ExpertRunner(ctx, GPTOSS["hidden"], GPTOSS["inter"], GPTOSS["act"], bias_dtype=gw.F32)
    assert err.value.status == GW_ERR_SHAPE and "overflow" in str(err.value)


def test_out_of_memory_is_reported_and_cleared(ctx):
    """An allocation beyond the device returns GW_ERR_OOM (gw_malloc, and the
    prefill scratch of an oversized batch), and the next launch still works."""
    with pytest.raises(gw.GodwitError) as err:
        ctx.empty(1 << 50)
    assert err.value.status == GW_ERR_OOM
    runner = gw.ExpertRunner(ctx, SMALL["hidden"], SMALL["inter"], SMALL["act"])
    with pytest.raises(gw.GodwitError) as err:
        runner.reserve_prefill(1 << 26, 8, 256)   # about 1.1 TB of scratch
    assert err.value.status == GW_ERR_OOM
    runner.close()
    b = ctx.empty(4096)
    ctx.fill_uniform_u8(b, 7, 7, 1)
    ctx.synchronize()
    assert (b.download(np.uint8) == 7).all()
    b.free()


def test_capture_guards(ctx):
    """gw_memset_zero refuses a capture (a memset node would be recorded); the
    zero-column GEMV records a fill kernel instead, and its replays write
    zeros."""
    b = ctx.empty(1024)
    with pytest.raises(gw.GodwitError) as err:
        gw.Graph.capture(ctx, lambda: check(lib.gw_memset_zero(ctx.handle, b.ptr, 1024)))
    assert err.value.status == GW_ERR_ARG and "capture" in str(err.value)
    rows = 300
    y = ctx.buffer(np.full(rows, 5.0, np.float32))
    p, s, x = ctx.empty(16), ctx.empty(16), ctx.empty(16)
    graph = gw.Graph.capture(ctx, lambda: gw.mxfp4_gemv(ctx, p, s, x, gw.F32, y, rows, 0))
    for _ in range(3):
        y.upload(np.full(rows, 5.0, np.float32))
        graph.launch()
        ctx.synchronize()
        assert (y.download(np.float32, rows) == 0).all()
    graph.destroy()
    for buf in (b, y, p, s, x):
        buf.free()
