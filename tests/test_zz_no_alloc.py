"""gw_moe_prefill_forward_static: the prefill with its scratch in the library's
fixed per-device array (resolved once per device at context creation) instead
of the runner's reserved buffer.  It runs the same kernels in the same order,
so its results equal gw_moe_prefill_forward's byte for byte: output, bf16
output, routing ids and weights.  Two calls in a row (the second smaller, so
the array holds the first call's bytes where the second carves its combine
counters), then the first size again; a batch too large for the array is
refused with GW_ERR_SHAPE.  The routed output also meets the oracle."""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from helpers import expert_metric, rng
from test_gpu_expert import GPTOSS, _make_layer
from test_gpu_prefill import _run, _x, _zipf_logits

pytestmark = pytest.mark.gpu


def test_static_scratch_prefill_equals_reserved(ctx):
    shape, E, K = GPTOSS, 16, 4
    H, F = shape["hidden"], shape["inter"]
    layout, experts, buf = _make_layer(ctx, shape, E, 4100)
    static = gw.ExpertRunner(ctx, H, F, shape["act"])
    reserved = gw.ExpertRunner(ctx, H, F, shape["act"])
    r = rng(4101)
    for T in (48, 12, 48):      # tile list + combine kernel; self-grouped + fused combine
        xb, xw = _x(ctx, r, T, H, gw.BF16)
        logits = _zipf_logits(r, T, E, K)
        lb = ctx.buffer(logits)
        got = _run(ctx, static, layout, buf, E, K, xb, gw.BF16, lb, T, H,
                   "prefill_forward_static")
        want = _run(ctx, reserved, layout, buf, E, K, xb, gw.BF16, lb, T, H, "prefill_forward")
        for i in range(4):
            assert np.array_equal(got[i], want[i]), (T, i)
        ref, rids, _ = oracle.moe_layer([e.oracle_expert() for e in experts[:E]], K, logits,
                                        xw, H, F, shape["oact"])
        assert np.array_equal(got[2], rids)
        m = max(expert_metric(got[0][t], ref[t]) for t in range(T))
        assert m < 1e-3, (T, m)
        for b in (xb, lb):
            b.free()
    # 2880 x 2880, top-4: about 116 KiB of scratch per token, so 256 tokens cannot fit
    T = 256
    xb = ctx.empty(T * H * 2)
    lb = ctx.buffer(np.zeros((T, E), np.float32))
    out = ctx.empty(T * H * 4)
    with pytest.raises(gw.GodwitError) as err:
        static.prefill_forward_static(buf.ptr, layout.stride, E, K, xb.ptr, gw.BF16, T, out.ptr,
                                      logits=lb.ptr)
    assert err.value.status == 2 and "static array" in str(err.value)
    for b in (xb, lb, out, buf):
        b.free()
    static.close()
    reserved.close()
