"""A .gwt installation loaded into HBM: the bytes on the device are the file's
bytes, whole layers and single experts, and a layer loaded this way runs the
MoE block against the oracle exactly as a layer filled in memory does."""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from gwt_install import write_install
from helpers import ExpertData, rng
from test_gpu_expert import GPTOSS, _close

pytestmark = pytest.mark.gpu


def test_load_layer_and_expert_bytes(ctx, tmp_path):
    layout = gw.ExpertLayout(2880, 2880, 6)
    r = rng(3100)
    blobs = [r.integers(0, 256, layout.stride * 6, dtype=np.uint8) for _ in range(2)]
    write_install(str(tmp_path), layout, blobs)
    m = gw.ModelReader(str(tmp_path))
    m.validate()
    for layer in (1, 0):
        buf = m.load_layer(ctx, layer)
        assert np.array_equal(buf.download(np.uint8, m.layer_file_size), blobs[layer])
        buf.free()
    one = m.load_expert(ctx, 1, 4)
    assert np.array_equal(one.download(np.uint8, m.expert_stride),
                          blobs[1][4 * layout.stride:5 * layout.stride])
    one.free()
    with pytest.raises(gw.GodwitError, match="layer 2 out of range"):
        m.load_layer(ctx, 2)
    m.close()


def test_loaded_layer_runs_the_moe_block(ctx, tmp_path):
    shape, E, K = GPTOSS, 8, 4
    H, F = shape["hidden"], shape["inter"]
    layout = gw.ExpertLayout(H, F, E)
    r = rng(3200)
    experts = [ExpertData(r, H, F, layout.offsets, layout.stride) for _ in range(E)]
    write_install(str(tmp_path), layout, [np.concatenate([e.blob for e in experts])], top_k=K)
    m = gw.ModelReader(str(tmp_path))
    runner = gw.ExpertRunner(ctx, m.hidden_size, m.intermediate_size, m.activation,
                             m.activation_limit, m.activation_alpha)
    buf = m.load_layer(ctx, 0)
    xbits = oracle.f32_to_bf16_bits(r.standard_normal(H).astype(np.float32))
    xw = oracle.bf16_bits_to_f32(xbits)
    logits = r.standard_normal(E).astype(np.float32)
    xb, lb, out = ctx.buffer(xbits), ctx.buffer(logits), ctx.empty(H * 4)
    runner.layer_forward(buf.ptr, m.expert_stride, m.expert_count, m.experts_per_token, xb.ptr,
                         gw.BF16, 1, out.ptr, logits=lb.ptr)
    ctx.synchronize()
    ref, _, _ = oracle.moe_layer([e.oracle_expert() for e in experts], K, logits[None, :], xw,
                                 H, F, shape["oact"])
    _close(out.download(np.float32, H), ref[0])
    for b in (buf, xb, lb, out):
        b.free()
    runner.close()
    m.close()
