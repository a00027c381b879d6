"""Benchmark config 4 at its own workload: one GPT-OSS-120B MoE layer (hidden =
intermediate = 2880, 128 experts, bf16 biases) and a 512-token batch with
Zipf(1.1)-popular top-4 routing and bf16 x, through gw_moe_layer_forward with
the launcher's default shapes (TransformerLayer.swift:175-230: route every
token, run each selected expert, combine in router order).

Checks: routing ids equal the oracle's Router.select for all 512 tokens; a
seeded sample of 32 tokens equals oracle.moe_layer at the expert metric
(GodwitCLI/main.swift:518-532) < 1e-3; and, for those tokens' 128 (token,
rank) entries, the layer taken apart stage by stage from the runner's prefill
scratch:
  * the fp16 activation (the scratch holds its bits) is within one fp16 ulp of the
    oracle's activation of the oracle's gate_up sums (expert.metal:92-101), or,
    where gate or up is near a point the activation magnifies, between the
    activations of gate and up moved by the fp32 summation bound;
  * the down projection + bias of the GPU's own activation is within the fp32
    summation bound (2^-16 of the sum of |terms|, which the oracle's own
    sequential GEMV meets too) of an fp64 evaluation, and its GEMV metric
    against the oracle (DequantGEMVBenchmark.swift:338-349) is reported;
  * the combine reproduces, bit for bit, the weighted sum of those outputs in
    router order with product and sum rounded separately (expert.metal:107-116).
Weights are filled on the device and only the sampled tokens' experts are
read back for the oracle."""
import ctypes

import numpy as np
import pytest

import godwit_amd as gw
import oracle
from godwit_amd._lib import check, lib
from helpers import expert_from_blob, expert_metric, fill_layer_device, gemv_metric, normal_bf16, rng
from test_gpu_prefill import _zipf_logits

pytestmark = pytest.mark.gpu

H = F = 2880
E, K, T = 128, 4, 512


def _download(ctx, addr, dtype, count):
    out = np.empty(count, dtype)
    check(lib.gw_memcpy_dtoh(ctx.handle, out.ctypes.data, addr, out.nbytes))
    return out


def _f16_ordered(bits):
    """fp16 bit patterns -> integers ordered like the values (ulp distance)."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def test_config4_layer_forward_512_tokens(ctx):
    layout = gw.ExpertLayout(H, F, E)
    buf = ctx.empty(layout.layer_file_size)
    fill_layer_device(ctx, buf, layout, E, 4400)
    r = rng(4401)
    logits = _zipf_logits(r, T, E, K)
    xbits, xw = normal_bf16(r, T * H)
    xb, lb = ctx.buffer(xbits), ctx.buffer(logits)
    out, out16 = ctx.empty(T * H * 4), ctx.empty(T * H * 2)
    ids_b, w_b = ctx.empty(T * K * 4), ctx.empty(T * K * 4)
    runner = gw.ExpertRunner(ctx, H, F, "gptOssClampedGLU", 7.0, 1.702)
    runner.layer_forward(buf.ptr, layout.stride, E, K, xb.ptr, gw.BF16, T, out.ptr,
                         logits=lb.ptr, out_bf16=out16.ptr, routing_ids=ids_b.ptr,
                         routing_weights=w_b.ptr)
    ctx.synchronize()
    got = out.download(np.float32, T * H).reshape(T, H)
    ids = ids_b.download(np.int32, T * K).reshape(T, K)
    wts = w_b.download(np.float32, T * K).reshape(T, K)
    assert np.array_equal(out16.download(np.uint16, T * H), oracle.f32_to_bf16_bits(got.ravel()))

    # Routing: every token, exactly.
    for t in range(T):
        rid, rw = oracle.router_select(logits[t], K)
        assert np.array_equal(ids[t], rid), t
        assert np.allclose(wts[t], rw, rtol=1e-6, atol=1e-7), t

    view = runner.prefill_view()
    assert view["tokens"] == T and view["top_k"] == K
    N = T * K
    assert view["activation_plane"] == 0          # one fp16 plane
    act = _download(ctx, view["activations"], np.uint16, N * F).reshape(N, F)
    y = _download(ctx, view["expert_outputs"], np.float32, N * H).reshape(N, H)
    assert np.array_equal(_download(ctx, view["routing_ids"], np.int32, N).reshape(T, K), ids)

    sample = np.sort(rng(4402).choice(T, 32, replace=False))
    needed = sorted(set(ids[sample].ravel().tolist()))
    experts = {e: expert_from_blob(buf.download(np.uint8, layout.stride, e * layout.stride),
                                   layout) for e in needed}
    slots = [experts.get(e, experts[needed[0]]) for e in range(E)]   # only routed slots are read
    oracle.set_threads(16)
    try:
        ref, rids, _ = oracle.moe_layer(slots, K, logits[sample], xw.reshape(T, H)[sample], H, F,
                                        oracle.ACT_GPTOSS)
        assert np.array_equal(rids, ids[sample])
        m = [expert_metric(got[t], ref[i]) for i, t in enumerate(sample)]
        assert max(m) < 1e-3, (max(m), sample[int(np.argmax(m))])

        flips, explained, worst_down, worst_gpu, worst_ora = 0, 0, 0.0, 0.0, 0.0
        for t in sample:
            x_t = xw[t * H:(t + 1) * H]
            comb = np.zeros(H, np.float32)
            for k in range(K):
                j = t * K + k
                ex = experts[int(ids[t, k])]
                gu = oracle.gemv_bias(*ex.arrays[:2], ex.arrays[4], x_t, 2 * F, H)
                want16 = oracle.activation(oracle.ACT_GPTOSS, gu).view(np.uint16)
                got16 = act[j].copy()
                act32 = got16.view(np.float16).astype(np.float32)
                d = np.abs(_f16_ordered(got16) - _f16_ordered(want16))
                flips += int((d == 1).sum())
                far = np.nonzero(d > 1)[0]
                if far.size:
                    # Off by more than one ulp only where the fp32 summation error
                    # of gate or up (at most 2^-16 of the sum of |terms| for the
                    # ~360 roundings of the K loop) moves the activation that far:
                    # the GPU value lies between the fp16 activations of the
                    # corners (gate +- delta, up +- delta).
                    w = np.abs(oracle.decode(*ex.arrays[:2], 2 * F * H // 32).reshape(2 * F, H))
                    delta = (w @ np.abs(x_t) + np.abs(ex.arrays[4])) * 2.0 ** -16
                    g, u, dg, du = gu[2 * far], gu[2 * far + 1], delta[2 * far], delta[2 * far + 1]
                    corners = []
                    for sg in (-1, 1):
                        for su in (-1, 1):
                            pair = np.stack([g + sg * dg, u + su * du], 1).ravel()
                            corners.append(oracle.activation(oracle.ACT_GPTOSS, pair)
                                           .astype(np.float32))
                    lo, hi = np.min(corners, 0), np.max(corners, 0)
                    v = act32[far]
                    assert ((v >= lo) & (v <= hi)).all(), (t, k, far[(v < lo) | (v > hi)])
                    explained += far.size
                # Down on the GPU's own activation: against the oracle's GEMV
                # (reported) and against an fp64 evaluation, within the fp32
                # summation bound 2^-16 * sum |terms| that the oracle's own
                # sequential loop meets too.
                yref = oracle.gemv_bias(*ex.arrays[2:4], ex.arrays[5], act32, H, F)
                gm = gemv_metric(y[j], yref)
                worst_down = max(worst_down, gm)
                wd = oracle.decode(*ex.arrays[2:4], H * F // 32).reshape(H, F).astype(np.float64)
                y64 = wd @ act32.astype(np.float64) + ex.arrays[5]
                bound = (np.abs(wd) @ np.abs(act32.astype(np.float64))) * 2.0 ** -16 + 1e-30
                e_gpu = np.abs(y[j] - y64) / bound
                e_ora = np.abs(yref - y64) / bound
                worst_gpu, worst_ora = max(worst_gpu, e_gpu.max()), max(worst_ora, e_ora.max())
                assert e_gpu.max() <= 1.0, (t, k, e_gpu.max())
                comb = comb + np.float32(wts[t, k]) * y[j]
            assert np.array_equal(comb, got[t]), t
        print(f"config 4: 32 tokens, worst expert metric {max(m):.2e}, "
              f"{flips} of {32 * K * F} activations one fp16 ulp from the oracle's, "
              f"{explained} further within the gate_up summation bound, "
              f"down: GEMV metric against the oracle {worst_down:.2e}, error / fp32 summation "
              f"bound {worst_gpu:.3f} (the oracle's own: {worst_ora:.3f})")
    finally:
        oracle.set_threads(1)
    for b in (xb, lb, out, out16, ids_b, w_b, buf):
        b.free()
    runner.close()
