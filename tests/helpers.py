"""Seeded synthetic inputs and error metrics shared by the tests.

Inputs follow the distributions of the benchmark configurations: e2m1 nibbles
uniform over 0..15 (bytes uniform), e8m0 scales uniform over 119..127, fp32
biases N(0, 0.02) rounded to bf16-representable values (the .gwt layout
stores bf16 biases), activations N(0, 1).
"""
import numpy as np

import oracle


def rng(seed):
    return np.random.default_rng(seed)


def mxfp4_matrix(r, rows, cols, scale_lo=119, scale_hi=127):
    packed = r.integers(0, 256, size=rows * cols // 2, dtype=np.uint8)
    scales = r.integers(scale_lo, scale_hi + 1, size=rows * cols // 32, dtype=np.uint8)
    return packed, scales


def bias_bf16(r, n, std=0.02):
    """Returns (bf16 bits, the same values as fp32)."""
    bits = oracle.f32_to_bf16_bits((r.standard_normal(n) * std).astype(np.float32))
    return bits, oracle.bf16_bits_to_f32(bits)


def normal_bf16(r, n):
    bits = oracle.f32_to_bf16_bits(r.standard_normal(n).astype(np.float32))
    return bits, oracle.bf16_bits_to_f32(bits)


def gemv_metric(got, ref):
    """DequantGEMVBenchmark.compareToReference (DequantGEMVBenchmark.swift:338-349):
    max |got - ref| / max(|ref|, 1)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), 1.0)))


def expert_metric(got, ref):
    """runExpertCheck (GodwitCLI/main.swift:518-532): max |got - ref| / mean |ref|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(got - ref)) / max(np.mean(np.abs(ref)), 1e-30))


def layer_check(got, ref):
    """runLayerCheck's acceptance (GodwitCLI/main.swift:697-718), applied to a
    layer's output: relative RMS error < 2e-3 and every |error| below
    4 * max|ref| * 2^-11 (four fp16 ulps at the output's peak).  Returns
    (relative_rms, worst_abs, bound_abs, passed)."""
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    rms = max(float(np.sqrt(np.mean(ref * ref))), 1e-6)
    err = np.abs(got - ref)
    rel_rms = float(np.sqrt(np.mean(err * err))) / rms
    worst = float(np.max(err))
    bound = 4.0 * float(np.max(np.abs(ref))) * 2.0 ** -11
    return rel_rms, worst, bound, rel_rms < 2e-3 and worst < bound


class ExpertData:
    """One expert's sections as host arrays, plus its bytes in the .gwt stride layout."""

    def __init__(self, r, hidden, inter, layout_offsets, stride, with_bias=True):
        self.gu_packed, self.gu_scales = mxfp4_matrix(r, 2 * inter, hidden)
        self.dn_packed, self.dn_scales = mxfp4_matrix(r, hidden, inter)
        if with_bias:
            self.gu_bias_bits, self.gu_bias = bias_bf16(r, 2 * inter)
            self.dn_bias_bits, self.dn_bias = bias_bf16(r, hidden)
        else:
            self.gu_bias_bits = np.zeros(2 * inter, np.uint16)
            self.dn_bias_bits = np.zeros(hidden, np.uint16)
            self.gu_bias = np.zeros(2 * inter, np.float32)
            self.dn_bias = np.zeros(hidden, np.float32)
        blob = np.zeros(stride, np.uint8)
        for name, arr in (("gate_up_blocks", self.gu_packed), ("gate_up_scales", self.gu_scales),
                          ("down_blocks", self.dn_packed), ("down_scales", self.dn_scales),
                          ("gate_up_bias", self.gu_bias_bits.view(np.uint8)),
                          ("down_bias", self.dn_bias_bits.view(np.uint8))):
            off = layout_offsets[name]
            blob[off:off + arr.nbytes] = arr.view(np.uint8)
        self.blob = blob

    def oracle_expert(self):
        return oracle.Expert(self.gu_packed, self.gu_scales, self.dn_packed, self.dn_scales,
                             self.gu_bias, self.dn_bias)


def fill_layer_device(ctx, buf, layout, n_experts, seed, biases=True):
    """A layer file of synthetic experts filled on the device in five launches:
    packed bytes U{0..255}, each scale section U{119..127} over all experts at
    once (rows of the expert stride), biases N(0, 0.02) bf16 or zeros."""
    import godwit_amd as gw
    o, sz = layout.offsets, layout.sizes
    ctx.fill_uniform_u8(buf, 0, 255, seed)
    for sec, k in (("gate_up_scales", 1), ("down_scales", 2)):
        ctx.fill_uniform_u8(buf, 119, 127, seed * 131 + k, offset=o[sec], count=sz[sec],
                            rows=n_experts, row_stride=layout.stride)
    for sec, k in (("gate_up_bias", 3), ("down_bias", 4)):
        if biases:
            ctx.fill_normal(buf, gw.BF16, sz[sec] // 2, 0.0, 0.02, seed * 131 + k, offset=o[sec],
                            rows=n_experts, row_stride=layout.stride)
        else:
            ctx.fill_uniform_u8(buf, 0, 0, 0, offset=o[sec], count=sz[sec], rows=n_experts,
                                row_stride=layout.stride)


def expert_from_blob(blob, layout):
    """oracle.Expert over one expert's bytes in the .gwt stride layout (bf16 biases
    widened to fp32)."""
    o, sz = layout.offsets, layout.sizes
    sec = {k: blob[o[k]:o[k] + sz[k]] for k in o}
    return oracle.Expert(sec["gate_up_blocks"], sec["gate_up_scales"], sec["down_blocks"],
                         sec["down_scales"],
                         oracle.bf16_bits_to_f32(sec["gate_up_bias"].view(np.uint16)),
                         oracle.bf16_bits_to_f32(sec["down_bias"].view(np.uint16)))
