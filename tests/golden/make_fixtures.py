"""Writes the golden fixtures of tests/golden/*.npz from the CPU oracle.

Run from the repository root: `python tests/golden/make_fixtures.py`.  Every
input is generated here from a fixed seed and stored in full next to the
oracle's outputs, so a fixture is plain data (numpy .npz, no pickles) that the
tests load without running this script.  The oracle itself is pinned by known
answers and closed forms (tests/test_oracle.py); these files freeze its outputs
on small cases of each function of the path so the device kernels are checked
against fixed numbers and any later change to the oracle shows up as a diff.

Cases (reference functions they exercise):
  dequant      MXFP4.decode (MXFP4.swift:48-93): every byte under 12 scale bytes
               including 0 (subnormal powers), 127 (x1), 254 and 255 (NaN).
  gemv         DequantGEMVBenchmark.referenceMXFP4 (DequantGEMVBenchmark.swift:100-120)
               on the reference test's xorshift inputs (DequantGEMVTests.swift:20-42).
  expert_*     ExpertRunner.apply (ExpertRunner.swift:275-331): gate_up GEMV + bias,
               GPT-OSS clamped SwiGLU (expert.metal:82-102) or SiLU-GLU
               (expert.metal:380-393), fp16 activation, down GEMV + bias.
  layer_*      TransformerLayer.forward's MoE block (TransformerLayer.swift:158-230):
               Router.select on given logits (Router.swift:78-98), experts,
               router-ordered combine (expert.metal:107-116).
  router       bf16_gemv_bias (router.metal:18-34) + Router.select.
  rmsnorm      rmsnorm (router.metal:36-60), fp16 output.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
from helpers import bias_bf16, mxfp4_matrix, normal_bf16, rng  # noqa: E402

# Small expert shape shared by the expert and layer cases (the grouped GEMMs
# need hidden and intermediate sizes that are multiples of 32 and >= 128).
H, F = 128, 128


def experts_arrays(r, n, with_bias):
    """n experts as the six section arrays, stacked: [n, ...]."""
    cols = {k: [] for k in ("gu_packed", "gu_scales", "dn_packed", "dn_scales",
                            "gu_bias_bits", "dn_bias_bits")}
    for _ in range(n):
        gp, gs = mxfp4_matrix(r, 2 * F, H)
        dp, ds = mxfp4_matrix(r, H, F)
        if with_bias:
            gb, _ = bias_bf16(r, 2 * F)
            db, _ = bias_bf16(r, H)
        else:
            gb, db = np.zeros(2 * F, np.uint16), np.zeros(H, np.uint16)
        for k, v in zip(cols, (gp, gs, dp, ds, gb, db)):
            cols[k].append(v)
    return {k: np.stack(v) for k, v in cols.items()}


def oracle_experts(ex):
    return [oracle.Expert(ex["gu_packed"][i], ex["gu_scales"][i], ex["dn_packed"][i],
                          ex["dn_scales"][i], oracle.bf16_bits_to_f32(ex["gu_bias_bits"][i]),
                          oracle.bf16_bits_to_f32(ex["dn_bias_bits"][i]))
            for i in range(ex["gu_packed"].shape[0])]


def make_dequant():
    scale_bytes = np.array([0, 1, 100, 119, 120, 126, 127, 128, 140, 200, 254, 255], np.uint8)
    blocks = len(scale_bytes) * 16
    packed = np.tile(np.arange(256, dtype=np.uint8), len(scale_bytes))
    scales = np.repeat(scale_bytes, 16)
    return dict(packed=packed, scales=scales,
                expected=oracle.decode(packed, scales, blocks).astype(np.float32))


def make_gemv():
    rows, cols = 64, 256
    packed = oracle.xorshift_bytes(0xA5A5, rows * cols // 2)
    scales = (120 + np.arange(rows * cols // 32) % 14).astype(np.uint8)
    x16 = oracle.xorshift_activations_f16(0x1234, cols)
    r = rng(9001)
    bias_bits, bias = bias_bf16(r, rows)
    return dict(rows=np.int32(rows), cols=np.int32(cols), packed=packed, scales=scales,
                x_f16=x16.view(np.uint16), bias_bf16=bias_bits,
                expected=oracle.gemv_bias(packed, scales, bias, x16.astype(np.float32), rows,
                                          cols).astype(np.float32))


def make_expert(act, seed, with_bias):
    r = rng(seed)
    ex = experts_arrays(r, 1, with_bias)
    xbits, xw = normal_bf16(r, H)
    out = oracle.expert_apply(oracle_experts(ex)[0], xw, H, F, act)
    return dict(hidden=np.int32(H), inter=np.int32(F), act=np.int32(act), x_bf16=xbits,
                expected=out.astype(np.float32), **ex)


def make_layer(act, seed, n_experts, top_k, tokens, with_bias):
    r = rng(seed)
    ex = experts_arrays(r, n_experts, with_bias)
    xbits, xw = normal_bf16(r, tokens * H)
    logits = r.standard_normal((tokens, n_experts)).astype(np.float32)
    out, ids, w = oracle.moe_layer(oracle_experts(ex), top_k, logits, xw, H, F, act)
    return dict(hidden=np.int32(H), inter=np.int32(F), act=np.int32(act),
                top_k=np.int32(top_k), tokens=np.int32(tokens), x_bf16=xbits, logits=logits,
                expected=out.astype(np.float32), expected_ids=ids, expected_weights=w, **ex)


def make_router():
    r = rng(9100)
    E, Hr, K = 32, 256, 4
    wbits = oracle.f32_to_bf16_bits((r.standard_normal(E * Hr) * 0.02).astype(np.float32))
    bbits, bf = bias_bf16(r, E)
    x16 = r.standard_normal(Hr).astype(np.float16)
    logits = oracle.router_logits(oracle.bf16_bits_to_f32(wbits), bf, x16.astype(np.float32),
                                  E, Hr)
    ids, w = oracle.router_select(logits, K)
    return dict(experts=np.int32(E), hidden=np.int32(Hr), top_k=np.int32(K), w_bf16=wbits,
                b_bf16=bbits, x_f16=x16.view(np.uint16), expected_logits=logits.astype(np.float32),
                expected_ids=np.asarray(ids, np.int32), expected_weights=np.asarray(w, np.float32))


def make_rmsnorm():
    r = rng(9200)
    T, W = 3, 256
    x = r.standard_normal((T, W)).astype(np.float32) * 3.0
    wbits, _ = normal_bf16(r, W)
    eps = np.float32(1e-5)
    out = oracle.rmsnorm_f16(x, wbits, float(eps))
    return dict(x=x, w_bf16=wbits, eps=eps, expected_f16=out.astype(np.uint16))


FIXTURES = {
    "dequant": make_dequant,
    "gemv": make_gemv,
    "expert_gptoss": lambda: make_expert(oracle.ACT_GPTOSS, 9300, True),
    "expert_qwen3": lambda: make_expert(oracle.ACT_SWIGLU, 9400, False),
    "layer_t1": lambda: make_layer(oracle.ACT_GPTOSS, 9500, 4, 2, 1, True),
    "layer_t3": lambda: make_layer(oracle.ACT_GPTOSS, 9600, 4, 2, 3, True),
    "layer_t40": lambda: make_layer(oracle.ACT_SWIGLU, 9700, 4, 2, 40, False),
    "router": make_router,
    "rmsnorm": make_rmsnorm,
}


def main():
    oracle.build()
    for name, fn in FIXTURES.items():
        path = os.path.join(HERE, name + ".npz")
        np.savez(path, **fn())
        print(f"{path}: {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
