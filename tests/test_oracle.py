"""Pins the CPU oracle (oracle/godwit_oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own code: the reference's known
answers (Tests/GodwitTests/*.swift), numpy closed forms, float64 brute force,
and invariants a plausible mistake would break.
"""
import math

import numpy as np
import pytest

import oracle
from helpers import mxfp4_matrix, rng

FP4 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], np.float32)


# ---- codec: MXFP4Tests.swift ------------------------------------------------

def test_codebook_shape():
    """MXFP4Tests.swift:7-16."""
    cb = np.array([oracle._lib.gwo_codebook(i) for i in range(16)], np.float32)
    assert cb[0] == 0.0 and cb[7] == 6.0
    for c in range(8):
        assert cb[c + 8] == -cb[c]
    assert np.signbit(cb[8])


def test_scale_decoding():
    """MXFP4Tests.swift:18-26."""
    assert oracle.decode_scale(127) == 1.0
    assert oracle.decode_scale(128) == 2.0
    assert oracle.decode_scale(126) == 0.5
    assert math.isnan(oracle.decode_scale(0xFF))
    assert oracle.decode_scale(0) > 0


def test_nibble_order():
    """MXFP4Tests.swift:28-43: 0x71 -> [0.5, 6.0]."""
    p = np.zeros(16, np.uint8)
    p[0] = 0x71
    d = oracle.decode(p, [127], 1)
    assert d[0] == 0.5 and d[1] == 6.0


def test_scale_applies_to_block():
    """MXFP4Tests.swift:45-58: 0x22 at scale 130 -> all 8.0."""
    d = oracle.decode(np.full(16, 0x22, np.uint8), [130], 1)
    assert np.all(d == 8.0)


def test_multi_block():
    """MXFP4Tests.swift:60-76: scales [127, 128, 126] -> 1, 2, 0.5."""
    d = oracle.decode(np.full(48, 0x22, np.uint8), [127, 128, 126], 3)
    assert d.size == 96 and d[0] == 1.0 and d[32] == 2.0 and d[64] == 0.5


def test_decode_exhaustive_against_closed_form():
    """All 256 bytes x 256 scale bytes against FP4[lo|hi] * 2^(s-127) built with numpy
    (ldexp is exact, including the subnormal 2^-127)."""
    packed = np.tile(np.arange(256, dtype=np.uint8), 256)
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)
    got = oracle.decode(packed, scales, 4096)
    with np.errstate(over="ignore"):
        scale = np.ldexp(np.float32(1.0), scales.astype(np.int32) - 127).astype(np.float32)
    scale[scales == 255] = np.nan
    per_byte = np.repeat(scale, 16)
    want = np.empty(4096 * 32, np.float32)
    want[0::2] = FP4[packed & 0x0F] * per_byte
    want[1::2] = FP4[packed >> 4] * per_byte
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


# ---- codec: MXFP4EncodeTests.swift ------------------------------------------

def test_grid_values_are_fixed_points():
    """MXFP4EncodeTests.swift:13-41."""
    weights = []
    for exponent in [-4, -1, 0, 3, 10]:
        s = 2.0 ** exponent
        block = []
        for m in FP4[:8]:
            block += [m * s, -m * s]
        block += [0.0] * (32 - len(block))
        weights += block
    w = np.array(weights, np.float32)
    p, sc = oracle.encode(w)
    d = oracle.decode(p, sc, sc.size)
    assert np.array_equal(d, w)


def test_scale_ceils():
    """MXFP4EncodeTests.swift:43-58."""
    assert oracle.decode_scale(oracle.scale_byte_for_peak(10)) == 2.0
    assert oracle.decode_scale(oracle.scale_byte_for_peak(6)) == 1.0
    assert oracle.decode_scale(oracle.scale_byte_for_peak(3)) == 0.5
    for step in range(200):
        peak = np.float32(2.0 ** (step / 8 - 12))
        s = oracle.decode_scale(oracle.scale_byte_for_peak(peak))
        assert peak / s <= 6.0 + 1e-6


def test_rounding_to_nearest():
    """MXFP4EncodeTests.swift:60-71."""
    cases = [(0.0, 0), (0.24, 0), (0.26, 1), (0.9, 2), (1.4, 3), (2.6, 5), (4.9, 6), (5.1, 7),
             (99, 7)]
    for v, c in cases:
        assert oracle.code_for_magnitude(v) == c


def test_sign_handling():
    """MXFP4EncodeTests.swift:73-91: -0.0 keeps its sign."""
    w = np.array([1.0, -1.0, 0.0, -0.0] + [0.0] * 28, np.float32)
    p, s = oracle.encode(w)
    d = oracle.decode(p, s, 1)
    assert d[0] == 1.0 and d[1] == -1.0
    assert not np.signbit(d[2]) and np.signbit(d[3])


def test_short_block_pads():
    """MXFP4EncodeTests.swift:93-106."""
    p, s = oracle.encode(np.array([1.0, 2.0, 3.0], np.float32))
    assert s.size == 1 and p.size == 16
    d = oracle.decode(p, s, 1)
    assert list(d[:3]) == [1.0, 2.0, 3.0] and np.all(d[3:] == 0)


def test_zero_block():
    """MXFP4EncodeTests.swift:108-114."""
    p, s = oracle.encode(np.zeros(32, np.float32))
    assert np.all(p == 0) and s[0] == 127


def test_error_bound():
    """MXFP4EncodeTests.swift:116-140."""
    w = rng(0).uniform(-3, 3, 32 * 64).astype(np.float32)
    p, s = oracle.encode(w)
    d = oracle.decode(p, s, s.size)
    for b in range(s.size):
        scale = oracle.decode_scale(s[b])
        assert np.all(np.abs(d[32 * b:32 * b + 32] - w[32 * b:32 * b + 32]) <= scale + 1e-6)


# ---- number formats ----------------------------------------------------------

def test_f16_matches_numpy_rne():
    r = rng(1)
    x = np.concatenate([r.standard_normal(20000) * 10 ** r.uniform(-9, 5, 20000),
                        [65504, 65519.99, 65520, 1e-8, 2 ** -25, 2 ** -24 * 1.5, np.inf,
                         -np.inf, 0.0, -0.0]]).astype(np.float32)
    assert np.array_equal(oracle.f32_to_f16_bits(x), x.astype(np.float16).view(np.uint16))


def test_bf16_rne_identities():
    """Int8Affine.swift:86-93 behaviour: exact values round-trip, ties go to even, NaN stays."""
    exact = np.array([1.0, -2.5, 3.140625, 0.0], np.float32)
    assert np.array_equal(oracle.round_to_bf16(exact), exact)
    # 1 + 2^-8 is halfway between bf16 1.0 and 1 + 2^-7: ties to even (1.0)
    assert oracle.round_to_bf16(np.array([1 + 2 ** -8], np.float32))[0] == 1.0
    assert oracle.round_to_bf16(np.array([1 + 3 * 2 ** -8], np.float32))[0] == 1 + 2 ** -6
    assert np.isnan(oracle.round_to_bf16(np.array([np.nan], np.float32))[0])


# ---- GEMV ----------------------------------------------------------------------

def test_gemv_hand_case():
    """DequantGEMVTests.swift:64-77."""
    y = oracle.reference_mxfp4(np.full(16, 0x22, np.uint8), [127], np.ones(32, np.float32), 1, 32)
    assert abs(y[0] - 32.0) < 1e-4


@pytest.mark.parametrize("rows,cols", [(64, 256), (32, 2880), (7, 96)])
def test_gemv_against_float64_brute_force(rows, cols):
    r = rng(rows + cols)
    packed, scales = mxfp4_matrix(r, rows, cols)
    x = r.standard_normal(cols).astype(np.float32)
    bias = (r.standard_normal(rows) * 0.02).astype(np.float32)
    w = oracle.decode(packed, scales, rows * cols // 32).astype(np.float64).reshape(rows, cols)
    exact = w @ x.astype(np.float64) + bias
    got = oracle.gemv_bias(packed, scales, bias, x, rows, cols)
    assert np.max(np.abs(got - exact) / np.maximum(np.abs(exact), 1)) < 1e-5


def test_gemv_row_and_column_order():
    """A transposed operand or swapped nibble order would fail: one-hot rows/cols."""
    rows, cols = 3, 64
    packed = np.zeros(rows * cols // 2, np.uint8)
    scales = np.full(rows * cols // 32, 127, np.uint8)
    packed[1 * 32 + 5] = 0x70   # row 1, column 11 (high nibble of byte 5) = 6.0
    x = np.zeros(cols, np.float32)
    x[11] = 2.0
    y = oracle.reference_mxfp4(packed, scales, x, rows, cols)
    assert list(y) == [0.0, 12.0, 0.0]


def test_gemv_row_parallel_is_identical():
    """The all-core CPU baseline splits GEMV rows over threads; each row keeps
    its serial summation order, so the bytes do not change."""
    r = np.random.default_rng(5)
    rows, cols = 333, 256
    packed = r.integers(0, 256, rows * cols // 2, dtype=np.uint8)
    scales = r.integers(110, 135, rows * cols // 32, dtype=np.uint8)
    bias = oracle.round_to_bf16((r.standard_normal(rows) * 0.02).astype(np.float32))
    x = r.standard_normal(cols).astype(np.float32)
    serial = oracle.gemv_bias(packed, scales, bias, x, rows, cols)
    try:
        oracle.set_threads(4)
        parallel = oracle.gemv_bias(packed, scales, bias, x, rows, cols)
    finally:
        oracle.set_threads(1)
    assert np.array_equal(serial, parallel)


def test_xorshift_generator_matches_swift_recipe():
    """DequantGEMVBenchmark.swift:35-54, restated independently in Python."""
    def ref_bytes(seed, n):
        s = (seed | 1) & 0xFFFFFFFF
        out = []
        for _ in range(n):
            s ^= (s << 13) & 0xFFFFFFFF
            s ^= s >> 17
            s ^= (s << 5) & 0xFFFFFFFF
            out.append((s >> 8) & 0xFF)
        return np.array(out, np.uint8)

    def ref_act(seed, n):
        s = (seed | 1) & 0xFFFFFFFF
        out = []
        for _ in range(n):
            s ^= (s << 13) & 0xFFFFFFFF
            s ^= s >> 17
            s ^= (s << 5) & 0xFFFFFFFF
            i = s - (1 << 32) if s >= 1 << 31 else s
            q = int(math.fmod(i, 200))
            out.append(np.float32(q) / np.float32(200.0))
        return np.array(out, np.float32).astype(np.float16)

    assert np.array_equal(oracle.xorshift_bytes(0xA5A5, 5000), ref_bytes(0xA5A5, 5000))
    assert np.array_equal(oracle.xorshift_activations_f16(0x1234, 3000), ref_act(0x1234, 3000))


# ---- activations: ArchitectureSpecTests.swift / ActivationTests.swift -------------

def _gptoss64(g, u, limit=7.0, alpha=1.702):
    g = min(g, limit)
    u = max(-limit, min(u, limit))
    return (u + 1) * (g / (1 + math.exp(-alpha * g)))


def test_gptoss_closed_form():
    r = rng(2)
    for g, u in zip(r.standard_normal(2000) * 12, r.standard_normal(2000) * 12):
        got = oracle.gptoss_activation(float(g), float(u))
        want = _gptoss64(float(np.float32(g)), float(np.float32(u)))
        assert abs(got - want) <= 1e-5 * max(1.0, abs(want))


def test_gptoss_invariants():
    """ArchitectureSpecTests.swift:86-107."""
    f = oracle.gptoss_activation
    assert f(2, 0) != 0                               # the +1 shift
    assert abs(f(-100, 1)) < 1e-3                     # gate unbounded below
    assert f(8, 1) == f(1000, 1)                      # gate clamped above
    assert f(1, 50) == f(1, 7) and f(1, -50) == f(1, -7)   # up clamped both ways


def test_swiglu_fixed_vectors():
    """ActivationTests.swift:62-83 (CPU side)."""
    gate = [-4, -2, -1, -0.5, 0, 0.5, 1, 2, 4, 8, -8, 0.1]
    up = [1, -1, 2, 0.5, 3, -2, 1, 0.25, -1, 2, 1, -3]
    for g, u in zip(gate, up):
        assert abs(oracle.swiglu(g, u) - g / (1 + math.exp(-g)) * u) < 1e-5


def test_activation_interleave_and_fp16():
    gate = np.array([1.0, -2.0, 9.0], np.float32)
    up = np.array([3.0, 0.5, -9.0], np.float32)
    gu = np.empty(6, np.float32)
    gu[0::2], gu[1::2] = gate, up
    out = oracle.activation(oracle.ACT_GPTOSS, gu)
    want = np.array([_gptoss64(g, u) for g, u in zip(gate, up)], np.float32).astype(np.float16)
    assert np.array_equal(out, want)


# ---- router: Router.swift ------------------------------------------------------------

def test_router_select_matches_sort_and_softmax():
    r = rng(3)
    for _ in range(200):
        lg = r.standard_normal(128).astype(np.float32)
        ids, w = oracle.router_select(lg, 4)
        order = np.argsort(-lg.astype(np.float64), kind="stable")[:4]
        assert list(ids) == list(order)
        e = np.exp(lg[order].astype(np.float64) - lg[order].max())
        assert np.allclose(w, e / e.sum(), rtol=1e-6)
        assert abs(float(w.astype(np.float64).sum()) - 1) < 1e-6


def test_router_select_tie_behaviour():
    """The partial selection sort's swap history decides ties: [5, 5, 7], k=2 picks
    expert 2, then expert 1 (position 1 after the swap holds expert 1, position 2
    holds expert 0, and 5 > 5 is false)."""
    ids, _ = oracle.router_select(np.array([5, 5, 7], np.float32), 2)
    assert list(ids) == [2, 1]


def test_router_select_permutation_invariant():
    r = rng(4)
    lg = r.standard_normal(32).astype(np.float32)
    perm = r.permutation(32)
    ids, w = oracle.router_select(lg, 4)
    ids2, w2 = oracle.router_select(lg[perm], 4)
    assert list(perm[ids2]) == list(ids) and np.array_equal(w, w2)


def test_router_logits_brute_force():
    r = rng(5)
    W = (r.standard_normal((32, 2880)) * 0.02).astype(np.float32)
    x = r.standard_normal(2880).astype(np.float32)
    got = oracle.router_logits(W, None, x, 32, 2880)
    assert np.allclose(got, W.astype(np.float64) @ x, rtol=1e-5, atol=1e-5)


# ---- composition (ExpertRunner, TransformerLayer) --------------------------------------

def _expert(r, hidden, inter):
    gp, gs = mxfp4_matrix(r, 2 * inter, hidden)
    dp, ds = mxfp4_matrix(r, hidden, inter)
    gb = oracle.round_to_bf16((r.standard_normal(2 * inter) * 0.02).astype(np.float32))
    db = oracle.round_to_bf16((r.standard_normal(hidden) * 0.02).astype(np.float32))
    return oracle.Expert(gp, gs, dp, ds, gb, db)


def _expert64(e, x, inter, act=oracle.ACT_GPTOSS):
    """float64 restatement of ExpertRunner.apply with the fp16 activation rounding."""
    gp, gs, dp, ds, gb, db = e.arrays
    hidden = x.size
    wg = oracle.decode(gp, gs, gs.size).astype(np.float64).reshape(2 * inter, hidden)
    wd = oracle.decode(dp, ds, ds.size).astype(np.float64).reshape(hidden, inter)
    gu = wg @ x.astype(np.float64) + gb
    g, u = gu[0::2], gu[1::2]
    if act == oracle.ACT_GPTOSS:
        g = np.minimum(g, 7.0)
        u = np.clip(u, -7.0, 7.0)
        a = (u + 1) * (g / (1 + np.exp(-1.702 * g)))
    else:
        a = g / (1 + np.exp(-g)) * u
    a = a.astype(np.float16).astype(np.float64)
    return wd @ a + db


def test_expert_apply_against_float64():
    r = rng(6)
    hidden, inter = 256, 128
    e = _expert(r, hidden, inter)
    x = r.standard_normal(hidden).astype(np.float32)
    got = oracle.expert_apply(e, x, hidden, inter)
    want = _expert64(e, x, inter)
    # fp16 rounding of the activation can flip an ulp between the two
    assert np.max(np.abs(got - want)) / np.mean(np.abs(want)) < 2e-3


def test_apply_batch_linearity():
    r = rng(7)
    hidden, inter = 256, 128
    es = [_expert(r, hidden, inter) for _ in range(4)]
    x = r.standard_normal(hidden).astype(np.float32)
    w = r.dirichlet(np.ones(4)).astype(np.float32)
    got = oracle.expert_apply_batch(es, w, x, hidden, inter)
    parts = sum(float(wi) * oracle.expert_apply(e, x, hidden, inter).astype(np.float64)
                for e, wi in zip(es, w))
    assert np.max(np.abs(got - parts) / np.maximum(np.abs(parts), 1)) < 1e-5


def test_moe_layer_composition():
    r = rng(8)
    hidden, inter, E, k, T = 256, 128, 8, 2, 3
    es = [_expert(r, hidden, inter) for _ in range(E)]
    logits = r.standard_normal((T, E)).astype(np.float32)
    x = r.standard_normal((T, hidden)).astype(np.float32)
    out, ids, w = oracle.moe_layer(es, k, logits, x, hidden, inter)
    for t in range(T):
        i2, w2 = oracle.router_select(logits[t], k)
        assert list(ids[t]) == list(i2) and np.array_equal(w[t], w2)
        want = sum(float(wi) * oracle.expert_apply(es[e], x[t], hidden, inter).astype(np.float64)
                   for e, wi in zip(i2, w2))
        assert np.max(np.abs(out[t] - want) / np.maximum(np.abs(want), 1)) < 1e-5
    # applyAssignments in token order reproduces the layer
    assigns = [(int(ids[t, j]), t, float(w[t, j])) for t in range(T) for j in range(k)]
    acc = oracle.apply_assignments(es, assigns, x, np.zeros((T, hidden), np.float32), hidden,
                                   inter)
    assert np.array_equal(acc, out)


# ---- around the MoE block: RMSNorm and the residual add --------------------

def _f16_ulp_diff(a_bits, b_bits):
    """Distance in fp16 ulps between finite fp16 bit patterns (sign-aware)."""
    def key(b):
        b = np.asarray(b, np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)
    return np.abs(key(a_bits) - key(b_bits))


def test_rmsnorm_against_float64_closed_form():
    """x / sqrt(mean(x^2) + eps) * w (layer_reference.py's rms_norm), in fp64, rounded
    once to fp16: the oracle's fp32 evaluation differs by at most one fp16 ulp.  A
    dropped mean (sum instead), eps outside the root or a missing weight all miss."""
    r = rng(41)
    for width, eps in ((2880, 1e-5), (2048, 1e-6), (64, 1e-5)):
        x = (r.standard_normal((3, width)) * np.array([[0.5], [2.0], [30.0]])).astype(np.float32)
        wbits = oracle.f32_to_bf16_bits((1.0 + 0.1 * r.standard_normal(width)).astype(np.float32))
        w = oracle.bf16_bits_to_f32(wbits).astype(np.float64)
        got = oracle.rmsnorm_f16(x, wbits, eps)
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + eps) * w
        assert _f16_ulp_diff(got, oracle.f32_to_f16_bits(ref.astype(np.float32)).reshape(got.shape)).max() <= 1


def test_rmsnorm_invariants_and_known_answers():
    # constant row c: every output is fp16(c / sqrt(c^2 + eps)) times the weight
    width = 2880
    ones = oracle.f32_to_bf16_bits(np.ones(width, np.float32))
    out = oracle.rmsnorm_f16(np.full((1, width), 3.0, np.float32), ones, 0.0)
    assert np.all(out == oracle.f32_to_f16_bits(np.float32(1.0)))
    # scale invariance (eps negligible): c * x normalises like x
    r = rng(42)
    x = r.standard_normal((1, width)).astype(np.float32)
    a = oracle.rmsnorm_f16(x, ones, 1e-30)
    b = oracle.rmsnorm_f16(np.float32(8.0) * x, ones, 1e-30)
    assert np.array_equal(a, b)                      # a power of two scales exactly
    # eps dominates for a tiny row, and a zero row stays zero (no NaN)
    tiny = np.full((1, width), 1e-6, np.float32)
    t = oracle.rmsnorm_f16(tiny, ones, 1e-2)
    expect = np.float32(1e-6) / np.sqrt(np.float32(1e-12) + np.float32(1e-2))
    assert _f16_ulp_diff(t[0], oracle.f32_to_f16_bits(np.full(width, expect, np.float32))).max() <= 1
    assert np.all(oracle.rmsnorm_f16(np.zeros((1, width), np.float32), ones, 1e-5) == 0)
    # the weight applies per element: a one-hot weight keeps only that element
    for i in (0, 17, width - 1):
        w = np.zeros(width, np.float32)
        w[i] = 1.0
        o = oracle.rmsnorm_f16(x, oracle.f32_to_bf16_bits(w), 1e-5)[0]
        nz = np.nonzero(o & 0x7FFF)[0]
        assert list(nz) == [i]


def test_residual_add_is_fp32_elementwise():
    r = rng(43)
    s = r.standard_normal(1000).astype(np.float32)
    c = r.standard_normal(1000).astype(np.float32)
    assert np.array_equal(oracle.residual_add(s, c), s + c)
