"""GPU parity of the kernel-level entry points against the CPU oracle.

Mirrors Tests/GodwitTests/DequantGEMVTests.swift (GEMV vs referenceMXFP4 at
64x256 and 32x2880, metric < 1e-3) and ActivationTests.swift (fixed vectors),
and adds the bit-exact dequant table and the benchmark config-0 shape.
"""
import numpy as np
import pytest

import godwit_amd as gw
import oracle
from helpers import bias_bf16, gemv_metric, mxfp4_matrix, normal_bf16, rng

pytestmark = pytest.mark.gpu


def _bits_equal(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    nan_a, nan_b = np.isnan(a), np.isnan(b)
    assert np.array_equal(nan_a, nan_b), "NaN positions differ"
    return np.array_equal(a[~nan_a].view(np.uint32), b[~nan_b].view(np.uint32))


def test_dequant_exhaustive_codes_and_scales(ctx):
    """Every (byte, scale) pair: 256 packed bytes x 256 scale bytes, bit-exact with
    MXFP4.decode (MXFP4.swift:69-93): subnormal scales, NaN for 0xFF, -0.0 for code 8."""
    blocks = 256 * 16   # block b: scale b // 16, bytes cover all 256 values once per scale
    packed = np.tile(np.arange(256, dtype=np.uint8), 256)
    scales = np.repeat(np.arange(256, dtype=np.uint8), 16)
    pb, sb, ob = ctx.buffer(packed), ctx.buffer(scales), ctx.empty(blocks * 32 * 4)
    gw.mxfp4_dequant(ctx, pb, sb, blocks, ob)
    got = ob.download(np.float32, blocks * 32)
    want = oracle.decode(packed, scales, blocks)
    assert _bits_equal(got, want)
    # spot checks of the special values
    assert got[0] == 0.0 and np.signbit(got[0]) is np.False_
    neg0 = got[(0x08 & 0xF) * 2 + 0]   # byte 0x08: low nibble code 8 -> -0.0
    assert neg0 == 0.0 and np.signbit(neg0)
    for b in (pb, sb, ob):
        b.free()


def test_dequant_random_large(ctx):
    r = rng(1)
    blocks = 5760 * 90
    packed, scales = mxfp4_matrix(r, 5760, 2880, 0, 255)
    pb, sb, ob = ctx.buffer(packed), ctx.buffer(scales), ctx.empty(blocks * 32 * 4)
    gw.mxfp4_dequant(ctx, pb, sb, blocks, ob)
    assert _bits_equal(ob.download(np.float32, blocks * 32), oracle.decode(packed, scales, blocks))
    for b in (pb, sb, ob):
        b.free()


def _run_gemv(ctx, packed, scales, x, x_dtype, rows, cols, bias=None, bias_dtype=gw.BF16):
    pb, sb, xb, yb = ctx.buffer(packed), ctx.buffer(scales), ctx.buffer(x), ctx.empty(rows * 4)
    bb = ctx.buffer(bias) if bias is not None else None
    gw.mxfp4_gemv_bias(ctx, pb, sb, bb, bias_dtype, xb, x_dtype, yb, rows, cols)
    y = yb.download(np.float32, rows)
    for b in (pb, sb, xb, yb, bb):
        if b is not None:
            b.free()
    return y


@pytest.mark.parametrize("rows,cols", [(64, 256), (32, 2880)])
def test_gemv_matches_reference_xorshift(ctx, rows, cols):
    """DequantGEMVTests.swift:20-42: the reference's own inputs (xorshift bytes seed
    0xA5A5, scales 120 + i % 14, fp16 x seed 0x1234), metric < 1e-3."""
    packed = oracle.xorshift_bytes(0xA5A5, rows * cols // 2)
    scales = (120 + np.arange(rows * cols // 32) % 14).astype(np.uint8)
    x16 = oracle.xorshift_activations_f16(0x1234, cols)
    ref = oracle.reference_mxfp4(packed, scales, x16.astype(np.float32), rows, cols)
    pb, sb, xb, yb = ctx.buffer(packed), ctx.buffer(scales), ctx.buffer(x16), ctx.empty(rows * 4)
    gw.mxfp4_gemv(ctx, pb, sb, xb, gw.F16, yb, rows, cols)
    got = yb.download(np.float32, rows)
    assert gemv_metric(got, ref) < 1e-3
    for b in (pb, sb, xb, yb):
        b.free()


def test_gemv_hand_case(ctx):
    """DequantGEMVTests.swift:64-77: 16 x 0x22 (code 2 = 1.0), scale 127, x = 1 -> 32."""
    y = _run_gemv(ctx, np.full(16, 0x22, np.uint8), np.array([127], np.uint8),
                  np.ones(32, np.float16), gw.F16, 1, 32)
    assert y[0] == 32.0


@pytest.mark.parametrize("x_dtype", [gw.F32, gw.F16, gw.BF16])
def test_gemv_config0_shape(ctx, x_dtype):
    """Benchmark config 0: 5760 x 2880, nibbles U{0..15}, scales U{119..127},
    fp32 bias N(0, 0.02); x ~ N(0,1) in each supported dtype."""
    r = rng(7)
    rows, cols = 5760, 2880
    packed, scales = mxfp4_matrix(r, rows, cols)
    bias = (r.standard_normal(rows) * 0.02).astype(np.float32)
    xf = r.standard_normal(cols).astype(np.float32)
    if x_dtype == gw.F32:
        x, xw = xf, xf
    elif x_dtype == gw.F16:
        x = xf.astype(np.float16)
        xw = x.astype(np.float32)
    else:
        x, xw = normal_bf16(r, cols)
    ref = oracle.gemv_bias(packed, scales, bias, xw, rows, cols)
    got = _run_gemv(ctx, packed, scales, x, x_dtype, rows, cols, bias=bias, bias_dtype=gw.F32)
    assert gemv_metric(got, ref) < 1e-3
    # float64 brute force bounds the oracle's own rounding too
    w = oracle.decode(packed, scales, rows * cols // 32).astype(np.float64).reshape(rows, cols)
    exact = w @ xw.astype(np.float64) + bias
    assert gemv_metric(got, exact) < 1e-4


@pytest.mark.parametrize("rows,cols", [(1, 32), (3, 64), (17, 768), (5, 4096), (33, 2048),
                                       (7, 32 * 600), (8196, 2880), (5000, 32 * 100),
                                       (9, 6144), (6000, 2176), (7000, 2304)])
@pytest.mark.parametrize("x_dtype", [gw.BF16, gw.F32], ids=["bf16", "f32"])
def test_gemv_ragged_shapes(ctx, rows, cols, x_dtype):
    """Ragged row counts and widths, bf16 and fp32 x, against the oracle and
    the float64 sum (rows past 512 workgroups' worth, rows wider than the
    register stages).  Between them they take every staging order of the
    kernels: a workgroup whose rows are one stage (dotted block by block as
    they land), several stages or chunks with x's loads issued first (8196
    rows; 6144 columns in bf16), x staged before any weight load (x wider
    than one batch of loads: 19200 columns, 6144 in fp32), and the
    one-workgroup-per-CU form for 17..32 rows a CU of 65..96 blocks, 384
    threads up to 24 rows (6000 x 2176; the config-0 shape too) and 512
    beyond (7000 x 2304, on 256 CUs)."""
    r = rng(rows * 1000 + cols)
    packed, scales = mxfp4_matrix(r, rows, cols)
    bits, bias = bias_bf16(r, rows)
    xb16, xw = normal_bf16(r, cols)
    if x_dtype == gw.F32:
        xw = r.standard_normal(cols).astype(np.float32)
    ref = oracle.gemv_bias(packed, scales, bias, xw, rows, cols)
    x = xb16 if x_dtype == gw.BF16 else xw
    got = _run_gemv(ctx, packed, scales, x, x_dtype, rows, cols, bias=bits, bias_dtype=gw.BF16)
    assert gemv_metric(got, ref) < 1e-3
    w = oracle.decode(packed, scales, rows * cols // 32).astype(np.float64).reshape(rows, cols)
    assert gemv_metric(got, w @ xw.astype(np.float64) + bias) < 1e-4


@pytest.mark.parametrize("x_dtype", [gw.F16, gw.F32], ids=["f16", "f32"])
def test_gemv_edge_scales(ctx, x_dtype):
    """Subnormal scale bytes 0/1, the largest scale 254 and NaN 0xFF flow through the GEMV
    as the CPU reference computes them."""
    r = rng(3)
    rows, cols = 8, 256
    packed, scales = mxfp4_matrix(r, rows, cols)
    scales = scales.reshape(rows, -1)
    scales[1, :] = 0
    scales[2, :] = 1
    scales[3, 3] = 254
    scales[4, 5] = 255
    scales = scales.ravel()
    x = np.ones(cols, np.float16 if x_dtype == gw.F16 else np.float32)
    ref = oracle.reference_mxfp4(packed, scales, x.astype(np.float32), rows, cols)
    got = _run_gemv(ctx, packed, scales, x, x_dtype, rows, cols)
    assert np.isnan(got[4]) and np.isnan(ref[4])
    keep = np.arange(rows) != 4
    assert np.allclose(got[keep], ref[keep], rtol=1e-6, atol=0)


def test_gemv_f32_large_scales(ctx):
    """Scale bytes 253 and 254 (2^126, 2^127) with small fp32 x, so the sums stay
    finite: rows mixing them with ordinary and subnormal scales match the
    oracle and the float64 sum."""
    r = rng(11)
    rows, cols = 40, 512
    packed, scales = mxfp4_matrix(r, rows, cols)
    scales = scales.reshape(rows, -1)
    scales[0, :] = 253
    scales[1, :] = 254
    scales[2, ::3] = 253
    scales[2, 1::3] = 0
    scales[5, 7] = 254
    scales[21, 2] = 253          # the second tile
    scales = scales.ravel()
    x = (r.standard_normal(cols) * 2.0 ** -20).astype(np.float32)
    ref = oracle.reference_mxfp4(packed, scales, x, rows, cols)
    got = _run_gemv(ctx, packed, scales, x, gw.F32, rows, cols)
    assert np.all(np.isfinite(ref)) and np.all(np.isfinite(got))
    # fp32 sums in any order stay within a small multiple of 2^-24 of the sum
    # of |products| from the exact value; rows of large blocks that cancel
    # are held to that, not to their (smaller) result
    nb = rows * cols // 32   # weights in float64: 6 * 2^127 overflows fp32
    codes = oracle.decode(packed, np.full(nb, 127, np.uint8), nb).astype(np.float64)
    w = (codes.reshape(nb, 32) * 2.0 ** (scales.astype(np.float64) - 127)[:, None]).reshape(rows, cols)
    exact = w @ x.astype(np.float64)
    mag = np.abs(w) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(ref - exact) <= 1e-5 * mag)   # the oracle itself
    assert np.all(np.abs(got - exact) <= 1e-5 * mag), np.max(np.abs(got - exact) / mag)


def test_gemv_shape_errors(ctx):
    b = ctx.empty(1024)
    with pytest.raises(gw.GodwitError) as e:
        gw.mxfp4_gemv(ctx, b, b, b, gw.F16, b, 4, 48)
    assert e.value.status == 2   # GW_ERR_SHAPE: cols % 32
    b.free()


GATE = np.array([-4, -2, -1, -0.5, 0, 0.5, 1, 2, 4, 8, -8, 0.1], np.float32)
UP = np.array([1, -1, 2, 0.5, 3, -2, 1, 0.25, -1, 2, 1, -3], np.float32)


def _run_activation(ctx, kind, gate, up):
    gu = np.empty(2 * gate.size, np.float32)
    gu[0::2], gu[1::2] = gate, up
    gb, ob = ctx.buffer(gu), ctx.empty(gate.size * 2)
    gw.expert_activation(ctx, kind, gb, ob, gate.size, 7.0, 1.702)
    out = ob.download(np.float16, gate.size)
    gb.free()
    ob.free()
    return out, gu


def test_swiglu_fixed_vectors(ctx):
    """ActivationTests.swift:62-83: silu(gate) * up within 0.01."""
    out, gu = _run_activation(ctx, "silu", GATE, UP)
    want = GATE / (1 + np.exp(-GATE.astype(np.float64))) * UP
    assert np.all(np.abs(out.astype(np.float64) - want) < 0.01)
    ref = oracle.activation(oracle.ACT_SWIGLU, gu)
    assert np.max(np.abs(out.astype(np.float32) - ref.astype(np.float32))
                  / np.maximum(np.abs(ref.astype(np.float32)), 1e-3)) <= 2 ** -10


def test_gptoss_activation_vectors(ctx):
    """gptoss_expert_activation (expert.metal:82-102) against the CPU closed form of
    ArchitectureSpecTests.swift:80-84 (the reference has no GPU test for it)."""
    r = rng(5)
    gate = np.concatenate([GATE, r.standard_normal(4000).astype(np.float32) * 20])
    up = np.concatenate([UP, r.standard_normal(4000).astype(np.float32) * 20])
    out, gu = _run_activation(ctx, "gptOssClampedGLU", gate, up)
    g = np.minimum(gate.astype(np.float64), 7)
    u = np.clip(up.astype(np.float64), -7, 7)
    want = (u + 1) * (g / (1 + np.exp(-1.702 * g)))
    assert np.all(np.abs(out.astype(np.float64) - want) <= 0.01 * np.maximum(1, np.abs(want)))
    ref = oracle.activation(oracle.ACT_GPTOSS, gu).astype(np.float32)
    o = out.astype(np.float32)
    # identical up to one fp16 ulp (exp may differ by an fp32 ulp before rounding)
    assert np.all(np.abs(o - ref) <= np.spacing(np.abs(ref).astype(np.float16)).astype(np.float32))


def test_accumulate(ctx):
    r = rng(11)
    src = r.standard_normal(2880).astype(np.float32)
    dst = r.standard_normal(2880).astype(np.float32)
    sb, db = ctx.buffer(src), ctx.buffer(dst)
    gw.expert_accumulate(ctx, sb, db, 0.37, 2880)
    got = db.download(np.float32, 2880)
    assert np.array_equal(got, oracle.accumulate(src, dst, 0.37))
    sb.free()
    db.free()


class _At:
    """A device address with the .ptr attribute the bindings read."""

    def __init__(self, ptr):
        self.ptr = ptr


@pytest.mark.parametrize("E,H,shift", [(32, 2880, 0), (20, 100, 0), (16, 512, 2)],
                         ids=["rows", "h100", "unaligned"])
def test_router_logits_forms(ctx, E, H, shift):
    """bf16_gemv_bias (router.metal:18-34) through both device forms: the
    row-per-workgroup kernel (H % 8 == 0, 16-byte aligned rows) and the
    one-wave-per-logit kernel it falls back to (H = 100; weights 2 bytes off
    alignment)."""
    r = rng(17 + H)
    wbits = oracle.f32_to_bf16_bits((r.standard_normal(E * H) * 0.02).astype(np.float32))
    bbits, bf = bias_bf16(r, E)
    x16 = r.standard_normal(H).astype(np.float16)
    store = np.zeros(E * H + 8, np.uint16)
    store[shift // 2:shift // 2 + E * H] = wbits
    wb, bb = ctx.buffer(store), ctx.buffer(bbits)
    router = gw.Router(ctx, E, H, 4)
    got = router.logits(x16, _At(wb.ptr + shift), bb)
    ref = oracle.router_logits(oracle.bf16_bits_to_f32(wbits), bf, x16.astype(np.float32), E, H)
    assert gemv_metric(got, ref) < 1e-5
    wb.free()
    bb.free()


def test_router_logits(ctx):
    """bf16_gemv_bias (router.metal:18-34) for 128 experts, bf16 weights and bias."""
    r = rng(13)
    E, H = 128, 2880
    wbits, wf = normal_bf16(r, E * H)
    wf = wf * 0.02
    wbits = oracle.f32_to_bf16_bits(wf)
    wf = oracle.bf16_bits_to_f32(wbits)
    bbits, bf = bias_bf16(r, E)
    x16 = r.standard_normal(H).astype(np.float16)
    router = gw.Router(ctx, E, H, 4)
    wb, bb = ctx.buffer(wbits), ctx.buffer(bbits)
    got = router.logits(x16, wb, bb)
    ref = oracle.router_logits(wf, bf, x16.astype(np.float32), E, H)
    assert gemv_metric(got, ref) < 1e-5
    d = router.route(x16, wb, bb)
    ids, w = oracle.router_select(got, 4)
    assert d.experts == list(ids) and np.allclose(d.weights, w, rtol=0, atol=0)
    wb.free()
    bb.free()


def test_fill_rows_equal_contiguous(ctx):
    """One strided fill launch over `rows` runs (one section of every expert of a
    layer, as the benchmark fills its weights) equals the contiguous fill of
    rows * count values cut into rows, and leaves the bytes between runs alone."""
    rows, count, stride = 5, 40, 72            # bytes: 8-byte units, rows not 8-aligned
    buf = ctx.buffer(np.full(rows * stride, 0xA5, np.uint8))
    ctx.fill_uniform_u8(buf, 3, 200, 99, count=count, rows=rows, row_stride=stride)
    ref = ctx.empty(rows * count)
    ctx.fill_uniform_u8(ref, 3, 200, 99, count=rows * count)
    ctx.synchronize()
    got = buf.download(np.uint8).reshape(rows, stride)
    want = ref.download(np.uint8).reshape(rows, count)
    assert np.array_equal(got[:, :count], want)
    assert (got[:, count:] == 0xA5).all()
    assert want.min() >= 3 and want.max() <= 200
    n, stride2 = 37, 100                       # bf16 normals, 2-byte aligned rows
    buf2 = ctx.buffer(np.full(3 * stride2, 0x5A, np.uint8))
    ctx.fill_normal(buf2, gw.BF16, n, 0.0, 1.0, 7, offset=2, rows=3, row_stride=stride2)
    ref2 = ctx.empty(3 * n * 2)
    ctx.fill_normal(ref2, gw.BF16, 3 * n, 0.0, 1.0, 7)
    ctx.synchronize()
    raw = buf2.download(np.uint8)
    want2 = ref2.download(np.uint16).reshape(3, n)
    for r in range(3):
        row = raw[r * stride2 + 2:r * stride2 + 2 + 2 * n].view(np.uint16)
        assert np.array_equal(row, want2[r]), r
        assert (raw[r * stride2 + 2 + 2 * n:(r + 1) * stride2 + 2][:stride2 - 2 * n] == 0x5A).all()
    for b in (buf, ref, buf2, ref2):
        b.free()
