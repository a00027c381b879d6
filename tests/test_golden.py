"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_fixtures.py from the CPU oracle).

CPU: every fixture is reproduced bit for bit by the oracle from the same
seeds; the dequantisation fixture agrees with the MXFP4 closed form and the
GEMV fixture with a float64 dot product of the decoded weights.  GPU: the HIP path run on the fixtures' inputs
matches their outputs — dequantisation bit-exact, routing exact, outputs within
the reference's metrics (rel. 1e-3)."""
import os
import sys

import numpy as np
import pytest

import oracle
from helpers import expert_metric, gemv_metric, layer_check

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import make_fixtures  # noqa: E402

NAMES = sorted(make_fixtures.FIXTURES)


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype.kind == "f":
        return a.shape == b.shape and np.array_equal(a, b, equal_nan=True)
    return a.shape == b.shape and np.array_equal(a, b)


@pytest.mark.parametrize("name", NAMES)
def test_oracle_reproduces_fixture(name):
    """The oracle, run again from the generator's seeds, gives the committed bytes."""
    want = load(name)
    got = make_fixtures.FIXTURES[name]()
    assert sorted(got) == sorted(want)
    for k in want:
        assert _same(got[k], want[k]), (name, k)


def test_dequant_fixture_closed_form():
    """MXFP4.decode (MXFP4.swift:37-40,60-61): value = codebook[c] * 2^(s-127),
    NaN for s = 0xFF, low nibble first."""
    z = load("dequant")
    cb = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6])
    exp = z["expected"].reshape(-1, 32)
    for b in range(exp.shape[0]):
        s = int(z["scales"][b])
        bytes_ = z["packed"][16 * b:16 * b + 16]
        codes = np.stack([bytes_ & 15, bytes_ >> 4], axis=1).ravel()
        if s == 255:
            assert np.all(np.isnan(exp[b]))
            continue
        with np.errstate(over="ignore"):   # 6 x 2^127 overflows fp32 to inf, as in Swift
            want = (cb[codes] * np.ldexp(1.0, s - 127)).astype(np.float32)
        assert np.array_equal(exp[b], want) and np.array_equal(np.signbit(exp[b]),
                                                               np.signbit(want))


def test_gemv_fixture_against_float64():
    """The GEMV fixture against a float64 dot product of the decoded weights."""
    z = load("gemv")
    rows, cols = int(z["rows"]), int(z["cols"])
    w = oracle.decode(z["packed"], z["scales"], rows * cols // 32).astype(np.float64)
    x = z["x_f16"].view(np.float16).astype(np.float64)
    bias = oracle.bf16_bits_to_f32(z["bias_bf16"]).astype(np.float64)
    exact = w.reshape(rows, cols) @ x + bias
    assert gemv_metric(z["expected"], exact) < 1e-5


# ---------------------------------------------------------------------------
# GPU: the HIP path on the fixtures' inputs
# ---------------------------------------------------------------------------

ACT_NAMES = {oracle.ACT_GPTOSS: "gptOssClampedGLU", oracle.ACT_SWIGLU: "silu"}


def _experts_buffer(ctx, gw, z):
    H, F = int(z["hidden"]), int(z["inter"])
    n = z["gu_packed"].shape[0]
    layout = gw.ExpertLayout(H, F, n)
    blob = np.zeros(n * layout.stride, np.uint8)
    for i in range(n):
        base = i * layout.stride
        for sec, key in (("gate_up_blocks", "gu_packed"), ("gate_up_scales", "gu_scales"),
                         ("down_blocks", "dn_packed"), ("down_scales", "dn_scales"),
                         ("gate_up_bias", "gu_bias_bits"), ("down_bias", "dn_bias_bits")):
            arr = z[key][i].view(np.uint8).ravel()
            off = base + layout.offsets[sec]
            blob[off:off + arr.size] = arr
    return layout, ctx.buffer(blob)


@pytest.mark.gpu
def test_gpu_dequant_fixture(ctx):
    import godwit_amd as gw
    z = load("dequant")
    blocks = z["scales"].size
    pb, sb, ob = ctx.buffer(z["packed"]), ctx.buffer(z["scales"]), ctx.empty(blocks * 32 * 4)
    gw.mxfp4_dequant(ctx, pb, sb, blocks, ob)
    got = ob.download(np.float32, blocks * 32)
    assert _same(got, z["expected"])
    assert np.array_equal(np.signbit(got), np.signbit(z["expected"]))
    for b in (pb, sb, ob):
        b.free()


@pytest.mark.gpu
def test_gpu_gemv_fixture(ctx):
    import godwit_amd as gw
    z = load("gemv")
    rows, cols = int(z["rows"]), int(z["cols"])
    pb, sb = ctx.buffer(z["packed"]), ctx.buffer(z["scales"])
    xb, bb, yb = ctx.buffer(z["x_f16"]), ctx.buffer(z["bias_bf16"]), ctx.empty(rows * 4)
    gw.mxfp4_gemv_bias(ctx, pb, sb, bb, gw.BF16, xb, gw.F16, yb, rows, cols)
    assert gemv_metric(yb.download(np.float32, rows), z["expected"]) < 1e-3
    for b in (pb, sb, xb, bb, yb):
        b.free()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["expert_gptoss", "expert_qwen3"])
def test_gpu_expert_fixture(ctx, name):
    import godwit_amd as gw
    z = load(name)
    H, F = int(z["hidden"]), int(z["inter"])
    layout, buf = _experts_buffer(ctx, gw, z)
    runner = gw.ExpertRunner(ctx, H, F, ACT_NAMES[int(z["act"])])
    got = runner.apply(z["x_bf16"], gw.Weights(buf, runner.section_offsets), dtype=gw.BF16)
    assert expert_metric(got, z["expected"]) < 1e-3
    runner.close()
    buf.free()


@pytest.mark.gpu
@pytest.mark.parametrize("name,path", [("layer_t1", "stream"), ("layer_t3", "stream"),
                                       ("layer_t3", "grouped"), ("layer_t40", "grouped")])
def test_gpu_layer_fixture(ctx, monkeypatch, name, path):
    """gw_moe_layer_forward on the fixture: 1 and 3 tokens on the streaming
    kernels, 3 and 40 tokens on the grouped GEMMs."""
    import godwit_amd as gw
    z = load(name)
    H, F, K, T = int(z["hidden"]), int(z["inter"]), int(z["top_k"]), int(z["tokens"])
    E = z["gu_packed"].shape[0]
    layout, buf = _experts_buffer(ctx, gw, z)
    monkeypatch.setenv("GODWIT_PREFILL_ABOVE", "8" if path == "stream" else "1")
    runner = gw.ExpertRunner(ctx, H, F, ACT_NAMES[int(z["act"])])
    xb, lb = ctx.buffer(z["x_bf16"]), ctx.buffer(z["logits"])
    out = ctx.empty(T * H * 4)
    ids_b, w_b = ctx.empty(T * K * 4), ctx.empty(T * K * 4)
    runner.layer_forward(buf.ptr, layout.stride, E, K, xb.ptr, gw.BF16, T, out.ptr,
                         logits=lb.ptr, routing_ids=ids_b.ptr, routing_weights=w_b.ptr)
    ctx.synchronize()
    got = out.download(np.float32, T * H).reshape(T, H)
    assert np.array_equal(ids_b.download(np.int32, T * K).reshape(T, K), z["expected_ids"])
    assert np.allclose(w_b.download(np.float32, T * K).reshape(T, K), z["expected_weights"],
                       rtol=1e-6, atol=1e-7)
    for t in range(T):
        assert expert_metric(got[t], z["expected"][t]) < 1e-3, t
    rel_rms, worst, bound, ok = layer_check(got, z["expected"])
    assert ok, (rel_rms, worst, bound)
    for b in (xb, lb, out, ids_b, w_b, buf):
        b.free()
    runner.close()


@pytest.mark.gpu
def test_gpu_router_fixture(ctx):
    import godwit_amd as gw
    z = load("router")
    E, H, K = int(z["experts"]), int(z["hidden"]), int(z["top_k"])
    router = gw.Router(ctx, E, H, K)
    wb, bb = ctx.buffer(z["w_bf16"]), ctx.buffer(z["b_bf16"])
    x16 = z["x_f16"].view(np.float16)
    got = router.logits(x16, wb, bb)
    assert gemv_metric(got, z["expected_logits"]) < 1e-5
    d = router.route(x16, wb, bb)
    assert d.experts == list(z["expected_ids"])
    assert np.allclose(d.weights, z["expected_weights"], rtol=1e-5, atol=1e-7)
    wb.free()
    bb.free()
