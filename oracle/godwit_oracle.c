/*
 * godwit_oracle.c — CPU restatement of rayl15/Godwit's MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the parity checker).  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library;
 * the HIP product path never calls it.
 *
 * Each function cites the reference function it restates (paths relative to
 * the reference repository root).  The reference is Swift + Metal and cannot
 * be built here, so this file is the executable statement of its CPU ground
 * truth.  Compiled with -O2 -ffp-contract=off and no fast-math: every `a += b*c`
 * below rounds the product and the sum separately, as the Swift source does.
 *
 * Pinning (what checks each function independently of this file):
 *   codec            known answers of Tests/GodwitTests/MXFP4Tests.swift and
 *                    MXFP4EncodeTests.swift, plus an exhaustive 16x256 table
 *                    built from the closed form with numpy (tests/test_oracle.py:59-77)
 *   f16 / bf16       numpy's float16 cast (RNE) and the bit identities of
 *                    Int8Affine.swift:86-93
 *   GEMV             DequantGEMVTests.swift:64-77 hand case, fp64 brute force
 *   activations      ArchitectureSpecTests.swift:80-107 closed form and
 *                    invariants, ActivationTests.swift:62-63 vectors
 *   router select    numpy argsort/softmax on distinct logits, permutation invariance
 *   composition      linearity: combined == sum_i w_i * expert_i (float64)
 */
#include "godwit_oracle.h"

#include <math.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- number formats ---------------------------------------------------- */

/* IEEE binary16 conversion with round-to-nearest-even, what Swift's
 * Float16(Float) and Metal's half(float) do (expert.metal:101). */
uint16_t gwo_f32_to_f16(float v)
{
    uint32_t x = f2u(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x47800000u) return (uint16_t)(sign | 0x7C00u);          /* >= 2^16: inf */
    uint32_t e = a >> 23;
    if (e >= 113) {                                                    /* normal half */
        uint32_t m = a & 0x7FFFFFu;
        uint32_t h = ((e - 112) << 10) | (m >> 13);
        uint32_t rem = m & 0x1FFFu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;       /* may carry to inf */
        return (uint16_t)(sign | h);
    }
    /* subnormal half: units of 2^-24 */
    uint32_t mant = (a & 0x7FFFFFu) | (e ? 0x800000u : 0u);
    int shift = 126 - (int)(e ? e : 1);
    if (shift > 24) return (uint16_t)sign;
    uint32_t h = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float gwo_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * 0x1p-24f;                                 /* exact */
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

/* BFloat16.fromFloat — Sources/Godwit/Install/Int8Affine.swift:86-93. */
uint16_t gwo_f32_to_bf16(float v)
{
    uint32_t bits = f2u(v);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t rounding = ((bits >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((bits + rounding) >> 16);
}

/* BFloat16.toFloat — Int8Affine.swift:80-83. */
float gwo_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

/* ---- MXFP4 codec ------------------------------------------------------- */

/* MXFP4.codebook — Sources/Godwit/Quant/MXFP4.swift:22-25. */
static const float kCodebook[16] = {
    0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f,
    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f,
};

float gwo_codebook(int code) { return kCodebook[code & 15]; }

/* MXFP4.decodeScale — MXFP4.swift:37-40.  exp2 of an integer is exact,
 * including the subnormal 2^-127 for byte 0; ldexpf states that directly. */
float gwo_decode_scale(uint8_t byte)
{
    if (byte == 0xFF) return NAN;
    return ldexpf(1.0f, (int)byte - 127);
}

/* MXFP4.decodeBlock — MXFP4.swift:48-63 (low nibble = even index, :59-61). */
void gwo_decode_block(const uint8_t *packed16, uint8_t scale_byte, float *dst32)
{
    float scale = gwo_decode_scale(scale_byte);
    for (int i = 0; i < 16; ++i) {
        uint8_t byte = packed16[i];
        dst32[2 * i] = kCodebook[byte & 0x0F] * scale;
        dst32[2 * i + 1] = kCodebook[byte >> 4] * scale;
    }
}

/* MXFP4.decode — MXFP4.swift:69-93. */
void gwo_decode(const uint8_t *packed, const uint8_t *scales, int64_t blocks, float *out)
{
    for (int64_t b = 0; b < blocks; ++b)
        gwo_decode_block(packed + 16 * b, scales[b], out + 32 * b);
}

/* MXFP4.scaleByte(forPeak:) — MXFP4.swift:118-123: ceil(log2(peak/6)) + 127,
 * 255 -> 254, clamped into a byte. */
uint8_t gwo_scale_byte_for_peak(float peak)
{
    if (!(peak > 0.0f) || !isfinite(peak)) return 127;
    float exponent = ceilf(log2f(peak / 6.0f));
    long biased = (long)exponent + 127;
    if (biased == 255) biased = 254;
    if (biased < 0) biased = 0;
    if (biased > 255) biased = 255;
    return (uint8_t)biased;
}

/* MXFP4.code(forMagnitude:) — MXFP4.swift:106,127-134. */
uint8_t gwo_code_for_magnitude(float value)
{
    static const float thresholds[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
    uint8_t code = 0;
    for (int i = 0; i < 7; ++i) {
        if (value < thresholds[i]) return code;
        code += 1;
    }
    return code;
}

/* MXFP4.encodeBlock — MXFP4.swift:143-182 (sign bit kept for -0, :175). */
uint8_t gwo_encode_block(const float *weights, int count, uint8_t *packed16)
{
    float peak = 0.0f;
    for (int i = 0; i < count; ++i)
        if (isfinite(weights[i])) peak = fmaxf(peak, fabsf(weights[i]));
    uint8_t sb = gwo_scale_byte_for_peak(peak);
    float inverse = 1.0f / gwo_decode_scale(sb);
    for (int byte_index = 0; byte_index < 16; ++byte_index) {
        uint8_t byte = 0;
        for (int half = 0; half < 2; ++half) {
            int index = byte_index * 2 + half;
            if (index >= count) continue;
            float w = weights[index];
            if (!isfinite(w)) continue;
            float scaled = fabsf(w) * inverse;
            uint8_t nibble = gwo_code_for_magnitude(scaled);
            if (signbit(w)) nibble |= 0x08;
            byte |= half == 0 ? nibble : (uint8_t)(nibble << 4);
        }
        packed16[byte_index] = byte;
    }
    return sb;
}

/* MXFP4.encode — MXFP4.swift:188-207 (short final block zero-padded). */
void gwo_encode(const float *weights, int64_t count, uint8_t *packed, uint8_t *scales)
{
    int64_t blocks = (count + 31) / 32;
    memset(packed, 0, (size_t)(blocks * 16));
    for (int64_t b = 0; b < blocks; ++b) {
        int64_t start = b * 32;
        int64_t end = start + 32 < count ? start + 32 : count;
        scales[b] = gwo_encode_block(weights + start, (int)(end - start), packed + 16 * b);
    }
}

/* ---- fused dequant GEMV ------------------------------------------------ */

/* DequantGEMVBenchmark.referenceMXFP4 —
 * Sources/Godwit/Benchmark/DequantGEMVBenchmark.swift:100-120.  Per-block
 * partial in element order, then acc += partial * scale over blocks in order. */
/* Threads for the row loop below (1 = the reference's serial loop).  Rows
 * are independent and each is summed by one thread in the order above, so
 * any count gives the same bytes; only the all-core CPU baseline raises it. */
static int g_threads = 1;

void gwo_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }

void gwo_reference_mxfp4(const uint8_t *packed, const uint8_t *scales, const float *x,
                         float *y, int64_t rows, int64_t cols)
{
    int64_t bpr = cols / 32;
#pragma omp parallel for num_threads(g_threads) if (g_threads > 1) schedule(static)
    for (int64_t row = 0; row < rows; ++row) {
        float acc = 0.0f;
        for (int64_t block = 0; block < bpr; ++block) {
            float scale = gwo_decode_scale(scales[row * bpr + block]);
            const uint8_t *base = packed + row * (cols / 2) + block * 16;
            const float *xb = x + block * 32;
            float partial = 0.0f;
            for (int i = 0; i < 16; ++i) {
                uint8_t byte = base[i];
                partial += kCodebook[byte & 0x0F] * xb[2 * i];
                partial += kCodebook[byte >> 4] * xb[2 * i + 1];
            }
            acc += partial * scale;
        }
        y[row] = acc;
    }
}

/* mxfp4_gemv_bias* — Sources/Godwit/Metal/MoE/expert.metal:46-77 (and the
 * multirow variant :311-368): the GEMV above plus `total + float(bias[row])`
 * (:76, :365). */
void gwo_gemv_bias(const uint8_t *packed, const uint8_t *scales, const float *bias,
                   const float *x, float *y, int64_t rows, int64_t cols)
{
    gwo_reference_mxfp4(packed, scales, x, y, rows, cols);
    if (bias)
        for (int64_t r = 0; r < rows; ++r) y[r] = y[r] + bias[r];
}

/* ---- activations, combine ---------------------------------------------- */

/* gptoss_expert_activation — expert.metal:92-101 (CPU closed form
 * Tests/GodwitTests/ArchitectureSpecTests.swift:80-84): gate clamped above
 * only, up clamped both ways, (up + 1) * gate * sigmoid(alpha * gate). */
float gwo_gptoss_activation_f32(float gate, float up, float limit, float alpha)
{
    gate = fminf(gate, limit);
    up = fminf(fmaxf(up, -limit), limit);
    float glu = gate * (1.0f / (1.0f + expf(-alpha * gate)));
    return (up + 1.0f) * glu;
}

/* expert_activation_swiglu — expert.metal:388-392: silu(gate) * up, no clamp,
 * no shift. */
float gwo_swiglu_f32(float gate, float up)
{
    float silu = gate * (1.0f / (1.0f + expf(-gate)));
    return silu * up;
}

/* Interleaved gate_up [2F] -> fp16 activation [F] — expert.metal:93-94,
 * 101 (gptoss) and :388-392 (swiglu). */
void gwo_activation(int kind, const float *gate_up, uint16_t *out_f16, int64_t width,
                    float limit, float alpha)
{
    for (int64_t i = 0; i < width; ++i) {
        float g = gate_up[2 * i], u = gate_up[2 * i + 1];
        float v = kind == GWO_ACT_GPTOSS ? gwo_gptoss_activation_f32(g, u, limit, alpha)
                                         : gwo_swiglu_f32(g, u);
        out_f16[i] = gwo_f32_to_f16(v);
    }
}

/* expert_accumulate — expert.metal:107-116: dst[i] += out[i] * w. */
void gwo_accumulate(const float *expert_out, float *dst, float weight, int64_t width)
{
    for (int64_t i = 0; i < width; ++i) dst[i] += expert_out[i] * weight;
}

/* ---- around the MoE block ------------------------------------------------ */

/* Post-attention RMSNorm of one token's fp32 residual-stream row to the fp16
 * MoE input — TransformerLayer.normalise, TransformerLayer.swift:265-285: the
 * sum of squares in element order, inverse = 1 / sqrt(sum / width + eps), then
 * out[i] = Float16(value * inverse * weight) with the bf16 weight widened and
 * the two products taken left to right (router.metal:36-60 is the same formula
 * on the GPU, with a SIMD-tree sum). */
void gwo_rmsnorm_f16(const float *x, const uint16_t *weight_bf16, int64_t width, float eps,
                     uint16_t *out_f16)
{
    float sum_squares = 0.0f;
    for (int64_t i = 0; i < width; ++i) sum_squares += x[i] * x[i];
    const float inverse = 1.0f / sqrtf(sum_squares / (float)width + eps);
    for (int64_t i = 0; i < width; ++i) {
        const float v = x[i] * inverse;
        out_f16[i] = gwo_f32_to_f16(v * gwo_bf16_to_f32(weight_bf16[i]));
    }
}

/* The residual add after the block — TransformerLayer.swift:232-238:
 * stream[i] += combined[i] in fp32. */
void gwo_residual_add(float *stream, const float *combined, int64_t count)
{
    for (int64_t i = 0; i < count; ++i) stream[i] += combined[i];
}

/* ---- router ------------------------------------------------------------ */

/* bf16_gemv_bias — Sources/Godwit/Metal/MoE/router.metal:18-34 (weights and
 * bias already widened to fp32), summed in column order. */
void gwo_router_logits(const float *weight, const float *bias, const float *x, float *logits,
                       int64_t experts, int64_t hidden)
{
    for (int64_t r = 0; r < experts; ++r) {
        float acc = 0.0f;
        for (int64_t c = 0; c < hidden; ++c) acc += weight[r * hidden + c] * x[c];
        logits[r] = acc + (bias ? bias[r] : 0.0f);
    }
}

/* Router.select — Sources/Godwit/Runtime/Router.swift:78-98: partial selection
 * sort (strict `>`, swapAt) for the top k, then softmax over those k logits with
 * the max subtracted. */
void gwo_router_select(const float *logits, int64_t experts, int64_t top_k,
                       int32_t *ids, float *weights)
{
    int32_t order[4096];
    for (int64_t i = 0; i < experts; ++i) order[i] = (int32_t)i;
    for (int64_t position = 0; position < top_k; ++position) {
        int64_t best = position;
        for (int64_t candidate = position + 1; candidate < experts; ++candidate)
            if (logits[order[candidate]] > logits[order[best]]) best = candidate;
        int32_t t = order[position]; order[position] = order[best]; order[best] = t;
    }
    float peak = 0.0f;
    for (int64_t i = 0; i < top_k; ++i) {
        float v = logits[order[i]];
        if (i == 0 || v > peak) peak = v;
    }
    float e[4096], total = 0.0f;
    for (int64_t i = 0; i < top_k; ++i) { e[i] = expf(logits[order[i]] - peak); total += e[i]; }
    for (int64_t i = 0; i < top_k; ++i) { ids[i] = order[i]; weights[i] = e[i] / total; }
}

/* ---- expert / layer composition ---------------------------------------- */

/* ExpertRunner.apply — Sources/Godwit/Runtime/ExpertRunner.swift:275-331:
 * gate_up GEMV + bias -> activation (fp16) -> down GEMV + bias; no routing
 * weight. */
void gwo_expert_apply(const gwo_expert *e, const float *x, float *out, int64_t hidden,
                      int64_t inter, int act, float limit, float alpha)
{
    static float gate_up[2 * 16384];
    static uint16_t activated[16384];
    static float activated_f32[16384];
    gwo_gemv_bias(e->gate_up_blocks, e->gate_up_scales, e->gate_up_bias, x, gate_up,
                  2 * inter, hidden);
    gwo_activation(act, gate_up, activated, inter, limit, alpha);
    for (int64_t i = 0; i < inter; ++i) activated_f32[i] = gwo_f16_to_f32(activated[i]);
    gwo_gemv_bias(e->down_blocks, e->down_scales, e->down_bias, activated_f32, out, hidden,
                  inter);
}

/* ExpertRunner.applyBatch — ExpertRunner.swift:191-269: combined starts at
 * zero, each expert then `expert_accumulate`s in list order. */
void gwo_expert_apply_batch(const gwo_expert *experts, const float *routing, int32_t n,
                            const float *x, float *out, int64_t hidden, int64_t inter,
                            int act, float limit, float alpha)
{
    static float one[16384];
    for (int64_t i = 0; i < hidden; ++i) out[i] = 0.0f;
    for (int32_t k = 0; k < n; ++k) {
        gwo_expert_apply(&experts[k], x, one, hidden, inter, act, limit, alpha);
        gwo_accumulate(one, out, routing[k], hidden);
    }
}

/* ExpertRunner.applyAssignments — ExpertRunner.swift:108-182: for each
 * (expert, token, weight) in order, outputs[token] += apply(expert,
 * inputs[token]) * weight (in place). */
void gwo_apply_assignments(const gwo_expert *experts, const gwo_assignment *a, int32_t n,
                           const float *inputs, float *outputs, int64_t hidden,
                           int64_t inter, int act, float limit, float alpha)
{
    static float one[16384];
    for (int32_t k = 0; k < n; ++k) {
        gwo_expert_apply(&experts[a[k].expert], inputs + (int64_t)a[k].token * hidden, one,
                         hidden, inter, act, limit, alpha);
        gwo_accumulate(one, outputs + (int64_t)a[k].token * hidden, a[k].weight, hidden);
    }
}

/* MoE block of TransformerLayer.forward —
 * Sources/Godwit/Runtime/TransformerLayer.swift:158-238 with the combine
 * order of Scripts/analysis/layer_reference.py:75-98: route each token
 * (Router.select), then per token combined = 0; combined += expert(x) * w in
 * router order.  The residual add (:232-238) is outside this block. */
void gwo_moe_layer(const gwo_expert *experts, int64_t expert_count, int64_t top_k,
                   const float *logits, const float *x, int32_t tokens, float *out,
                   int32_t *ids, float *weights, int64_t hidden, int64_t inter,
                   int act, float limit, float alpha)
{
    static float one[16384];
    for (int32_t t = 0; t < tokens; ++t) {
        int32_t *tid = ids + (int64_t)t * top_k;
        float *tw = weights + (int64_t)t * top_k;
        gwo_router_select(logits + (int64_t)t * expert_count, expert_count, top_k, tid, tw);
        float *dst = out + (int64_t)t * hidden;
        for (int64_t i = 0; i < hidden; ++i) dst[i] = 0.0f;
        for (int64_t k = 0; k < top_k; ++k) {
            gwo_expert_apply(&experts[tid[k]], x + (int64_t)t * hidden, one, hidden, inter,
                             act, limit, alpha);
            gwo_accumulate(one, dst, tw[k], hidden);
        }
    }
}

/* ---- deterministic inputs ---------------------------------------------- */

/* DequantGEMVBenchmark.pseudoRandomBytes — DequantGEMVBenchmark.swift:35-43. */
void gwo_xorshift_bytes(uint32_t seed, uint8_t *out, int64_t count)
{
    uint32_t state = seed | 1u;
    for (int64_t i = 0; i < count; ++i) {
        state ^= state << 13;
        state ^= state >> 17;
        state ^= state << 5;
        out[i] = (uint8_t)(state >> 8);
    }
}

/* DequantGEMVBenchmark.activations — DequantGEMVBenchmark.swift:45-54. */
void gwo_xorshift_activations_f16(uint32_t seed, uint16_t *out, int64_t count)
{
    uint32_t state = seed | 1u;
    for (int64_t i = 0; i < count; ++i) {
        state ^= state << 13;
        state ^= state >> 17;
        state ^= state << 5;
        int32_t s = (int32_t)state;
        float v = (float)(s % 200) / 200.0f;
        out[i] = gwo_f32_to_f16(v);
    }
}
