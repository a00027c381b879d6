/*
 * godwit_oracle.h — CPU restatement of rayl15/Godwit's MoE expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the parity checker for the HIP library
 * (godwit_amd/libgodwit_hip.so).  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product path never links or
 * calls it.
 *
 * Every function follows a reference function; the citation (path:line,
 * relative to the reference repository root) is on each definition in
 * godwit_oracle.c.  Build: gcc -O2 -ffp-contract=off (no fast-math), so fp32
 * arithmetic happens in the scalar order the reference writes it.
 */
#ifndef GODWIT_ORACLE_H
#define GODWIT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- number formats ---------------------------------------------------- */
uint16_t gwo_f32_to_f16(float v);         /* IEEE binary16, round-to-nearest-even */
float    gwo_f16_to_f32(uint16_t h);
uint16_t gwo_f32_to_bf16(float v);        /* BFloat16.fromFloat (RNE, NaN kept) */
float    gwo_bf16_to_f32(uint16_t b);     /* BFloat16.toFloat */

/* ---- MXFP4 codec ------------------------------------------------------- */
float   gwo_codebook(int code);
float   gwo_decode_scale(uint8_t byte);
void    gwo_decode_block(const uint8_t *packed16, uint8_t scale, float *dst32);
void    gwo_decode(const uint8_t *packed, const uint8_t *scales, int64_t blocks, float *out);
uint8_t gwo_scale_byte_for_peak(float peak);
uint8_t gwo_code_for_magnitude(float value);
uint8_t gwo_encode_block(const float *weights, int count, uint8_t *packed16);
void    gwo_encode(const float *weights, int64_t count, uint8_t *packed, uint8_t *scales);

/* ---- fused dequant GEMV ------------------------------------------------ */
/* x is already widened to fp32 (the reference widens fp16 x with Float(x)). */
/* Row-parallel threads for the GEMVs (default 1; results do not depend on it). */
void gwo_set_threads(int threads);
void gwo_reference_mxfp4(const uint8_t *packed, const uint8_t *scales, const float *x,
                         float *y, int64_t rows, int64_t cols);
/* bias may be NULL (no bias); otherwise fp32 values (bf16 biases are widened first). */
void gwo_gemv_bias(const uint8_t *packed, const uint8_t *scales, const float *bias,
                   const float *x, float *y, int64_t rows, int64_t cols);

/* ---- activations, combine ---------------------------------------------- */
enum { GWO_ACT_GPTOSS = 0, GWO_ACT_SWIGLU = 1 };
float gwo_gptoss_activation_f32(float gate, float up, float limit, float alpha);
float gwo_swiglu_f32(float gate, float up);
void  gwo_activation(int kind, const float *gate_up, uint16_t *out_f16, int64_t width,
                     float limit, float alpha);
void  gwo_accumulate(const float *expert_out, float *dst, float weight, int64_t width);

/* ---- router ------------------------------------------------------------ */
/* around the MoE block */
void gwo_rmsnorm_f16(const float *x, const uint16_t *weight_bf16, int64_t width, float eps,
                     uint16_t *out_f16);
void gwo_residual_add(float *stream, const float *combined, int64_t count);

void gwo_router_logits(const float *weight, const float *bias, const float *x, float *logits,
                       int64_t experts, int64_t hidden);
void gwo_router_select(const float *logits, int64_t experts, int64_t top_k,
                       int32_t *ids, float *weights);

/* ---- expert / layer composition ---------------------------------------- */
/* One expert as six section pointers (ExpertRunner.Weights + ExpertLayout). */
typedef struct {
    const uint8_t *gate_up_blocks, *gate_up_scales, *down_blocks, *down_scales;
    const float *gate_up_bias, *down_bias;    /* fp32 widened; NULL = zero */
} gwo_expert;

void gwo_expert_apply(const gwo_expert *e, const float *x, float *out, int64_t hidden,
                      int64_t inter, int act, float limit, float alpha);
void gwo_expert_apply_batch(const gwo_expert *experts, const float *routing, int32_t n,
                            const float *x, float *out, int64_t hidden, int64_t inter,
                            int act, float limit, float alpha);
typedef struct { int32_t expert; int32_t token; float weight; } gwo_assignment;
void gwo_apply_assignments(const gwo_expert *experts, const gwo_assignment *a, int32_t n,
                           const float *inputs, float *outputs, int64_t hidden,
                           int64_t inter, int act, float limit, float alpha);
/* MoE block of TransformerLayer.forward for `tokens` tokens, logits given
 * ([tokens, experts]); writes ids/weights ([tokens, top_k]) and out ([tokens, hidden],
 * overwritten). */
void gwo_moe_layer(const gwo_expert *experts, int64_t expert_count, int64_t top_k,
                   const float *logits, const float *x, int32_t tokens, float *out,
                   int32_t *ids, float *weights, int64_t hidden, int64_t inter,
                   int act, float limit, float alpha);

/* ---- deterministic inputs ---------------------------------------------- */
void gwo_xorshift_bytes(uint32_t seed, uint8_t *out, int64_t count);
void gwo_xorshift_activations_f16(uint32_t seed, uint16_t *out, int64_t count);

#ifdef __cplusplus
}
#endif
#endif
