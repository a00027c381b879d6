/*
 * godwit_hip.h — C ABI of the MI355X (gfx950) MoE expert hot-path library
 * (libgodwit_hip.so).
 *
 * This is the drop-in boundary for rayl15/Godwit's MoE expert path.  Each
 * entry point names the reference interface it replaces (paths relative to the
 * reference repository root).  Plain pointers and sizes only: device buffers
 * are `void*` device addresses from gw_malloc (or any hipMalloc'd memory of
 * this process), host buffers are ordinary host memory.
 *
 * Conventions
 *  - Every call returns an int status (gw_status); 0 is success.  On failure
 *    gw_last_error() returns a thread-local message.  No C++ exception crosses
 *    the ABI.  Shape violations return GW_ERR_SHAPE instead of trapping (the
 *    reference traps with `precondition`).
 *  - Calls on a context are stream-ordered on its stream.  Calls whose Swift
 *    counterpart blocks (ExpertRunner.apply*, Router.logits, which run
 *    MetalContext.run = commit + waitUntilCompleted) block here too;
 *    gw_*_async variants and the layer/kernel calls only enqueue.
 *  - A context and everything created from it is single-threaded; callers
 *    serialise access.
 *
 * MXFP4 data (MXFP4.swift:3-31): a block is 32 e2m1 codes, two per byte, low
 * nibble = even element, plus one e8m0 scale byte (2^(b-127), 0xFF = NaN).
 * A matrix [rows, cols] is packed [rows, cols/32, 16] bytes + scales
 * [rows, cols/32] bytes, row-major, cols % 32 == 0.
 */
#ifndef GODWIT_HIP_H
#define GODWIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility push(default)
#endif

/* ---- status, dtypes ---------------------------------------------------- */

/* Replaces MetalError (Sources/Godwit/Infrastructure/Metal/MetalContext.swift:4-33)
 * and the precondition traps of ExpertRunner.swift:194,276 / Router.swift:41,79. */
typedef enum gw_status {
    GW_OK = 0,
    GW_ERR_ARG = 1,         /* null pointer, bad enum, negative size */
    GW_ERR_SHAPE = 2,       /* cols % 32 != 0, size mismatch, limits exceeded */
    GW_ERR_OOM = 3,         /* device allocation failed */
    GW_ERR_HIP = 4,         /* HIP runtime error (message has hipGetErrorString) */
    GW_ERR_NO_DEVICE = 5,   /* no HIP device / device index out of range */
    GW_ERR_UNSUPPORTED = 6, /* valid request this build does not implement */
    GW_ERR_EXCHANGE = 7     /* a one-token layer's bounded wait gave up: see
                               gw_expert_runner_sync_errors */
} gw_status;

typedef enum gw_dtype { GW_F32 = 0, GW_F16 = 1, GW_BF16 = 2 } gw_dtype;

/* FeedForwardActivation (Sources/Godwit/Model/ArchitectureSpec.swift:14-38):
 * .gptOssClampedGLU -> gptoss_expert_activation (expert.metal:82-102),
 * .silu -> expert_activation_swiglu (expert.metal:380-393). */
typedef enum gw_activation { GW_ACT_GPTOSS_CLAMPED_GLU = 0, GW_ACT_SILU = 1 } gw_activation;

/* Thread-local message of the last failing call on this thread ("" if none). */
const char *gw_last_error(void);
/* Library version string. */
const char *gw_version(void);

/* ---- context (replaces MetalContext, MetalContext.swift:36-179) -------- */

typedef struct gw_context gw_context;

int gw_device_count(int *count);
/* MetalContext.init: binds `device`, creates the context's stream. */
int gw_context_create(int device, gw_context **out);
int gw_context_destroy(gw_context *ctx);
/* Blocks until all work enqueued on the context's stream is done. */
int gw_context_synchronize(gw_context *ctx);
/* The context's hipStream_t (as void*). */
void *gw_context_stream(gw_context *ctx);
/* Number of compute units of the context's device. */
int gw_context_cu_count(gw_context *ctx, int *cus);

/* Per-kernel timing (replaces Profiler, Infrastructure/Metal/Profiler.swift:11-98):
 * while enabled, every launch is bracketed by hipEvents on the context stream.
 * gw_context_profile_read synchronises and returns the summed GPU milliseconds
 * and launch count of the kernel family `name` ("gate_up", "down", "route",
 * "router", "gemv", "dequant", "activation", "accumulate"). */
int gw_context_set_profiling(gw_context *ctx, int enabled);
int gw_context_profile_read(gw_context *ctx, const char *name, double *total_ms,
                            int64_t *launches);
int gw_context_profile_reset(gw_context *ctx);

/* ---- device memory (MetalContext.buffer / emptyBuffer, :161-178) ------- */

int gw_malloc(gw_context *ctx, size_t bytes, void **out);
int gw_free(gw_context *ctx, void *ptr);
int gw_memcpy_htod(gw_context *ctx, void *dst, const void *src, size_t bytes);
int gw_memcpy_dtoh(gw_context *ctx, void *dst, const void *src, size_t bytes);
int gw_memcpy_dtod(gw_context *ctx, void *dst, const void *src, size_t bytes);
/* Blocking zero fill; GW_ERR_ARG while the context's stream is being captured
 * (a memset node would be recorded). */
int gw_memset_zero(gw_context *ctx, void *dst, size_t bytes);
/* Enqueue-only device-to-device copy on the context stream (no wait). */
int gw_memcpy_dtod_async(gw_context *ctx, void *dst, const void *src, size_t bytes);

/* Seeded synthetic data on the device (counter-based: element i depends only
 * on (seed, i)).  Replaces the xorshift inputs of
 * DequantGEMVBenchmark.swift:35-54 for the large configurations.  One launch
 * fills `rows` runs of `count` elements whose starts are `row_stride` bytes
 * apart (one section of every expert of a layer, say); element i is
 * row * count + position, so rows == 1 is the plain contiguous fill.
 *  - bytes uniform over [lo, hi] inclusive;
 *  - normal(mean, std) written as f32, f16 or bf16 (RNE). */
int gw_fill_uniform_u8(gw_context *ctx, void *dst, size_t count, size_t rows,
                       size_t row_stride, int lo, int hi, uint64_t seed);
int gw_fill_normal(gw_context *ctx, void *dst, gw_dtype dtype, size_t count, size_t rows,
                   size_t row_stride, float mean, float std, uint64_t seed);

/* ---- expert weight layout (ExpertLayout, Install/InstallLayout.swift:14-121) */

/* Section order is ExpertLayout.Section (InstallLayout.swift:18-24). */
enum {
    GW_SECTION_GATE_UP_BLOCKS = 0,
    GW_SECTION_GATE_UP_SCALES = 1,
    GW_SECTION_DOWN_BLOCKS = 2,
    GW_SECTION_DOWN_SCALES = 3,
    GW_SECTION_GATE_UP_BIAS = 4,  /* bf16 [2F] */
    GW_SECTION_DOWN_BIAS = 5,     /* bf16 [H] */
    GW_SECTION_COUNT = 6
};

typedef struct gw_expert_layout {
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t expert_count;
    int64_t offsets[GW_SECTION_COUNT]; /* byte offset within one expert stride */
    int64_t sizes[GW_SECTION_COUNT];
    int64_t stride;                    /* page-aligned (16384) bytes per expert */
    int64_t page_size;
} gw_expert_layout;

/* ExpertLayout.init(hiddenSize:intermediateSize:expertCount:) — InstallLayout.swift:50-92.
 * Host-only; no device needed. */
int gw_expert_layout_init(int64_t hidden_size, int64_t intermediate_size,
                          int64_t expert_count, gw_expert_layout *out);

/* ---- kernel-level entry points (the Metal argument tables) ------------- */

/* mxfp4_dequant_reference / mxfp4_dequant_wide — Metal/Quant/mxfp4.metal:36-77.
 * `blocks` blocks -> out[blocks*32] fp32, bit-exact with MXFP4.decode
 * (MXFP4.swift:69-93): subnormal scales kept, 0xFF -> NaN, code 8 -> -0.0. */
int gw_mxfp4_dequant(gw_context *ctx, const uint8_t *packed, const uint8_t *scales,
                     int64_t blocks, float *out);

/* mxfp4_gemv — Metal/Quant/dequant_gemv.metal:37-67 (no bias).
 * y[r] = sum_b scale(r,b) * sum_i code(r,b,i) * x[32b+i], fp32 accumulation. */
int gw_mxfp4_gemv(gw_context *ctx, const uint8_t *packed, const uint8_t *scales,
                  const void *x, gw_dtype x_dtype, float *y, int64_t rows, int64_t cols);

/* mxfp4_gemv_bias{,_persistent,_staged,_lut,_multirow} — Metal/MoE/expert.metal:46-77,
 * 138-368: the GEMV plus bias[r] (bias_dtype GW_BF16 as in the .gwt layout, or
 * GW_F32; bias may be NULL = no bias). */
int gw_mxfp4_gemv_bias(gw_context *ctx, const uint8_t *packed, const uint8_t *scales,
                       const void *bias, gw_dtype bias_dtype, const void *x,
                       gw_dtype x_dtype, float *y, int64_t rows, int64_t cols);

/* gptoss_expert_activation (expert.metal:82-102) / expert_activation_swiglu
 * (expert.metal:380-393): interleaved fp32 gate_up[2*width] -> fp16 out[width]. */
int gw_expert_activation(gw_context *ctx, gw_activation kind, const float *gate_up,
                         uint16_t *out_f16, int64_t width, float limit, float alpha);

/* expert_accumulate — expert.metal:107-116: dst[i] += expert_out[i] * weight. */
int gw_expert_accumulate(gw_context *ctx, const float *expert_out, float *dst, float weight,
                         int64_t width);

/* bf16_gemv_bias — Metal/MoE/router.metal:18-34, as called by Router.logits
 * (Runtime/Router.swift:38-66): logits[t, e] = W[e,:] . x[t,:] + bias[e] for
 * `tokens` rows of x.  W is bf16 (reference) or f32; bias may be NULL. */
int gw_router_logits(gw_context *ctx, const void *weight, gw_dtype weight_dtype,
                     const void *bias, gw_dtype bias_dtype, const void *x, gw_dtype x_dtype,
                     float *logits, int64_t experts, int64_t hidden, int32_t tokens);

/* Router.select — Runtime/Router.swift:78-98, on the host: top_k by partial
 * selection sort (strict >, swapAt), softmax over the k selected logits.
 * ids highest-logit first. */
int gw_router_select(const float *logits, int64_t experts, int64_t top_k, int32_t *ids,
                     float *weights);

/* ---- ExpertRunner (Runtime/ExpertRunner.swift:10-363) ------------------ */

/* ExpertRunner.Weights (:54-64): one expert stride in device memory plus the
 * byte offsets of its six sections (ExpertRunner.sectionOffsets, :67-75). */
typedef struct gw_expert_weights {
    const uint8_t *buffer;
    int64_t offsets[GW_SECTION_COUNT];
} gw_expert_weights;

/* ExpertRunner.Assignment (:88-98). */
typedef struct gw_assignment {
    gw_expert_weights weights;
    int32_t token;
    float routing_weight;
} gw_assignment;

typedef struct gw_expert_runner gw_expert_runner;

/* ExpertRunner.init(context:reader:swigluLimit:swigluAlpha:) (:37-47).
 * limit/alpha are the model's activationLimit/activationAlpha (7.0 / 1.702 for
 * GPT-OSS, ArchitectureSpec.swift:102-104).  Bias sections are bf16 as written
 * by the installer; gw_expert_runner_set_bias_dtype switches to f32 sections,
 * and returns GW_ERR_SHAPE where the layout's bias pages cannot hold fp32
 * values (a gate_up bias of 2 x intermediate fp32 values must end before the
 * down bias section, the down bias before the expert stride: GPT-OSS's 5760
 * gate_up biases do not fit). */
int gw_expert_runner_create(gw_context *ctx, int64_t hidden_size, int64_t intermediate_size,
                            gw_activation activation, float swiglu_limit, float swiglu_alpha,
                            gw_expert_runner **out);
int gw_expert_runner_destroy(gw_expert_runner *runner);
int gw_expert_runner_set_bias_dtype(gw_expert_runner *runner, gw_dtype bias_dtype);
/* ExpertRunner.sectionOffsets (:67-75) for this runner's shape. */
int gw_expert_runner_section_offsets(gw_expert_runner *runner,
                                     int64_t offsets[GW_SECTION_COUNT]);

/* ExpertRunner.apply(_:weights:) (:275-331): one expert, one token, no routing
 * weight.  x [hidden] device, out [hidden] fp32 device (overwritten).  Blocks. */
int gw_expert_apply(gw_expert_runner *runner, const void *x, gw_dtype x_dtype,
                    const gw_expert_weights *weights, float *out);

/* ExpertRunner.applyBatch(_:experts:) (:191-269): out = sum_i w_i * expert_i(x),
 * accumulated in list order.  out [hidden] fp32 device (overwritten).  Blocks. */
int gw_expert_apply_batch(gw_expert_runner *runner, const void *x, gw_dtype x_dtype,
                          const gw_expert_weights *experts, const float *routing_weights,
                          int32_t count, float *out);

/* ExpertRunner.applyAssignments(inputs:assignments:outputs:) (:108-182):
 * outputs[token] += routing_weight * expert(inputs[token]) for every
 * assignment (in place; the caller zero-fills, TransformerLayer.swift:173).
 * inputs [tokens, hidden], outputs [tokens, hidden] fp32, device.  Each
 * distinct expert is read once per group of up to 8 tokens.  Blocks; the
 * _async variant only enqueues. */
int gw_expert_apply_assignments(gw_expert_runner *runner, const void *inputs,
                                gw_dtype x_dtype, const gw_assignment *assignments,
                                int32_t count, float *outputs);
int gw_expert_apply_assignments_async(gw_expert_runner *runner, const void *inputs,
                                      gw_dtype x_dtype, const gw_assignment *assignments,
                                      int32_t count, float *outputs);

/* ---- MoE block of TransformerLayer.forward (Runtime/TransformerLayer.swift:140-238) */

/* One layer's MoE block for `tokens` decode tokens, entirely on the
 * device: router (bf16_gemv_bias, or given logits) -> top-k + softmax
 * (Router.select) -> expert-major grouping (the demand map, :175-181) ->
 * fused gate_up + activation -> fused down + weighted combine.
 * Experts are HBM-resident at experts_base + e * expert_stride with the
 * runner's section offsets (the .gwt layer file, ExpertLayout).
 * out [tokens, hidden] fp32 is overwritten with the combined expert output
 * (the residual add stays with the caller, :232-238).  Batches of more than
 * 8 tokens run the grouped GEMMs of gw_moe_prefill_forward; so do batches of
 * 2..8 tokens (more than GODWIT_PREFILL_ABOVE at runner creation, default 1)
 * when hidden and intermediate sizes are multiples of 32 and >= 128, x is
 * 16-byte aligned, there are at most 256 experts and, during graph capture,
 * the prefill scratch is already reserved.  Batches of up to 12 tokens are
 * routed and grouped inside the grouped GEMMs themselves (every expert then
 * holds at most one 32-entry tile); GODWIT_SELF_GROUP_TOKENS at runner
 * creation (0..32, default 12) sets that bound, larger batches use the
 * group kernel's tile list.  Up to GODWIT_FUSED_COMBINE_TOKENS tokens (default
 * 32, 0 disables) the weighted combine runs inside the down GEMM instead of
 * a kernel of its own; results are the same bytes either way.  Enqueue only. */
typedef struct gw_moe_layer_args {
    const uint8_t *experts_base;
    int64_t expert_stride;
    int64_t expert_count;
    int64_t top_k;
    const float *logits;              /* [tokens, expert_count] or NULL -> router runs */
    const void *router_weight;        /* [expert_count, hidden] when logits == NULL */
    gw_dtype router_weight_dtype;
    const void *router_bias;          /* [expert_count] or NULL (Qwen3: no bias) */
    gw_dtype router_bias_dtype;
    const void *x;                    /* [tokens, hidden] */
    gw_dtype x_dtype;
    int32_t tokens;
    float *out;                       /* [tokens, hidden] fp32 */
    uint16_t *out_bf16;               /* optional bf16 copy of out (next layer's input) */
    int32_t *routing_ids;             /* optional [tokens, top_k] */
    float *routing_weights;           /* optional [tokens, top_k] */
} gw_moe_layer_args;

int gw_moe_layer_forward(gw_expert_runner *runner, const gw_moe_layer_args *args);

/* Batched prefill of the same MoE block for any number of tokens
 * (TransformerLayer.forward with T > 1, :140-238), as grouped GEMMs on the
 * matrix cores: route every token, sort the T*k (token, rank) entries by
 * expert (the demand map, :175-181), run each expert's gate_up and down over
 * its whole token group (weights widened exactly to bf16 with the block
 * scale folded in; activations as exact sums of bf16 parts; fp32
 * accumulation), then combine each token's experts in router order.  Same
 * arguments as gw_moe_layer_forward; up to 256 experts.  Scratch grows on
 * demand (or up front with gw_expert_runner_reserve_prefill, which a caller
 * about to capture a graph must use).  gw_moe_layer_forward itself sends
 * batches of more than 8 tokens here, and smaller batches as it describes.
 * Enqueue only. */
int gw_expert_runner_reserve_prefill(gw_expert_runner *runner, int32_t max_tokens, int32_t top_k,
                                     int32_t expert_count);
int gw_moe_prefill_forward(gw_expert_runner *runner, const gw_moe_layer_args *args);

/* Inspection, no counterpart in the reference (the Metal runner exposes its
 * intermediate buffers to its own tests the same way): device pointers into
 * this runner's prefill scratch as the last batch through it left them
 * (gw_moe_prefill_forward, or gw_moe_layer_forward / gw_moe_block_forward on
 * the grouped GEMMs), valid until the next such call.  Entry j = token *
 * top_k + rank.  activations: fp16 [tokens * top_k][intermediate], each
 * entry's activation as the reference rounds it (activation_plane is 0: one
 * plane); expert_outputs: [tokens * top_k][hidden] fp32, down
 * projection plus bias, before the weighted combine.  Returns GW_ERR_ARG
 * before the first batch. */
typedef struct gw_prefill_view {
    const int32_t *routing_ids;        /* [tokens * top_k] */
    const float *routing_weights;      /* [tokens * top_k] */
    const uint16_t *activations;
    int64_t activation_plane;          /* 0: the activations are one plane */
    const float *expert_outputs;
    int32_t tokens, top_k;
} gw_prefill_view;
int gw_expert_runner_prefill_view(gw_expert_runner *runner, gw_prefill_view *view);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): gw_moe_prefill_forward with its scratch (routing ids and
 * weights, the tile list, the split x planes, the fp16 activations, the
 * expert outputs, the combine counters) carved from a fixed per-device array
 * of GW_STATIC_SCRATCH_BYTES instead of the runner's reserved buffer.  It
 * calls no allocator (with profiling off).  A batch whose scratch exceeds the
 * array returns GW_ERR_SHAPE: about 90 tokens of GPT-OSS-120B (2880 x 2880,
 * top-4) or 88 of Qwen3-30B-A3B fit.  Same arguments and results, byte for
 * byte, as gw_moe_prefill_forward.  Every call on one device shares that
 * device's array and leaves its contents behind: calls that overlap on one GPU
 * (two streams, two runners, two threads) race, and the caller serialises
 * them.  Enqueue only. */
#define GW_STATIC_SCRATCH_BYTES ((size_t)8 << 20)
int gw_moe_prefill_forward_static(gw_expert_runner *runner, const gw_moe_layer_args *args);

/* ---- .gwt installations ---------------------------------------------------
 * A .gwt install is a directory with manifest.json (GodwitManifest,
 * Install/GodwitManifest.swift:8-105) and experts/layer_NN.bin, each
 * expertCount strides of expertStride bytes in ExpertLayout section order
 * (Install/InstallLayout.swift:14-121).  gw_model_open replaces ModelReader.init
 * (Runtime/ModelReader.swift:17-37: manifest required, format version 2);
 * gw_model_validate is GodwitManifest.validate (:79-104, layer file sizes);
 * gw_model_load_layer / _load_expert replace ModelReader.loadExpertStride and
 * read (:72-110): pread into pinned staging, copied to HBM by the context's
 * stream; they return when the bytes are on the device.  The loaded layer is
 * the experts_base of gw_moe_layer_forward, unchanged bytes.  A gw_model keeps
 * its two 32 MiB pinned staging buffers from the first load until
 * gw_model_close, so loads through one handle must not overlap (use one handle
 * per loading thread). */
#define GW_GWT_FORMAT_VERSION 2

typedef struct gw_model gw_model;

typedef struct gw_model_info {
    int64_t format_version;
    int64_t layer_count;              /* installed layers */
    int64_t expert_count;
    int64_t expert_stride;            /* bytes per expert within a layer file */
    int64_t section_offset[GW_SECTION_COUNT];   /* ExpertLayout.Section order */
    int64_t section_length[GW_SECTION_COUNT];
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t experts_per_token;        /* largest spec.layers[].expertsPerToken */
    float rms_norm_epsilon;
    float activation_limit;           /* spec.activationLimit (default 7.0) */
    float activation_alpha;           /* spec.activationAlpha (default 1.702) */
    gw_activation activation;         /* spec.activation */
    int32_t expert_bias;              /* spec.expertBias (default false) */
    int32_t router_bias;              /* spec.routerBias (default false) */
} gw_model_info;

int gw_model_open(const char *directory, gw_model **out);
int gw_model_close(gw_model *model);
int gw_model_info_get(const gw_model *model, gw_model_info *info);
int gw_model_validate(const gw_model *model);
int gw_model_load_layer(gw_context *ctx, gw_model *model, int32_t layer, void *device_dst,
                        size_t capacity);
int gw_model_load_expert(gw_context *ctx, gw_model *model, int32_t layer, int32_t expert,
                         void *device_dst);

/* The MoE block with the steps either side of it (TransformerLayer.forward,
 * TransformerLayer.swift:140-143 and 232-238): normed = RMSNorm(stream) in fp16
 * (TransformerLayer.normalise, :265-285; rmsnorm, router.metal:36-60: the sum
 * of squares in fp32, x * rsqrt(mean + eps) * weight), then the block of
 * gw_moe_layer_forward on `normed` (the router, when logits is NULL, sees it
 * too), then stream += the combined expert output, in fp32, the sum finished
 * before it is added.  `layer.x`, `layer.x_dtype` and `layer.out` are ignored;
 * `layer.out_bf16`, when set, receives a bf16 copy of the updated stream.
 * Batches take the prefill path as in gw_moe_layer_forward (reserve it
 * before capture).  Enqueue only. */
typedef struct gw_moe_block_args {
    gw_moe_layer_args layer;
    float *stream;                    /* [tokens, hidden] fp32 residual stream, in place */
    const void *norm_weight;          /* [hidden] post-attention norm weight */
    gw_dtype norm_weight_dtype;       /* GW_BF16 (the .gwt trunk) or GW_F32 */
    float epsilon;                    /* ArchitectureSpec.rmsNormEpsilon (1e-5 GPT-OSS) */
} gw_moe_block_args;

int gw_moe_block_forward(gw_expert_runner *runner, const gw_moe_block_args *args);

/* For one token (the decode step of a single sequence) with 16-bit x the
 * layer above runs as ONE kernel, one workgroup per compute unit, whose
 * workgroups exchange the activations through device memory.  Eligible:
 * 16-bit x, top-k <= 8, up to 256 experts, and either GPT-OSS-class rows
 * (hidden and intermediate both 65..96 blocks of 32) with top-k <= 4, or
 * Qwen3-class rows (hidden 25..64 blocks, intermediate 9..24 blocks); other
 * cases, and GODWIT_DECODE_LAYER=0 in the environment when the runner is
 * created, use a gate_up and a down kernel.  Given router weights instead of
 * logits (up to 128 experts, 16-byte aligned weights and x, and the CU count
 * a multiple of expert_count with each logit's hidden / (CUs / experts)
 * slice whole 8-element units, at most 2048), the kernel computes the
 * logits too: each workgroup dots one slice of one weight row, the grid
 * exchanges the partials and every workgroup adds each logit's partials in
 * slice order plus the bias.  The standalone router adds the same slices in
 * the same order for one 16-bit token, so both forms route alike.
 *
 * Co-residency contract: the kernel's workgroups wait for each other, so all
 * of them must run at once.  The host checks that one workgroup fits each
 * compute unit of an idle device; nothing else may run on the GPU during a
 * one-token layer (no other stream, runner or process).  With
 * GODWIT_DECODE_COOP=1 in the environment when the context is created the
 * kernel goes through hipLaunchCooperativeKernel, whose runtime refuses a
 * grid that cannot be resident at once (it captures into graphs, but costs
 * about 18 us a launch on MI355X with ROCm 7, so it is off by default).  The waits are
 * bounded: a wait that gives up is counted instead of hanging the device,
 * and that launch's outputs are invalid.  gw_context_synchronize then
 * returns GW_ERR_EXCHANGE, and the runner runs later one-token layers with
 * the two-kernel form, which has no such wait.
 *
 * No counterpart in the reference (there the command buffer's encoder
 * boundaries order the stages).  Blocks until the runner's stream is idle
 * (GW_ERR_ARG during graph capture); *count is the number of waves whose
 * wait gave up since the runner was created (0 when every result is valid). */
int gw_expert_runner_sync_errors(gw_expert_runner *runner, uint32_t *count);

/* The bounded wait of the one-token layer: polls of the exchange before a
 * wait gives up (0 restores the default, 2^18, some milliseconds).  Waits on
 * a workgroup's own waves keep the fixed 2^18 bound whatever is set here.  No
 * counterpart in the reference. */
int gw_expert_runner_set_wait_limit(gw_expert_runner *runner, uint32_t polls);

/* Test hook for the failure path above: with enable != 0 the one-token
 * layer's workgroups read an exchange slot that no launch writes, so every
 * wait runs to its limit and gives up while every kernel still exits
 * normally.  Never set in normal use.  No counterpart in the reference. */
int gw_expert_runner_inject_exchange_fault(gw_expert_runner *runner, int enable);

/* ---- graphs (replace per-call command buffers with one replayable graph) */

typedef struct gw_graph gw_graph;
/* Starts stream capture on the context's stream; calls until end_capture are
 * recorded, not run (only enqueue-only calls may be captured). */
int gw_graph_begin_capture(gw_context *ctx);
int gw_graph_end_capture(gw_context *ctx, gw_graph **out);
int gw_graph_launch(gw_graph *graph);
int gw_graph_destroy(gw_graph *graph);

#if defined(__GNUC__) || defined(__clang__)
#pragma GCC visibility pop
#endif

#ifdef __cplusplus
}
#endif
#endif
