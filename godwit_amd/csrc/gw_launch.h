// gw_launch.h — host-side launchers of the gfx950 kernels (gw_kernels.hip).
// Internal to libgodwit_hip.so; the public surface is include/godwit_hip.h.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gw_plan.h"

namespace gw {

// Launches on the Launch's stream; when the Launch carries a start/stop event
// pair (profiling), they are attached to the kernel's own dispatch, so they
// time the kernel alone, not the gaps around it.
#define GW_LAUNCH(KERNEL, GRID, BLOCK, LDS, L, ...)                                          \
    do {                                                                                      \
        if ((L).ev_start)                                                                     \
            hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, (L).stream, (L).ev_start,          \
                                  (L).ev_stop, 0, __VA_ARGS__);                               \
        else                                                                                  \
            hipLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, (L).stream, __VA_ARGS__);            \
    } while (0)

struct Launch {
    hipStream_t stream;
    int cus;        // compute units of the device
    int grid_a;     // workgroups of the gate_up kernel (0 = default)
    int grid_b;     // workgroups of the down kernel (0 = default)
    hipEvent_t ev_start = nullptr;   // set: recorded by the kernel's dispatch (profiling)
    hipEvent_t ev_stop = nullptr;
    int coop = 0;   // one-token layer through hipLaunchCooperativeKernel
};

// Device routing from logits (Router.select + the demand map), done by the
// route kernel or fused into the gate_up kernel's prologue.
struct RouteArgs {
    const float *logits;          // [tokens, experts]; null = the plan is given
    int experts, top_k, tokens;
    const uint8_t *experts_base;  // expert e at experts_base + e * stride
    int64_t stride;
    int32_t *ids_out;             // optional [tokens, top_k]
    float *w_out;                 // optional [tokens, top_k]
};

// State of the fused layer kernel's in-kernel exchange (owned by a runner).
struct SyncArgs {
    unsigned *counters;   // 16 counters, 4352 bytes apart
    unsigned *epochs;     // per workgroup: launches it has completed
    unsigned *err;        // nonzero once a bounded wait gave up
};
constexpr int kSyncWords = 16 * 1088;

// Lanes per row and blocks per lane chosen for a row of `bpr` MXFP4 blocks.
struct RowShape { int tpr; int m; int chunks; };
RowShape row_shape(int bpr);

hipError_t launch_dequant(const Launch &L, const uint8_t *packed, const uint8_t *scales,
                          int64_t blocks, float *out);
hipError_t launch_gemv(const Launch &L, const uint8_t *packed, const uint8_t *scales,
                       const void *bias, int bias_dt, const void *x, int x_dt, float *y,
                       int rows, int cols);
hipError_t launch_activation(const Launch &L, int kind, const float *gate_up, uint16_t *out,
                             int64_t width, float limit, float alpha);
hipError_t launch_rmsnorm(const Launch &L, const float *x, const void *weight, int w_dt,
                          int rows, int width, float eps, uint16_t *out);
hipError_t launch_accumulate(const Launch &L, const float *src, float *dst, float w,
                             int64_t width);
hipError_t launch_router(const Launch &L, const void *W, int w_dt, const void *b, int b_dt,
                         const void *x, int x_dt, float *logits, int experts, int hidden,
                         int tokens);
hipError_t launch_route(const Launch &L, const RouteArgs &route, Plan *plan);
// route == null: the plan is read from `plan`; otherwise every workgroup routes
// and workgroup 0 writes the plan to `plan` for the down kernel.
hipError_t launch_gate_up(const Launch &L, Plan *plan, const RouteArgs *route, int max_tokens,
                          const void *x, int x_dt, int hidden, int inter, const Sections &sec,
                          int bias_dt, uint16_t *act, int act_kind, float limit, float alpha);
constexpr int kFusedRouteExperts = 256;
hipError_t launch_down(const Launch &L, const Plan *plan, int max_tokens, int max_slots,
                       const uint16_t *act, int hidden, int inter, const Sections &sec,
                       int bias_dt, float *out, uint16_t *out_bf16, int accumulate);
// ---- one-token layer in one kernel (gw_decode.hip)

constexpr int kSyncEpochCapacity = 8192;      // per-workgroup epochs a runner keeps
constexpr int kDecodeLdsMax = 160 * 1024;     // LDS of one gfx950 compute unit
constexpr int kDecodeMaxGrid = 256;           // workgroups of the one-kernel layer at most
// The one-kernel layer's exchange: launches alternate between two slots of
// 8-byte activation words (four fp16 each); a third slot is never written.
constexpr int kDecodeXchgSlotBytes = 256 * 1024;
// three activation slots, then three slots of router partials (one word a workgroup)
constexpr int kDecodeXchgBytes = 3 * kDecodeXchgSlotBytes + 3 * kDecodeMaxGrid * 8;
constexpr uint32_t kDecodeSpinLimit = 1u << 18;   // polls before a wait gives up

struct DecodeArgs {
    const float *logits;          // [experts] router logits of the token
    int experts, top_k;
    const uint8_t *base;          // expert e at base + e * stride
    int64_t stride;
    uint32_t base_bytes;          // experts * stride (< 2^31: 32-bit buffer offsets)
    int32_t *ids_out;             // optional [top_k]
    float *w_out;                 // optional [top_k]
    const void *x;                // [hidden] bf16 or fp16
    int hidden, inter;
    Sections sec;
    int bias_dt;                  // -1: none
    uint64_t *xchg;               // kDecodeXchgBytes of activation words; all ones initially
    int act_kind;
    float limit, alpha;
    float *out;                   // [hidden]
    uint16_t *out_bf16;           // optional bf16 copy of out
    int accumulate;               // 0 overwrite, 1 add to out, 2 residual: out += sum
    SyncArgs sync;
    int nrmax;                    // most down rows a workgroup owns (ceil(hidden / grid))
    uint32_t spin_limit;          // polls of the exchange before a wait gives up
    int poll_fault;               // 1: read the never-written slot (tests the give-up path)
    // In-kernel router (rw != null, logits unused): workgroup b computes the
    // partial (b / rslices, b % rslices) of router_partial, the grid exchanges
    // them and every workgroup adds each logit's rslices partials in order.
    const void *rw;               // [experts, hidden] router weights
    int rw_dt;
    const void *rb;               // optional [experts] router bias
    int rb_dt;
    int rslices;
};
struct DecodeLds { int route, xs, actl, dma, scl, part, bx, total; };

// Grid (one workgroup per CU) of the one-kernel layer for this shape, or 0
// when it is not available (shape, dtype or top-k not built, LDS, or the grid
// cannot be resident).  Fills args->nrmax / base_bytes and the LDS size.
int decode_layer_plan(const Launch &L, int hidden, int inter, int x_dt, int top_k, int experts,
                      int64_t stride, int bias_dt, DecodeArgs *args, size_t *lds_bytes);
hipError_t launch_decode_layer(const Launch &L, int grid, size_t lds, int x_dt,
                               const DecodeArgs &a);
// ---- prefill (batched tokens) on the matrix cores

// One grouped GEMM launch (gate_up or down) over the work items of a grouping.
struct PrefillGemm {
    const int32_t *tiles, *ntiles, *offsets, *order;
    const uint16_t *in;           // bf16 planes of [rows, kdim] (down: one fp16 plane)
    int64_t in_plane;             // elements between planes
    int in_row_div;               // entry -> input row divisor (top_k for x, 1 for act)
    const uint8_t *experts_base;
    int64_t stride;
    int64_t blocks_off, scales_off, bias_off;
    int bias_dt;                  // -1: none
    int kdim, fdim;
    uint16_t *act_out;            // gate_up: fp16 activations [entries, fdim/2]
    float *y_out;                 // down: [entries, fdim] fp32
    int act_kind;
    float limit, alpha;
    // Self-grouped batch (sg_tokens > 0): the GEMM builds its own work list;
    // gate_up routes from sg_logits and writes sg_ids_out / sg_w_out, down
    // reads sg_ids.  tiles / ntiles / offsets / order are then unused.
    int sg_tokens = 0, sg_topk = 0, sg_experts = 0;
    const float *sg_logits = nullptr;
    const int32_t *sg_ids = nullptr;
    int32_t *sg_ids_out = nullptr;
    float *sg_w_out = nullptr;
    // Forced workgroup shape (waves 8 or 12, ring depth 2 or 4; 0: chosen per
    // launch).  12 waves run 4 deep and three activation planes 2 deep
    // whatever is asked; a shape whose LDS does not fit is not forced.  Same
    // results either way.
    int force_waves = 0, force_depth = 0;
    // Down launch with the combine fused in (arrive != null): arrive holds
    // arrive_count zeroed counters (left zeroed), one per token and feature
    // tile of the chosen shape (prefill_arrive_count covers every shape),
    // y_bytes the size of y_out, and the combine writes out [comb_tokens,
    // fdim] (+ out_bf16) from weights [comb_tokens, K], adding to out when
    // residual.
    uint32_t *arrive = nullptr;
    int64_t arrive_count = 0;
    int comb_tokens = 0;
    int64_t y_bytes = 0;
    const float *comb_w = nullptr;
    float *comb_out = nullptr;
    uint16_t *comb_out_bf16 = nullptr;
    int comb_topk = 0, comb_residual = 0;
};
int prefill_max_tiles(int T, int K, int E);
// Combine counters for T tokens of a down GEMM with fdim output rows: one per
// token and feature tile of the narrowest built shape.
int64_t prefill_arrive_count(int T, int fdim);
// True when the down GEMM of a batch (fdim output rows, K = kdim, tiles_hint
// entries, max_tiles work items) runs the 4-wave shape: the shape that keeps
// the fused combine cheap.
bool prefill_down_four_wave(int fdim, int kdim, int tiles_hint, int max_tiles, int cus);
// True when a batch is small enough for the self-grouped GEMMs (every expert
// at most one 32-entry tile); max_tiles is then min(E, T*K).
bool prefill_self_groups(int T, int K, int E);
int prefill_planes(int in_dt);        // bf16 planes that hold a dtype exactly: 1, 2 or 3
int prefill_gemm_lds_bytes(int planes, int kdim, int waves, int depth);
hipError_t launch_prefill_route(const Launch &L, const float *logits, int T, int E, int K,
                                int32_t *ids, float *weights);
// True when launch_prefill_group can route the batch itself (logits given).
bool prefill_routes_in_group(int T, int K);
// Groups entries t*K+k by expert.  With logits non-null it first routes the
// batch (writing ids and weights), which needs prefill_routes_in_group(T, K);
// with logits null it reads ids written by launch_prefill_route.
hipError_t launch_prefill_group(const Launch &L, const float *logits, int T, int K, float *weights,
                                int32_t *ids, int E, int32_t *offsets, int32_t *order,
                                int32_t *tiles, int32_t *ntiles, int max_tiles);
hipError_t launch_prefill_split(const Launch &L, const void *in, int in_dt, int64_t n,
                                uint16_t *out);
// tiles_hint: an upper bound on the work list's length (the entry count for
// small batches), used to size the workgroups.
hipError_t launch_prefill_gemm(const Launch &L, bool gate_up, int planes, const PrefillGemm &g,
                               int max_tiles, int tiles_hint);
hipError_t launch_prefill_combine(const Launch &L, const float *y, const float *w, int T, int K,
                                  int H, float *out, uint16_t *out_bf16, int residual);

hipError_t launch_fill_u8(const Launch &L, void *dst, size_t count, size_t rows,
                          size_t row_stride, int lo, int hi, uint64_t seed);
hipError_t launch_fill_normal(const Launch &L, void *dst, int dt, size_t count, size_t rows,
                              size_t row_stride, float mean, float stddev, uint64_t seed);

// LDS bytes the down kernel needs per slot of staged activations and the
// fixed part; used by the host to bound slots per chunk.
int down_lds_bytes(int hidden, int inter, int grid, int smax);
int gate_up_lds_bytes(int hidden, int x_dt, int max_tokens);

constexpr int kLdsBudget = 64 * 1024;

}  // namespace gw
