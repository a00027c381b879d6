// gw_api.hip — the C ABI of libgodwit_hip.so (declared in include/godwit_hip.h).
//
// Host-side mirror of the reference's engine API: MetalContext ->
// gw_context, ExpertRunner -> gw_expert_runner, Router -> gw_router_*,
// TransformerLayer's MoE block -> gw_moe_layer_forward.  Plans (the device
// form of the demand map) are built here for the host-driven calls and by the
// route kernel for the device-driven layer call.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/godwit_hip.h"
#include "gw_error.h"
#include "gw_host.h"
#include "gw_launch.h"
#include "gw_plan.h"

using gw::HostPlan;
using gw::Plan;
using gw::plan_add;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------

#define fail gw::set_error

#define GW_HIP(call)                                                                     \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess)                                                            \
            return fail(e_ == hipErrorOutOfMemory ? GW_ERR_OOM : GW_ERR_HIP, "%s: %s (%s:%d)", \
                        #call, hipGetErrorString(e_), __FILE__, __LINE__);               \
    } while (0)

#define GW_CHECK(cond, code, ...) \
    do {                          \
        if (!(cond)) return fail(code, __VA_ARGS__); \
    } while (0)

extern "C" const char *gw_version(void) { return "godwit_hip 0.1 (gfx950)"; }

static bool dtype_ok(int dt) { return dt == GW_F32 || dt == GW_F16 || dt == GW_BF16; }
static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

struct ProfEvent {
    const char *name;
    hipEvent_t start, end;
};

struct gw_context {
    int device = 0;
    hipStream_t stream = nullptr;
    int cus = 0;
    int grid_a = 0, grid_b = 0;
    int coop = 0;
    bool capturing = false;
    bool profiling = false;
    std::vector<ProfEvent> events;       // recorded pairs, in order
    std::vector<hipEvent_t> event_pool;  // reusable events
    std::vector<std::pair<std::string, std::pair<double, int64_t>>> totals;
    std::vector<gw_expert_runner *> runners;   // checked for failed exchanges at synchronize
};

// True while the context's stream is being captured, by gw_graph_begin_capture
// or by a caller's own capture of that stream.
static bool is_capturing(const gw_context *ctx)
{
    if (ctx->capturing) return true;
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(ctx->stream, &st) == hipSuccess &&
           st == hipStreamCaptureStatusActive;
}

static gw::Launch launch_of(gw_context *ctx)
{
    gw::Launch L;
    L.stream = ctx->stream;
    L.cus = ctx->cus;
    L.grid_a = ctx->grid_a;
    L.grid_b = ctx->grid_b;
    L.coop = ctx->coop;
    return L;
}

static hipEvent_t take_event(gw_context *ctx)
{
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// Brackets one launch with events when profiling (never inside a capture).
// Times one kernel launch under a name.  launch(L) hands the launcher an
// event pair that the kernel's own dispatch records (hipExtLaunchKernel), so
// the figure is the kernel's duration, without the gaps that separate event
// packets would add around it.
struct ProfScope {
    gw_context *ctx;
    const char *name;
    hipEvent_t start = nullptr, end = nullptr;
    ProfScope(gw_context *c, const char *n) : ctx(c), name(n) {}
    gw::Launch launch(gw::Launch L)
    {
        if (ctx->profiling && !is_capturing(ctx) && !start) {
            start = take_event(ctx);
            end = start ? take_event(ctx) : nullptr;
            if (start && end) {
                L.ev_start = start;
                L.ev_stop = end;
            }
        }
        return L;
    }
    ~ProfScope()
    {
        if (start && end) ctx->events.push_back({name, start, end});
        else if (start) ctx->event_pool.push_back(start);
    }
};

static int get_env_int(const char *name, int dflt)
{
    const char *v = getenv(name);
    return v ? atoi(v) : dflt;
}

extern "C" int gw_device_count(int *count)
{
    GW_CHECK(count, GW_ERR_ARG, "count is null");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return GW_OK;
}

// The allocation-free prefill's scratch (gw_moe_prefill_forward_static): one
// copy of this array per device.  Host code never uses its name as an
// address: gw_context_create resolves each device's copy once, with that
// device current, into g_scratch_ptr.
static __device__ __align__(256) unsigned char scratch[GW_STATIC_SCRATCH_BYTES];
static constexpr int kScratchDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kScratchDevices] = {};

extern "C" int gw_context_create(int device, gw_context **out)
{
    GW_CHECK(out, GW_ERR_ARG, "out is null");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(GW_ERR_NO_DEVICE, "no HIP device visible");
    GW_CHECK(device >= 0 && device < n, GW_ERR_NO_DEVICE, "device %d out of range (%d)", device,
             n);
    GW_HIP(hipSetDevice(device));
    hipDeviceProp_t prop;
    GW_HIP(hipGetDeviceProperties(&prop, device));
    if (device < kScratchDevices) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_ptr[device]) {
            void *p = nullptr;
            GW_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
            g_scratch_ptr[device] = p;
        }
    }
    gw_context *ctx = new gw_context();
    ctx->device = device;
    ctx->cus = prop.multiProcessorCount;
    ctx->grid_a = get_env_int("GODWIT_GRID_A", 0);
    ctx->grid_b = get_env_int("GODWIT_GRID_B", 0);
    ctx->coop = get_env_int("GODWIT_DECODE_COOP", 0);
    hipError_t e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return fail(GW_ERR_HIP, "hipStreamCreate: %s", hipGetErrorString(e));
    }
    *out = ctx;
    return GW_OK;
}

static void release_events(gw_context *ctx)
{
    for (auto &p : ctx->events) {
        ctx->event_pool.push_back(p.start);
        ctx->event_pool.push_back(p.end);
    }
    ctx->events.clear();
}

extern "C" int gw_context_destroy(gw_context *ctx)
{
    if (!ctx) return GW_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    release_events(ctx);
    for (hipEvent_t e : ctx->event_pool) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return GW_OK;
}

static int check_exchanges(gw_context *ctx);

extern "C" int gw_context_synchronize(gw_context *ctx)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(!is_capturing(ctx), GW_ERR_ARG, "synchronize during graph capture");
    GW_HIP(hipStreamSynchronize(ctx->stream));
    return check_exchanges(ctx);
}

extern "C" void *gw_context_stream(gw_context *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" int gw_context_cu_count(gw_context *ctx, int *cus)
{
    GW_CHECK(ctx && cus, GW_ERR_ARG, "null argument");
    *cus = ctx->cus;
    return GW_OK;
}

extern "C" int gw_context_set_profiling(gw_context *ctx, int enabled)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    ctx->profiling = enabled != 0;
    return GW_OK;
}

static int collect_events(gw_context *ctx)
{
    if (ctx->events.empty()) return GW_OK;
    GW_HIP(hipStreamSynchronize(ctx->stream));
    for (auto &p : ctx->events) {
        float ms = 0.0f;
        // A launcher that returned before launching (empty input) left its
        // events unrecorded: that entry is skipped.
        if (hipEventElapsedTime(&ms, p.start, p.end) != hipSuccess) {
            (void)hipGetLastError();
            continue;
        }
        bool found = false;
        for (auto &t : ctx->totals) {
            if (t.first == p.name) {
                t.second.first += ms;
                t.second.second += 1;
                found = true;
                break;
            }
        }
        if (!found) ctx->totals.push_back({p.name, {(double)ms, 1}});
    }
    release_events(ctx);
    return GW_OK;
}

extern "C" int gw_context_profile_read(gw_context *ctx, const char *name, double *total_ms,
                                       int64_t *launches)
{
    GW_CHECK(ctx && name && total_ms && launches, GW_ERR_ARG, "null argument");
    int rc = collect_events(ctx);
    if (rc) return rc;
    *total_ms = 0.0;
    *launches = 0;
    for (auto &t : ctx->totals)
        if (t.first == name) {
            *total_ms = t.second.first;
            *launches = t.second.second;
        }
    return GW_OK;
}

extern "C" int gw_context_profile_reset(gw_context *ctx)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    int rc = collect_events(ctx);
    ctx->totals.clear();
    return rc;
}

// ---------------------------------------------------------------------------
// memory
// ---------------------------------------------------------------------------

// A failed allocation: the status (GW_ERR_OOM for out-of-memory), and the
// runtime's last-error record cleared, so that the next launch's
// hipGetLastError does not report this failure again.
static int alloc_failed(hipError_t e, const char *what, size_t bytes)
{
    (void)hipGetLastError();
    return fail(e == hipErrorOutOfMemory ? GW_ERR_OOM : GW_ERR_HIP, "%s(%zu): %s", what, bytes,
                hipGetErrorString(e));
}

extern "C" int gw_malloc(gw_context *ctx, size_t bytes, void **out)
{
    GW_CHECK(ctx && out, GW_ERR_ARG, "null argument");
    *out = nullptr;
    if (bytes == 0) return GW_OK;
    GW_HIP(hipSetDevice(ctx->device));
    hipError_t e = hipMalloc(out, bytes);
    if (e != hipSuccess) {
        *out = nullptr;
        return alloc_failed(e, "hipMalloc", bytes);
    }
    return GW_OK;
}

extern "C" int gw_free(gw_context *ctx, void *ptr)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    if (!ptr) return GW_OK;
    GW_HIP(hipFree(ptr));
    return GW_OK;
}

static int copy(gw_context *ctx, void *dst, const void *src, size_t n, hipMemcpyKind kind)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    if (n == 0) return GW_OK;
    GW_CHECK(dst && src, GW_ERR_ARG, "null pointer");
    GW_CHECK(!is_capturing(ctx), GW_ERR_ARG, "blocking copy during graph capture");
    GW_HIP(hipMemcpyAsync(dst, src, n, kind, ctx->stream));
    GW_HIP(hipStreamSynchronize(ctx->stream));
    return GW_OK;
}

extern "C" int gw_memcpy_htod(gw_context *ctx, void *dst, const void *src, size_t bytes)
{ return copy(ctx, dst, src, bytes, hipMemcpyHostToDevice); }
extern "C" int gw_memcpy_dtoh(gw_context *ctx, void *dst, const void *src, size_t bytes)
{ return copy(ctx, dst, src, bytes, hipMemcpyDeviceToHost); }
extern "C" int gw_memcpy_dtod(gw_context *ctx, void *dst, const void *src, size_t bytes)
{ return copy(ctx, dst, src, bytes, hipMemcpyDeviceToDevice); }

extern "C" int gw_memcpy_dtod_async(gw_context *ctx, void *dst, const void *src, size_t bytes)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    if (bytes == 0) return GW_OK;
    GW_CHECK(dst && src, GW_ERR_ARG, "null pointer");
    GW_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return GW_OK;
}

extern "C" int gw_memset_zero(gw_context *ctx, void *dst, size_t bytes)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    if (bytes == 0) return GW_OK;
    GW_CHECK(dst, GW_ERR_ARG, "null pointer");
    GW_CHECK(!is_capturing(ctx), GW_ERR_ARG, "memset during graph capture");
    GW_HIP(hipMemsetAsync(dst, 0, bytes, ctx->stream));
    GW_HIP(hipStreamSynchronize(ctx->stream));
    return GW_OK;
}

extern "C" int gw_fill_uniform_u8(gw_context *ctx, void *dst, size_t count, size_t rows,
                                  size_t row_stride, int lo, int hi, uint64_t seed)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(count == 0 || rows == 0 || dst, GW_ERR_ARG, "null pointer");
    GW_CHECK(rows <= 65535 && (rows <= 1 || row_stride >= count), GW_ERR_ARG,
             "rows %zu (at most 65535) of %zu bytes need a stride of at least that (got %zu)",
             rows, count, row_stride);
    GW_CHECK(lo >= 0 && hi <= 255 && lo <= hi, GW_ERR_ARG, "bad range [%d, %d]", lo, hi);
    ProfScope ps(ctx, "fill");
    GW_HIP(gw::launch_fill_u8(ps.launch(launch_of(ctx)), dst, count, rows, row_stride, lo, hi,
                              seed));
    return GW_OK;
}

extern "C" int gw_fill_normal(gw_context *ctx, void *dst, gw_dtype dtype, size_t count,
                              size_t rows, size_t row_stride, float mean, float stddev,
                              uint64_t seed)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(count == 0 || rows == 0 || dst, GW_ERR_ARG, "null pointer");
    GW_CHECK(dtype_ok(dtype), GW_ERR_ARG, "bad dtype %d", (int)dtype);
    const size_t esz = dtype == GW_F32 ? 4 : 2;
    GW_CHECK(rows <= 65535 && (rows <= 1 || (row_stride >= count * esz && row_stride % esz == 0)),
             GW_ERR_ARG, "rows %zu (at most 65535) of %zu elements need a stride of at least "
             "that many bytes, a multiple of the element size (got %zu)", rows, count, row_stride);
    ProfScope ps(ctx, "fill");
    GW_HIP(gw::launch_fill_normal(ps.launch(launch_of(ctx)), dst, dtype, count, rows, row_stride,
                                  mean, stddev, seed));
    return GW_OK;
}

// ---------------------------------------------------------------------------
// layout (ExpertLayout, InstallLayout.swift:50-92)
// ---------------------------------------------------------------------------

extern "C" int gw_expert_layout_init(int64_t hidden_size, int64_t intermediate_size,
                                     int64_t expert_count, gw_expert_layout *out)
{
    GW_CHECK(out, GW_ERR_ARG, "out is null");
    GW_CHECK(hidden_size > 0 && intermediate_size > 0 && expert_count > 0, GW_ERR_ARG,
             "sizes must be positive");
    GW_CHECK(hidden_size % 32 == 0 && intermediate_size % 32 == 0, GW_ERR_SHAPE,
             "hidden (%lld) and intermediate (%lld) must be multiples of 32",
             (long long)hidden_size, (long long)intermediate_size);
    const int64_t page = 16384;
    const int64_t gate_up_rows = 2 * intermediate_size;
    const int64_t down_rows = hidden_size;
    const int64_t bpr = hidden_size / 32;
    int64_t sizes[GW_SECTION_COUNT];
    sizes[GW_SECTION_GATE_UP_BLOCKS] = gate_up_rows * bpr * 16;
    sizes[GW_SECTION_GATE_UP_SCALES] = gate_up_rows * bpr;
    sizes[GW_SECTION_DOWN_BLOCKS] = down_rows * (intermediate_size / 32) * 16;
    sizes[GW_SECTION_DOWN_SCALES] = down_rows * (intermediate_size / 32);
    sizes[GW_SECTION_GATE_UP_BIAS] = gate_up_rows * 2;
    sizes[GW_SECTION_DOWN_BIAS] = down_rows * 2;
    int64_t cursor = 0;
    for (int s = 0; s < GW_SECTION_COUNT; ++s) {
        cursor = (cursor + page - 1) / page * page;
        out->offsets[s] = cursor;
        out->sizes[s] = sizes[s];
        cursor += sizes[s];
    }
    out->stride = (cursor + page - 1) / page * page;
    out->hidden_size = hidden_size;
    out->intermediate_size = intermediate_size;
    out->expert_count = expert_count;
    out->page_size = page;
    return GW_OK;
}

// ---------------------------------------------------------------------------
// kernel-level entry points
// ---------------------------------------------------------------------------

extern "C" int gw_mxfp4_dequant(gw_context *ctx, const uint8_t *packed, const uint8_t *scales,
                                int64_t blocks, float *out)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(blocks >= 0, GW_ERR_ARG, "negative block count");
    if (blocks == 0) return GW_OK;
    GW_CHECK(packed && scales && out, GW_ERR_ARG, "null pointer");
    GW_CHECK(aligned16(packed) && aligned16(out), GW_ERR_ARG,
             "packed and out must be 16-byte aligned");
    ProfScope ps(ctx, "dequant");
    GW_HIP(gw::launch_dequant(ps.launch(launch_of(ctx)), packed, scales, blocks, out));
    return GW_OK;
}

static int check_gemv(const uint8_t *packed, const uint8_t *scales, const void *x, int x_dt,
                      const float *y, int64_t rows, int64_t cols)
{
    GW_CHECK(rows >= 0 && cols >= 0, GW_ERR_ARG, "negative shape");
    GW_CHECK(cols % 32 == 0, GW_ERR_SHAPE, "MXFP4 needs cols to be a multiple of 32 (got %lld)",
             (long long)cols);
    GW_CHECK(rows < (1ll << 31) && cols <= 32 * 4096, GW_ERR_SHAPE, "shape too large");
    GW_CHECK(dtype_ok(x_dt), GW_ERR_ARG, "bad x dtype %d", x_dt);
    if (rows == 0 || cols == 0) return GW_OK;
    GW_CHECK(packed && scales && x && y, GW_ERR_ARG, "null pointer");
    GW_CHECK(aligned16(packed), GW_ERR_ARG, "packed must be 16-byte aligned");
    GW_CHECK((reinterpret_cast<uintptr_t>(x) & 3u) == 0, GW_ERR_ARG,
             "x must be 4-byte aligned");
    return GW_OK;
}

extern "C" int gw_mxfp4_gemv_bias(gw_context *ctx, const uint8_t *packed, const uint8_t *scales,
                                  const void *bias, gw_dtype bias_dtype, const void *x,
                                  gw_dtype x_dtype, float *y, int64_t rows, int64_t cols)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    int rc = check_gemv(packed, scales, x, x_dtype, y, rows, cols);
    if (rc) return rc;
    GW_CHECK(!bias || dtype_ok(bias_dtype), GW_ERR_ARG, "bad bias dtype %d", (int)bias_dtype);
    if (rows == 0) return GW_OK;
    if (cols == 0) {
        // y = 0: a fill kernel rather than a memset, so that the call can be
        // captured into a graph (no memset node).
        GW_CHECK(!bias, GW_ERR_UNSUPPORTED, "cols == 0 with bias");
        ProfScope ps(ctx, "fill");
        GW_HIP(gw::launch_fill_u8(ps.launch(launch_of(ctx)), y, (size_t)rows * 4, 1, 0, 0, 0, 0));
        return GW_OK;
    }
    ProfScope ps(ctx, "gemv");
    GW_HIP(gw::launch_gemv(ps.launch(launch_of(ctx)), packed, scales, bias, bias ? (int)bias_dtype : -1, x,
                           x_dtype, y, (int)rows, (int)cols));
    return GW_OK;
}

extern "C" int gw_mxfp4_gemv(gw_context *ctx, const uint8_t *packed, const uint8_t *scales,
                             const void *x, gw_dtype x_dtype, float *y, int64_t rows,
                             int64_t cols)
{
    return gw_mxfp4_gemv_bias(ctx, packed, scales, nullptr, GW_F32, x, x_dtype, y, rows, cols);
}

extern "C" int gw_expert_activation(gw_context *ctx, gw_activation kind, const float *gate_up,
                                    uint16_t *out_f16, int64_t width, float limit, float alpha)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(kind == GW_ACT_GPTOSS_CLAMPED_GLU || kind == GW_ACT_SILU, GW_ERR_ARG,
             "bad activation %d", (int)kind);
    GW_CHECK(width >= 0, GW_ERR_ARG, "negative width");
    if (width == 0) return GW_OK;
    GW_CHECK(gate_up && out_f16, GW_ERR_ARG, "null pointer");
    ProfScope ps(ctx, "activation");
    GW_HIP(gw::launch_activation(ps.launch(launch_of(ctx)), (int)kind, gate_up, out_f16, width, limit,
                                 alpha));
    return GW_OK;
}

extern "C" int gw_expert_accumulate(gw_context *ctx, const float *expert_out, float *dst,
                                    float weight, int64_t width)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(width >= 0, GW_ERR_ARG, "negative width");
    if (width == 0) return GW_OK;
    GW_CHECK(expert_out && dst, GW_ERR_ARG, "null pointer");
    ProfScope ps(ctx, "accumulate");
    GW_HIP(gw::launch_accumulate(ps.launch(launch_of(ctx)), expert_out, dst, weight, width));
    return GW_OK;
}

extern "C" int gw_router_logits(gw_context *ctx, const void *weight, gw_dtype weight_dtype,
                                const void *bias, gw_dtype bias_dtype, const void *x,
                                gw_dtype x_dtype, float *logits, int64_t experts,
                                int64_t hidden, int32_t tokens)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(experts >= 0 && hidden >= 0 && tokens >= 0, GW_ERR_ARG, "negative shape");
    GW_CHECK(dtype_ok(weight_dtype) && dtype_ok(x_dtype) && (!bias || dtype_ok(bias_dtype)),
             GW_ERR_ARG, "bad dtype");
    GW_CHECK(experts * tokens < (1ll << 31), GW_ERR_SHAPE, "shape too large");
    if (experts == 0 || tokens == 0) return GW_OK;
    GW_CHECK(weight && x && logits, GW_ERR_ARG, "null pointer");
    ProfScope ps(ctx, "router");
    GW_HIP(gw::launch_router(ps.launch(launch_of(ctx)), weight, weight_dtype, bias,
                             bias ? (int)bias_dtype : -1, x, x_dtype, logits, (int)experts,
                             (int)hidden, tokens));
    return GW_OK;
}

// Router.select (Router.swift:78-98), host side like the reference.
extern "C" int gw_router_select(const float *logits, int64_t experts, int64_t top_k,
                                int32_t *ids, float *weights)
{
    GW_CHECK(logits && ids && weights, GW_ERR_ARG, "null pointer");
    GW_CHECK(top_k >= 1 && top_k <= experts, GW_ERR_SHAPE, "top_k %lld of %lld experts",
             (long long)top_k, (long long)experts);
    std::vector<int32_t> order((size_t)experts);
    for (int64_t i = 0; i < experts; ++i) order[(size_t)i] = (int32_t)i;
    for (int64_t position = 0; position < top_k; ++position) {
        int64_t best = position;
        for (int64_t c = position + 1; c < experts; ++c)
            if (logits[order[(size_t)c]] > logits[order[(size_t)best]]) best = c;
        std::swap(order[(size_t)position], order[(size_t)best]);
    }
    float peak = 0.0f;
    for (int64_t i = 0; i < top_k; ++i) {
        const float v = logits[order[(size_t)i]];
        if (i == 0 || v > peak) peak = v;
    }
    std::vector<float> e((size_t)top_k);
    float total = 0.0f;
    for (int64_t i = 0; i < top_k; ++i) {
        e[(size_t)i] = std::exp(logits[order[(size_t)i]] - peak);
        total += e[(size_t)i];
    }
    for (int64_t i = 0; i < top_k; ++i) {
        ids[i] = order[(size_t)i];
        weights[i] = e[(size_t)i] / total;
    }
    return GW_OK;
}

// ---------------------------------------------------------------------------
// ExpertRunner
// ---------------------------------------------------------------------------

static constexpr int kPlanRing = 64;
static constexpr int kMaxExperts = 1024;

struct gw_expert_runner {
    gw_context *ctx = nullptr;
    int64_t hidden = 0, inter = 0;
    int act = 0;
    float limit = 7.0f, alpha = 1.702f;
    int bias_dt = GW_BF16;
    int64_t offsets[GW_SECTION_COUNT] = {};
    // device scratch
    Plan *plans = nullptr;           // [kPlanRing] host-built plans
    Plan *route_plan = nullptr;      // device-built plan of gw_moe_layer_forward
    uint16_t *act_buf = nullptr;     // [kMaxSlots, inter] fp16 activations
    uint16_t *normed_buf = nullptr;  // [kMaxTokens, hidden] fp16 RMSNorm output
    float *logits = nullptr;         // [kMaxTokens, kMaxExperts]
    Plan *staging = nullptr;         // pinned host mirror of `plans`
    unsigned *sync_buf = nullptr;    // fused layer exchange: counters | epochs | error word
    uint64_t *xchg_buf = nullptr;    // one-kernel layer: activation words (all ones once)
    uint32_t spin_limit = gw::kDecodeSpinLimit;   // exchange polls before a wait gives up
    int poll_fault = 0;              // test hook: read the never-written exchange slot
    uint32_t xchg_errors_seen = 0;   // failed exchange waits already reported
    // prefill scratch, sized for pf_tokens tokens x pf_topk ranks x pf_experts
    int pf_tokens = 0, pf_topk = 0, pf_experts = 0;
    int pf_last_tokens = 0, pf_last_topk = 0;   // of the last batch in pf_buf
    void *pf_buf = nullptr;
    bool decode_layer = true;        // one-token layers in one kernel (GODWIT_DECODE_LAYER=0: two)
    int prefill_above = 1;           // batches larger than this run the grouped GEMMs
    int self_group_max = 16;         // grouped batches up to this size group inside the GEMMs
    int gemm_waves = 0, gemm_depth = 0;   // forced grouped-GEMM shape (0: chosen per launch)
    int fused_combine_max = 32;      // grouped batches up to this size combine inside the down GEMM
    int ring_next = 0;
    int ring_used = 0;
};

static constexpr int kSyncEpochWords = gw::kSyncEpochCapacity;

static gw::SyncArgs sync_of(gw_expert_runner *r)
{
    gw::SyncArgs s;
    s.counters = r->sync_buf;
    s.epochs = r->sync_buf + gw::kSyncWords;
    s.err = r->sync_buf + gw::kSyncWords + kSyncEpochWords;
    return s;
}

extern "C" int gw_expert_runner_destroy(gw_expert_runner *r)
{
    if (!r) return GW_OK;
    if (r->ctx) {
        (void)hipStreamSynchronize(r->ctx->stream);
        auto &v = r->ctx->runners;
        v.erase(std::remove(v.begin(), v.end(), r), v.end());
    }
    (void)hipFree(r->plans);
    (void)hipFree(r->route_plan);
    (void)hipFree(r->act_buf);
    (void)hipFree(r->normed_buf);
    (void)hipFree(r->logits);
    (void)hipHostFree(r->staging);
    (void)hipFree(r->sync_buf);
    (void)hipFree(r->xchg_buf);
    (void)hipFree(r->pf_buf);
    delete r;
    return GW_OK;
}

extern "C" int gw_expert_runner_create(gw_context *ctx, int64_t hidden_size,
                                       int64_t intermediate_size, gw_activation activation,
                                       float swiglu_limit, float swiglu_alpha,
                                       gw_expert_runner **out)
{
    GW_CHECK(ctx && out, GW_ERR_ARG, "null argument");
    *out = nullptr;
    GW_CHECK(activation == GW_ACT_GPTOSS_CLAMPED_GLU || activation == GW_ACT_SILU, GW_ERR_ARG,
             "bad activation %d", (int)activation);
    gw_expert_layout layout;
    int rc = gw_expert_layout_init(hidden_size, intermediate_size, 1, &layout);
    if (rc) return rc;
    GW_CHECK(hidden_size <= 32 * 4096 && intermediate_size <= 32 * 4096, GW_ERR_SHAPE,
             "shape too large");
    GW_CHECK(gw::gate_up_lds_bytes((int)hidden_size, GW_F32, 1) <= gw::kLdsBudget, GW_ERR_SHAPE,
             "hidden size %lld too large for the LDS-staged activation", (long long)hidden_size);
    gw_expert_runner *r = new gw_expert_runner();
    r->ctx = ctx;
    r->hidden = hidden_size;
    r->inter = intermediate_size;
    r->act = activation;
    r->limit = swiglu_limit;
    r->alpha = swiglu_alpha;
    for (int s = 0; s < GW_SECTION_COUNT; ++s) r->offsets[s] = layout.offsets[s];
    hipError_t e = hipSetDevice(ctx->device);
    if (e == hipSuccess) e = hipMalloc((void **)&r->plans, sizeof(Plan) * kPlanRing);
    if (e == hipSuccess) e = hipMalloc((void **)&r->route_plan, sizeof(Plan));
    if (e == hipSuccess)
        e = hipMalloc((void **)&r->act_buf, sizeof(uint16_t) * gw::kMaxSlots * intermediate_size);
    if (e == hipSuccess)
        e = hipMalloc((void **)&r->normed_buf, sizeof(uint16_t) * gw::kMaxTokens * hidden_size);
    if (e == hipSuccess)
        e = hipMalloc((void **)&r->logits, sizeof(float) * gw::kMaxTokens * kMaxExperts);
    if (e == hipSuccess) e = hipHostMalloc((void **)&r->staging, sizeof(Plan) * kPlanRing);
    const size_t sync_bytes = sizeof(unsigned) * (gw::kSyncWords + kSyncEpochWords + 64);
    if (e == hipSuccess) e = hipMalloc((void **)&r->sync_buf, sync_bytes);
    if (e == hipSuccess) e = hipMemset(r->sync_buf, 0, sync_bytes);
    // the exchange ring gets a 2 MiB block of its own: a block of the ring's own
    // size measured 1-2% slower per layer on the same box
    const size_t xchg_bytes = std::max<size_t>(gw::kDecodeXchgBytes, 2u << 20);
    if (e == hipSuccess) e = hipMalloc((void **)&r->xchg_buf, xchg_bytes);
    if (e == hipSuccess) e = hipMemset(r->xchg_buf, 0xFF, xchg_bytes);   // every word empty
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        gw_expert_runner_destroy(r);
        return alloc_failed(e, "runner scratch", 0);
    }
    r->decode_layer = get_env_int("GODWIT_DECODE_LAYER", 1) != 0;
    ctx->runners.push_back(r);
    const int pa = get_env_int("GODWIT_PREFILL_ABOVE", 1);
    r->prefill_above = pa < 1 ? 1 : pa > gw::kMaxTokens ? gw::kMaxTokens : pa;
    // 12: Qwen3 per token, self-grouped against the route and group kernels
    // in front: 296.1 / 305.3 us at 10 tokens, 273.7 / 277.1 at 12, 283.0 /
    // 237.7 at 14, 255.1 / 214.3 at 16, 257.2 / 208.8 at 17 (the selection
    // in every gate_up workgroup grows with the batch; the kernels in front
    // cost a fixed ~9 us a layer).
    const int sg = get_env_int("GODWIT_SELF_GROUP_TOKENS", 12);
    r->self_group_max = sg < 0 ? 0 : sg > 32 ? 32 : sg;
    const int fc = get_env_int("GODWIT_FUSED_COMBINE_TOKENS", 32);
    r->fused_combine_max = fc < 0 ? 0 : fc;
    if (const char *shape = getenv("GODWIT_PREFILL_SHAPE")) {
        int w = 0, d = 0;
        if (sscanf(shape, "%dx%d", &w, &d) == 2 && (w == 4 || w == 8 || w == 12) &&
            (d == 2 || d == 4)) {
            r->gemm_waves = w;
            r->gemm_depth = d;
        }
    }
    *out = r;
    return GW_OK;
}

// After the stream is idle: a runner whose one-token layers counted a failed
// exchange since the last check reports it, and runs its later one-token
// layers with the two-kernel form (no cross-workgroup wait).
static int check_exchanges(gw_context *ctx)
{
    for (gw_expert_runner *r : ctx->runners) {
        uint32_t n = 0;
        GW_HIP(hipMemcpy(&n, sync_of(r).err, sizeof(uint32_t), hipMemcpyDeviceToHost));
        if (n != r->xchg_errors_seen) {
            const uint32_t fresh = n - r->xchg_errors_seen;
            r->xchg_errors_seen = n;
            r->decode_layer = false;
            return fail(GW_ERR_EXCHANGE,
                        "%u wave(s) of a one-token layer gave up waiting for the activation "
                        "exchange (the GPU was shared, or the wait limit is too small): those "
                        "layers' outputs are invalid; this runner now uses the two-kernel form",
                        fresh);
        }
    }
    return GW_OK;
}

extern "C" int gw_expert_runner_sync_errors(gw_expert_runner *r, uint32_t *count)
{
    GW_CHECK(r && count, GW_ERR_ARG, "null argument");
    GW_CHECK(!is_capturing(r->ctx), GW_ERR_ARG, "sync_errors during graph capture");
    GW_HIP(hipStreamSynchronize(r->ctx->stream));
    GW_HIP(hipMemcpy(count, sync_of(r).err, sizeof(uint32_t), hipMemcpyDeviceToHost));
    return GW_OK;
}

extern "C" int gw_expert_runner_set_wait_limit(gw_expert_runner *r, uint32_t polls)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    r->spin_limit = polls ? polls : gw::kDecodeSpinLimit;
    return GW_OK;
}

extern "C" int gw_expert_runner_inject_exchange_fault(gw_expert_runner *r, int enable)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    r->poll_fault = enable != 0;
    return GW_OK;
}

extern "C" int gw_expert_runner_set_bias_dtype(gw_expert_runner *r, gw_dtype bias_dtype)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    GW_CHECK(bias_dtype == GW_BF16 || bias_dtype == GW_F32, GW_ERR_ARG, "bad bias dtype");
    if (bias_dtype == GW_F32) {
        // The .gwt layout sizes the bias sections for bf16; fp32 values need
        // twice the bytes, which must still end before the next section (the
        // gate_up bias) or the expert stride (the down bias).
        gw_expert_layout lay;
        int rc = gw_expert_layout_init(r->hidden, r->inter, 1, &lay);
        if (rc) return rc;
        const int64_t gu_end = r->offsets[GW_SECTION_GATE_UP_BIAS] + 4 * 2 * r->inter;
        const int64_t dn_end = r->offsets[GW_SECTION_DOWN_BIAS] + 4 * r->hidden;
        GW_CHECK(gu_end <= r->offsets[GW_SECTION_DOWN_BIAS] && dn_end <= lay.stride, GW_ERR_SHAPE,
                 "fp32 biases of %lld + %lld rows overflow their sections in the expert layout "
                 "(gate_up bias ends at %lld, down bias at %lld; limits %lld and %lld)",
                 (long long)(2 * r->inter), (long long)r->hidden, (long long)gu_end,
                 (long long)dn_end, (long long)r->offsets[GW_SECTION_DOWN_BIAS],
                 (long long)lay.stride);
    }
    r->bias_dt = bias_dtype;
    return GW_OK;
}

extern "C" int gw_expert_runner_section_offsets(gw_expert_runner *r,
                                                int64_t offsets[GW_SECTION_COUNT])
{
    GW_CHECK(r && offsets, GW_ERR_ARG, "null argument");
    for (int s = 0; s < GW_SECTION_COUNT; ++s) offsets[s] = r->offsets[s];
    return GW_OK;
}

static gw::Sections sections_of(const int64_t off[GW_SECTION_COUNT])
{
    gw::Sections s;
    s.gu_blocks = off[GW_SECTION_GATE_UP_BLOCKS];
    s.gu_scales = off[GW_SECTION_GATE_UP_SCALES];
    s.dn_blocks = off[GW_SECTION_DOWN_BLOCKS];
    s.dn_scales = off[GW_SECTION_DOWN_SCALES];
    s.gu_bias = off[GW_SECTION_GATE_UP_BIAS];
    s.dn_bias = off[GW_SECTION_DOWN_BIAS];
    return s;
}

// Runs one plan: upload, fused gate_up + activation, fused down + combine.
// All groups of a plan share one set of section offsets (the runner launches
// a separate plan per distinct offset set).
static int run_plan(gw_expert_runner *r, HostPlan &hp, const int64_t offsets[GW_SECTION_COUNT],
                    const void *inputs, int x_dt, float *outputs, int accumulate)
{
    gw_context *ctx = r->ctx;
    Plan q;
    gw::plan_regroup(hp, q);

    if (r->ring_used == kPlanRing) {   // staging slots are reused only after their copies ran
        GW_HIP(hipStreamSynchronize(ctx->stream));
        r->ring_used = 0;
    }
    const int slot = r->ring_next;
    r->ring_next = (r->ring_next + 1) % kPlanRing;
    r->ring_used += 1;
    r->staging[slot] = q;
    GW_HIP(hipMemcpyAsync(r->plans + slot, r->staging + slot, sizeof(Plan),
                          hipMemcpyHostToDevice, ctx->stream));
    const gw::Sections sec = sections_of(offsets);
    const gw::Launch L = launch_of(ctx);
    // The staged inputs bound every group's width, so q.ntokens picks the
    // kernel width (1, or the 8-wide variant) for both kernels.
    GW_CHECK(gw::gate_up_lds_bytes((int)r->hidden, x_dt, q.ntokens) <= gw::kLdsBudget,
             GW_ERR_SHAPE, "%d staged inputs of width %lld exceed the LDS budget", q.ntokens,
             (long long)r->hidden);
    {
        ProfScope ps(ctx, "gate_up");
        GW_HIP(gw::launch_gate_up(ps.launch(L), r->plans + slot, nullptr, q.ntokens, inputs, x_dt,
                                  (int)r->hidden,
                                  (int)r->inter, sec, r->bias_dt, r->act_buf, r->act, r->limit,
                                  r->alpha));
    }
    {
        ProfScope ps(ctx, "down");
        GW_HIP(gw::launch_down(ps.launch(L), r->plans + slot, q.ntokens, q.nslots, r->act_buf,
                               (int)r->hidden, (int)r->inter, sec, r->bias_dt, outputs, nullptr,
                               accumulate));
    }
    return GW_OK;
}

static bool same_offsets(const gw_expert_weights *a, const gw_expert_weights *b)
{
    for (int s = 0; s < GW_SECTION_COUNT; ++s)
        if (a->offsets[s] != b->offsets[s]) return false;
    return true;
}

static int check_weights(gw_expert_runner *r, const gw_expert_weights *w)
{
    GW_CHECK(w && w->buffer, GW_ERR_ARG, "null expert weights");
    GW_CHECK(aligned16(w->buffer), GW_ERR_ARG, "expert buffer must be 16-byte aligned");
    for (int s = 0; s < 4; ++s)
        GW_CHECK(w->offsets[s] >= 0 && (w->offsets[s] & 15) == 0, GW_ERR_ARG,
                 "section %d offset %lld must be non-negative and 16-byte aligned", s,
                 (long long)w->offsets[s]);
    const int bias_align = r->bias_dt == GW_F32 ? 4 : 2;
    for (int s = 4; s < 6; ++s)
        GW_CHECK(w->offsets[s] >= 0 && (w->offsets[s] % bias_align) == 0, GW_ERR_ARG,
                 "bias section %d offset misaligned", s);
    return GW_OK;
}

// Shared driver of apply / applyBatch / applyAssignments.
static int run_assignments(gw_expert_runner *r, const void *inputs, int x_dt,
                           const gw_assignment *a, int32_t n, float *outputs, int accumulate,
                           bool merge)
{
    GW_CHECK(dtype_ok(x_dt), GW_ERR_ARG, "bad x dtype %d", x_dt);
    GW_CHECK(inputs && outputs, GW_ERR_ARG, "null pointer");
    GW_CHECK((reinterpret_cast<uintptr_t>(inputs) & 3u) == 0, GW_ERR_ARG,
             "inputs must be 4-byte aligned");
    GW_CHECK(!is_capturing(r->ctx), GW_ERR_ARG, "host-planned calls cannot be captured");
    for (int32_t i = 0; i < n; ++i) {
        int rc = check_weights(r, &a[i].weights);
        if (rc) return rc;
        GW_CHECK(a[i].token >= 0, GW_ERR_ARG, "negative token index");
    }
    HostPlan hp;
    hp.clear();
    const gw_expert_weights *plan_offsets = nullptr;
    int first_run = 1;
    for (int32_t i = 0; i < n; ++i) {
        const gw_expert_weights *w = &a[i].weights;
        const bool fits_offsets = !plan_offsets || same_offsets(plan_offsets, w);
        if (!fits_offsets || !plan_add(hp, w, a[i].token, a[i].routing_weight, merge)) {
            int rc = run_plan(r, hp, plan_offsets->offsets, inputs, x_dt, outputs,
                              accumulate || !first_run);
            if (rc) return rc;
            first_run = 0;
            hp.clear();
            plan_offsets = nullptr;
            if (!plan_add(hp, w, a[i].token, a[i].routing_weight, merge))
                return fail(GW_ERR_SHAPE, "assignment does not fit an empty plan");
        }
        if (!plan_offsets) plan_offsets = w;
    }
    if (hp.p.nslots > 0) {
        int rc = run_plan(r, hp, plan_offsets->offsets, inputs, x_dt, outputs,
                          accumulate || !first_run);
        if (rc) return rc;
    }
    return GW_OK;
}

extern "C" int gw_expert_apply(gw_expert_runner *r, const void *x, gw_dtype x_dtype,
                               const gw_expert_weights *weights, float *out)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    GW_CHECK(weights, GW_ERR_ARG, "weights is null");
    gw_assignment a;
    a.weights = *weights;
    a.token = 0;
    a.routing_weight = 1.0f;   // combine: 0 + out * 1 == out exactly
    int rc = run_assignments(r, x, x_dtype, &a, 1, out, 0, false);
    if (rc) return rc;
    GW_HIP(hipStreamSynchronize(r->ctx->stream));
    return GW_OK;
}

extern "C" int gw_expert_apply_batch(gw_expert_runner *r, const void *x, gw_dtype x_dtype,
                                     const gw_expert_weights *experts,
                                     const float *routing_weights, int32_t count, float *out)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    GW_CHECK(count >= 0, GW_ERR_ARG, "negative count");
    GW_CHECK(count == 0 || (experts && routing_weights), GW_ERR_ARG, "null pointer");
    GW_CHECK(out, GW_ERR_ARG, "out is null");
    if (count == 0) {   // the reference returns zeros (ExpertRunner.swift:195)
        GW_CHECK(!is_capturing(r->ctx), GW_ERR_ARG, "cannot capture");
        GW_HIP(hipMemsetAsync(out, 0, sizeof(float) * r->hidden, r->ctx->stream));
        GW_HIP(hipStreamSynchronize(r->ctx->stream));
        return GW_OK;
    }
    std::vector<gw_assignment> a((size_t)count);
    for (int32_t i = 0; i < count; ++i) {
        a[(size_t)i].weights = experts[i];
        a[(size_t)i].token = 0;
        a[(size_t)i].routing_weight = routing_weights[i];
    }
    int rc = run_assignments(r, x, x_dtype, a.data(), count, out, 0, false);
    if (rc) return rc;
    GW_HIP(hipStreamSynchronize(r->ctx->stream));
    return GW_OK;
}

extern "C" int gw_expert_apply_assignments_async(gw_expert_runner *r, const void *inputs,
                                                 gw_dtype x_dtype,
                                                 const gw_assignment *assignments,
                                                 int32_t count, float *outputs)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    GW_CHECK(count >= 0, GW_ERR_ARG, "negative count");
    if (count == 0) return GW_OK;   // ExpertRunner.swift:111
    GW_CHECK(assignments, GW_ERR_ARG, "assignments is null");
    return run_assignments(r, inputs, x_dtype, assignments, count, outputs, 1, true);
}

extern "C" int gw_expert_apply_assignments(gw_expert_runner *r, const void *inputs,
                                           gw_dtype x_dtype, const gw_assignment *assignments,
                                           int32_t count, float *outputs)
{
    int rc = gw_expert_apply_assignments_async(r, inputs, x_dtype, assignments, count, outputs);
    if (rc) return rc;
    GW_HIP(hipStreamSynchronize(r->ctx->stream));
    return GW_OK;
}

// ---------------------------------------------------------------------------
// MoE layer (device-routed)
// ---------------------------------------------------------------------------

// out_mode 0: out = MoE output; 2: out += MoE output (the residual add).
static int moe_prefill_impl(gw_expert_runner *r, const gw_moe_layer_args *a, int out_mode,
                            bool use_static = false);

// A batch of up to kMaxTokens tokens runs either the streaming decode kernels,
// which read each selected expert once per token group of a workgroup, or the
// grouped GEMMs, which read each distinct expert once for the whole batch but
// pay for routing, grouping and combining in kernels of their own.  Above
// prefill_above tokens (GODWIT_PREFILL_ABOVE at creation, default 1) the
// grouped GEMMs win; they are taken when the shape is one they accept and,
// under graph capture, when their scratch is already large enough.
static bool batch_takes_grouped_gemm(const gw_expert_runner *r, const gw_moe_layer_args *a)
{
    if (a->tokens <= r->prefill_above) return false;
    if (r->hidden % 32 || r->inter % 32 || r->hidden < 128 || r->inter < 128) return false;
    if (a->expert_count < 1 || a->expert_count > 256 || !aligned16(a->x) ||
        !aligned16(a->experts_base) || a->expert_stride % 16)
        return false;
    if (is_capturing(r->ctx) &&
        !(r->pf_buf && a->tokens <= r->pf_tokens && a->top_k <= r->pf_topk &&
          a->expert_count <= r->pf_experts))
        return false;
    return true;
}

static int moe_layer_impl(gw_expert_runner *r, const gw_moe_layer_args *a, int out_mode)
{
    GW_CHECK(r && a, GW_ERR_ARG, "null argument");
    if (a->tokens > gw::kMaxTokens || batch_takes_grouped_gemm(r, a))
        return moe_prefill_impl(r, a, out_mode);
    GW_CHECK(a->tokens >= 1, GW_ERR_SHAPE, "tokens must be positive (got %d)", a->tokens);
    GW_CHECK(a->expert_count >= 1 && a->expert_count <= kMaxExperts, GW_ERR_SHAPE,
             "expert_count %lld out of range", (long long)a->expert_count);
    GW_CHECK(a->top_k >= 1 && a->top_k <= gw::kMaxTopK && a->top_k <= a->expert_count,
             GW_ERR_SHAPE, "top_k %lld out of range", (long long)a->top_k);
    GW_CHECK(a->experts_base && a->x && a->out, GW_ERR_ARG, "null pointer");
    GW_CHECK(aligned16(a->experts_base) && a->expert_stride > 0 && a->expert_stride % 16 == 0,
             GW_ERR_ARG, "experts_base/stride must be 16-byte aligned");
    GW_CHECK(dtype_ok(a->x_dtype), GW_ERR_ARG, "bad x dtype");
    GW_CHECK((reinterpret_cast<uintptr_t>(a->x) & 3u) == 0, GW_ERR_ARG, "x must be 4-byte aligned");
    GW_CHECK(a->logits || a->router_weight, GW_ERR_ARG, "need logits or router weights");
    gw_context *ctx = r->ctx;
    const gw::Launch L = launch_of(ctx);
    if (!a->logits) GW_CHECK(dtype_ok(a->router_weight_dtype), GW_ERR_ARG, "bad router dtype");
    // One token: the whole layer in one kernel when the shape, the dtype and
    // the occupancy allow it, which also computes the router logits when the
    // router rows split evenly over its grid (16-bit x, up to 128 experts).
    gw::DecodeArgs d = {};
    size_t dlds = 0;
    const int dgrid = a->tokens == 1 && r->decode_layer
                          ? gw::decode_layer_plan(L, (int)r->hidden, (int)r->inter, a->x_dtype,
                                                  (int)a->top_k, (int)a->expert_count,
                                                  a->expert_stride, r->bias_dt, &d, &dlds)
                          : 0;
    const int rslices = dgrid > 0 && !a->logits && a->expert_count <= 128 &&
                                aligned16(a->router_weight) && aligned16(a->x)
                            ? gw::router_slices((int)a->expert_count, (int)r->hidden, dgrid)
                            : 0;
    const float *logits = a->logits;
    if (!logits && rslices == 0) {
        ProfScope ps(ctx, "router");
        GW_HIP(gw::launch_router(ps.launch(L), a->router_weight, a->router_weight_dtype, a->router_bias,
                                 a->router_bias ? (int)a->router_bias_dtype : -1, a->x,
                                 a->x_dtype, r->logits, (int)a->expert_count, (int)r->hidden,
                                 a->tokens));
        logits = r->logits;
    }
    GW_CHECK(gw::gate_up_lds_bytes((int)r->hidden, a->x_dtype, a->tokens) <= gw::kLdsBudget,
             GW_ERR_SHAPE, "%d tokens of width %lld exceed the LDS budget", a->tokens,
             (long long)r->hidden);
    gw::RouteArgs route;
    route.logits = logits;
    route.experts = (int)a->expert_count;
    route.top_k = (int)a->top_k;
    route.tokens = a->tokens;
    route.experts_base = a->experts_base;
    route.stride = a->expert_stride;
    route.ids_out = a->routing_ids;
    route.w_out = a->routing_weights;
    const gw::Sections sec = sections_of(r->offsets);
    {
        const int grid = dgrid;
        const size_t lds = dlds;
        if (grid > 0) {
            d.logits = logits;
            if (rslices > 0) {
                d.rw = a->router_weight;
                d.rw_dt = (int)a->router_weight_dtype;
                d.rb = a->router_bias;
                d.rb_dt = a->router_bias ? (int)a->router_bias_dtype : -1;
                d.rslices = rslices;
            }
            d.experts = (int)a->expert_count;
            d.top_k = (int)a->top_k;
            d.base = a->experts_base;
            d.stride = a->expert_stride;
            d.ids_out = a->routing_ids;
            d.w_out = a->routing_weights;
            d.x = a->x;
            d.hidden = (int)r->hidden;
            d.inter = (int)r->inter;
            d.sec = sec;
            d.bias_dt = r->bias_dt;
            d.xchg = r->xchg_buf;
            d.act_kind = r->act;
            d.limit = r->limit;
            d.alpha = r->alpha;
            d.out = a->out;
            d.out_bf16 = a->out_bf16;
            d.accumulate = out_mode;
            d.sync = sync_of(r);
            d.spin_limit = r->spin_limit;
            d.poll_fault = r->poll_fault;
            ProfScope ps(ctx, "moe_layer");
            GW_HIP(gw::launch_decode_layer(ps.launch(L), grid, lds, a->x_dtype, d));
            return GW_OK;
        }
    }
    // Up to 256 experts the gate_up kernel routes in its prologue; beyond that
    // the route kernel builds the plan first.
    const bool fused = a->expert_count <= gw::kFusedRouteExperts;
    if (!fused) {
        ProfScope ps(ctx, "route");
        GW_HIP(gw::launch_route(ps.launch(L), route, r->route_plan));
    }
    {
        ProfScope ps(ctx, "gate_up");
        GW_HIP(gw::launch_gate_up(ps.launch(L), r->route_plan, fused ? &route : nullptr, a->tokens, a->x,
                                  a->x_dtype, (int)r->hidden, (int)r->inter, sec, r->bias_dt,
                                  r->act_buf, r->act, r->limit, r->alpha));
    }
    {
        ProfScope ps(ctx, "down");
        GW_HIP(gw::launch_down(ps.launch(L), r->route_plan, a->tokens, (int)(a->tokens * a->top_k), r->act_buf,
                               (int)r->hidden, (int)r->inter, sec, r->bias_dt, a->out,
                               a->out_bf16, out_mode));
    }
    return GW_OK;
}

extern "C" int gw_moe_layer_forward(gw_expert_runner *r, const gw_moe_layer_args *a)
{
    return moe_layer_impl(r, a, 0);
}

// ---------------------------------------------------------------------------
// prefill: many tokens through one layer on the matrix cores
// ---------------------------------------------------------------------------

namespace {
struct PrefillScratch {
    float *logits;
    int32_t *ids;
    float *weights;
    int32_t *offsets, *order, *tiles, *ntiles;
    uint16_t *normed;   // [T, hidden] fp16 RMSNorm output (gw_moe_block_forward)
    uint16_t *xsplit;   // [planes][T, hidden] bf16 planes of a fp16 or fp32 x
    uint16_t *act;      // [N, inter] fp16 activations
    float *y;
    uint32_t *arrive;   // prefill_arrive_count(T, hidden) combine counters, zero between launches
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// Carves the runner's prefill buffer; returns the bytes needed for (T, K, E).
size_t prefill_layout(const gw_expert_runner *r, int T, int K, int E, char *base,
                      PrefillScratch *ps)
{
    const size_t N = (size_t)T * K;
    const size_t tiles = (size_t)gw::prefill_max_tiles(T, K, E);
    size_t o = 0;
    auto take = [&](size_t bytes) {
        char *p = base ? base + o : nullptr;
        o += align256(bytes);
        return p;
    };
    PrefillScratch s;
    s.logits = reinterpret_cast<float *>(take(sizeof(float) * (size_t)T * E));
    s.ids = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * N));
    s.weights = reinterpret_cast<float *>(take(sizeof(float) * N));
    s.offsets = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * (E + 1)));
    s.order = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * N));
    s.tiles = reinterpret_cast<int32_t *>(take(sizeof(int32_t) * tiles));
    s.ntiles = reinterpret_cast<int32_t *>(take(sizeof(int32_t)));
    s.normed = reinterpret_cast<uint16_t *>(take(sizeof(uint16_t) * (size_t)T * r->hidden));
    s.xsplit = reinterpret_cast<uint16_t *>(take(sizeof(uint16_t) * 3 * (size_t)T * r->hidden));
    s.act = reinterpret_cast<uint16_t *>(take(sizeof(uint16_t) * N * r->inter));
    s.y = reinterpret_cast<float *>(take(sizeof(float) * N * r->hidden));
    s.arrive = reinterpret_cast<uint32_t *>(
        take(sizeof(uint32_t) * (size_t)gw::prefill_arrive_count(T, (int)r->hidden)));
    if (ps) *ps = s;
    return o;
}
}  // namespace

extern "C" int gw_expert_runner_reserve_prefill(gw_expert_runner *r, int32_t max_tokens,
                                                int32_t top_k, int32_t expert_count)
{
    GW_CHECK(r, GW_ERR_ARG, "runner is null");
    GW_CHECK(max_tokens >= 1 && top_k >= 1 && top_k <= gw::kMaxTopK && expert_count >= top_k &&
                 expert_count <= 256,
             GW_ERR_SHAPE, "prefill shape out of range (tokens %d, top_k %d, experts %d)",
             max_tokens, top_k, expert_count);
    if (r->pf_buf && max_tokens <= r->pf_tokens && top_k <= r->pf_topk &&
        expert_count <= r->pf_experts)
        return GW_OK;
    GW_CHECK(!is_capturing(r->ctx), GW_ERR_ARG,
             "prefill scratch must be reserved before graph capture");
    const int T = max_tokens > r->pf_tokens ? max_tokens : r->pf_tokens;
    const int K = top_k > r->pf_topk ? top_k : r->pf_topk;
    const int E = expert_count > r->pf_experts ? expert_count : r->pf_experts;
    const size_t bytes = prefill_layout(r, T, K, E, nullptr, nullptr);
    GW_HIP(hipStreamSynchronize(r->ctx->stream));
    (void)hipFree(r->pf_buf);
    r->pf_buf = nullptr;
    r->pf_tokens = r->pf_topk = r->pf_experts = 0;
    if (hipError_t e = hipMalloc(&r->pf_buf, bytes); e != hipSuccess) {
        r->pf_buf = nullptr;
        return alloc_failed(e, "prefill scratch hipMalloc", bytes);
    }
    PrefillScratch ps;
    prefill_layout(r, T, K, E, static_cast<char *>(r->pf_buf), &ps);
    GW_HIP(hipMemsetAsync(ps.arrive, 0, sizeof(uint32_t) * (size_t)gw::prefill_arrive_count(T, (int)r->hidden),
                          r->ctx->stream));
    GW_HIP(hipStreamSynchronize(r->ctx->stream));
    r->pf_tokens = T;
    r->pf_topk = K;
    r->pf_experts = E;
    return GW_OK;
}

// use_static: scratch carved from the device's static array (exactly T, K, E)
// instead of the runner's reserved buffer, and no allocation.
static int moe_prefill_impl(gw_expert_runner *r, const gw_moe_layer_args *a, int out_mode,
                            bool use_static)
{
    GW_CHECK(r && a, GW_ERR_ARG, "null argument");
    GW_CHECK(a->tokens >= 1, GW_ERR_SHAPE, "tokens must be positive (got %d)", a->tokens);
    GW_CHECK(a->expert_count >= 1 && a->expert_count <= 256, GW_ERR_SHAPE,
             "prefill takes 1..256 experts (got %lld)", (long long)a->expert_count);
    GW_CHECK(a->top_k >= 1 && a->top_k <= gw::kMaxTopK && a->top_k <= a->expert_count,
             GW_ERR_SHAPE, "top_k %lld out of range", (long long)a->top_k);
    GW_CHECK(a->experts_base && a->x && a->out, GW_ERR_ARG, "null pointer");
    GW_CHECK(aligned16(a->experts_base) && a->expert_stride > 0 && a->expert_stride % 16 == 0,
             GW_ERR_ARG, "experts_base/stride must be 16-byte aligned");
    GW_CHECK(dtype_ok(a->x_dtype), GW_ERR_ARG, "bad x dtype");
    GW_CHECK(aligned16(a->x), GW_ERR_ARG, "x must be 16-byte aligned for prefill");
    GW_CHECK(a->logits || a->router_weight, GW_ERR_ARG, "need logits or router weights");
    GW_CHECK(r->hidden % 32 == 0 && r->inter % 32 == 0 && r->hidden >= 128 && r->inter >= 128,
             GW_ERR_SHAPE, "prefill needs hidden and intermediate sizes that are multiples of 32 "
             "and at least 128 (got %lld, %lld)", (long long)r->hidden, (long long)r->inter);
    const int T = a->tokens, K = (int)a->top_k, E = (int)a->expert_count;
    gw_context *ctx = r->ctx;
    const gw::Launch L = launch_of(ctx);
    PrefillScratch ps;
    if (use_static) {
        void *base = ctx->device < kScratchDevices ? g_scratch_ptr[ctx->device] : nullptr;
        GW_CHECK(base, GW_ERR_ARG, "no static scratch on device %d", ctx->device);
        const size_t need = prefill_layout(r, T, K, E, nullptr, nullptr);
        GW_CHECK(need <= GW_STATIC_SCRATCH_BYTES, GW_ERR_SHAPE,
                 "%d tokens x top-%d over %d experts need %zu bytes of prefill scratch; the "
                 "static array holds %zu", T, K, E, need, (size_t)GW_STATIC_SCRATCH_BYTES);
        prefill_layout(r, T, K, E, static_cast<char *>(base), &ps);
    } else {
        int rc = gw_expert_runner_reserve_prefill(r, T, K, E);
        if (rc) return rc;
        prefill_layout(r, r->pf_tokens, r->pf_topk, r->pf_experts,
                       static_cast<char *>(r->pf_buf), &ps);
    }
    const float *logits = a->logits;
    if (!logits) {
        GW_CHECK(dtype_ok(a->router_weight_dtype), GW_ERR_ARG, "bad router dtype");
        ProfScope p(ctx, "router");
        GW_HIP(gw::launch_router(p.launch(L), a->router_weight, a->router_weight_dtype,
                                 a->router_bias, a->router_bias ? (int)a->router_bias_dtype : -1,
                                 a->x, a->x_dtype, ps.logits, E, (int)r->hidden, T));
        logits = ps.logits;
    }
    // Up to self_group_max tokens every expert holds at most one tile, and
    // the GEMMs route and group the batch themselves (no route or group
    // kernel); larger batches get the tile list from the group kernel.
    const bool self_group = T <= r->self_group_max && gw::prefill_self_groups(T, K, E);
    const int max_tiles = self_group ? std::min(E, T * K) : gw::prefill_max_tiles(T, K, E);
    if (!self_group) {
        const bool route_in_group = gw::prefill_routes_in_group(T, K);
        if (!route_in_group) {
            ProfScope p(ctx, "prefill_route");
            GW_HIP(gw::launch_prefill_route(p.launch(L), logits, T, E, K, ps.ids, ps.weights));
        }
        ProfScope p(ctx, "prefill_group");
        GW_HIP(gw::launch_prefill_group(p.launch(L), route_in_group ? logits : nullptr, T, K,
                                        ps.weights, ps.ids, E, ps.offsets, ps.order, ps.tiles,
                                        ps.ntiles, max_tiles));
    }
    const gw::Sections sec = sections_of(r->offsets);
    // Up to fused_combine_max tokens the combine runs inside the down GEMM
    // (the workgroup that completes a token's feature tile sums it), saving a
    // launch.  Larger batches keep the combine kernel where the coherent
    // write-through of y costs more than the launch (Qwen3 batch 512: down
    // 49 -> 63 us against an 8.3 us combine), except when the down GEMM runs
    // the 4-wave shape, where it costs less (GPT-OSS 512 tokens: down 191 ->
    // 195 us against a 9 us combine and its launch gap).
    const bool fuse_combine =
        (T <= r->fused_combine_max ||
         (r->fused_combine_max > 0 &&
          gw::prefill_down_four_wave((int)r->hidden, (int)r->inter, T * K, max_tiles, L.cus))) &&
        (int64_t)sizeof(float) * T * K * r->hidden < ((int64_t)1 << 31);
    gw::PrefillGemm g;
    g.force_waves = r->gemm_waves;
    g.force_depth = r->gemm_depth;
    if (self_group) {
        g.sg_tokens = T;
        g.sg_topk = K;
        g.sg_experts = E;
        g.sg_logits = logits;
        g.sg_ids_out = ps.ids;
        g.sg_w_out = ps.weights;
    }
    g.tiles = ps.tiles;
    g.ntiles = ps.ntiles;
    g.offsets = ps.offsets;
    g.order = ps.order;
    g.experts_base = a->experts_base;
    g.stride = a->expert_stride;
    g.bias_dt = r->bias_dt;
    g.act_kind = r->act;
    g.limit = r->limit;
    g.alpha = r->alpha;
    {
        const int planes = gw::prefill_planes(a->x_dtype);
        const int64_t nx = (int64_t)T * r->hidden;
        g.in = static_cast<const uint16_t *>(a->x);
        g.in_plane = nx;
        if (planes > 1) {
            ProfScope p(ctx, "prefill_split");
            GW_HIP(gw::launch_prefill_split(p.launch(L), a->x, a->x_dtype, nx, ps.xsplit));
            g.in = ps.xsplit;
        }
        g.in_row_div = K;
        g.blocks_off = sec.gu_blocks;
        g.scales_off = sec.gu_scales;
        g.bias_off = sec.gu_bias;
        g.kdim = (int)r->hidden;
        g.fdim = (int)(2 * r->inter);
        g.act_out = ps.act;
        g.y_out = nullptr;
        ProfScope p(ctx, "prefill_gate_up");
        GW_HIP(gw::launch_prefill_gemm(p.launch(L), true, planes, g, max_tiles, T * K));
    }
    {
        g.sg_logits = nullptr;
        g.sg_ids = self_group ? ps.ids : nullptr;
        g.in = ps.act;
        g.in_plane = (int64_t)T * K * r->inter;
        g.in_row_div = 1;
        g.blocks_off = sec.dn_blocks;
        g.scales_off = sec.dn_scales;
        g.bias_off = sec.dn_bias;
        g.kdim = (int)r->inter;
        g.fdim = (int)r->hidden;
        g.act_out = nullptr;
        g.y_out = ps.y;
        g.y_bytes = (int64_t)sizeof(float) * T * K * r->hidden;
        if (fuse_combine) {
            if (use_static) {
                // The array holds the previous call's bytes: the counters
                // start from zero by a fill kernel (no memset node in a
                // captured graph).
                ProfScope p(ctx, "prefill_clear");
                GW_HIP(gw::launch_fill_u8(
                    p.launch(L), ps.arrive,
                    sizeof(uint32_t) * (size_t)gw::prefill_arrive_count(T, (int)r->hidden), 1, 0,
                    0, 0, 0));
            }
            g.arrive = ps.arrive;
            g.arrive_count = gw::prefill_arrive_count(T, (int)r->hidden);
            g.comb_tokens = T;
            g.comb_w = ps.weights;
            g.comb_out = a->out;
            g.comb_out_bf16 = a->out_bf16;
            g.comb_topk = K;
            g.comb_residual = out_mode == 2 ? 1 : 0;
        }
        ProfScope p(ctx, "prefill_down");
        GW_HIP(gw::launch_prefill_gemm(p.launch(L), false, 1, g, max_tiles, T * K));
    }
    if (!fuse_combine) {
        ProfScope p(ctx, "prefill_combine");
        GW_HIP(gw::launch_prefill_combine(p.launch(L), ps.y, ps.weights, T, K, (int)r->hidden,
                                          a->out, a->out_bf16, out_mode == 2 ? 1 : 0));
    }
    if (a->routing_ids)
        GW_HIP(hipMemcpyAsync(a->routing_ids, ps.ids, sizeof(int32_t) * T * K,
                              hipMemcpyDeviceToDevice, ctx->stream));
    if (a->routing_weights)
        GW_HIP(hipMemcpyAsync(a->routing_weights, ps.weights, sizeof(float) * T * K,
                              hipMemcpyDeviceToDevice, ctx->stream));
    if (!use_static) {
        r->pf_last_tokens = T;
        r->pf_last_topk = K;
    }
    return GW_OK;
}

extern "C" int gw_moe_prefill_forward(gw_expert_runner *r, const gw_moe_layer_args *a)
{
    return moe_prefill_impl(r, a, 0);
}

extern "C" int gw_expert_runner_prefill_view(gw_expert_runner *r, gw_prefill_view *v)
{
    GW_CHECK(r && v, GW_ERR_ARG, "null argument");
    GW_CHECK(r->pf_buf && r->pf_last_tokens > 0, GW_ERR_ARG,
             "no batch has run through this runner's prefill scratch");
    PrefillScratch ps;
    prefill_layout(r, r->pf_tokens, r->pf_topk, r->pf_experts, static_cast<char *>(r->pf_buf),
                   &ps);
    v->routing_ids = ps.ids;
    v->routing_weights = ps.weights;
    v->activations = ps.act;
    v->activation_plane = 0;
    v->expert_outputs = ps.y;
    v->tokens = r->pf_last_tokens;
    v->top_k = r->pf_last_topk;
    return GW_OK;
}

extern "C" int gw_moe_prefill_forward_static(gw_expert_runner *r, const gw_moe_layer_args *a)
{
    return moe_prefill_impl(r, a, 0, true);
}

// ---------------------------------------------------------------------------
// the MoE block with its surroundings: RMSNorm before, residual add after
// ---------------------------------------------------------------------------

extern "C" int gw_moe_block_forward(gw_expert_runner *r, const gw_moe_block_args *b)
{
    GW_CHECK(r && b, GW_ERR_ARG, "null argument");
    GW_CHECK(b->stream && b->norm_weight, GW_ERR_ARG, "null stream or norm weight");
    GW_CHECK(b->norm_weight_dtype == GW_BF16 || b->norm_weight_dtype == GW_F32, GW_ERR_ARG,
             "norm weight must be bf16 or fp32");
    GW_CHECK(b->epsilon >= 0.0f, GW_ERR_ARG, "epsilon must be non-negative");
    const int T = b->layer.tokens;
    GW_CHECK(T >= 1, GW_ERR_SHAPE, "tokens must be positive (got %d)", T);
    gw_context *ctx = r->ctx;
    uint16_t *normed = r->normed_buf;
    if (T > gw::kMaxTokens) {
        // The batched path: normalised rows live in the prefill scratch.
        int rc = gw_expert_runner_reserve_prefill(r, T, (int)b->layer.top_k,
                                                  (int)b->layer.expert_count);
        if (rc) return rc;
        PrefillScratch ps;
        prefill_layout(r, r->pf_tokens, r->pf_topk, r->pf_experts,
                       static_cast<char *>(r->pf_buf), &ps);
        normed = ps.normed;
    }
    const gw::Launch L = launch_of(ctx);
    {
        ProfScope ps(ctx, "rmsnorm");
        GW_HIP(gw::launch_rmsnorm(ps.launch(L), b->stream, b->norm_weight, b->norm_weight_dtype,
                                  T, (int)r->hidden, b->epsilon, normed));
    }
    gw_moe_layer_args a = b->layer;
    a.x = normed;
    a.x_dtype = GW_F16;
    a.out = b->stream;
    return moe_layer_impl(r, &a, 2);
}

// ---------------------------------------------------------------------------
// graphs
// ---------------------------------------------------------------------------

struct gw_graph {
    gw_context *ctx;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

extern "C" int gw_graph_begin_capture(gw_context *ctx)
{
    GW_CHECK(ctx, GW_ERR_ARG, "context is null");
    GW_CHECK(!ctx->capturing, GW_ERR_ARG, "already capturing");
    GW_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return GW_OK;
}

extern "C" int gw_graph_end_capture(gw_context *ctx, gw_graph **out)
{
    GW_CHECK(ctx && out, GW_ERR_ARG, "null argument");
    GW_CHECK(ctx->capturing, GW_ERR_ARG, "not capturing");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    GW_HIP(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(GW_ERR_HIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
    }
    gw_graph *gr = new gw_graph{ctx, g, ex};
    *out = gr;
    return GW_OK;
}

extern "C" int gw_graph_launch(gw_graph *g)
{
    GW_CHECK(g, GW_ERR_ARG, "graph is null");
    GW_HIP(hipGraphLaunch(g->exec, g->ctx->stream));
    return GW_OK;
}

extern "C" int gw_graph_destroy(gw_graph *g)
{
    if (!g) return GW_OK;
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
    return GW_OK;
}
