// gw_kernels.hip — gfx950 kernels of the MXFP4 MoE expert hot path.
//
// Decode is HBM-bound (about 3.7 flop per byte), so every kernel here is a
// streaming GEMV built around one mapping ("row segments"):
//   * a 256-thread workgroup works on RG = 256/TPR rows at a time, TPR lanes
//     per row; lane l of a row owns column blocks l, l+TPR, ... (M of them),
//     so each wave-wide load is TPR contiguous 16-byte blocks per row;
//   * the activation vector(s) sit in LDS, widened weights are dotted against
//     them with v_dot2c_f32_{bf16,f16} (or v_fma_f32 for f32 x), one fp32
//     partial per block scaled by its e8m0 scale, accumulated per lane;
//   * the row sum is a TPR-lane shuffle reduction;
//   * loads for the next row group are issued before the current one is
//     consumed (register double buffering), so a workgroup keeps two row
//     groups of weights in flight.
// Rows are split over a fixed grid in contiguous, balanced ranges (the
// reference's persistent kernel, expert.metal:138-183, strides rows over 64
// threadgroups instead).
#include "gw_device.h"
#include "gw_launch.h"

namespace gw {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMMax = 8;   // column blocks per lane per row chunk

RowShape row_shape(int bpr)
{
    // Pick lanes-per-row so M*TPR covers bpr with little waste.
    RowShape s;
    if (bpr <= 8) { s.tpr = 8; s.m = 1; }
    else if (bpr <= 24) { s.tpr = 8; s.m = (bpr + 7) / 8; }
    else { s.tpr = 16; s.m = (bpr + 15) / 16; }
    if (s.m > kMMax) { s.chunks = (bpr + kMMax * s.tpr - 1) / (kMMax * s.tpr); s.m = kMMax; }
    else s.chunks = 1;
    return s;
}

__device__ __forceinline__ void widen_u(const u32x4 &w, WBlock<DT_BF16> &o)
{ uint4 v; v.x = w.x; v.y = w.y; v.z = w.z; v.w = w.w; widen<DT_BF16>(v, o); }
__device__ __forceinline__ void widen_u(const u32x4 &w, WBlock<DT_F16> &o)
{ uint4 v; v.x = w.x; v.y = w.y; v.z = w.z; v.w = w.w; widen<DT_F16>(v, o); }
__device__ __forceinline__ void widen_u(const u32x4 &w, WBlock<DT_F32> &o)
{ uint4 v; v.x = w.x; v.y = w.y; v.z = w.z; v.w = w.w; widen<DT_F32>(v, o); }

// ---------------------------------------------------------------------------
// Row-segment engine
// ---------------------------------------------------------------------------

template <int MT> struct RowRef {
    const uint8_t *packed;   // first block of the row
    const uint8_t *scales;   // first scale byte of the row
    int ntok;                // activation vectors this row is dotted with
    int xoff[MT];            // LDS dword offset of each vector
};

template <int MT> struct Stage {
    u32x4 w[kMMax];
    uint32_t s[kMMax];
    int item, chunk, ntok;
    int xoff[MT];
    bool valid;
};

template <int TPR> __device__ __forceinline__ float seg_sum(float v)
{
#pragma unroll
    for (int o = TPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

template <int MT, int TPR, class RowFn>
__device__ __forceinline__ void issue(Stage<MT> &S, int it, int chunks, int M, int bpr,
                                      int n_items, RowFn &rowfn)
{
    constexpr int RG = kNT / TPR;
    const int rg = it / chunks;
    const int c = it - rg * chunks;
    const int seg = threadIdx.x / TPR, lane = threadIdx.x % TPR;
    const int item = rg * RG + seg;
    S.item = item;
    S.chunk = c;
    S.valid = item < n_items;
    RowRef<MT> ref;
    ref.ntok = 0;
    if (S.valid) ref = rowfn(item);
    S.ntok = ref.ntok;
#pragma unroll
    for (int t = 0; t < MT; ++t) S.xoff[t] = S.valid ? ref.xoff[t] : 0;
    const int cb0 = c * kMMax * TPR + lane;
#pragma unroll
    for (int m = 0; m < kMMax; ++m) {
        const int cb = cb0 + m * TPR;
        if (m < M && S.valid && cb < bpr) {
            S.w[m] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4 *>(ref.packed) + cb);
            S.s[m] = ref.scales[cb];
        }
    }
}

template <int XK, int MT, int TPR, class EpiFn>
__device__ __forceinline__ void consume(Stage<MT> &S, float (&acc)[MT], int chunks, int M,
                                        int bpr, const uint32_t *xs, EpiFn &epi)
{
    constexpr int BD = XL<XK>::kBlockDw;
    const int lane = threadIdx.x % TPR;
    const int cb0 = S.chunk * kMMax * TPR + lane;
#pragma unroll
    for (int m = 0; m < kMMax; ++m) {
        const int cb = cb0 + m * TPR;
        if (m < M && S.valid && cb < bpr) {
            WBlock<XK> wb;
            widen_u(S.w[m], wb);
            const float sc = decode_scale(S.s[m]);
            const uint32_t *xb = xs + cb * BD;
#pragma unroll
            for (int t = 0; t < MT; ++t)
                if (t < S.ntok) acc[t] += block_dot<XK>(wb, xb + S.xoff[t]) * sc;
        }
    }
    if (S.chunk == chunks - 1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = seg_sum<TPR>(acc[t]);
        epi(S.item, S.valid, S.ntok, acc);
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    }
}

// Runs `n_items` rows (RowFn maps item -> RowRef) through the engine, calling
// EpiFn(item, valid, ntok, acc) once per row group with every lane holding its
// row's fp32 sums.  All threads of the workgroup must call it.
template <int XK, int MT, int TPR, class RowFn, class EpiFn>
__device__ __forceinline__ void row_engine(int n_items, int chunks, int M, int bpr,
                                           const uint32_t *xs, RowFn rowfn, EpiFn epi)
{
    constexpr int RG = kNT / TPR;
    const int nit = ((n_items + RG - 1) / RG) * chunks;
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    Stage<MT> A, B;
    if (nit > 0) issue<MT, TPR>(A, 0, chunks, M, bpr, n_items, rowfn);
    for (int it = 0; it < nit; it += 2) {
        if (it + 1 < nit) issue<MT, TPR>(B, it + 1, chunks, M, bpr, n_items, rowfn);
        consume<XK, MT, TPR>(A, acc, chunks, M, bpr, xs, epi);
        if (it + 1 < nit) {
            if (it + 2 < nit) issue<MT, TPR>(A, it + 2, chunks, M, bpr, n_items, rowfn);
            consume<XK, MT, TPR>(B, acc, chunks, M, bpr, xs, epi);
        }
    }
}

__device__ __forceinline__ void copy_plan(Plan *dst, const Plan *src)
{
    const uint32_t *s = reinterpret_cast<const uint32_t *>(src);
    uint32_t *d = reinterpret_cast<uint32_t *>(dst);
    for (int i = threadIdx.x; i < (int)(sizeof(Plan) / 4); i += blockDim.x) d[i] = s[i];
}

// ---------------------------------------------------------------------------
// Standalone GEMV (mxfp4_gemv / mxfp4_gemv_bias*, dequant_gemv.metal:37-67,
// expert.metal:46-368)
// ---------------------------------------------------------------------------

template <int XK, int TPR>
__global__ __launch_bounds__(kNT) void gemv_kernel(const uint8_t *__restrict__ packed,
                                                   const uint8_t *__restrict__ scales,
                                                   const void *__restrict__ bias, int bias_dt,
                                                   const void *__restrict__ x,
                                                   float *__restrict__ y, int rows, int bpr,
                                                   int M, int chunks)
{
    extern __shared__ uint32_t lds[];
    uint32_t *xs = lds;
    stage_vector<XK>(xs, x, bpr * 32);
    __syncthreads();
    const int r0 = (int)((int64_t)blockIdx.x * rows / gridDim.x);
    const int r1 = (int)((int64_t)(blockIdx.x + 1) * rows / gridDim.x);
    const int64_t row_bytes = (int64_t)bpr * 16;
    auto rowfn = [&](int item) {
        RowRef<1> r;
        const int64_t row = r0 + item;
        r.packed = packed + row * row_bytes;
        r.scales = scales + row * bpr;
        r.ntok = 1;
        r.xoff[0] = 0;
        return r;
    };
    auto epi = [&](int item, bool valid, int, float (&acc)[1]) {
        if (valid && (threadIdx.x % TPR) == 0) {
            const int row = r0 + item;
            y[row] = acc[0] + load_bias(bias, bias_dt, row);
        }
    };
    row_engine<XK, 1, TPR>(r1 - r0, chunks, M, bpr, xs, rowfn, epi);
}

// ---------------------------------------------------------------------------
// Fused gate_up GEMV + bias + activation (expert.metal:311-368 then :82-102 or
// :380-393), all groups of a plan.  Rows 2i and 2i+1 of an expert are gate i
// and up i (interleaved, expert.metal:9-17); they are neighbouring segments
// of one wave, so the activation is applied straight from the reduction.
// ---------------------------------------------------------------------------

template <int XK, int MT, int TPR>
__global__ __launch_bounds__(kNT) void gate_up_kernel(
    const Plan *__restrict__ gplan, const void *__restrict__ x, int hidden, int inter,
    Sections sec, int bias_dt, uint16_t *__restrict__ act, int act_kind, float limit,
    float alpha, int max_tokens, int M, int chunks)
{
    extern __shared__ uint32_t lds[];
    constexpr int BD = XL<XK>::kBlockDw;
    constexpr int ES = XK == DT_F32 ? 4 : 2;
    Plan *plan = reinterpret_cast<Plan *>(lds);
    uint32_t *xs = lds + sizeof(Plan) / 4;
    const int bpr = hidden >> 5;
    const int xstride = bpr * BD;
    copy_plan(plan, gplan);
    __syncthreads();
    const int ntokens = plan->ntokens;
    for (int t = 0; t < ntokens && t < max_tokens; ++t)
        stage_vector<XK>(xs + t * xstride,
                         static_cast<const char *>(x) + (int64_t)plan->tok_global[t] * hidden * ES,
                         hidden);
    __syncthreads();

    const int64_t total = (int64_t)plan->ngroups * inter;   // (group, pair) space
    const int64_t p0 = (int64_t)blockIdx.x * total / gridDim.x;
    const int64_t p1 = (int64_t)(blockIdx.x + 1) * total / gridDim.x;
    const int64_t row_bytes = (int64_t)bpr * 16;
    auto rowfn = [&](int item) {
        RowRef<MT> r;
        const int64_t p = p0 + (item >> 1);
        const int g = (int)(p / inter);
        const int64_t row = 2 * (p - (int64_t)g * inter) + (item & 1);
        const uint8_t *base = plan->group_base[g];
        r.packed = base + sec.gu_blocks + row * row_bytes;
        r.scales = base + sec.gu_scales + row * bpr;
        r.ntok = plan->group_ntok[g];
        const int s0 = plan->group_slot0[g];
#pragma unroll
        for (int t = 0; t < MT; ++t)
            r.xoff[t] = t < r.ntok ? plan->slot_token[s0 + t] * xstride : 0;
        return r;
    };
    auto epi = [&](int item, bool valid, int ntok, float (&acc)[MT]) {
        float up[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) up[t] = __shfl_down(acc[t], TPR);
        if (valid && (item & 1) == 0 && (threadIdx.x % TPR) == 0) {
            const int64_t p = p0 + (item >> 1);
            const int g = (int)(p / inter);
            const int64_t i = p - (int64_t)g * inter;
            const uint8_t *base = plan->group_base[g];
            const void *bias = bias_dt >= 0 ? (const void *)(base + sec.gu_bias) : nullptr;
            const float bg = load_bias(bias, bias_dt, 2 * i);
            const float bu = load_bias(bias, bias_dt, 2 * i + 1);
            const int s0 = plan->group_slot0[g];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (t < ntok) {
                    const float v = apply_activation(act_kind, acc[t] + bg, up[t] + bu, limit,
                                                     alpha);
                    act[(int64_t)(s0 + t) * inter + i] = f32_to_f16_bits(v);
                }
            }
        }
    };
    row_engine<XK, MT, TPR>((int)(2 * (p1 - p0)), chunks, M, bpr, xs, rowfn, epi);
}

// ---------------------------------------------------------------------------
// Fused down GEMV + bias + weighted combine (expert.metal:311-368 then
// :107-116).  A workgroup owns output rows [r0, r1) for every group, so the
// combine happens in LDS without atomics, in each token's slot order.
// ---------------------------------------------------------------------------

template <int MT, int TPR>
__global__ __launch_bounds__(kNT) void down_kernel(
    const Plan *__restrict__ gplan, const uint16_t *__restrict__ act, int hidden, int inter,
    Sections sec, int bias_dt, float *__restrict__ out, uint16_t *__restrict__ out_bf16,
    int accumulate, int smax, int nmax, int M, int chunks)
{
    extern __shared__ uint32_t lds[];
    constexpr int BD = XL<DT_F16>::kBlockDw;
    Plan *plan = reinterpret_cast<Plan *>(lds);
    const int bpr = inter >> 5;
    const int astride = bpr * BD;
    uint32_t *as = lds + sizeof(Plan) / 4;                          // [smax][astride]
    float *vals = reinterpret_cast<float *>(as + smax * astride);   // [kMaxSlots][nmax]
    copy_plan(plan, gplan);
    __syncthreads();

    const int r0 = (int)((int64_t)blockIdx.x * hidden / gridDim.x);
    const int r1 = (int)((int64_t)(blockIdx.x + 1) * hidden / gridDim.x);
    const int n = r1 - r0;
    const int ngroups = plan->ngroups;
    const int64_t row_bytes = (int64_t)bpr * 16;

    int g = 0;
    while (g < ngroups) {
        // Next chunk of whole groups whose slots fit the LDS staging area.
        const int s0 = plan->group_slot0[g];
        int g1 = g, s1 = s0;
        while (g1 < ngroups && s1 + plan->group_ntok[g1] - s0 <= smax) {
            s1 += plan->group_ntok[g1];
            ++g1;
        }
        if (g1 == g) break;   // a group wider than the staging area (the host prevents it)
        for (int s = s0; s < s1; ++s)
            stage_vector<DT_F16>(as + (s - s0) * astride, act + (int64_t)s * inter, inter);
        __syncthreads();
        const int gbase = g;
        auto rowfn = [&](int item) {
            RowRef<MT> r;
            const int gl = item / n;
            const int q = item - gl * n;
            const int gg = gbase + gl;
            const uint8_t *base = plan->group_base[gg];
            const int64_t row = r0 + q;
            r.packed = base + sec.dn_blocks + row * row_bytes;
            r.scales = base + sec.dn_scales + row * bpr;
            r.ntok = plan->group_ntok[gg];
            const int sl = plan->group_slot0[gg] - s0;
#pragma unroll
            for (int t = 0; t < MT; ++t) r.xoff[t] = (sl + (t < r.ntok ? t : 0)) * astride;
            return r;
        };
        auto epi = [&](int item, bool valid, int ntok, float (&acc)[MT]) {
            if (valid && (threadIdx.x % TPR) == 0) {
                const int gl = item / n;
                const int q = item - gl * n;
                const int gg = gbase + gl;
                const void *bias = bias_dt >= 0
                                       ? (const void *)(plan->group_base[gg] + sec.dn_bias)
                                       : nullptr;
                const float b = load_bias(bias, bias_dt, r0 + q);
                const int sg = plan->group_slot0[gg];
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    if (t < ntok) vals[(sg + t) * nmax + q] = acc[t] + b;
            }
        };
        row_engine<DT_F16, MT, TPR>((g1 - g) * n, chunks, M, bpr, as, rowfn, epi);
        __syncthreads();
        g = g1;
    }

    // Weighted combine in each token's slot order: dst += out * w, the product
    // and the sum rounded separately as expert_accumulate does.
    const int ntokens = plan->ntokens;
    for (int p = threadIdx.x; p < ntokens * n; p += kNT) {
        const int t = p / n;
        const int q = p - t * n;
        const int64_t o = (int64_t)plan->tok_global[t] * hidden + r0 + q;
        float dst = accumulate ? out[o] : 0.0f;
        for (int k = 0; k < plan->tok_nslots[t]; ++k) {
            const int s = plan->tok_slots[t][k];
            dst = add_scaled_rn(dst, vals[s * nmax + q], plan->slot_weight[s]);
        }
        out[o] = dst;
        if (out_bf16) out_bf16[o] = f32_to_bf16_bits(dst);
    }
}

// ---------------------------------------------------------------------------
// Router: logits (bf16_gemv_bias, router.metal:18-34) and selection + plan
// (Router.select, Router.swift:78-98; demand map, TransformerLayer.swift:175-181)
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void router_kernel(const void *__restrict__ W, int w_dt,
                                                     const void *__restrict__ b, int b_dt,
                                                     const void *__restrict__ x, int x_dt,
                                                     float *__restrict__ logits, int E, int H,
                                                     int T)
{
    const int wave = blockIdx.x * 4 + threadIdx.x / 64;
    const int lane = threadIdx.x & 63;
    if (wave >= E * T) return;
    const int t = wave / E, e = wave - (wave / E) * E;
    float acc = 0.0f;
    for (int c = lane; c < H; c += 64)
        acc += load_as_f32(W, w_dt, (int64_t)e * H + c) * load_as_f32(x, x_dt, (int64_t)t * H + c);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (lane == 0) logits[(int64_t)t * E + e] = acc + (b ? load_as_f32(b, b_dt, e) : 0.0f);
}

constexpr int kMaxExperts = 1024;

// One wave.  Selection replicates the reference's partial selection sort
// exactly, including its tie behaviour: at position p the sort keeps the
// first position (in the partially permuted order) holding the largest
// non-NaN logit, or p itself when logits[order[p]] is NaN.
__global__ __launch_bounds__(64) void route_kernel(const float *__restrict__ logits, int E,
                                                   int K, int T,
                                                   const uint8_t *__restrict__ experts_base,
                                                   int64_t stride, Plan *__restrict__ plan,
                                                   int32_t *__restrict__ ids_out,
                                                   float *__restrict__ w_out)
{
    __shared__ float lg[kMaxExperts];
    __shared__ int ord[kMaxExperts];
    __shared__ int sel_id[kMaxSlots];
    __shared__ float sel_w[kMaxSlots];
    __shared__ int first_of[kMaxSlots];
    const int lane = threadIdx.x;

    for (int t = 0; t < T; ++t) {
        for (int i = lane; i < E; i += 64) {
            lg[i] = logits[(int64_t)t * E + i];
            ord[i] = i;
        }
        __syncthreads();
        for (int pos = 0; pos < K; ++pos) {
            float bv = 0.0f;
            int bp = -1;
            for (int i = pos + lane; i < E; i += 64) {
                const float v = lg[ord[i]];
                if (!__builtin_isnan(v) && (bp < 0 || v > bv)) { bv = v; bp = i; }
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) {
                const float ov = __shfl_xor(bv, o);
                const int op = __shfl_xor(bp, o);
                const bool take = op >= 0 && (bp < 0 || ov > bv || (ov == bv && op < bp));
                bv = take ? ov : bv;
                bp = take ? op : bp;
            }
            if (lane == 0) {
                int best = bp;
                if (__builtin_isnan(lg[ord[pos]]) || best < 0) best = pos;
                const int tmp = ord[pos];
                ord[pos] = ord[best];
                ord[best] = tmp;
            }
            __syncthreads();
        }
        if (lane == 0) {
            float peak = 0.0f;
            for (int i = 0; i < K; ++i) {
                const float v = lg[ord[i]];
                if (i == 0 || v > peak) peak = v;
            }
            float e[kMaxTopK];
            float total = 0.0f;
            for (int i = 0; i < K; ++i) { e[i] = expf(lg[ord[i]] - peak); total += e[i]; }
            for (int i = 0; i < K; ++i) {
                sel_id[t * K + i] = ord[i];
                sel_w[t * K + i] = e[i] / total;
                if (ids_out) ids_out[(int64_t)t * K + i] = ord[i];
                if (w_out) w_out[(int64_t)t * K + i] = e[i] / total;
            }
        }
        __syncthreads();
    }

    // Expert-major grouping of the T*K (token, rank) entries by first appearance.
    const int n = T * K;
    int my_e = -1, first = lane, before = 0, same = 0;
    if (lane < n) {
        my_e = sel_id[lane];
        first = -1;
        for (int j = 0; j < n; ++j) {
            if (sel_id[j] == my_e) {
                if (first < 0) first = j;
                if (j < lane) ++before;
                ++same;
            }
        }
        first_of[lane] = first;
    }
    __syncthreads();
    const bool leader = lane < n && first == lane;
    const unsigned long long leaders = __ballot(leader);
    if (lane < n) {
        const int gi = __popcll(leaders & ((1ull << first) - 1ull));
        int slot0 = 0;
        for (int j = 0; j < n; ++j) slot0 += first_of[j] < first ? 1 : 0;
        const int slot = slot0 + before;
        const int t = lane / K, r = lane - (lane / K) * K;
        plan->slot_token[slot] = t;
        plan->slot_group[slot] = gi;
        plan->slot_weight[slot] = sel_w[lane];
        plan->tok_slots[t][r] = slot;
        if (leader) {
            plan->group_base[gi] = experts_base + (int64_t)my_e * stride;
            plan->group_slot0[gi] = slot0;
            plan->group_ntok[gi] = same;
        }
    }
    if (lane < T) {
        plan->tok_global[lane] = lane;
        plan->tok_nslots[lane] = K;
    }
    if (lane == 0) {
        plan->ngroups = __popcll(leaders);
        plan->nslots = n;
        plan->ntokens = T;
        plan->pad0 = 0;
    }
}

// ---------------------------------------------------------------------------
// Element-wise kernels
// ---------------------------------------------------------------------------

// mxfp4_dequant_reference / _wide (mxfp4.metal:36-77), fp32 out, through the
// same widening instruction the GEMVs use: one thread per 4 packed bytes.
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t *__restrict__ packed,
                                                      const uint8_t *__restrict__ scales,
                                                      int64_t words, float4 *__restrict__ out)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const uint32_t w = packed[i];
    const float s = decode_scale(scales[i >> 2]);
    const f32x2 a = GW_CVT_F32(w, 0), b = GW_CVT_F32(w, 1);
    const f32x2 c = GW_CVT_F32(w, 2), d = GW_CVT_F32(w, 3);
    out[2 * i] = make_float4(a.x * s, a.y * s, b.x * s, b.y * s);
    out[2 * i + 1] = make_float4(c.x * s, c.y * s, d.x * s, d.y * s);
}

__global__ __launch_bounds__(256) void activation_kernel(int kind,
                                                         const float *__restrict__ gate_up,
                                                         uint16_t *__restrict__ out,
                                                         int64_t width, float limit,
                                                         float alpha)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= width) return;
    out[i] = f32_to_f16_bits(apply_activation(kind, gate_up[2 * i], gate_up[2 * i + 1],
                                              limit, alpha));
}

__global__ __launch_bounds__(256) void accumulate_kernel(const float *__restrict__ src,
                                                         float *__restrict__ dst, float w,
                                                         int64_t width)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= width) return;
    dst[i] = add_scaled_rn(dst[i], src[i], w);
}

// Counter-based generator: splitmix64 finaliser of (seed, index).
__device__ __forceinline__ uint64_t mix64(uint64_t z)
{
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ __launch_bounds__(256) void fill_u8_kernel(uint8_t *__restrict__ dst, int64_t count,
                                                      uint32_t lo, uint32_t range,
                                                      uint64_t seed)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // 8 bytes each
    const int64_t b0 = i * 8;
    if (b0 >= count) return;
    const uint64_t h0 = mix64(seed ^ mix64((uint64_t)i * 2));
    const uint64_t h1 = mix64(seed ^ mix64((uint64_t)i * 2 + 1));
    uint64_t word = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t r16 = (uint32_t)(((k < 4 ? h0 : h1) >> (16 * (k & 3))) & 0xFFFFu);
        const uint32_t v = lo + ((r16 * range) >> 16);
        word |= (uint64_t)(v & 0xFFu) << (8 * k);
    }
    if (b0 + 8 <= count && (reinterpret_cast<uintptr_t>(dst) & 7) == 0) {
        *reinterpret_cast<uint64_t *>(dst + b0) = word;
    } else {
        for (int k = 0; k < 8 && b0 + k < count; ++k) dst[b0 + k] = (uint8_t)(word >> (8 * k));
    }
}

__global__ __launch_bounds__(256) void fill_normal_kernel(void *__restrict__ dst, int dt,
                                                          int64_t count, float mean,
                                                          float stddev, uint64_t seed)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const uint64_t h = mix64(seed ^ mix64((uint64_t)i));
    const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);        // (0, 1]
    const float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);  // [0, 1)
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    const float v = mean + stddev * z;
    if (dt == DT_F32) static_cast<float *>(dst)[i] = v;
    else if (dt == DT_BF16) static_cast<uint16_t *>(dst)[i] = f32_to_bf16_bits(v);
    else static_cast<uint16_t *>(dst)[i] = f32_to_f16_bits(v);
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------

static inline int div_up(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

hipError_t launch_dequant(const Launch &L, const uint8_t *packed, const uint8_t *scales,
                          int64_t blocks, float *out)
{
    const int64_t words = blocks * 4;
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(dequant_kernel, dim3(div_up(words, 256)), dim3(256), 0, L.stream,
                       reinterpret_cast<const uint32_t *>(packed), scales, words,
                       reinterpret_cast<float4 *>(out));
    return hipGetLastError();
}

static int x_block_dw(int x_dt) { return x_dt == DT_F32 ? 36 : 20; }

template <int XK>
static hipError_t gemv_dispatch(const Launch &L, const RowShape &s, dim3 grid, size_t lds,
                                const uint8_t *packed, const uint8_t *scales, const void *bias,
                                int bias_dt, const void *x, float *y, int rows, int bpr)
{
    if (s.tpr == 8)
        hipLaunchKernelGGL((gemv_kernel<XK, 8>), grid, dim3(kNT), lds, L.stream, packed, scales,
                           bias, bias_dt, x, y, rows, bpr, s.m, s.chunks);
    else
        hipLaunchKernelGGL((gemv_kernel<XK, 16>), grid, dim3(kNT), lds, L.stream, packed,
                           scales, bias, bias_dt, x, y, rows, bpr, s.m, s.chunks);
    return hipGetLastError();
}

hipError_t launch_gemv(const Launch &L, const uint8_t *packed, const uint8_t *scales,
                       const void *bias, int bias_dt, const void *x, int x_dt, float *y,
                       int rows, int cols)
{
    if (rows == 0) return hipSuccess;
    const int bpr = cols / 32;
    const RowShape s = row_shape(bpr);
    const int rg = kNT / s.tpr;
    int grid = L.grid_a > 0 ? L.grid_a : 2 * L.cus;
    grid = grid < div_up(rows, rg) ? grid : div_up(rows, rg);
    const size_t lds = (size_t)bpr * x_block_dw(x_dt) * 4;
    if (x_dt == DT_F32)
        return gemv_dispatch<DT_F32>(L, s, dim3(grid), lds, packed, scales, bias, bias_dt, x, y,
                                     rows, bpr);
    if (x_dt == DT_F16)
        return gemv_dispatch<DT_F16>(L, s, dim3(grid), lds, packed, scales, bias, bias_dt, x, y,
                                     rows, bpr);
    return gemv_dispatch<DT_BF16>(L, s, dim3(grid), lds, packed, scales, bias, bias_dt, x, y,
                                  rows, bpr);
}

int gate_up_lds_bytes(int hidden, int x_dt, int max_tokens)
{
    return (int)sizeof(Plan) + max_tokens * (hidden / 32) * x_block_dw(x_dt) * 4;
}

template <int XK, int MT>
static hipError_t gate_up_dispatch(const Launch &L, const RowShape &s, dim3 grid, size_t lds,
                                   const Plan *plan, int max_tokens, const void *x, int hidden,
                                   int inter, const Sections &sec, int bias_dt, uint16_t *act,
                                   int act_kind, float limit, float alpha)
{
    if (s.tpr == 8)
        hipLaunchKernelGGL((gate_up_kernel<XK, MT, 8>), grid, dim3(kNT), lds, L.stream, plan, x,
                           hidden, inter, sec, bias_dt, act, act_kind, limit, alpha,
                           max_tokens, s.m, s.chunks);
    else
        hipLaunchKernelGGL((gate_up_kernel<XK, MT, 16>), grid, dim3(kNT), lds, L.stream, plan,
                           x, hidden, inter, sec, bias_dt, act, act_kind, limit, alpha,
                           max_tokens, s.m, s.chunks);
    return hipGetLastError();
}

hipError_t launch_gate_up(const Launch &L, const Plan *plan, int max_tokens, const void *x,
                          int x_dt, int hidden, int inter, const Sections &sec, int bias_dt,
                          uint16_t *act, int act_kind, float limit, float alpha)
{
    const RowShape s = row_shape(hidden / 32);
    const int grid = L.grid_a > 0 ? L.grid_a : 2 * L.cus;
    const size_t lds = (size_t)gate_up_lds_bytes(hidden, x_dt, max_tokens);
    const bool one = max_tokens == 1;
#define GW_GU(XK)                                                                             \
    return one ? gate_up_dispatch<XK, 1>(L, s, dim3(grid), lds, plan, max_tokens, x, hidden, \
                                         inter, sec, bias_dt, act, act_kind, limit, alpha)   \
               : gate_up_dispatch<XK, kMaxTokens>(L, s, dim3(grid), lds, plan, max_tokens,   \
                                                  x, hidden, inter, sec, bias_dt, act,       \
                                                  act_kind, limit, alpha)
    if (x_dt == DT_F32) { GW_GU(DT_F32); }
    if (x_dt == DT_F16) { GW_GU(DT_F16); }
    GW_GU(DT_BF16);
#undef GW_GU
}

int down_lds_bytes(int hidden, int inter, int grid, int smax)
{
    const int nmax = (hidden + grid - 1) / grid;
    return (int)sizeof(Plan) + smax * (inter / 32) * 20 * 4 + kMaxSlots * nmax * 4;
}

hipError_t launch_down(const Launch &L, const Plan *plan, int max_tokens, int max_slots,
                       const uint16_t *act, int hidden, int inter, const Sections &sec,
                       int bias_dt, float *out, uint16_t *out_bf16, int accumulate)
{
    const RowShape s = row_shape(inter / 32);
    int grid = L.grid_b > 0 ? L.grid_b : L.cus;
    if (grid > hidden) grid = hidden;
    // As many staged slots as fit the LDS budget, at least a full group.
    int smax = max_slots;
    while (smax > 1 && down_lds_bytes(hidden, inter, grid, smax) > kLdsBudget) --smax;
    const int need = max_tokens < kMaxTokens ? max_tokens : kMaxTokens;
    while (smax < need && grid < hidden) {   // shrink rows per workgroup instead
        grid *= 2;
        if (grid > hidden) grid = hidden;
        smax = max_slots;
        while (smax > 1 && down_lds_bytes(hidden, inter, grid, smax) > kLdsBudget) --smax;
    }
    if (smax < need) return hipErrorInvalidValue;
    const int nmax = (hidden + grid - 1) / grid;
    const size_t lds = (size_t)down_lds_bytes(hidden, inter, grid, smax);
    if (max_tokens == 1) {
        if (s.tpr == 8)
            hipLaunchKernelGGL((down_kernel<1, 8>), dim3(grid), dim3(kNT), lds, L.stream, plan,
                               act, hidden, inter, sec, bias_dt, out, out_bf16, accumulate, smax,
                               nmax, s.m, s.chunks);
        else
            hipLaunchKernelGGL((down_kernel<1, 16>), dim3(grid), dim3(kNT), lds, L.stream, plan,
                               act, hidden, inter, sec, bias_dt, out, out_bf16, accumulate, smax,
                               nmax, s.m, s.chunks);
    } else {
        if (s.tpr == 8)
            hipLaunchKernelGGL((down_kernel<kMaxTokens, 8>), dim3(grid), dim3(kNT), lds,
                               L.stream, plan, act, hidden, inter, sec, bias_dt, out, out_bf16,
                               accumulate, smax, nmax, s.m, s.chunks);
        else
            hipLaunchKernelGGL((down_kernel<kMaxTokens, 16>), dim3(grid), dim3(kNT), lds,
                               L.stream, plan, act, hidden, inter, sec, bias_dt, out, out_bf16,
                               accumulate, smax, nmax, s.m, s.chunks);
    }
    return hipGetLastError();
}

hipError_t launch_activation(const Launch &L, int kind, const float *gate_up, uint16_t *out,
                             int64_t width, float limit, float alpha)
{
    if (width == 0) return hipSuccess;
    hipLaunchKernelGGL(activation_kernel, dim3(div_up(width, 256)), dim3(256), 0, L.stream,
                       kind, gate_up, out, width, limit, alpha);
    return hipGetLastError();
}

hipError_t launch_accumulate(const Launch &L, const float *src, float *dst, float w,
                             int64_t width)
{
    if (width == 0) return hipSuccess;
    hipLaunchKernelGGL(accumulate_kernel, dim3(div_up(width, 256)), dim3(256), 0, L.stream,
                       src, dst, w, width);
    return hipGetLastError();
}

hipError_t launch_router(const Launch &L, const void *W, int w_dt, const void *b, int b_dt,
                         const void *x, int x_dt, float *logits, int experts, int hidden,
                         int tokens)
{
    const int waves = experts * tokens;
    if (waves == 0) return hipSuccess;
    hipLaunchKernelGGL(router_kernel, dim3(div_up(waves, 4)), dim3(256), 0, L.stream, W, w_dt,
                       b, b_dt, x, x_dt, logits, experts, hidden, tokens);
    return hipGetLastError();
}

hipError_t launch_route(const Launch &L, const float *logits, int experts, int top_k,
                        int tokens, const uint8_t *experts_base, int64_t stride, Plan *plan,
                        int32_t *ids_out, float *w_out)
{
    if (experts > kMaxExperts || top_k > kMaxTopK || tokens > kMaxTokens || top_k > experts)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(route_kernel, dim3(1), dim3(64), 0, L.stream, logits, experts, top_k,
                       tokens, experts_base, stride, plan, ids_out, w_out);
    return hipGetLastError();
}

hipError_t launch_fill_u8(const Launch &L, void *dst, size_t count, int lo, int hi,
                          uint64_t seed)
{
    if (count == 0) return hipSuccess;
    const int64_t threads = ((int64_t)count + 7) / 8;
    const uint32_t range = (uint32_t)(hi - lo + 1);
    hipLaunchKernelGGL(fill_u8_kernel, dim3(div_up(threads, 256)), dim3(256), 0, L.stream,
                       static_cast<uint8_t *>(dst), (int64_t)count, (uint32_t)lo, range, seed);
    return hipGetLastError();
}

hipError_t launch_fill_normal(const Launch &L, void *dst, int dt, size_t count, float mean,
                              float stddev, uint64_t seed)
{
    if (count == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_normal_kernel, dim3(div_up((int64_t)count, 256)), dim3(256), 0,
                       L.stream, dst, dt, (int64_t)count, mean, stddev, seed);
    return hipGetLastError();
}

}  // namespace gw
