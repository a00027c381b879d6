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
//   * a ring of row groups (stages) in registers keeps several groups' loads
//     in flight; on the decode shapes the ring holds a workgroup's whole share,
//     so every load goes out at once and compute follows the data.
// Rows are split over a fixed grid in contiguous, balanced ranges (the
// reference's persistent kernel, expert.metal:138-183, strides rows over 64
// threadgroups instead).
#include <hip/hip_ext.h>

#include <type_traits>

#include "gw_device.h"
#include "gw_launch.h"
#include "gw_route.h"

namespace gw {


typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Weight streams are read through explicitly global (address space 1)
// pointers.  Expert bases come out of the LDS-resident plan as generic
// pointers; left generic, the loads become flat loads, which also count
// against lgkmcnt, so every LDS read of the activations would wait for all
// outstanding weight loads and the double buffering below would be lost.
typedef const __attribute__((address_space(1))) u32x4 g_u32x4;
typedef const __attribute__((address_space(1))) uint8_t g_u8;

__device__ __forceinline__ u32x4 load_block(const uint8_t *row, int cb)
{
    return __builtin_nontemporal_load((g_u32x4 *)row + cb);
}

__device__ __forceinline__ uint32_t load_scale(const uint8_t *row, int cb)
{
    return ((g_u8 *)row)[cb];
}

// Shape classes: TPR lanes per row, M column blocks per lane (per chunk of
// M*TPR blocks).  Compile-time, so every stage issues a fixed number of loads
// and the compiler can wait for exactly the older stage (s_waitcnt vmcnt(N))
// instead of draining the prefetched one too.
template <int TPR_, int M_, bool CHUNKED_ = false> struct Shape {
    static constexpr int TPR = TPR_;
    static constexpr int M = M_;
    static constexpr bool CHUNKED = CHUNKED_;   // rows may span several chunks
};
using S0 = Shape<8, 1>;    // bpr <= 8
using S1 = Shape<8, 3>;    // bpr <= 24   (Qwen3 down: 24)
using S2 = Shape<16, 4>;   // bpr <= 64   (Qwen3 gate_up: 64)
using S3 = Shape<16, 6>;   // bpr <= 96   (GPT-OSS: 90)
using S4 = Shape<16, 8, true>;   // wider rows, in chunks of 128 blocks

// A lane sees the same activation blocks in every stage (blocks lane + m*TPR
// of one chunk), so when every row is dotted with the same 16-bit vector
// (UNIFORM: one token, one shared input) and rows are unchunked, the blocks
// are read from LDS once, into registers, instead of once per stage.  (The
// down projection dots each expert's rows with that expert's own activation,
// so it never qualifies.)
template <int XK, int MT, class SH, bool UNIFORM> struct XRegs {
    static constexpr bool kOn = UNIFORM && MT == 1 && XK != DT_F32 && !SH::CHUNKED;
    uint4 v[kOn ? SH::M : 1][4];
};

// Stages in flight per engine: a decode workgroup's gate_up share is three
// 16-row stages (GPT-OSS, 512 workgroups) and its down share two.
constexpr int kGateUpDepth = 3;
constexpr int kDownDepth = 2;
constexpr int kGemvDepth = 3;

RowShape row_shape(int bpr)
{
    RowShape s;
    s.chunks = 1;
    if (bpr <= 8) { s.tpr = 8; s.m = 1; }
    else if (bpr <= 24) { s.tpr = 8; s.m = 3; }
    else if (bpr <= 64) { s.tpr = 16; s.m = 4; }
    else if (bpr <= 96) { s.tpr = 16; s.m = 6; }
    else { s.tpr = 16; s.m = 8; s.chunks = (bpr + 127) / 128; }
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
    const uint8_t *bias;     // the row's bias element (any readable address if none)
    int ntok;                // activation vectors this row is dotted with
    int xoff[MT];            // LDS dword offset of each vector
};

template <int MT, int M> struct Stage {
    u32x4 w[M];
    uint32_t s[M];
    uint32_t bw;             // aligned dword holding the row's bias
    int bshift;              // bit offset of a bf16 bias within bw
    int item, chunk, ntok;
    int xoff[MT];
    bool valid;
};

// The bias element is read with the stage as the aligned dword containing it
// (one load whatever the dtype), so the epilogue needs no young load.
__device__ __forceinline__ float decode_bias(uint32_t bw, int bshift, int bias_dt)
{
    if (bias_dt < 0) return 0.0f;
    if (bias_dt == DT_F32) return __uint_as_float(bw);
    const uint16_t b = (uint16_t)(bw >> bshift);
    return bias_dt == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Issues the M block loads (and M scale loads) of one stage.  Every lane issues
// all of them: a column past the end re-reads the row's last block, and a row
// past the end reads the last row's first block on every lane (one cache line
// per load instruction); consume() ignores those values.
template <int MT, class SH, class RowFn>
__device__ __forceinline__ void issue(Stage<MT, SH::M> &S, int it, int chunks, int bpr,
                                      int n_items, RowFn &rowfn)
{
    constexpr int TPR = SH::TPR, M = SH::M, RG = kNT / TPR;
    const int rg = chunks == 1 ? it : it / chunks;
    const int c = it - rg * chunks;
    const int seg = threadIdx.x / TPR, lane = threadIdx.x % TPR;
    const int item = rg * RG + seg;
    S.item = item;
    S.chunk = c;
    S.valid = item < n_items;
    const RowRef<MT> ref = rowfn(S.valid ? item : n_items - 1);
    S.ntok = S.valid ? ref.ntok : 0;
#pragma unroll
    for (int t = 0; t < MT; ++t) S.xoff[t] = ref.xoff[t];
    const int cb0 = c * M * TPR + lane;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int cb = S.valid ? min(cb0 + m * TPR, bpr - 1) : 0;
        S.w[m] = load_block(ref.packed, cb);
        S.s[m] = load_scale(ref.scales, cb);
    }
    const uintptr_t ba = reinterpret_cast<uintptr_t>(ref.bias);
    S.bshift = (int)(ba & 2u) * 8;
    S.bw = *(const __attribute__((address_space(1))) uint32_t *)(ba & ~(uintptr_t)3);
}

template <int XK, int MT, class SH, bool U>
__device__ __forceinline__ void load_xregs(XRegs<XK, MT, SH, U> &X, const uint32_t *xs, int bpr)
{
    if constexpr (XRegs<XK, MT, SH, U>::kOn) {
        constexpr int BD = XL<XK>::kBlockDw;
        const int lane = threadIdx.x % SH::TPR;
#pragma unroll
        for (int m = 0; m < SH::M; ++m) {
            const int cb = lane + m * SH::TPR;
            const uint4 *xv = reinterpret_cast<const uint4 *>(xs + (cb < bpr ? cb : 0) * BD);
#pragma unroll
            for (int q = 0; q < 4; ++q) X.v[m][q] = xv[q];
        }
    }
}

template <int XK, int MT, class SH, bool U, class EpiFn>
__device__ __forceinline__ void consume(Stage<MT, SH::M> &S, float (&acc)[MT], int chunks,
                                        int bpr, const uint32_t *xs,
                                        const XRegs<XK, MT, SH, U> &X, EpiFn &epi)
{
    constexpr int TPR = SH::TPR, M = SH::M;
    constexpr int BD = XL<XK>::kBlockDw;
    const int lane = threadIdx.x % TPR;
    const int cb0 = S.chunk * M * TPR + lane;
    // Every block is computed; a block past the row's end (or of a row past
    // the end) contributes through a select, never a branch.  Its activation
    // read stays inside the staged vectors' LDS (block 0 for such rows).
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int cb = cb0 + m * TPR;
        const bool use = S.valid && cb < bpr;
        WBlock<XK> wb;
        widen_u(S.w[m], wb);
        const float sc = decode_scale(S.s[m]);
        if constexpr (XRegs<XK, MT, SH, U>::kOn) {
            const float d = block_dot_r<XK>(wb, X.v[m]) * sc;
            acc[0] += use ? d : 0.0f;
        } else {
            const uint32_t *xb = xs + (use ? cb : 0) * BD;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float d = block_dot<XK>(wb, xb + S.xoff[t]) * sc;
                acc[t] += (use && t < S.ntok) ? d : 0.0f;
            }
        }
    }
    if (S.chunk == chunks - 1) {
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = seg_sum<TPR>(acc[t]);
        epi(S.item, S.valid, S.ntok, acc, S.bw, S.bshift);
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    }
}

// A ring of D stages in registers.  prime() issues the first D stages (the
// loads only); run() consumes every stage in order and reissues each ring
// slot D stages ahead, so up to D stages are in flight.  On the decode shapes
// D covers a workgroup's whole share, so all of its loads go out at once and
// compute follows the data as it arrives; a launch is one pass, not a steady
// state, so a shallower ring leaves the memory system idle while every
// workgroup computes its first stage.
template <int D, int MT, class SH> struct EngineRing {
    Stage<MT, SH::M> S[D];
};

template <int D, int MT, class SH, class RowFn>
__device__ __forceinline__ void engine_prime(EngineRing<D, MT, SH> &E, int n_items, int chunks,
                                             int bpr, RowFn &rowfn)
{
#pragma unroll
    for (int d = 0; d < D; ++d) issue<MT, SH>(E.S[d], d, chunks, bpr, n_items, rowfn);
    __builtin_amdgcn_sched_barrier(0);
}

// The scheduling barriers keep every issue ahead of the next consume: left
// free, the scheduler sinks loads below that consume's wait (their addresses
// come from LDS).  Stages past the end are never issued by run(); prime()
// issues them unconditionally (one line per load), so the compiler always
// waits for exactly the stage it consumes (s_waitcnt vmcnt(N)).
template <int D, int XK, int MT, class SH, bool UNIFORM, class RowFn, class EpiFn>
__device__ __forceinline__ void engine_run(EngineRing<D, MT, SH> &E, int n_items, int chunks,
                                           int bpr, const uint32_t *xs, RowFn &rowfn, EpiFn &epi)
{
    constexpr int RG = kNT / SH::TPR;
    const int nit = ((n_items + RG - 1) / RG) * chunks;
    XRegs<XK, MT, SH, UNIFORM> X;
    load_xregs(X, xs, bpr);
    float acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = 0.0f;
    for (int base = 0; base < nit; base += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (base + d < nit) {
                consume(E.S[d], acc, chunks, bpr, xs, X, epi);
                if (base + d + D < nit) issue<MT, SH>(E.S[d], base + d + D, chunks, bpr, n_items, rowfn);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
}

// Runs `n_items` rows (RowFn maps item -> RowRef) through the engine, calling
// EpiFn(item, valid, ntok, acc, bias_word, bias_shift) once per row group with
// every lane holding its row's fp32 sums.  All threads of the workgroup must
// call it.  The loop body holds one copy of each ring slot's (consume, issue)
// pair, so the code stays small.
template <int D, int XK, int MT, class SH, bool UNIFORM, class RowFn, class EpiFn>
__device__ __forceinline__ void row_engine(int n_items, int chunks, int bpr,
                                           const uint32_t *xs, RowFn rowfn, EpiFn epi)
{
    EngineRing<D, MT, SH> E;
    engine_prime<D, MT, SH>(E, n_items, chunks, bpr, rowfn);
    engine_run<D, XK, MT, SH, UNIFORM>(E, n_items, chunks, bpr, xs, rowfn, epi);
}

static_assert(sizeof(Plan) % 16 == 0, "plans are copied in 16-byte chunks");

__device__ __forceinline__ void copy_plan(Plan *dst, const Plan *src)
{
    const uint4 *s = reinterpret_cast<const uint4 *>(src);
    uint4 *d = reinterpret_cast<uint4 *>(dst);
    for (int i = threadIdx.x; i < (int)(sizeof(Plan) / 16); i += blockDim.x) d[i] = s[i];
}

constexpr int kFusedRouteR = 4;      // fused routing handles up to 256 experts
constexpr int kMaxRouterTokens = 8;  // token rows per router_rows_kernel workgroup
constexpr int kMaxExperts = 1024;    // the standalone route kernel, up to 1024

// ---------------------------------------------------------------------------
// Standalone GEMV (mxfp4_gemv / mxfp4_gemv_bias*, dequant_gemv.metal:37-67,
// expert.metal:46-368)
// ---------------------------------------------------------------------------

template <int XK, class SH>
__global__ __launch_bounds__(kNT) void gemv_kernel(const uint8_t *__restrict__ packed,
                                                   const uint8_t *__restrict__ scales,
                                                   const void *__restrict__ bias, int bias_dt,
                                                   const void *__restrict__ x,
                                                   float *__restrict__ y, int rows, int bpr,
                                                   int chunks)
{
    constexpr int TPR = SH::TPR;
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t *xs = lds;
    int r0, r1;
    slice_of(rows, r0, r1);
    const int64_t row_bytes = (int64_t)bpr * 16;
    const int bsz = bias_dt == DT_F32 ? 4 : 2;
    auto rowfn = [&](int item) {
        RowRef<1> r;
        const int64_t row = r0 + item;
        r.packed = packed + row * row_bytes;
        r.scales = scales + row * bpr;
        r.bias = bias_dt >= 0 ? static_cast<const uint8_t *>(bias) + row * bsz : r.scales;
        r.ntok = 1;
        r.xoff[0] = 0;
        return r;
    };
    auto epi = [&](int item, bool valid, int, float (&acc)[1], uint32_t bw, int bsh) {
        if (valid && (threadIdx.x % TPR) == 0) y[r0 + item] = acc[0] + decode_bias(bw, bsh, bias_dt);
    };
    const bool fits = vector_batch_fits<XK>(x, bpr * 32, kNT);
    const int n4 = (XK == DT_F32 ? 8 : 4) * bpr, last = n4 - 1;
    const int t = (int)threadIdx.x;
    const uint4 *xg = static_cast<const uint4 *>(x);
    // x's loads first, the weight loads queued right behind them, then x into
    // LDS: loads complete in issue order, so x lands first and its round trip
    // overlaps the weights'.  A bare barrier (a fenced one would also wait for
    // the weights in flight).  Each form issues its own x loads, so the
    // compiler's waits see one straight path from them to the weight loads.
    auto store_x = [&](const uint4 &x0, const uint4 &x1, const uint4 &x2, const uint4 &x3) {
        vector_store<XK>(xs, min(t, last), x0);
        vector_store<XK>(xs, min(t + kNT, last), x1);
        vector_store<XK>(xs, min(t + 2 * kNT, last), x2);
        vector_store<XK>(xs, min(t + 3 * kNT, last), x3);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    if (fits && chunks == 1 && r1 - r0 <= kNT / TPR) {
        // The workgroup's rows are one stage (the launch shapes of the
        // standalone GEMV): that stage's loads only, then each block dotted
        // as it lands (its loads complete in issue order: a block, its scale
        // byte, the next block ...), in order.
        const uint4 x0 = xg[min(t, last)], x1 = xg[min(t + kNT, last)];
        const uint4 x2 = xg[min(t + 2 * kNT, last)], x3 = xg[min(t + 3 * kNT, last)];
        __builtin_amdgcn_sched_barrier(0);
        Stage<1, SH::M> S;
        issue<1, SH>(S, 0, 1, bpr, r1 - r0, rowfn);
        __builtin_amdgcn_sched_barrier(0);
        store_x(x0, x1, x2, x3);
        constexpr int BD = XL<XK>::kBlockDw;
        const int lane = threadIdx.x % TPR;
        float acc[1] = {0.0f};
        Unroll<0, SH::M>::run([&](auto mc) {
            constexpr int m = decltype(mc)::value;
            __builtin_amdgcn_sched_barrier(0);
            u32x4 w = S.w[m];
            uint32_t sb = S.s[m];
            asm volatile("" : "+v"(w), "+v"(sb));   // block m's wait here, not hoisted
            const int cb = lane + m * TPR;
            const bool use = S.valid && cb < bpr;
            WBlock<XK> wb;
            widen_u(w, wb);
            const float d = block_dot<XK>(wb, xs + (use ? cb : 0) * BD) * decode_scale(sb);
            acc[0] += use ? d : 0.0f;
        });
        acc[0] = seg_sum<TPR>(acc[0]);
        epi(S.item, S.valid, S.ntok, acc, S.bw, S.bshift);
    } else if (fits) {
        const uint4 x0 = xg[min(t, last)], x1 = xg[min(t + kNT, last)];
        const uint4 x2 = xg[min(t + 2 * kNT, last)], x3 = xg[min(t + 3 * kNT, last)];
        __builtin_amdgcn_sched_barrier(0);
        EngineRing<kGemvDepth, 1, SH> E;
        engine_prime<kGemvDepth, 1, SH>(E, r1 - r0, chunks, bpr, rowfn);
        store_x(x0, x1, x2, x3);
        engine_run<kGemvDepth, XK, 1, SH, true>(E, r1 - r0, chunks, bpr, xs, rowfn, epi);
    } else {
        stage_vector<XK>(xs, x, bpr * 32);
        __syncthreads();
        row_engine<kGemvDepth, XK, 1, SH, true>(r1 - r0, chunks, bpr, xs, rowfn, epi);
    }
}

// One workgroup of NT threads (384 or 512) per CU, each holding its rows (at
// most NT / 16: 16 lanes a row, 6 blocks a lane, rows of 65..96 blocks) in
// one stage, for 17..32 rows per CU: every CU then streams the same share,
// where 256-thread workgroups of 16 rows would leave some CUs two of them.
// The order of gemv_kernel's one-stage form: x's loads, the stage's loads, x
// into LDS, a bare barrier, each block dotted as it lands.  The same blocks,
// lanes and sums as gemv_kernel, so the same bits.
template <int XK, int NT>
__global__ __launch_bounds__(NT) void gemv_wide_kernel(const uint8_t *__restrict__ packed,
                                                                const uint8_t *__restrict__ scales,
                                                                const void *__restrict__ bias,
                                                                int bias_dt,
                                                                const void *__restrict__ x,
                                                                float *__restrict__ y, int rows, int bpr)
{
    constexpr int TPR = 16, M = 6, BD = XL<XK>::kBlockDw;
    extern __shared__ __align__(16) uint32_t lds[];
    uint32_t *xs = lds;
    int r0, r1;
    slice_of(rows, r0, r1);
    const int t = (int)threadIdx.x, lane = t % TPR;
    const int item = t / TPR, row = r0 + min(item, r1 - r0 - 1);
    const bool valid = r0 + item < r1;
    // x: two 16-byte loads per thread cover up to NT * 32 bytes (the host checks)
    const int n4 = (XK == DT_F32 ? 8 : 4) * bpr, last = n4 - 1;
    const uint4 xv0 = static_cast<const uint4 *>(x)[min(t, last)];
    const uint4 xv1 = static_cast<const uint4 *>(x)[min(t + NT, last)];
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t *prow = packed + (int64_t)row * bpr * 16;
    const uint8_t *srow = scales + (int64_t)row * bpr;
    u32x4 w[M];
    uint32_t sb[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int cb = valid ? min(lane + m * TPR, bpr - 1) : 0;
        w[m] = load_block(prow, cb);
        sb[m] = load_scale(srow, cb);
    }
    const int bsz = bias_dt == DT_F32 ? 4 : 2;
    const uintptr_t ba = reinterpret_cast<uintptr_t>(bias_dt >= 0 ? static_cast<const uint8_t *>(bias) +
                                                                         (int64_t)row * bsz
                                                                   : srow);
    const uint32_t bw = *(const __attribute__((address_space(1))) uint32_t *)(ba & ~(uintptr_t)3);
    __builtin_amdgcn_sched_barrier(0);
    vector_store<XK>(xs, min(t, last), xv0);   // spares store the last piece again
    vector_store<XK>(xs, min(t + NT, last), xv1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    float acc = 0.0f;
    Unroll<0, M>::run([&](auto mc) {
        constexpr int m = decltype(mc)::value;
        __builtin_amdgcn_sched_barrier(0);
        u32x4 wm = w[m];
        uint32_t sm = sb[m];
        asm volatile("" : "+v"(wm), "+v"(sm));   // block m's wait here, not hoisted
        const int cb = lane + m * TPR;
        const bool use = valid && cb < bpr;
        WBlock<XK> wb;
        widen_u(wm, wb);
        const float d = block_dot<XK>(wb, xs + (use ? cb : 0) * BD) * decode_scale(sm);
        acc += use ? d : 0.0f;
    });
    acc = seg_sum<TPR>(acc);
    if (valid && lane == 0) y[row] = acc + decode_bias(bw, (int)(ba & 2u) * 8, bias_dt);
}

// ---------------------------------------------------------------------------
// Fused gate_up GEMV + bias + activation (expert.metal:311-368 then :82-102 or
// :380-393), all groups of a plan.  Rows 2i and 2i+1 of an expert are gate i
// and up i (interleaved, expert.metal:9-17); they are neighbouring segments
// of one wave, so the activation is applied straight from the reduction.
// ---------------------------------------------------------------------------

template <int XK, int MT, class SH>
__global__ __launch_bounds__(kNT) void gate_up_kernel(
    Plan *__restrict__ gplan, RouteArgs route, const void *__restrict__ x, int hidden,
    int inter, Sections sec, int bias_dt, uint16_t *__restrict__ act, int act_kind,
    float limit, float alpha, int max_tokens, int chunks)
{
    constexpr int TPR = SH::TPR;
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int BD = XL<XK>::kBlockDw;
    constexpr int ES = XK == DT_F32 ? 4 : 2;
    Plan *plan = reinterpret_cast<Plan *>(lds);
    uint32_t *xs = lds + sizeof(Plan) / 4;
    const int bpr = hidden >> 5;
    const int xstride = bpr * BD;
    if (route.logits) {
        // Wave 0 routes (every workgroup, redundantly: 4 x 128 logits) while the
        // other waves stage the inputs, which are rows 0..T-1 of x.
        if (threadIdx.x < 64) {
            if constexpr (MT == 1) {
                // This workgroup streams rows of the experts of rank < need
                // only; workgroup 0 routes in full for the down kernel's plan.
                // 128 experts or fewer fit two logits per lane.
                int q0, q1;
                slice_of(route.top_k * inter, q0, q1);
                const int need = blockIdx.x == 0 ? route.top_k : q1 > q0 ? (q1 - 1) / inter + 1 : 0;
                int32_t *ids = blockIdx.x == 0 ? route.ids_out : nullptr;
                float *ws = blockIdx.x == 0 ? route.w_out : nullptr;
                if (route.experts <= 128)
                    route_one<2>(route.logits, route.experts, route.top_k, route.experts_base,
                                 route.stride, plan, ids, ws, need);
                else
                    route_one<kFusedRouteR>(route.logits, route.experts, route.top_k,
                                            route.experts_base, route.stride, plan, ids, ws,
                                            need);
            } else
                route_wave<kFusedRouteR>(route.logits, route.experts, route.top_k, route.tokens,
                                         route.experts_base, route.stride, plan,
                                         blockIdx.x == 0 ? route.ids_out : nullptr,
                                         blockIdx.x == 0 ? route.w_out : nullptr);
        } else {
            for (int t = 0; t < route.tokens && t < max_tokens; ++t)
                stage_vector<XK>(xs + t * xstride,
                                 static_cast<const char *>(x) + (int64_t)t * hidden * ES, hidden,
                                 threadIdx.x - 64, kNT - 64);
        }
        __syncthreads();
        if (blockIdx.x == 0) copy_plan(gplan, plan);   // for the down kernel
    } else {
        copy_plan(plan, gplan);
        __syncthreads();
        const int ntokens = plan->ntokens;
        for (int t = 0; t < ntokens && t < max_tokens; ++t)
            stage_vector<XK>(xs + t * xstride,
                             static_cast<const char *>(x) +
                                 (int64_t)plan->tok_global[t] * hidden * ES,
                             hidden);
        __syncthreads();
    }

    int p0, p1;                                        // (group, pair) space
    slice_of(plan->ngroups * inter, p0, p1);
    const int64_t row_bytes = (int64_t)bpr * 16;
    const int bsz = bias_dt == DT_F32 ? 4 : 2;
    // (group, pair) of the range start, once; items step through pairs with
    // 32-bit arithmetic (a workgroup's range spans few groups).
    const int g_start = (int)((unsigned)p0 / (unsigned)inter);
    const int i_start = p0 - g_start * inter;
    const float inv_inter = 1.0f / (float)inter;
    auto locate = [&](int item, int &g, int &i) {
        int q, r;
        divmod_small(i_start + (item >> 1), inter, inv_inter, q, r);
        g = g_start + q;
        i = r;
    };
    auto rowfn = [&](int item) {
        RowRef<MT> r;
        int g, i;
        locate(item, g, i);
        const int row = 2 * i + (item & 1);
        const uint8_t *base = plan->group_base[g];
        r.packed = base + sec.gu_blocks + row * row_bytes;
        r.scales = base + sec.gu_scales + row * bpr;
        r.bias = bias_dt >= 0 ? base + sec.gu_bias + row * bsz : r.scales;
        r.ntok = plan->group_ntok[g];
        const int s0 = plan->group_slot0[g];
#pragma unroll
        for (int t = 0; t < MT; ++t)
            r.xoff[t] = t < r.ntok ? plan->slot_token[s0 + t] * xstride : 0;
        return r;
    };
    auto epi = [&](int item, bool valid, int ntok, float (&acc)[MT], uint32_t bw, int bsh) {
        float up[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) up[t] = __shfl_down(acc[t], TPR);
        const float b_own = decode_bias(bw, bsh, bias_dt);
        const float b_next = __shfl_down(b_own, TPR);
        if (valid && (item & 1) == 0 && (threadIdx.x % TPR) == 0) {
            int g, i;
            locate(item, g, i);
            const float bg = b_own;    // gate row 2i
            const float bu = b_next;   // up row 2i+1 (the next segment)
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
    row_engine<(MT == 1 ? kGateUpDepth : 2), XK, MT, SH, true>(2 * (p1 - p0), chunks, bpr, xs,
                                                                rowfn, epi);
}

// ---------------------------------------------------------------------------
// Fused down GEMV + bias + weighted combine (expert.metal:311-368 then
// :107-116).  A workgroup owns output rows [r0, r1) for every group, so the
// combine happens in LDS without atomics, in each token's slot order.
// ---------------------------------------------------------------------------

template <int MT, class SH>
__global__ __launch_bounds__(kNT) void down_kernel(
    const Plan *__restrict__ gplan, const uint16_t *__restrict__ act, int hidden, int inter,
    Sections sec, int bias_dt, float *__restrict__ out, uint16_t *__restrict__ out_bf16,
    int accumulate, int smax, int nmax, int chunks)
{
    constexpr int TPR = SH::TPR;
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int BD = XL<DT_F16>::kBlockDw;
    Plan *plan = reinterpret_cast<Plan *>(lds);
    const int bpr = inter >> 5;
    const int astride = bpr * BD;
    uint32_t *as = lds + sizeof(Plan) / 4;                          // [smax][astride]
    float *vals = reinterpret_cast<float *>(as + smax * astride);   // [kMaxSlots][nmax]
    // The plan comes first: the weights' addresses depend on it.  Each chunk
    // of groups below issues its first weight stages before it stages its
    // activations, so those two round trips overlap.
    copy_plan(plan, gplan);
    __syncthreads();

    int r0, r1;
    slice_of(hidden, r0, r1);
    const int n = r1 - r0;
    const int ngroups = plan->ngroups;
    const int64_t row_bytes = (int64_t)bpr * 16;
    const int bsz = bias_dt == DT_F32 ? 4 : 2;

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
        const int gbase = g;
        const float inv_n = 1.0f / (float)n;
        auto split = [&](int item, int &gl, int &q) { divmod_small(item, n, inv_n, gl, q); };
        auto rowfn = [&](int item) {
            RowRef<MT> r;
            int gl, q;
            split(item, gl, q);
            const int gg = gbase + gl;
            const uint8_t *base = plan->group_base[gg];
            const int64_t row = r0 + q;
            r.packed = base + sec.dn_blocks + row * row_bytes;
            r.scales = base + sec.dn_scales + row * bpr;
            r.bias = bias_dt >= 0 ? base + sec.dn_bias + row * bsz : r.scales;
            r.ntok = plan->group_ntok[gg];
            const int sl = plan->group_slot0[gg] - s0;
#pragma unroll
            for (int t = 0; t < MT; ++t) r.xoff[t] = (sl + (t < r.ntok ? t : 0)) * astride;
            return r;
        };
        auto epi = [&](int item, bool valid, int ntok, float (&acc)[MT], uint32_t bw, int bsh) {
            if (valid && (threadIdx.x % TPR) == 0) {
                int gl, q;
                split(item, gl, q);
                const int gg = gbase + gl;
                const float b = decode_bias(bw, bsh, bias_dt);
                const int sg = plan->group_slot0[gg];
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    if (t < ntok) vals[(sg + t) * nmax + q] = acc[t] + b;
            }
        };
        // Weights first, then this chunk's activations (slot-major in act);
        // the barrier publishes the staged activations before any consume.
        constexpr int DD = MT == 1 ? kDownDepth : 2;
        EngineRing<DD, MT, SH> E;
        engine_prime<DD, MT, SH>(E, (g1 - g) * n, chunks, bpr, rowfn);
        for (int s = s0; s < s1; ++s)
            stage_vector<DT_F16>(as + (s - s0) * astride, act + (int64_t)s * inter, inter);
        __syncthreads();
        engine_run<DD, DT_F16, MT, SH, false>(E, (g1 - g) * n, chunks, bpr, as, rowfn, epi);
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
        // accumulate: 0 overwrite; 1 continue the sum from out (applyAssignments);
        // 2 the residual add after the block, out += finished sum
        // (TransformerLayer.swift:232-238).
        float dst = accumulate == 1 ? out[o] : 0.0f;
        for (int k = 0; k < plan->tok_nslots[t]; ++k) {
            const int s = plan->tok_slots[t][k];
            dst = add_scaled_rn(dst, vals[s * nmax + q], plan->slot_weight[s]);
        }
        if (accumulate == 2) dst = out[o] + dst;
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

// Router logits, wide form: workgroup (e, token block) reads expert e's
// weight row in 8-element units (16-byte loads, all units of a thread in
// flight together) and dots it with up to 8 token rows; the per-thread sums
// are reduced across the workgroup.  Needs H % 8 == 0 and 16-byte aligned
// rows; router_kernel covers the rest.
template <int WDT, int XDT>
__global__ __launch_bounds__(256) void router_rows_kernel(const void *__restrict__ W,
                                                          const void *__restrict__ b, int b_dt,
                                                          const void *__restrict__ x,
                                                          float *__restrict__ logits, int E,
                                                          int H, int T)
{
    __shared__ float red[4][kMaxRouterTokens];
    const int e = blockIdx.x, t0 = blockIdx.y * kMaxRouterTokens;
    const int nt = min(kMaxRouterTokens, T - t0);
    const int H8 = H >> 3;
    // The bias as the aligned dword holding it, read with the first loads
    // (a branchy load here would make the compiler drain them at the join).
    const int bsz = b_dt == DT_F32 ? 4 : 2;
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void *>(b ? b : W), (short)0, b ? (E * bsz + 3) & ~3 : 0, 0x00020000);
    const uint32_t b_at = (uint32_t)(e * bsz);
    uint32_t bias_word;
    float acc[kMaxRouterTokens];
#pragma unroll
    for (int t = 0; t < kMaxRouterTokens; ++t) acc[t] = 0.0f;
    // The first two units of every thread (H up to 4096): every weight and x
    // load in flight before the first product, out-of-range units clamped
    // to unit 0 and their products dropped.
    {
        float w[2][8];
        bool has[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int u = (int)threadIdx.x + 256 * k;
            has[k] = u < H8;
            load8_f32<WDT>(W, (int64_t)e * H + 8 * (has[k] ? u : 0), w[k]);
        }
        const uint32_t bw = __builtin_amdgcn_raw_buffer_load_b32(br, b_at & ~3u, 0, 0);
        float xv[kMaxRouterTokens][2][8];
#pragma unroll
        for (int t = 0; t < kMaxRouterTokens; ++t)
            if (t < nt)
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int u = (int)threadIdx.x + 256 * k;
                    load8_f32<XDT>(x, (int64_t)(t0 + t) * H + 8 * (u < H8 ? u : 0), xv[t][k]);
                }
        // the same products in the same order as one unit after another
#pragma unroll
        for (int t = 0; t < kMaxRouterTokens; ++t)
            if (t < nt)
#pragma unroll
                for (int k = 0; k < 2; ++k)
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const float nv = acc[t] + w[k][q] * xv[t][k][q];
                        acc[t] = has[k] ? nv : acc[t];
                    }
        bias_word = bw;
    }
    for (int u = (int)threadIdx.x + 512; u < H8; u += 256) {
        float w[8];
        load8_f32<WDT>(W, (int64_t)e * H + 8 * u, w);
#pragma unroll
        for (int t = 0; t < kMaxRouterTokens; ++t) {
            if (t < nt) {
                float xv[8];
                load8_f32<XDT>(x, (int64_t)(t0 + t) * H + 8 * u, xv);
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[t] += w[k] * xv[k];
            }
        }
    }
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < kMaxRouterTokens; ++t) {
        float v = acc[t];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) red[wv][t] = v;
    }
    __syncthreads();
    if ((int)threadIdx.x < nt) {
        const int t = threadIdx.x;
        const float sum = (red[0][t] + red[1][t]) + (red[2][t] + red[3][t]);
        logits[(int64_t)(t0 + t) * E + e] = sum + (b ? decode_bias(bias_word, (int)(b_at & 2u) * 8, b_dt) : 0.0f);
    }
}

// Router logits of one token by slices (router_partial, the same order as the
// one-token layer kernel's in-kernel router): workgroup e, wave s.
template <int WDT, int XDT>
__global__ __launch_bounds__(64 * kRouterMaxSlices) void router_split_kernel(
    const void *__restrict__ W, const void *__restrict__ b, int b_dt, const void *__restrict__ x,
    float *__restrict__ logits, int H, int S)
{
    __shared__ float part[kRouterMaxSlices];
    const int e = blockIdx.x, s = (int)threadIdx.x >> 6, lane = (int)threadIdx.x & 63;
    const float p = router_partial<WDT, XDT>(W, x, e, s, H / S, H, lane);
    if (lane == 0) part[s] = p;
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = part[0];
        for (int k = 1; k < S; ++k) v += part[k];
        logits[e] = v + (b ? load_as_f32(b, b_dt, e) : 0.0f);
    }
}

// Standalone routing (more than 256 experts, or a host that wants the plan
// only): one wave builds the plan in LDS and copies it out.
__global__ __launch_bounds__(64) void route_kernel(RouteArgs route, Plan *__restrict__ gplan)
{
    __shared__ __align__(16) Plan plan;
    route_wave<kMaxExperts / 64>(route.logits, route.experts, route.top_k, route.tokens,
                                 route.experts_base, route.stride, &plan, route.ids_out,
                                 route.w_out);
    __syncthreads();
    copy_plan(gplan, &plan);
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

// Post-attention RMSNorm of fp32 residual-stream rows to the fp16 MoE input
// (TransformerLayer.normalise, TransformerLayer.swift:265-285; rmsnorm,
// router.metal:36-60): one workgroup per row, the sum of squares as a
// workgroup tree in fp32, inverse = 1 / sqrt(sum / width + eps) (correctly
// rounded), out = fp16((x * inverse) * weight).
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x,
                                                      const void *__restrict__ weight, int w_dt,
                                                      int width, float eps,
                                                      uint16_t *__restrict__ out)
{
    __shared__ float partial[4];
    const float *row = x + (int64_t)blockIdx.x * width;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < width; i += 256) ss += row[i] * row[i];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if ((threadIdx.x & 63) == 0) partial[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float inverse = 1.0f / sqrtf(total / (float)width + eps);
    uint16_t *dst = out + (int64_t)blockIdx.x * width;
    for (int i = threadIdx.x; i < width; i += 256)
        dst[i] = f32_to_f16_bits((row[i] * inverse) * load_as_f32(weight, w_dt, i));
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

// Row blockIdx.y of rows spaced row_stride bytes apart; value i of the fill
// (row * count + element; 8-byte units for bytes) depends only on (seed, i),
// so one row is the plain contiguous fill.
__global__ __launch_bounds__(256) void fill_u8_kernel(uint8_t *__restrict__ dst, int64_t count,
                                                      int64_t row_stride, uint32_t lo,
                                                      uint32_t range, uint64_t seed)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // 8 bytes each
    const int64_t b0 = i * 8;
    if (b0 >= count) return;
    const int64_t unit = (int64_t)blockIdx.y * ((count + 7) / 8) + i;
    uint8_t *row = dst + (int64_t)blockIdx.y * row_stride;
    const uint64_t h0 = mix64(seed ^ mix64((uint64_t)unit * 2));
    const uint64_t h1 = mix64(seed ^ mix64((uint64_t)unit * 2 + 1));
    uint64_t word = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const uint32_t r16 = (uint32_t)(((k < 4 ? h0 : h1) >> (16 * (k & 3))) & 0xFFFFu);
        const uint32_t v = lo + ((r16 * range) >> 16);
        word |= (uint64_t)(v & 0xFFu) << (8 * k);
    }
    if (b0 + 8 <= count && (reinterpret_cast<uintptr_t>(row) & 7) == 0) {
        *reinterpret_cast<uint64_t *>(row + b0) = word;
    } else {
        for (int k = 0; k < 8 && b0 + k < count; ++k) row[b0 + k] = (uint8_t)(word >> (8 * k));
    }
}

__global__ __launch_bounds__(256) void fill_normal_kernel(void *__restrict__ dst, int dt,
                                                          int64_t count, int64_t row_stride,
                                                          float mean, float stddev,
                                                          uint64_t seed)
{
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= count) return;
    const int64_t i = (int64_t)blockIdx.y * count + e;
    void *row = static_cast<uint8_t *>(dst) + (int64_t)blockIdx.y * row_stride;
    const uint64_t h = mix64(seed ^ mix64((uint64_t)i));
    const float u1 = ((float)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);        // (0, 1]
    const float u2 = (float)((h >> 16) & 0xFFFFFFull) * (1.0f / 16777216.0f);  // [0, 1)
    const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    const float v = mean + stddev * z;
    if (dt == DT_F32) static_cast<float *>(row)[e] = v;
    else if (dt == DT_BF16) static_cast<uint16_t *>(row)[e] = f32_to_bf16_bits(v);
    else static_cast<uint16_t *>(row)[e] = f32_to_f16_bits(v);
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
    GW_LAUNCH(dequant_kernel, dim3(div_up(words, 256)), dim3(256), 0, L,
              reinterpret_cast<const uint32_t *>(packed), scales, words,
              reinterpret_cast<float4 *>(out));
    return hipGetLastError();
}

static int x_block_dw(int x_dt) { return x_dt == DT_F32 ? 36 : 20; }

// Calls f(SH{}) with the shape class row_shape() chose.
template <class F> static void with_shape(const RowShape &s, F &&f)
{
    if (s.tpr == 8 && s.m == 1) f(S0{});
    else if (s.tpr == 8) f(S1{});
    else if (s.m == 4) f(S2{});
    else if (s.m == 6) f(S3{});
    else f(S4{});
}

hipError_t launch_gemv(const Launch &L, const uint8_t *packed, const uint8_t *scales,
                       const void *bias, int bias_dt, const void *x, int x_dt, float *y,
                       int rows, int cols)
{
    if (rows == 0) return hipSuccess;
    const int bpr = cols / 32;
    const RowShape s = row_shape(bpr);
    const int rg = kNT / s.tpr;
    const size_t x_bytes = (size_t)cols * (x_dt == DT_F32 ? 4 : 2);
    const int per_cu = div_up(rows, L.cus);
    if (L.grid_a <= 0 && s.tpr == 16 && s.m == 6 && s.chunks == 1 && per_cu > rg && per_cu <= 32 &&
        (reinterpret_cast<uintptr_t>(x) & 15u) == 0) {
        // 17..32 rows a CU: one workgroup per CU, all its rows in one stage
        const int nt = per_cu <= 24 ? 384 : 512;
        if (x_bytes <= (size_t)nt * 32) {
            const size_t lds = (size_t)bpr * x_block_dw(x_dt) * 4;
            auto go = [&](auto ntc) {
                constexpr int NT = decltype(ntc)::value;
                if (x_dt == DT_F32)
                    GW_LAUNCH((gemv_wide_kernel<DT_F32, NT>), dim3(L.cus), dim3(NT), lds, L, packed,
                              scales, bias, bias_dt, x, y, rows, bpr);
                else if (x_dt == DT_F16)
                    GW_LAUNCH((gemv_wide_kernel<DT_F16, NT>), dim3(L.cus), dim3(NT), lds, L, packed,
                              scales, bias, bias_dt, x, y, rows, bpr);
                else
                    GW_LAUNCH((gemv_wide_kernel<DT_BF16, NT>), dim3(L.cus), dim3(NT), lds, L, packed,
                              scales, bias, bias_dt, x, y, rows, bpr);
            };
            if (nt == 384) go(std::integral_constant<int, 384>{});
            else go(std::integral_constant<int, 512>{});
            return hipGetLastError();
        }
    }
    int grid = L.grid_a > 0 ? L.grid_a : 2 * L.cus;
    grid = grid < div_up(rows, rg) ? grid : div_up(rows, rg);
    const size_t lds = (size_t)bpr * x_block_dw(x_dt) * 4;
    with_shape(s, [&](auto sh) {
        using SH = decltype(sh);
        if (x_dt == DT_F32)
            GW_LAUNCH((gemv_kernel<DT_F32, SH>), dim3(grid), dim3(kNT), lds, L,
                               packed, scales, bias, bias_dt, x, y, rows, bpr, s.chunks);
        else if (x_dt == DT_F16)
            GW_LAUNCH((gemv_kernel<DT_F16, SH>), dim3(grid), dim3(kNT), lds, L,
                               packed, scales, bias, bias_dt, x, y, rows, bpr, s.chunks);
        else
            GW_LAUNCH((gemv_kernel<DT_BF16, SH>), dim3(grid), dim3(kNT), lds, L,
                               packed, scales, bias, bias_dt, x, y, rows, bpr, s.chunks);
    });
    return hipGetLastError();
}

int gate_up_lds_bytes(int hidden, int x_dt, int max_tokens)
{
    return (int)sizeof(Plan) + max_tokens * (hidden / 32) * x_block_dw(x_dt) * 4;
}

hipError_t launch_gate_up(const Launch &L, Plan *plan, const RouteArgs *route, int max_tokens,
                          const void *x, int x_dt, int hidden, int inter, const Sections &sec,
                          int bias_dt, uint16_t *act, int act_kind, float limit, float alpha)
{
    RouteArgs r = {};
    if (route) {
        if (route->experts > 64 * kFusedRouteR || route->top_k > kMaxTopK ||
            route->tokens > kMaxTokens || route->tokens != max_tokens)
            return hipErrorInvalidValue;
        r = *route;
    }
    const RowShape s = row_shape(hidden / 32);
    const int grid = L.grid_a > 0 ? L.grid_a : 2 * L.cus;
    const size_t lds = (size_t)gate_up_lds_bytes(hidden, x_dt, max_tokens);
    with_shape(s, [&](auto sh) {
        using SH = decltype(sh);
        auto go = [&](auto xk, auto mt) {
            constexpr int XK = decltype(xk)::value, MT = decltype(mt)::value;
            GW_LAUNCH((gate_up_kernel<XK, MT, SH>), dim3(grid), dim3(kNT), lds, L, plan, r, x, hidden, inter, sec, bias_dt, act, act_kind,
                               limit, alpha, max_tokens, s.chunks);
        };
        using One = std::integral_constant<int, 1>;
        using Many = std::integral_constant<int, kMaxTokens>;
        if (x_dt == DT_F32) {
            if (max_tokens == 1) go(std::integral_constant<int, DT_F32>{}, One{});
            else go(std::integral_constant<int, DT_F32>{}, Many{});
        } else if (x_dt == DT_F16) {
            if (max_tokens == 1) go(std::integral_constant<int, DT_F16>{}, One{});
            else go(std::integral_constant<int, DT_F16>{}, Many{});
        } else {
            if (max_tokens == 1) go(std::integral_constant<int, DT_BF16>{}, One{});
            else go(std::integral_constant<int, DT_BF16>{}, Many{});
        }
    });
    return hipGetLastError();
}

int down_lds_bytes(int hidden, int inter, int grid, int smax)
{
    const int nmax = (hidden + grid - 1) / grid;
    return (int)sizeof(Plan) + smax * (inter / 32) * 20 * 4 + kMaxSlots * nmax * 4;
}

template <int MT>
static void down_dispatch(const Launch &L, const RowShape &s, int grid, size_t lds,
                          const Plan *plan, const uint16_t *act, int hidden, int inter,
                          const Sections &sec, int bias_dt, float *out, uint16_t *out_bf16,
                          int accumulate, int smax, int nmax)
{
    with_shape(s, [&](auto sh) {
        using SH = decltype(sh);
        GW_LAUNCH((down_kernel<MT, SH>), dim3(grid), dim3(kNT), lds, L, plan,
                           act, hidden, inter, sec, bias_dt, out, out_bf16, accumulate, smax,
                           nmax, s.chunks);
    });
}

hipError_t launch_down(const Launch &L, const Plan *plan, int max_tokens, int max_slots,
                       const uint16_t *act, int hidden, int inter, const Sections &sec,
                       int bias_dt, float *out, uint16_t *out_bf16, int accumulate)
{
    const RowShape s = row_shape(inter / 32);
    int grid = L.grid_b > 0 ? L.grid_b : 2 * L.cus;
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
    if (max_tokens == 1)
        down_dispatch<1>(L, s, grid, lds, plan, act, hidden, inter, sec, bias_dt, out, out_bf16,
                         accumulate, smax, nmax);
    else
        down_dispatch<kMaxTokens>(L, s, grid, lds, plan, act, hidden, inter, sec, bias_dt, out,
                                  out_bf16, accumulate, smax, nmax);
    return hipGetLastError();
}

hipError_t launch_activation(const Launch &L, int kind, const float *gate_up, uint16_t *out,
                             int64_t width, float limit, float alpha)
{
    if (width == 0) return hipSuccess;
    GW_LAUNCH(activation_kernel, dim3(div_up(width, 256)), dim3(256), 0, L, kind, gate_up, out,
              width, limit, alpha);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const Launch &L, const float *x, const void *weight, int w_dt,
                          int rows, int width, float eps, uint16_t *out)
{
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    GW_LAUNCH(rmsnorm_kernel, dim3(rows), dim3(256), 0, L, x, weight, w_dt, width, eps, out);
    return hipGetLastError();
}

hipError_t launch_accumulate(const Launch &L, const float *src, float *dst, float w,
                             int64_t width)
{
    if (width == 0) return hipSuccess;
    GW_LAUNCH(accumulate_kernel, dim3(div_up(width, 256)), dim3(256), 0, L, src, dst, w, width);
    return hipGetLastError();
}

hipError_t launch_router(const Launch &L, const void *W, int w_dt, const void *b, int b_dt,
                         const void *x, int x_dt, float *logits, int experts, int hidden,
                         int tokens)
{
    const int waves = experts * tokens;
    if (waves == 0) return hipSuccess;
    const int S = router_slices(experts, hidden, L.cus);
    if (tokens == 1 && S > 0 && x_dt != DT_F32 && ((uintptr_t)W & 15u) == 0 &&
        ((uintptr_t)x & 15u) == 0) {
        // one 16-bit token: the sliced order of the one-token layer's router
        auto go = [&](auto wdt, auto xdt) {
            constexpr int WD = decltype(wdt)::value, XD = decltype(xdt)::value;
            GW_LAUNCH((router_split_kernel<WD, XD>), dim3(experts), dim3(64 * S), 0, L, W, b, b_dt,
                      x, logits, hidden, S);
        };
        auto with_x = [&](auto wdt) {
            if (x_dt == DT_F16) go(wdt, std::integral_constant<int, DT_F16>{});
            else go(wdt, std::integral_constant<int, DT_BF16>{});
        };
        if (w_dt == DT_F32) with_x(std::integral_constant<int, DT_F32>{});
        else if (w_dt == DT_F16) with_x(std::integral_constant<int, DT_F16>{});
        else with_x(std::integral_constant<int, DT_BF16>{});
        return hipGetLastError();
    }
    const bool wide = hidden % 8 == 0 && ((uintptr_t)W & 15u) == 0 &&
                      ((uintptr_t)x & 15u) == 0 && div_up(tokens, kMaxRouterTokens) <= 65535;
    if (wide) {
        const dim3 grid(experts, div_up(tokens, kMaxRouterTokens));
        auto go = [&](auto wdt, auto xdt) {
            constexpr int WD = decltype(wdt)::value, XD = decltype(xdt)::value;
            GW_LAUNCH((router_rows_kernel<WD, XD>), grid, dim3(256), 0, L, W, b, b_dt, x, logits,
                      experts, hidden, tokens);
        };
        auto with_x = [&](auto wdt) {
            if (x_dt == DT_F32) go(wdt, std::integral_constant<int, DT_F32>{});
            else if (x_dt == DT_F16) go(wdt, std::integral_constant<int, DT_F16>{});
            else go(wdt, std::integral_constant<int, DT_BF16>{});
        };
        if (w_dt == DT_F32) with_x(std::integral_constant<int, DT_F32>{});
        else if (w_dt == DT_F16) with_x(std::integral_constant<int, DT_F16>{});
        else with_x(std::integral_constant<int, DT_BF16>{});
        return hipGetLastError();
    }
    GW_LAUNCH(router_kernel, dim3(div_up(waves, 4)), dim3(256), 0, L, W, w_dt, b, b_dt, x, x_dt,
              logits, experts, hidden, tokens);
    return hipGetLastError();
}

hipError_t launch_route(const Launch &L, const RouteArgs &route, Plan *plan)
{
    if (route.experts > kMaxExperts || route.top_k > kMaxTopK || route.tokens > kMaxTokens ||
        route.top_k > route.experts)
        return hipErrorInvalidValue;
    GW_LAUNCH(route_kernel, dim3(1), dim3(64), 0, L, route, plan);
    return hipGetLastError();
}

hipError_t launch_fill_u8(const Launch &L, void *dst, size_t count, size_t rows,
                          size_t row_stride, int lo, int hi, uint64_t seed)
{
    if (count == 0 || rows == 0) return hipSuccess;
    const int64_t threads = ((int64_t)count + 7) / 8;
    const uint32_t range = (uint32_t)(hi - lo + 1);
    GW_LAUNCH(fill_u8_kernel, dim3(div_up(threads, 256), (unsigned)rows), dim3(256), 0, L,
              static_cast<uint8_t *>(dst), (int64_t)count, (int64_t)row_stride, (uint32_t)lo,
              range, seed);
    return hipGetLastError();
}

hipError_t launch_fill_normal(const Launch &L, void *dst, int dt, size_t count, size_t rows,
                              size_t row_stride, float mean, float stddev, uint64_t seed)
{
    if (count == 0 || rows == 0) return hipSuccess;
    GW_LAUNCH(fill_normal_kernel, dim3(div_up((int64_t)count, 256), (unsigned)rows), dim3(256), 0,
              L, dst, dt, (int64_t)count, (int64_t)row_stride, mean, stddev, seed);
    return hipGetLastError();
}

}  // namespace gw
