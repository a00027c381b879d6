// gw_prefill.hip — batched prefill of one MoE layer on CDNA4 matrix cores.
//
// A prefill batch routes T tokens to K experts each (TransformerLayer.swift:
// 158-181), so every selected expert sees a group of tokens and its weights
// are used by the whole group: the one true contraction of the path.  Steps:
//   1. route: one wave per token selects top-k + softmax (Router.select);
//   2. group: counting sort of the T*K (token, rank) entries by expert, and
//      the list of (expert, 32-token tile) work items;
//   3. gate_up grouped GEMM + bias + activation -> fp16 activations per entry;
//   4. down grouped GEMM + bias -> fp32 expert outputs per entry;
//   5. combine: out[t] = sum_k w[t,k] * y[t,k] in router order
//      (expert_accumulate, expert.metal:107-116).
//
// GEMM numerics.  Weights are widened by v_cvt_scalef32_pk_bf16_fp4 with the
// block's e8m0 scale folded in: every e2m1 value times a power of two is
// exact in bf16 (two significant bits; the whole e8m0 range, subnormal
// scales included, checked exhaustively on gfx950).  Activations enter the
// bf16 matrix cores as exact sums of bf16 planes: bf16 x is one plane, fp16
// two (hi = bf16(v), lo = v - hi) and fp32 three.  Every product is then
// exact in fp32 and v_mfma_f32_32x32x16_bf16 accumulates in fp32, so the
// results differ from the reference's scalar loop only in summation order.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include "gw_device.h"
#include "gw_launch.h"
#include "gw_route.h"

namespace gw {

#define GW_LAUNCH(KERNEL, GRID, BLOCK, LDS, L, ...)                                          \
    do {                                                                                      \
        if ((L).ev_start)                                                                     \
            hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, (L).stream, (L).ev_start,          \
                                  (L).ev_stop, 0, __VA_ARGS__);                               \
        else                                                                                  \
            hipLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, (L).stream, __VA_ARGS__);            \
    } while (0)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4v g_u32x4v;
typedef const __attribute__((address_space(1))) uint8_t g_u8c;

constexpr int kPT = 32;                 // tokens per tile (MFMA columns)
constexpr int kPWaves = 8;              // waves per workgroup, 32 features each
constexpr int kPThreads = 64 * kPWaves;
constexpr int kPF = 32 * kPWaves;       // features per workgroup
constexpr int kKC = 8;                  // 32-element blocks per staged activation chunk
constexpr int kXPitch = kKC * 32 + 8;   // bf16 per staged token row (16-byte pad: banks)
constexpr int kWChunks = 2;             // weight chunks in flight per wave (ring depth)
constexpr int kPrefillMaxExperts = 256;

// ---------------------------------------------------------------------------
// 1. Routing: one wave per token.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void prefill_route_kernel(const float *__restrict__ logits,
                                                            int T, int E, int K,
                                                            int32_t *__restrict__ ids,
                                                            float *__restrict__ weights)
{
    const int t = blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    if (t >= T) return;   // whole waves leave together
    int sid;
    float w;
    select_one<4>(logits + (int64_t)t * E, E, K, sid, w);
    const int lane = threadIdx.x & 63;
    if (lane < K) {
        ids[(int64_t)t * K + lane] = sid;
        weights[(int64_t)t * K + lane] = w;
    }
}

// ---------------------------------------------------------------------------
// 2. Grouping (one workgroup).  Entry j = t*K + k.  offsets[e]..offsets[e+1]
// index `order`, which lists expert e's entries; a work item is one 32-entry
// tile of one expert, encoded (e << 16) | m.  Positions inside a group come
// from LDS atomics: each entry's results depend only on its own token row, so
// the order inside a group never changes a value.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void prefill_group_kernel(const int32_t *__restrict__ ids, int N,
                                                             int E, int32_t *__restrict__ offsets,
                                                             int32_t *__restrict__ order,
                                                             int32_t *__restrict__ tiles,
                                                             int32_t *__restrict__ ntiles,
                                                             int max_tiles)
{
    __shared__ int cnt[kPrefillMaxExperts];
    __shared__ int cur[kPrefillMaxExperts];
    __shared__ int off[kPrefillMaxExperts + 1];
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        cnt[e] = 0;
        cur[e] = 0;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < N; j += blockDim.x) atomicAdd(&cnt[ids[j]], 1);
    __syncthreads();
    if (threadIdx.x == 0) {
        int o = 0, nt = 0;
        for (int e = 0; e < E; ++e) {
            off[e] = o;
            o += cnt[e];
            for (int m = 0; m * kPT < cnt[e]; ++m)
                if (nt < max_tiles) tiles[nt++] = (e << 16) | m;
        }
        off[E] = o;
        *ntiles = nt;
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= E; e += blockDim.x) offsets[e] = off[e];
    for (int j = threadIdx.x; j < N; j += blockDim.x) {
        const int e = ids[j];
        order[off[e] + atomicAdd(&cur[e], 1)] = j;
    }
}

// ---------------------------------------------------------------------------
// 3./4. Grouped GEMM: workgroup (feature tile f, work item) computes
// C[256 features x 32 entries] = W_e[f-tile, :] . X[entries, :]^T over K, one
// 32x32 block per wave.  Per 32-element K block a lane (row r = lane & 31,
// half h = lane >> 5) holds dwords 2h, 2h+1 of row r's 16-byte block, i.e.
// elements 16h .. 16h+15, widened with the scale folded in; MFMA j (0, 1)
// takes elements 16h + 8j .. +7 from both A (weights) and B (the staged
// activation row of entry r' = lane & 31), so A and B share one K order.
// C element v of a lane is feature row 8(v/4) + 4h + (v%4), entry column
// lane & 31.
// ---------------------------------------------------------------------------

struct GemmArgs {
    const int32_t *tiles;
    const int32_t *ntiles;
    const int32_t *offsets;
    const int32_t *order;
    const void *in;               // activations: [rows, kdim] of in_dt
    int in_row_div;               // entry -> input row: entry / in_row_div (K for x, 1 for act)
    const uint8_t *experts_base;
    int64_t stride;
    int64_t blocks_off, scales_off, bias_off;   // section offsets within an expert
    int bias_dt;                  // -1: no bias
    int kdim, fdim;               // K (input width) and weight rows
    uint16_t *act_out;            // gate_up: [N, fdim/2] fp16
    float *y_out;                 // down: [N, fdim] fp32
    int act_kind;
    float limit, alpha;
};

// Splits 8 input values into PL bf16 planes whose sum is exact.
template <int IN_DT, int PL>
__device__ __forceinline__ void split_planes(const float (&v)[8], uint32_t (&out)[PL][4])
{
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = v[i];
#pragma unroll
    for (int p = 0; p < PL; ++p) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint16_t a = f32_to_bf16_bits(r[2 * i]), b = f32_to_bf16_bits(r[2 * i + 1]);
            out[p][i] = (uint32_t)a | ((uint32_t)b << 16);
            r[2 * i] -= bf16_bits_to_f32(a);
            r[2 * i + 1] -= bf16_bits_to_f32(b);
        }
    }
}

template <int IN_DT, int PL, bool GATE_UP>
__global__ __launch_bounds__(kPThreads) void prefill_gemm_kernel(GemmArgs a)
{
    // Dynamic LDS only (a static __shared__ variable would shift the dynamic
    // area off its 16-byte alignment): [kPT] entries, then [2][PL][kPT][kXPitch].
    extern __shared__ __align__(16) uint32_t plds[];
    int *ent = reinterpret_cast<int *>(plds);
    uint16_t *xs = reinterpret_cast<uint16_t *>(plds + kPT);
    const int item = blockIdx.y;
    if (item >= *a.ntiles) return;                    // uniform: the workgroup leaves
    const int te = a.tiles[item];
    const int e = te >> 16, m = te & 0xFFFF;
    const int g0 = a.offsets[e] + m * kPT;
    const int ntok = min(kPT, a.offsets[e + 1] - g0);
    if (threadIdx.x < kPT) ent[threadIdx.x] = a.order[g0 + min((int)threadIdx.x, ntok - 1)];
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = lane >> 5, c = lane & 31;
    const int fbase = blockIdx.x * kPF + wave * 32;
    const int row = min(fbase + c, a.fdim - 1);       // clamped: rows past fdim are never stored
    const int nb = a.kdim >> 5;
    const uint8_t *ex = a.experts_base + (int64_t)e * a.stride;
    const uint8_t *wrow = ex + a.blocks_off + (int64_t)row * nb * 16;
    const uint8_t *srow = ex + a.scales_off + (int64_t)row * nb;

    // Activation staging: unit u = (token, 8-element piece) of a chunk.  A
    // thread's units keep their token and piece for every chunk, so their row
    // offsets are computed once.  Loads keep the raw bits in registers until
    // the store at the chunk's end converts them (a conversion right after
    // the load would wait for every older load still in flight).
    constexpr int kUnits = kPT * kKC * 4;             // 8-element pieces per chunk
    constexpr int kPer = kUnits / kPThreads;          // units per thread
    constexpr int kRawQ = IN_DT == DT_F32 ? 2 : 1;    // 16-byte loads per unit
    const size_t plane_elems = (size_t)kPT * kXPitch;
    int64_t urow[kPer];
    int upiece[kPer];
#pragma unroll
    for (int s = 0; s < kPer; ++s) {
        const int u = s * kPThreads + (int)threadIdx.x;
        const int t = u / (kKC * 4);
        upiece[s] = u % (kKC * 4);
        urow[s] = (int64_t)(ent[t] / a.in_row_div) * a.kdim;
    }
    uint4 raw[kPer][kRawQ];
    auto stage_load = [&](int q) {
#pragma unroll
        for (int s = 0; s < kPer; ++s) {
            const int k = min(q * kKC * 32 + upiece[s] * 8, a.kdim - 8);
#pragma unroll
            for (int j = 0; j < kRawQ; ++j)
                raw[s][j] = reinterpret_cast<const uint4 *>(
                    static_cast<const uint8_t *>(a.in) +
                    (urow[s] + k) * (IN_DT == DT_F32 ? 4 : 2))[j];
        }
    };
    // Pieces past kdim (the last chunks' tails) are stored as zeros, so the
    // unconditional chunk loop below multiplies them by finite weights only.
    auto stage_store = [&](int buf, int q) {
#pragma unroll
        for (int s = 0; s < kPer; ++s) {
            const int u = s * kPThreads + (int)threadIdx.x;
            const int t = u / (kKC * 4);
            const bool live = q * kKC * 32 + upiece[s] * 8 < a.kdim;
            float v[8];
            if constexpr (IN_DT == DT_F32) {
                const uint32_t w[8] = {raw[s][0].x, raw[s][0].y, raw[s][0].z, raw[s][0].w,
                                       raw[s][1].x, raw[s][1].y, raw[s][1].z, raw[s][1].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = live ? __uint_as_float(w[i]) : 0.0f;
            } else {
                const uint32_t w[4] = {raw[s][0].x, raw[s][0].y, raw[s][0].z, raw[s][0].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint16_t lo = (uint16_t)(w[i] & 0xFFFFu), hi = (uint16_t)(w[i] >> 16);
                    const float flo = IN_DT == DT_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
                    const float fhi = IN_DT == DT_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
                    v[2 * i] = live ? flo : 0.0f;
                    v[2 * i + 1] = live ? fhi : 0.0f;
                }
            }
            uint32_t pl[PL][4];
            split_planes<IN_DT, PL>(v, pl);
#pragma unroll
            for (int p = 0; p < PL; ++p) {
                uint16_t *dst = xs + ((size_t)buf * PL + p) * plane_elems + t * kXPitch + upiece[s] * 8;
                *reinterpret_cast<uint4 *>(dst) = make_uint4(pl[p][0], pl[p][1], pl[p][2], pl[p][3]);
            }
        }
    };

    // Weight ring, kWChunks chunks deep: per chunk a lane holds its row's
    // blocks 4h .. 4h+3 of the chunk (64 contiguous bytes, four 16-byte loads
    // that the wave issues back to back, so each 128-byte line is fetched
    // once) and their four scale bytes.  Block indices past nb clamp to the
    // row's last block; their activations are staged as zeros.
    u32x4v wq[kWChunks][4];
    uint32_t sq[kWChunks][4];
    auto wload = [&](int slot, int q) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int bb = min(q * kKC + 4 * h + i, nb - 1);
            wq[slot][i] = *(g_u32x4v *)(wrow + (int64_t)bb * 16);
            sq[slot][i] = ((g_u8c *)srow)[bb];
        }
    };

    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

    // Chunk q from ring slot s and activation buffer s: MFMA 4i+d takes dword d
    // of block 4h+i, i.e. elements 128h + 32i + 8d .. +7 of the chunk, from
    // both the weights (A) and the staged activation row of entry c (B).
    auto chunk = [&](int q, auto s_const) {
        constexpr int s = decltype(s_const)::value;
        stage_load(q + 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float sc = decode_scale(sq[s][i]);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t w = wq[s][i][d];
                const uint4 au = make_uint4(
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2)),
                    __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3)));
                const bf16x8 A = __builtin_bit_cast(bf16x8, au);
#pragma unroll
                for (int p = 0; p < PL; ++p) {
                    const uint16_t *xr = xs + ((size_t)s * PL + p) * plane_elems + c * kXPitch +
                                         128 * h + 32 * i + 8 * d;
                    const bf16x8 B = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(xr));
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A, B, acc, 0, 0, 0);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        wload(s, q + kWChunks);
        __builtin_amdgcn_sched_barrier(0);
        stage_store(s ^ 1, q + 1);
        __syncthreads();
    };

    // nq rounded up to the ring depth: a padding chunk sees zero activations.
    const int nq = (nb + kKC - 1) / kKC;
    const int nq_pad = (nq + kWChunks - 1) / kWChunks * kWChunks;
#pragma unroll
    for (int s = 0; s < kWChunks; ++s) wload(s, s);
    stage_load(0);
    stage_store(0, 0);
    __syncthreads();
    for (int q = 0; q < nq_pad; q += kWChunks) {
        chunk(q, std::integral_constant<int, 0>{});
        chunk(q + 1, std::integral_constant<int, 1>{});
    }

    // Epilogue: lane holds entry column c, feature rows 8(v/4) + 4h + (v%4).
    const bool col_ok = c < ntok;
    const int entry = ent[c];
    const uint8_t *bias = ex + a.bias_off;
    // The lane's 16 bias values, loaded together before any is used.
    float bv[16];
    {
        uint32_t raw[16];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = min(fbase + 8 * (v >> 2) + 4 * h + (v & 3), a.fdim - 1);
            raw[v] = a.bias_dt == DT_F32 ? reinterpret_cast<const uint32_t *>(bias)[r]
                                         : (uint32_t)reinterpret_cast<const uint16_t *>(bias)[r];
        }
#pragma unroll
        for (int v = 0; v < 16; ++v)
            bv[v] = a.bias_dt < 0 ? 0.0f
                    : a.bias_dt == DT_F32 ? __uint_as_float(raw[v])
                    : a.bias_dt == DT_BF16 ? bf16_bits_to_f32((uint16_t)raw[v])
                                           : f16_bits_to_f32((uint16_t)raw[v]);
    }
    if constexpr (GATE_UP) {
        const int half = a.fdim >> 1;
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
            const int r = fbase + 8 * (v >> 2) + 4 * h + (v & 3);   // even: gate, r+1: up
            if (col_ok && r + 1 < a.fdim) {
                const float gate = acc[v] + bv[v];
                const float up = acc[v + 1] + bv[v + 1];
                const float y = apply_activation(a.act_kind, gate, up, a.limit, a.alpha);
                a.act_out[(int64_t)entry * half + (r >> 1)] = f32_to_f16_bits(y);
            }
        }
    } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int r = fbase + 8 * (v >> 2) + 4 * h + (v & 3);
            if (col_ok && r < a.fdim)
                a.y_out[(int64_t)entry * a.fdim + r] = acc[v] + bv[v];
        }
    }
}

// ---------------------------------------------------------------------------
// 5. Combine: out[t] = sum_k w[t,k] * y[t*K+k], product and sum rounded
// separately in router order (expert_accumulate), starting from zero.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void prefill_combine_kernel(const float *__restrict__ y,
                                                              const float *__restrict__ w,
                                                              int T, int K, int H,
                                                              float *__restrict__ out,
                                                              uint16_t *__restrict__ out_bf16)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * H) return;
    const int t = (int)(i / H), col = (int)(i - (int64_t)t * H);
    float dst = 0.0f;
    for (int k = 0; k < K; ++k)
        dst = add_scaled_rn(dst, y[((int64_t)t * K + k) * H + col], w[(int64_t)t * K + k]);
    out[i] = dst;
    if (out_bf16) out_bf16[i] = f32_to_bf16_bits(dst);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

static inline int pdiv_up(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

hipError_t launch_prefill_route(const Launch &L, const float *logits, int T, int E, int K,
                                int32_t *ids, float *weights)
{
    if (E > 256 || K > kMaxTopK || T <= 0) return hipErrorInvalidValue;
    GW_LAUNCH(prefill_route_kernel, dim3(pdiv_up(T, 4)), dim3(256), 0, L, logits, T, E, K, ids,
              weights);
    return hipGetLastError();
}

int prefill_max_tiles(int T, int K, int E) { return pdiv_up((int64_t)T * K, kPT) + E; }

hipError_t launch_prefill_group(const Launch &L, const int32_t *ids, int N, int E,
                                int32_t *offsets, int32_t *order, int32_t *tiles,
                                int32_t *ntiles, int max_tiles)
{
    if (E > kPrefillMaxExperts) return hipErrorInvalidValue;
    GW_LAUNCH(prefill_group_kernel, dim3(1), dim3(1024), 0, L, ids, N, E, offsets, order, tiles,
              ntiles, max_tiles);
    return hipGetLastError();
}

int prefill_gemm_lds_bytes(int in_dt)
{
    const int pl = in_dt == DT_BF16 ? 1 : in_dt == DT_F16 ? 2 : 3;
    return kPT * 4 + 2 * pl * kPT * kXPitch * 2;
}

hipError_t launch_prefill_gemm(const Launch &L, bool gate_up, int in_dt, const PrefillGemm &g,
                               int max_tiles)
{
    if (g.kdim % 32 != 0 || g.kdim < 32 || g.fdim <= 0 || max_tiles <= 0)
        return hipErrorInvalidValue;
    GemmArgs a;
    a.tiles = g.tiles;
    a.ntiles = g.ntiles;
    a.offsets = g.offsets;
    a.order = g.order;
    a.in = g.in;
    a.in_row_div = g.in_row_div;
    a.experts_base = g.experts_base;
    a.stride = g.stride;
    a.blocks_off = g.blocks_off;
    a.scales_off = g.scales_off;
    a.bias_off = g.bias_off;
    a.bias_dt = g.bias_dt;
    a.kdim = g.kdim;
    a.fdim = g.fdim;
    a.act_out = g.act_out;
    a.y_out = g.y_out;
    a.act_kind = g.act_kind;
    a.limit = g.limit;
    a.alpha = g.alpha;
    const dim3 grid(pdiv_up(g.fdim, kPF), max_tiles);
    const size_t lds = (size_t)prefill_gemm_lds_bytes(in_dt);
    hipError_t err = hipSuccess;
    auto go = [&](auto dt, auto pl, auto gu) {
        constexpr int DT = decltype(dt)::value, PL = decltype(pl)::value;
        constexpr bool GU = decltype(gu)::value;
        // More than 64 KiB of dynamic LDS (two or three planes) must be allowed
        // explicitly, once per instantiation.
        static bool lds_ok = false;
        if (!lds_ok) {
            err = hipFuncSetAttribute(reinterpret_cast<const void *>(&prefill_gemm_kernel<DT, PL, GU>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (err != hipSuccess) return;
            lds_ok = true;
        }
        GW_LAUNCH((prefill_gemm_kernel<DT, PL, GU>), grid, dim3(kPThreads), lds, L, a);
    };
    using B1 = std::integral_constant<int, DT_BF16>;
    using H2 = std::integral_constant<int, DT_F16>;
    using F3 = std::integral_constant<int, DT_F32>;
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;
    using Y = std::true_type;
    using N = std::false_type;
    if (gate_up) {
        if (in_dt == DT_BF16) go(B1{}, P1{}, Y{});
        else if (in_dt == DT_F16) go(H2{}, P2{}, Y{});
        else go(F3{}, P3{}, Y{});
    } else {
        if (in_dt != DT_F16) return hipErrorInvalidValue;   // the activation is fp16
        go(H2{}, P2{}, N{});
    }
    if (err != hipSuccess) return err;
    return hipGetLastError();
}

hipError_t launch_prefill_combine(const Launch &L, const float *y, const float *w, int T, int K,
                                  int H, float *out, uint16_t *out_bf16)
{
    GW_LAUNCH(prefill_combine_kernel, dim3(pdiv_up((int64_t)T * H, 256)), dim3(256), 0, L, y, w,
              T, K, H, out, out_bf16);
    return hipGetLastError();
}

}  // namespace gw
