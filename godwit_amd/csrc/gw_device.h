// gw_device.h — gfx950 device helpers for the MXFP4 decode kernels.
//
// MXFP4 (Sources/Godwit/Quant/MXFP4.swift:3-31): 32 e2m1 codes per block, two
// per byte with the low nibble the even element, one e8m0 scale per block.
// Codes are widened by CDNA4's v_cvt_scalef32_pk_{f32,f16,bf16}_fp4 (one
// instruction per packed byte, scale operand 1.0 so the result is the exact
// codebook value of MXFP4.swift:22-25), and dotted with the activation in
// fp32 by v_dot2c_f32_{f16,bf16} (two products per lane-op) or v_fma_f32.
// The block scale multiplies the block's fp32 partial afterwards, as in
// referenceMXFP4 (Benchmark/DequantGEMVBenchmark.swift:106-116).
#pragma once
#include <type_traits>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gw_plan.h"

namespace gw {

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };   // == gw_dtype

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Calls f(std::integral_constant<int, i>) for i = B .. E-1: a loop whose
// index is a compile-time constant in the body.
template <int B, int E> struct Unroll {
    template <class F> __device__ __forceinline__ static void run(F &&f)
    {
        f(std::integral_constant<int, B>{});
        Unroll<B + 1, E>::run(f);
    }
};
template <int E> struct Unroll<E, E> {
    template <class F> __device__ __forceinline__ static void run(F &&) {}
};

constexpr int kNT = 256;   // threads per workgroup of the streaming kernels

// e8m0 -> fp32, exactly 2^(b-127): b<<23 is the normal encoding, b == 0 is the
// subnormal 2^-127, 0xFF is NaN (MXFP4.decodeScale, MXFP4.swift:37-40).
__device__ __forceinline__ float decode_scale(uint32_t b)
{
    uint32_t bits = b << 23;
    bits = (b == 0u) ? 0x00400000u : bits;
    bits = (b == 255u) ? 0x7FC00000u : bits;
    return __uint_as_float(bits);
}

// Activation vector layout in LDS: one block of 32 elements per row of
// kBlockDw dwords; the 4-dword pad staggers consecutive blocks across banks
// (lanes of a wave read consecutive blocks).
template <int XK> struct XL { static constexpr int kBlockDw = 20; };   // 16-bit: 16 + 4
template <> struct XL<DT_F32> { static constexpr int kBlockDw = 36; }; // f32: 32 + 4

// --- one block: 16 packed bytes . 32 activations -> fp32 partial ----------

#define GW_CVT_BF16(word, sel) __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4((word), 1.0f, (sel))
#define GW_CVT_F16(word, sel) __builtin_amdgcn_cvt_scalef32_pk_f16_fp4((word), 1.0f, (sel))
#define GW_CVT_F32(word, sel) __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((word), 1.0f, (sel))

// Widened weights of one block, kept in registers so several token vectors can
// reuse them.
template <int XK> struct WBlock { uint32_t v[16]; };       // 16 packed 16-bit pairs
template <> struct WBlock<DT_F32> { f32x2 v[16]; };

template <int XK> __device__ __forceinline__ void widen(const uint4 &w, WBlock<XK> &o);

template <> __device__ __forceinline__ void widen<DT_BF16>(const uint4 &w, WBlock<DT_BF16> &o)
{
#define GW_W(i, word, sel) o.v[i] = __builtin_bit_cast(uint32_t, GW_CVT_BF16(word, sel))
    GW_W(0, w.x, 0); GW_W(1, w.x, 1); GW_W(2, w.x, 2); GW_W(3, w.x, 3);
    GW_W(4, w.y, 0); GW_W(5, w.y, 1); GW_W(6, w.y, 2); GW_W(7, w.y, 3);
    GW_W(8, w.z, 0); GW_W(9, w.z, 1); GW_W(10, w.z, 2); GW_W(11, w.z, 3);
    GW_W(12, w.w, 0); GW_W(13, w.w, 1); GW_W(14, w.w, 2); GW_W(15, w.w, 3);
#undef GW_W
}

template <> __device__ __forceinline__ void widen<DT_F16>(const uint4 &w, WBlock<DT_F16> &o)
{
#define GW_W(i, word, sel) o.v[i] = __builtin_bit_cast(uint32_t, GW_CVT_F16(word, sel))
    GW_W(0, w.x, 0); GW_W(1, w.x, 1); GW_W(2, w.x, 2); GW_W(3, w.x, 3);
    GW_W(4, w.y, 0); GW_W(5, w.y, 1); GW_W(6, w.y, 2); GW_W(7, w.y, 3);
    GW_W(8, w.z, 0); GW_W(9, w.z, 1); GW_W(10, w.z, 2); GW_W(11, w.z, 3);
    GW_W(12, w.w, 0); GW_W(13, w.w, 1); GW_W(14, w.w, 2); GW_W(15, w.w, 3);
#undef GW_W
}

template <> __device__ __forceinline__ void widen<DT_F32>(const uint4 &w, WBlock<DT_F32> &o)
{
#define GW_W(i, word, sel) o.v[i] = GW_CVT_F32(word, sel)
    GW_W(0, w.x, 0); GW_W(1, w.x, 1); GW_W(2, w.x, 2); GW_W(3, w.x, 3);
    GW_W(4, w.y, 0); GW_W(5, w.y, 1); GW_W(6, w.y, 2); GW_W(7, w.y, 3);
    GW_W(8, w.z, 0); GW_W(9, w.z, 1); GW_W(10, w.z, 2); GW_W(11, w.z, 3);
    GW_W(12, w.w, 0); GW_W(13, w.w, 1); GW_W(14, w.w, 2); GW_W(15, w.w, 3);
#undef GW_W
}

// Dot of a widened block with one activation block in LDS (layout XL<XK>).
template <int XK> __device__ __forceinline__ float block_dot(const WBlock<XK> &w,
                                                            const uint32_t *xb);

// The same dot with the activation block already in registers (16-bit x).
template <int XK> __device__ __forceinline__ float block_dot_r(const WBlock<XK> &w,
                                                              const uint4 (&x)[4]);

template <> __device__ __forceinline__ float block_dot_r<DT_BF16>(const WBlock<DT_BF16> &w,
                                                                 const uint4 (&xv)[4])
{
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 x = xv[q];
        a0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.v[4 * q + 0]),
                                             __builtin_bit_cast(bf16x2, x.x), a0, false);
        a1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.v[4 * q + 1]),
                                             __builtin_bit_cast(bf16x2, x.y), a1, false);
        a0 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.v[4 * q + 2]),
                                             __builtin_bit_cast(bf16x2, x.z), a0, false);
        a1 = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w.v[4 * q + 3]),
                                             __builtin_bit_cast(bf16x2, x.w), a1, false);
    }
    return a0 + a1;
}

template <> __device__ __forceinline__ float block_dot_r<DT_F16>(const WBlock<DT_F16> &w,
                                                                const uint4 (&xv)[4])
{
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint4 x = xv[q];
        a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.v[4 * q + 0]),
                                    __builtin_bit_cast(f16x2, x.x), a0, false);
        a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.v[4 * q + 1]),
                                    __builtin_bit_cast(f16x2, x.y), a1, false);
        a0 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.v[4 * q + 2]),
                                    __builtin_bit_cast(f16x2, x.z), a0, false);
        a1 = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w.v[4 * q + 3]),
                                    __builtin_bit_cast(f16x2, x.w), a1, false);
    }
    return a0 + a1;
}

template <> __device__ __forceinline__ float block_dot<DT_BF16>(const WBlock<DT_BF16> &w,
                                                               const uint32_t *xb)
{
    const uint4 *xv = reinterpret_cast<const uint4 *>(xb);
    const uint4 x[4] = {xv[0], xv[1], xv[2], xv[3]};
    return block_dot_r<DT_BF16>(w, x);
}

template <> __device__ __forceinline__ float block_dot<DT_F16>(const WBlock<DT_F16> &w,
                                                              const uint32_t *xb)
{
    const uint4 *xv = reinterpret_cast<const uint4 *>(xb);
    const uint4 x[4] = {xv[0], xv[1], xv[2], xv[3]};
    return block_dot_r<DT_F16>(w, x);
}

template <> __device__ __forceinline__ float block_dot<DT_F32>(const WBlock<DT_F32> &w,
                                                              const uint32_t *xb)
{
    const float4 *xv = reinterpret_cast<const float4 *>(xb);
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 x = xv[q];
        a0 = fmaf(w.v[2 * q].x, x.x, a0);
        a1 = fmaf(w.v[2 * q].y, x.y, a1);
        a0 = fmaf(w.v[2 * q + 1].x, x.z, a0);
        a1 = fmaf(w.v[2 * q + 1].y, x.w, a1);
    }
    return a0 + a1;
}

// --- activation vector staging ---------------------------------------------

// Copies one activation vector of `n` elements (n % 32 == 0) of dtype XK from
// global memory into LDS layout XL<XK>, using threads [tid0, tid0 + nthr) of
// the block.  16-byte loads when the source is 16-byte aligned; the loop is
// unrolled so a thread's loads are all in flight before its first LDS store.
template <int XK>
__device__ __forceinline__ void stage_vector(uint32_t *dst, const void *src, int n, int tid,
                                             int nthr)
{
    constexpr int BD = XL<XK>::kBlockDw;
    if ((reinterpret_cast<uintptr_t>(src) & 15u) == 0) {
        // Batches of 4 loads per thread in flight together.  Indices are
        // clamped rather than guarded, so loads and stores are unconditional
        // (a guard lets the compiler sink each load to its store, one round
        // trip per load); the clamped duplicates store equal values.
        constexpr int Q = XK == DT_F32 ? 8 : 4;        // 16-byte chunks of data per block
        constexpr int BQ = BD / 4;                      // 16-byte chunks per block in LDS
        const uint4 *s = static_cast<const uint4 *>(src);
        uint4 *d = reinterpret_cast<uint4 *>(dst);
        const int n4 = XK == DT_F32 ? n / 4 : n / 8;
        for (int base = 0; base < n4; base += 4 * nthr) {
            uint4 v[4];
            int idx[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                idx[u] = min(base + u * nthr + tid, n4 - 1);
                v[u] = s[idx[u]];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) d[(idx[u] / Q) * BQ + (idx[u] % Q)] = v[u];
        }
    } else if constexpr (XK == DT_F32) {
        const float *s = static_cast<const float *>(src);
#pragma unroll 4
        for (int i = tid; i < n; i += nthr) dst[(i >> 5) * BD + (i & 31)] = __float_as_uint(s[i]);
    } else {
        const uint32_t *s = static_cast<const uint32_t *>(src);   // element pairs
#pragma unroll 4
        for (int i = tid; i < n / 2; i += nthr) dst[(i >> 4) * BD + (i & 15)] = s[i];
    }
}

// Whether stage_vector's aligned form covers the vector with one batch of 4
// loads per thread (n4 <= 4 * nthr): a kernel can then issue those loads, queue
// other loads behind them and store the values to LDS afterwards (the compiler
// waits for these loads only, the older ones).
template <int XK> __device__ __forceinline__ bool vector_batch_fits(const void *src, int n, int nthr)
{
    const int n4 = XK == DT_F32 ? n / 4 : n / 8;
    return (reinterpret_cast<uintptr_t>(src) & 15u) == 0 && n4 <= 4 * nthr;
}

// The 16-byte piece `i` of such a vector into its place in the LDS layout.
template <int XK> __device__ __forceinline__ void vector_store(uint32_t *dst, int i, const uint4 &v)
{
    constexpr int Q = XK == DT_F32 ? 8 : 4, BQ = XL<XK>::kBlockDw / 4;
    reinterpret_cast<uint4 *>(dst)[(i / Q) * BQ + (i % Q)] = v;
}

template <int XK>
__device__ __forceinline__ void stage_vector(uint32_t *dst, const void *src, int n)
{
    stage_vector<XK>(dst, src, n, threadIdx.x, blockDim.x);
}

// --- small numerics ----------------------------------------------------------

// BFloat16.fromFloat (Install/Int8Affine.swift:86-93): RNE, NaN kept a NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float v)
{
    uint32_t bits = __float_as_uint(v);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((bits >> 16) | 0x0040u);
    uint32_t rounding = ((bits >> 16) & 1u) + 0x7FFFu;
    return (uint16_t)((bits + rounding) >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b)
{
    return __uint_as_float((uint32_t)b << 16);
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float v)
{
    return __builtin_bit_cast(uint16_t, (_Float16)v);   // v_cvt_f16_f32, RNE
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h)
{
    return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ float load_as_f32(const void *p, int dtype, int64_t i)
{
    if (dtype == DT_F32) return static_cast<const float *>(p)[i];
    const uint16_t b = static_cast<const uint16_t *>(p)[i];
    return dtype == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

// Bias of row r: bf16 (the .gwt layout, InstallLayout.swift:76-77), f32, or none.
__device__ __forceinline__ float load_bias(const void *bias, int dtype, int64_t r)
{
    return bias ? load_as_f32(bias, dtype, r) : 0.0f;
}

// dst + a * w with the product and the sum rounded separately (no FMA), the
// arithmetic of expert_accumulate (expert.metal:115).
__device__ __forceinline__ float add_scaled_rn(float dst, float a, float w)
{
#pragma clang fp contract(off)
    return dst + a * w;
}

// GPT-OSS expert gate (expert.metal:93-101) and SiLU-GLU (expert.metal:388-392),
// written in the kernels' operation order; fp16 rounding is the caller's.
__device__ __forceinline__ float gptoss_glu(float gate, float up, float limit, float alpha)
{
    gate = fminf(gate, limit);
    up = fminf(fmaxf(up, -limit), limit);
    const float glu = gate * (1.0f / (1.0f + expf(-alpha * gate)));
    return (up + 1.0f) * glu;
}

__device__ __forceinline__ float silu_glu(float gate, float up)
{
    const float silu = gate * (1.0f / (1.0f + expf(-gate)));
    return silu * up;
}

__device__ __forceinline__ float apply_activation(int kind, float g, float u, float limit,
                                                  float alpha)
{
    return kind == 0 ? gptoss_glu(g, u, limit, alpha) : silu_glu(g, u);
}

// --- work split and row reductions (shared by the streaming kernels) ------

// a = q*d + r for 0 <= a < 2^22, without a loop or an integer divide: the
// float quotient is off by at most one and is corrected with selects (the
// engine keeps control flow out of its load path).
__device__ __forceinline__ void divmod_small(int a, int d, float inv_d, int &q, int &r)
{
    q = (int)((float)a * inv_d);
    r = a - q * d;
    q = r < 0 ? q - 1 : q;
    r = r < 0 ? r + d : r;
    q = r >= d ? q + 1 : q;
    r = r >= d ? r - d : r;
}

// This workgroup's share [lo, hi) of `total` items in balanced contiguous
// ranges (the first total % G workgroups take one more), with one 32-bit
// division instead of 64-bit products and quotients.
__device__ __forceinline__ void slice_of(int total, int &lo, int &hi)
{
    const unsigned G = gridDim.x, b = blockIdx.x;
    const unsigned q = (unsigned)total / G, r = (unsigned)total - q * G;
    lo = (int)(b * q + min(b, r));
    hi = lo + (int)q + (b < r ? 1 : 0);
}

// Sum over the TPR lanes of a row segment with DPP butterflies inside a
// 16-lane row (pair swap, quad swap, half mirror, mirror): every lane ends with
// the same bits (each step adds two equal partial sums in either order).
#define GW_DPPF(x, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), (ctrl), 0xF, 0xF, false))
// 32-lane segments add the neighbouring 16-lane row last (permlane16 swap),
// the same two partial sums in the same order in both rows.
template <int TPR> __device__ __forceinline__ float seg_sum(float v)
{
    static_assert(TPR == 8 || TPR == 16 || TPR == 32, "row segments are 8, 16 or 32 lanes");
    v += GW_DPPF(v, 0xB1);                      // quad_perm [1,0,3,2]
    v += GW_DPPF(v, 0x4E);                      // quad_perm [2,3,0,1]
    v += GW_DPPF(v, 0x141);                     // row_half_mirror
    if constexpr (TPR >= 16) v += GW_DPPF(v, 0x140);   // row_mirror
    if constexpr (TPR == 32) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                        false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}
#undef GW_DPPF

// Eight consecutive elements as fp32 from a 16-byte aligned position (one
// 16-byte load for 16-bit data, two for fp32).
template <int DT>
__device__ __forceinline__ void load8_f32(const void *p, int64_t i, float (&v)[8])
{
    if constexpr (DT == DT_F32) {
        const float4 *q = reinterpret_cast<const float4 *>(static_cast<const float *>(p) + i);
        const float4 a = q[0], c = q[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
        const uint4 a = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(p) + i);
        const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint16_t lo = (uint16_t)(w[k] & 0xFFFFu), hi = (uint16_t)(w[k] >> 16);
            v[2 * k] = DT == DT_BF16 ? bf16_bits_to_f32(lo) : f16_bits_to_f32(lo);
            v[2 * k + 1] = DT == DT_BF16 ? bf16_bits_to_f32(hi) : f16_bits_to_f32(hi);
        }
    }
}

// ---- router logits by slices ------------------------------------------------
// For one token, the E logits (bf16_gemv_bias, router.metal:18-34) can be
// computed by E * S waves, wave (e, s) dotting weight row e with x over slice
// s of S (L = H / S elements): the one-token layer kernel does this in its
// workgroups and the standalone router in the same order, so both give the
// same logit bits.  Lane l dots the 8-element units l, l + 64, ... of the
// slice in order (fused multiply-adds into one sum), the wave sum is a fixed
// xor butterfly, and a logit is its S partials added in slice order plus the
// bias.

template <int WDT, int XDT>
__device__ __forceinline__ float router_partial(const void *W, const void *x, int e, int s, int L,
                                                int H, int lane)
{
    const int units = L >> 3;
    float w[kRouterUnits][8], xv[kRouterUnits][8];
    bool ok[kRouterUnits];
#pragma unroll
    for (int u = 0; u < kRouterUnits; ++u) {
        const int unit = lane + 64 * u;
        ok[u] = unit < units;
        const int at = s * L + 8 * (ok[u] ? unit : 0);
        load8_f32<WDT>(W, (int64_t)e * H + at, w[u]);
        load8_f32<XDT>(x, at, xv[u]);
    }
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < kRouterUnits; ++u)
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float nv = acc + w[u][q] * xv[u][q];
            acc = ok[u] ? nv : acc;
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    return acc;
}

// router_partial with the weight dtype chosen at run time.
template <int XDT>
__device__ __forceinline__ float router_partial_dt(const void *W, int w_dt, const void *x, int e,
                                                   int s, int L, int H, int lane)
{
    if (w_dt == DT_F32) return router_partial<DT_F32, XDT>(W, x, e, s, L, H, lane);
    if (w_dt == DT_F16) return router_partial<DT_F16, XDT>(W, x, e, s, L, H, lane);
    return router_partial<DT_BF16, XDT>(W, x, e, s, L, H, lane);
}

}  // namespace gw
