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
// block's e8m0 scale folded in: e2m1 * 2^(b-127) is exact in bf16 (two
// significant bits) for every byte up to 252, subnormal 2^-127 included, and
// byte 255 widens to NaN.  The reference multiplies each finite block partial
// by the scale (referenceMXFP4, DequantGEMVBenchmark.swift:106-116), whereas a
// folded 2^126 or 2^127 (bytes 253, 254) would overflow bf16 for |code| >= 4
// and >= 2.  So a row that holds a 253 or 254 byte folds 2^(b-129) into every
// block and its fp32 accumulator is multiplied by 4 after the K loop (a
// prologue pass finds such rows and lowers their staged bytes by 2).  The
// conversion reads a subnormal scale as 2^-127, so in such a row bytes 0 and
// 1 widen 4x and 2x too large: their products are 2^-250 of a 253/254 block's for activations
// of like size, and differ from the reference only where every 253/254 block
// of the row sums to exactly zero.  The gate_up input enters the bf16 matrix
// cores as exact sums of bf16 planes: bf16 x is one plane, fp16 two (hi =
// bf16(v), lo = v - hi) and fp32 three.  The down input is the fp16
// activation itself (one plane): a wave whose scale bytes all lie in [104,
// 140] widens its weights to fp16, exactly, and multiplies on
// v_mfma_f32_32x32x16_f16; any other wave splits each activation into two
// bf16 values as it reads it.  Every product in the fp32 normal range is then
// exact and the matrix cores accumulate in fp32, so the results differ from
// the reference's scalar loop only in summation order.
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>

#include "gw_device.h"
#include "gw_launch.h"
#include "gw_route.h"

namespace gw {


typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(1))) u32x4v g_u32x4v;
typedef const __attribute__((address_space(1))) uint8_t g_u8c;

constexpr int kPT = 32;                 // tokens per tile (MFMA columns)
constexpr int kCachePolicySc1 = 16;     // buffer access cache policy: device-coherent (sc1)
constexpr int kKC = 8;                  // 32-element blocks per staged activation chunk
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
    if (E <= 128) select_one<2>(logits + (int64_t)t * E, E, K, sid, w);
    else select_one<4>(logits + (int64_t)t * E, E, K, sid, w);
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
// the order inside a group never changes a value.  The expert offsets and the
// tile list come from one exclusive scan over the experts (waves 0..3 hold
// one expert per lane).  Batches of at most kRouteGroupTokens tokens (one
// per wave) are routed in the same workgroup first and skip the route kernel
// (batches above the GEMMs' own grouping reach this only when that grouping
// is lowered); with two tokens a wave the route kernel in front was faster.
// ---------------------------------------------------------------------------

constexpr int kGroupThreads = 1024;
constexpr int kRouteGroupTokens = 16;
constexpr int kRouteGroupEntries = kRouteGroupTokens * kMaxTopK;

__global__ __launch_bounds__(kGroupThreads) void prefill_group_kernel(
    const float *__restrict__ logits, int T, int K, float *__restrict__ weights,
    int32_t *__restrict__ ids, int E, int32_t *__restrict__ offsets,
    int32_t *__restrict__ order, int32_t *__restrict__ tiles, int32_t *__restrict__ ntiles,
    int max_tiles)
{
    __shared__ int cnt[kPrefillMaxExperts];
    __shared__ int cur[kPrefillMaxExperts];
    __shared__ int off[kPrefillMaxExperts + 1];
    __shared__ int wtot[2][kPrefillMaxExperts / 64];
    __shared__ int sids[kRouteGroupEntries];
    const int tid = (int)threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int N = T * K;
    for (int e = tid; e < E; e += kGroupThreads) {
        cnt[e] = 0;
        cur[e] = 0;
    }
    if (logits) {
        // routing fused in: the launcher only passes logits for N <= kRouteGroupEntries
        for (int t = wv; t < T; t += kGroupThreads / 64) {
            int sid;
            float w;
            if (E <= 128) select_one<2>(logits + (int64_t)t * E, E, K, sid, w);
            else select_one<4>(logits + (int64_t)t * E, E, K, sid, w);
            if (lane < K) {
                ids[t * K + lane] = sid;
                weights[t * K + lane] = w;
                sids[t * K + lane] = sid;
            }
        }
    }
    __syncthreads();
    for (int j = tid; j < N; j += kGroupThreads) atomicAdd(&cnt[logits ? sids[j] : ids[j]], 1);
    __syncthreads();
    // inclusive wave scans of (entries, tiles) per expert, then wave totals
    int c = 0, n = 0;
    if (tid < kPrefillMaxExperts && tid < E) {
        c = cnt[tid];
        n = (c + kPT - 1) / kPT;
    }
    int ic = c, in = n;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int uc = __shfl_up(ic, d, 64), un = __shfl_up(in, d, 64);
        if (lane >= d) {
            ic += uc;
            in += un;
        }
    }
    if (tid < kPrefillMaxExperts && lane == 63) {
        wtot[0][wv] = ic;
        wtot[1][wv] = in;
    }
    __syncthreads();
    if (tid < E) {
        int bc = 0, bn = 0;
        for (int w = 0; w < wv; ++w) {
            bc += wtot[0][w];
            bn += wtot[1][w];
        }
        const int ec = bc + ic - c, en = bn + in - n;   // exclusive prefix of expert tid
        off[tid] = ec;
        for (int m = 0; m < n && en + m < max_tiles; ++m) tiles[en + m] = (tid << 16) | m;
        if (tid == E - 1) {
            off[E] = ec + c;
            *ntiles = min(en + n, max_tiles);
        }
    }
    __syncthreads();
    for (int e = tid; e <= E; e += kGroupThreads) offsets[e] = off[e];
    for (int j = tid; j < N; j += kGroupThreads) {
        const int e = logits ? sids[j] : ids[j];
        order[off[e] + atomicAdd(&cur[e], 1)] = j;
    }
}

// ---------------------------------------------------------------------------
// 3./4. Grouped GEMM: workgroup (feature tile f, work item) computes
// C[256 features x 32 entries] = W_e[f-tile, :] . X[entries, :]^T over K, one
// 32x32 block per wave, in chunks of kKC 32-element blocks (256 K elements).
//
// Operands.  The gate_up input arrives as PL bf16 planes whose sum is exact
// (bf16 x: the input itself; fp16 or fp32 x: split beforehand); the down
// input is one plane of fp16 activations, written by the gate_up epilogue.  Per
// chunk a lane (row r = lane & 31, half h = lane >> 5) holds its row's blocks
// 2i + h, i = 0..3 (so the two lanes of a row read 32 contiguous bytes per
// load instruction), widened to bf16 with the block scale folded in; MFMA
// 4i+d takes dword d of block 2i+h, i.e. chunk elements 64i + 32h + 8d .. +7,
// from A (weights) and from B (the staged activation row of entry r), so A
// and B share one K order.  C element v of a lane is feature row 8(v/4) +
// 4h + (v%4), entry column lane & 31.
//
// Pipeline.  A chunk's activations are staged by LDS-DMA (16 bytes per lane
// straight into LDS, no registers) and its weights are loaded into a
// register ring; both are issued together kDepth-1 chunks ahead, activation
// first.  The vector-memory counter completes in issue order, so waiting for
// a chunk's activations leaves every younger load in flight: kDepth-1 chunks
// of weights stream while one chunk is multiplied.  Staged rows are 512
// bytes (32 pieces of 16 bytes); piece j of row t sits in slot j ^ (t & 15),
// which keeps the B reads of 16 consecutive rows on distinct LDS banks.
// ---------------------------------------------------------------------------

struct GemmArgs {
    const int32_t *tiles;
    const int32_t *ntiles;
    const int32_t *offsets;
    const int32_t *order;
    const uint16_t *in;           // PL bf16 planes of [rows, kdim] (down: fp16, PL 1)
    int64_t in_plane;             // elements between planes
    uint32_t in_bytes;            // bytes of all planes (below 2^31)
    int in_row_div;               // entry -> input row: entry / in_row_div (K for x, 1 for act)
    const uint8_t *experts_base;
    int64_t stride;
    int64_t blocks_off, scales_off, bias_off;   // section offsets within an expert
    int bias_dt;                  // -1: no bias
    int kdim, fdim;               // K (input width) and weight rows
    uint16_t *act_out;            // gate_up: fp16 activations [N, fdim/2]
    float *y_out;                 // down: [N, fdim] fp32
    int act_kind;
    float limit, alpha;
    // Self-grouped batches (sg_tokens > 0, at most kSelfGroupTokens tokens):
    // the gate_up launch routes from sg_logits [T, E] in every workgroup and
    // workgroup 0 writes the routing to sg_ids_out / sg_w_out; the down
    // launch groups from those ids (sg_ids).  The tile list is unused.
    int sg_tokens, sg_topk, sg_experts;
    const float *sg_logits;
    const int32_t *sg_ids;
    int32_t *sg_ids_out;
    float *sg_w_out;
    // Combine fused into the down launch (arrive != null): y rows are stored
    // device-coherent, every entry counts itself on arrive[token * tiles +
    // feature tile], and the workgroup whose count completes a token's tile
    // sums that tile into comb_out (weights comb_w [T, K], router order).
    uint32_t *arrive;
    uint32_t y_bytes;             // bytes of y_out (below 2^31)
    const float *comb_w;
    float *comb_out;
    uint16_t *comb_out_bf16;
    int comb_topk, comb_residual;
};

// A batch of at most this many tokens gives every expert at most one tile.
constexpr int kSelfGroupTokens = kPT;


// Calls f(integral_constant<int, S>) for S = B .. E-1 in order.
constexpr int kRowBytes = kKC * 32 * 2;       // one staged chunk row: 256 bf16
constexpr int kPlaneBytes = kPT * kRowBytes;  // one staged plane of a chunk
constexpr int kPrefillLdsMax = 160 * 1024;

// LDS layout of one GEMM workgroup (byte offsets): the kPT entry ids, the
// [depth][planes] staged activation chunks (also the output tile at the end),
// a copy of the workgroup's 32 x waves rows of scale bytes (whole 1 KiB DMA pieces
// from a 16-byte aligned start, plus room for reads one dword past the last
// byte), and the bias tile.
struct PrefillLds { int ring, scales, bias, total; };
__host__ __device__ inline PrefillLds prefill_lds(int planes, int depth, int nb, int waves)
{
    PrefillLds l;
    l.ring = kPT * 4;
    l.scales = l.ring + depth * planes * kPlaneBytes;
    l.bias = l.scales + ((32 * waves * nb + 32 + 1023) & ~1023);
    l.total = l.bias + ((32 * waves * 4 + 1023) & ~1023);
    return l;
}

typedef __attribute__((address_space(3))) void l_void;

// s_waitcnt with only the vector-memory count limited (gfx9 encoding: vmcnt
// in bits 3:0 and 15:14; expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
template <int N> __device__ __forceinline__ void wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// The staged activations are read with ds_read_b128 written out here: the
// compiler's own wait insertion treats any LDS read after an LDS-DMA as
// possibly dependent on the newest DMA and would drain the whole pipeline;
// the kernel orders DMA and reads itself (a counted vmcnt wait and a barrier
// per chunk), and lds_wait for the reads before their values are used.
__device__ __forceinline__ uint32_t lds_address(const void *p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ uint32_t lds_read4(uint32_t addr)
{
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

__device__ __forceinline__ void lds_write1(uint32_t addr, uint32_t v)
{
    asm volatile("ds_write_b8 %0, %1" : : "v"(addr), "v"(v) : "memory");
}

__device__ __forceinline__ bf16x8 lds_read16(uint32_t addr)
{
    bf16x8 v;
    asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
    return v;
}

// Waits until at most N of this wave's LDS reads are outstanding (they
// complete in order); the caller then passes each register it reads through
// an empty asm so that no use is scheduled above the wait.
template <int N> __device__ __forceinline__ void lds_wait()
{
    static_assert(N >= 0 && N < 16, "lgkmcnt out of range");
    if constexpr (N == 0) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    else if constexpr (N == 2) asm volatile("s_waitcnt lgkmcnt(2)" ::: "memory");
    else if constexpr (N == 3) asm volatile("s_waitcnt lgkmcnt(3)" ::: "memory");
    else if constexpr (N == 4) asm volatile("s_waitcnt lgkmcnt(4)" ::: "memory");
    else static_assert(N == 0 || N == 2 || N == 3 || N == 4, "unsupported count");
}

// W waves, D-deep ring.  The 8-wave, 2-deep form is held to 128 VGPRs (four
// waves per SIMD), so two of its workgroups share a CU when their LDS fits,
// and the 4-wave form to 168 (three workgroups per CU); the others hold ~165
// VGPRs and one workgroup per CU.
template <int PL, bool GATE_UP, int W, int D, bool COMB>
__global__ __launch_bounds__(64 * W, W == 8 && D == 2 ? 4 : W == 4 ? 3 : 1) void prefill_gemm_kernel(GemmArgs a)
{
    // W waves, 32 features each: a workgroup computes kF features x kPT entries.
    constexpr int kF = 32 * W, kThreads = 64 * W;
    static_assert(D >= 2 && D <= 4, "ring depth");
    constexpr int kNW = 4;                    // weight-ring loads per chunk (4 x 16 B)
    // Two-row LDS-DMA loads per wave per plane and chunk: 4 waves stage the
    // 32 rows four loads each, 8 or 12 waves two each.
    constexpr int kXR = W == 4 ? 4 : 2;
    constexpr int kNX = kXR * PL;             // LDS-DMA loads per chunk per wave
    // The down GEMM takes one plane of fp16 activations: a wave whose rows'
    // scale bytes all lie in [104, 140] widens its weights to fp16, where
    // e2m1 * 2^(b-127) is exact (the smallest, 2^(b-128), is at least the
    // fp16 subnormal step 2^-24, and 6 * 2^13 < 65504), and multiplies on the
    // fp16 MFMA; other waves split each activation into two bf16 values.
    constexpr bool F16IN = PL == 1 && !GATE_UP;
    // Loads a wave issues after a chunk's DMA until it waits for that DMA.
    constexpr int kYounger = kNW + (D - 2) * (kNX + kNW);
    // Weight loads four lanes to a row with a pair swap (kSwap), or, in the
    // 8-wave 2-deep shape held to 128 registers, two lanes to a row reading
    // their own blocks (the swap's extra registers would spill there); the
    // lane's blocks, and so every product and sum, are the same either way.
    constexpr bool kSwap = !(W == 8 && D == 2);
    static_assert(D * PL * kPlaneBytes >= 2048, "the self-grouping lists must fit in the ring");
    // Dynamic LDS only (a static __shared__ variable would shift the dynamic
    // area off its alignment); layout in prefill_lds.
    extern __shared__ __align__(16) uint32_t plds[];
    uint8_t *lds8 = reinterpret_cast<uint8_t *>(plds);
    int *ent = reinterpret_cast<int *>(plds);
    const int nb = a.kdim >> 5;
    const PrefillLds lay = prefill_lds(PL, D, nb, W);
    uint8_t *xring = lds8 + lay.ring;
    // Work unit -> (expert e, feature tile, entry tile m).  Units run expert by
    // expert, feature tile by feature tile, with the entry tiles of one
    // (expert, feature tile) adjacent, so the workgroups that read the same
    // weights run together; and each XCD (workgroup ids congruent mod 8) takes
    // one contiguous eighth of the units, so those workgroups share one L2.
    // floor(unit / nft) is always one of the unit's expert's tiles.
    const int nft = (a.fdim + kF - 1) / kF;
    const int jx = (int)(blockIdx.x >> 3);
    int e, fidx, ntok;
    if (a.sg_tokens > 0) {
        // Self-grouped batch: every expert has at most sg_tokens <= kPT
        // entries (top-k picks distinct experts), so a work unit is
        // (active expert, feature tile) and each workgroup derives the whole
        // list from the routing in its own LDS: the expert ids of the entries
        // (selected here from the logits, or read from the routing the
        // gate_up launch wrote), a 256-bit mask of active experts, and the
        // unit's expert as the tq-th set bit.  Scratch lives in the staging
        // ring, which no DMA targets yet.
        const int tid = (int)threadIdx.x, T = a.sg_tokens, K = a.sg_topk, E = a.sg_experts;
        const int N = T * K;
        int *sid_l = reinterpret_cast<int *>(xring);                          // [N <= 256]
        uint32_t *amask = reinterpret_cast<uint32_t *>(xring + 1024);         // [8]
        int *ecount = reinterpret_cast<int *>(xring + 1024 + 32);
        float *lg = reinterpret_cast<float *>(xring + 2048);                  // [T, E]
        if (tid < 8) amask[tid] = 0u;
        if (tid == 8) *ecount = 0;
        if (a.sg_logits) {
            // All logits into LDS with every load in flight when they fit
            // the ring (else each wave reads its tokens' rows itself), then
            // one wave per token selects.
            constexpr int kRing = D * PL * kPlaneBytes - 2048;
            constexpr int kLU = (kRing / 4 + kThreads - 1) / kThreads;
            const int n = T * E;
            const bool staged = n * 4 <= kRing;
            if (staged) {
                float v[kLU];
#pragma unroll
                for (int u = 0; u < kLU; ++u) {
                    const int i = tid + u * kThreads;
                    v[u] = i < n ? a.sg_logits[i] : 0.0f;
                }
#pragma unroll
                for (int u = 0; u < kLU; ++u) {
                    const int i = tid + u * kThreads;
                    if (i < n) lg[i] = v[u];
                }
                __syncthreads();
            }
            const float *src = staged ? lg : a.sg_logits;
            const int wv = __builtin_amdgcn_readfirstlane(tid >> 6), ln = tid & 63;
            for (int t = wv; t < T; t += W) {
                int sid;
                float w;
                if (E <= 128) select_one<2>(src + t * E, E, K, sid, w);
                else select_one<4>(src + t * E, E, K, sid, w);
                if (ln < K) {
                    sid_l[t * K + ln] = sid;
                    if (blockIdx.x == 0) {                // one copy for down and combine
                        a.sg_ids_out[t * K + ln] = sid;
                        a.sg_w_out[t * K + ln] = w;
                    }
                }
            }
        } else if (tid < N) {
            sid_l[tid] = a.sg_ids[tid];
        }
        __syncthreads();
        if (tid < N && (unsigned)sid_l[tid] < (unsigned)E)
            atomicOr(&amask[sid_l[tid] >> 5], 1u << (sid_l[tid] & 31));
        __syncthreads();
        uint32_t words[8];
        int active = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            words[i] = __builtin_amdgcn_readfirstlane(amask[i]);
            active += __builtin_popcount(words[i]);
        }
        const int units = active * nft;
        const int per = (units + 7) >> 3;
        const int unit = (int)(blockIdx.x & 7) * per + jx;
        if (jx >= per || unit >= units) return;       // uniform: the workgroup leaves
        const int tq = unit / nft;
        fidx = unit - tq * nft;
        // The tq-th active expert in id order.
        int rem = tq, wi = 0;
        while (wi < 7 && rem >= __builtin_popcount(words[wi])) rem -= __builtin_popcount(words[wi++]);
        uint32_t x = words[wi];
        for (int i = 0; i < rem; ++i) x &= x - 1;
        e = wi * 32 + __builtin_ctz(x);
        // Its entries, in any order (an entry's results depend on its row only).
        if (tid < N && sid_l[tid] == e) {
            const int pos = atomicAdd(ecount, 1);
            if (pos < kPT) ent[pos] = tid;   // always: a token picks an expert once
        }
        __syncthreads();
        ntok = min(__builtin_amdgcn_readfirstlane(*ecount), kPT);
        if (tid < kPT && tid >= ntok) ent[tid] = ent[ntok - 1];
    } else {
        const int units = *a.ntiles * nft;
        const int per = (units + 7) >> 3;
        const int unit = (int)(blockIdx.x & 7) * per + jx;
        if (jx >= per || unit >= units) return;       // uniform: the workgroup leaves
        const int tq = unit / nft;
        const int te = a.tiles[tq];
        e = te >> 16;
        const int t0 = tq - (te & 0xFFFF);
        const int ecnt = a.offsets[e + 1] - a.offsets[e];
        const int ne = (ecnt + kPT - 1) / kPT;
        const int local = unit - t0 * nft;
        fidx = local / ne;
        const int m = local - fidx * ne;
        const int g0 = a.offsets[e] + m * kPT;
        ntok = min(kPT, a.offsets[e + 1] - g0);
        if (threadIdx.x < kPT) ent[threadIdx.x] = a.order[g0 + min((int)threadIdx.x, ntok - 1)];
    }

    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5, c = lane & 31;
    const int f0 = fidx * kF;
    const int fbase = f0 + wave * 32;
    const int row = min(fbase + c, a.fdim - 1);       // clamped: rows past fdim are never stored
    const uint8_t *ex = a.experts_base + (int64_t)e * a.stride;
    const uint8_t *wrow = ex + a.blocks_off + (int64_t)row * nb * 16;
    // The weight loads read the lane's row pair (rows c & ~1 and c | 1 of the
    // tile, clamped like row): four lanes to a row per load; byte offsets of
    // the two rows from the expert's blocks (an expert's section is far below
    // 4 GiB).
    const uint8_t *wbase = ex + a.blocks_off;
    const uint32_t wrow0 = (uint32_t)min(fbase + (c & ~1), a.fdim - 1) * (uint32_t)(nb * 16);
    const uint32_t wrow1 = (uint32_t)min(fbase + (c | 1), a.fdim - 1) * (uint32_t)(nb * 16);

    __syncthreads();                                  // ent[] is written

    // The workgroup's scale bytes (rows f0 .. f0+kF-1 are contiguous in the
    // scales section) and its bias tile, copied once by LDS-DMA in 1 KiB
    // pieces from a 16-byte aligned start; reads past a section's end
    // return zeros (buffer bounds).
    const uint32_t s0 = (uint32_t)(f0 * nb) & ~15u;
    const int sshift = f0 * nb - (int)s0;
    {
        const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t *>(ex + a.scales_off), (short)0, a.fdim * nb, 0x00020000);
        const int ninst = (sshift + kF * nb + 1023) >> 10;
        for (int k = wave; k < ninst; k += W)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sres, (l_void *)(lds8 + lay.scales + k * 1024),
                                                     16, s0 + k * 1024 + lane * 16, 0, 0, 0);
        const int esz = a.bias_dt == DT_F32 ? 4 : 2;
        if (a.bias_dt >= 0 && wave < (kF * esz + 1023) >> 10) {
            const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint8_t *>(ex + a.bias_off), (short)0, a.fdim * esz, 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(bres, (l_void *)(lds8 + lay.bias + wave * 1024),
                                                     16, f0 * esz + wave * 1024 + lane * 16, 0, 0,
                                                     0);
        }
    }

    // Staging: wave w copies rows 4w' .. 4w'+3 of each plane (w' = w mod 8;
    // waves past 8 repeat waves 0.. with the same bytes to the same slots, so
    // every wave issues the same loads), two rows per DMA (lanes 0-31 row
    // 4w'+2n, lanes 32-63 the next); with 4 waves, wave w copies rows 8w ..
    // 8w+7 in four DMAs.  A lane's slot is lane & 31.  The padding
    // rows of a partial tile (t >= ntok) are read past the buffer's end: the
    // DMA puts zeros in their slots without a memory access, and their
    // columns of the tile are never stored.
    const int sw = wave & 7;
    auto xrow0 = [&](int n) { return W == 4 ? 8 * wave + 2 * n : 4 * sw + 2 * n; };
    int64_t xrow[kXR];
    int xpiece[kXR];
#pragma unroll
    for (int n = 0; n < kXR; ++n) {
        const int t = xrow0(n) + h;
        xpiece[n] = (lane & 31) ^ (t & 15);
        xrow[n] = t < ntok ? (int64_t)(ent[t] / a.in_row_div) * a.kdim : -1;
    }
    // Pieces past kdim read the row's last piece instead; the weights of the
    // blocks there are zeroed, so they add exact zeros (for finite inputs).
    // The buffer form of the LDS-DMA (not the global one) keeps the
    // compiler's own waits for the weight ring exact.
    const __amdgpu_buffer_rsrc_t xres =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(a.in), (short)0,
                                          (int)a.in_bytes, 0x00020000);
    auto xload = [&](int buf, int q) {
#pragma unroll
        for (int p = 0; p < PL; ++p) {
#pragma unroll
            for (int n = 0; n < kXR; ++n) {
                const int k = min(q * (kKC * 32) + xpiece[n] * 8, a.kdim - 8);
                const uint32_t voff =
                    xrow[n] < 0 ? 0x80000000u   // >= in_bytes (< 2^31): out of range
                                : (uint32_t)((p * a.in_plane + xrow[n] + k) * 2);
                uint8_t *dst = xring + (size_t)(buf * PL + p) * kPlaneBytes +
                               xrow0(n) * kRowBytes;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (l_void *)dst, 16, voff, 0, 0, 0);
            }
        }
    };

    // Weight ring: load 2j + t of a chunk reads, for row 2p + t of each of the
    // tile's 16 row pairs (p = c >> 1), the 64 contiguous bytes of blocks 4j ..
    // 4j+3: lane (h, c) block 4j + 2 (c & 1) + h.  The fewer lines a load
    // instruction touches, the fewer requests the texture path makes.  A lane
    // and its pair partner (lane ^ 1) then swap the blocks each read of the
    // other's row (take_blocks), so that the lane holds blocks 2i + h of its
    // own row.  Block indices past nb clamp to the row's last block.  The
    // loaded words are used only when their chunk is multiplied (arithmetic on
    // them here would wait for the load just issued).
    u32x4v wq[D][4];
    auto wload = [&](int slot, int q) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (kSwap) {
                const int bb = min(q * kKC + 4 * (i >> 1) + 2 * (c & 1) + h, nb - 1);
                wq[slot][i] = *(g_u32x4v *)(wbase + ((i & 1) ? wrow1 : wrow0) + (uint32_t)bb * 16u);
            } else {
                wq[slot][i] = *(g_u32x4v *)(wrow + (int64_t)min(q * kKC + 2 * i + h, nb - 1) * 16);
            }
        }
    };
    // Dword d of block 2i + h of the lane's own row, from the chunk's loads
    // as loaded: of the row pair's two loads of blocks 4j .. 4j+3 (j = i >> 1),
    // the one of the lane's own row holds it for one parity of i, and for the
    // other the partner (lane ^ 1) read it: a lane swap by DPP.  Taken where
    // it is used, so no second copy of the chunk's words is held.
    const bool odd_row = (c & 1) != 0;
    auto wdw = [&](const u32x4v (&ld)[4], int i, int d) __attribute__((always_inline)) -> uint32_t {
        if constexpr (!kSwap) return (uint32_t)ld[i][d];
        const int jj = i >> 1;
        if (i & 1) {
            const uint32_t x0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)ld[2 * jj][d], 0xB1, 0xF, 0xF, true);
            return odd_row ? (uint32_t)ld[2 * jj + 1][d] : x0;
        }
        const uint32_t x1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)ld[2 * jj + 1][d], 0xB1, 0xF, 0xF, true);
        return odd_row ? x1 : (uint32_t)ld[2 * jj][d];
    };

    f32x16 acc, acc1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        acc[i] = 0.0f;
        acc1[i] = 0.0f;
    }

    // B read address of piece p for entry c: row c, slot p ^ (c & 15).  MFMA
    // m = 4i + d reads piece 4 (2i + h) + d = (8i + d) ^ 4h (bits apart), so
    // its offset is this lane's base XOR a constant of m.
    const uint32_t rb = (uint32_t)(c * kRowBytes + (((4 * h) ^ (c & 15)) << 4));

    const uint32_t xbase = lds_address(xring);
    // The scale bytes of chunk q of the lane's row start at byte srel + 8q of
    // the copy; the lane's are those of blocks h, h+2, h+4, h+6.
    const uint32_t sbase = lds_address(lds8 + lay.scales);
    const int srel = sshift + (row - f0) * nb + h;

    // Chunk q from ring slot / staging buffer s.  A block past nb is widened
    // from a zero word with scale 1: exact zeros.  The 16 MFMAs (m = 4i + d)
    // run in groups of G whose B reads are issued one group ahead, and
    // alternate between two accumulators so consecutive MFMAs are independent.
    constexpr int G = PL == 1 ? 4 : PL == 2 ? 2 : 1;
    constexpr int NG = 16 / G;
    // FB: the wave's scale bytes leave the fp16 range (F16IN only).  wsrc:
    // the chunk's weight words.
    auto multiply = [&](int q, auto s_const, auto fb_const, const u32x4v (&wsrc)[4]) __attribute__((always_inline)) {
        constexpr int s = decltype(s_const)::value;
        constexpr bool FB = decltype(fb_const)::value;
        // Recomputed per chunk rather than kept in 16 registers per plane.
        uint32_t rbs = rb;
        asm volatile("" : "+v"(rbs));
        auto read_group = [&](int g, bf16x8 (&dst)[G][PL]) {
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const int mm = g * G + j;
                const uint32_t off = rbs ^ (uint32_t)((((mm >> 2) << 3) | (mm & 3)) << 4);
#pragma unroll
                for (int p = 0; p < PL; ++p)
                    dst[j][p] = lds_read16(xbase + (uint32_t)((s * PL + p) * kPlaneBytes) + off);
            }
        };
        // The lane's four scale bytes, every other byte of the seven from
        // its first: three aligned dwords and a byte shift, read ahead of the
        // first B group.  (Byte reads into 16-bit halves would save a
        // register, but with SRAM ECC on, as on this part, a 16-bit load
        // clears the other half.)
        const uint32_t sb0 = sbase + (uint32_t)(srel + 8 * q);
        uint32_t slo = lds_read4(sb0 & ~3u), smid = lds_read4((sb0 & ~3u) + 4),
                 shi = lds_read4((sb0 & ~3u) + 8);
        // Bit masks rather than selects, so no branch separates a load from
        // its use.
        uint32_t keep[4];
        float sc[4];
        auto scales = [&]() {
            asm volatile("" : "+v"(slo), "+v"(smid), "+v"(shi));
            const uint32_t b03 = __builtin_amdgcn_alignbyte(smid, slo, sb0 & 3u);
            const uint32_t b47 = __builtin_amdgcn_alignbyte(shi, smid, sb0 & 3u);
            const uint32_t sword = __builtin_amdgcn_perm(b47, b03, 0x06040200u);   // bytes 0, 2, 4, 6
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                keep[i] = q * kKC + 2 * i + h < nb ? 0xFFFFFFFFu : 0u;
                const uint32_t sb = (sword >> (8 * i)) & 0xFFu;
                sc[i] = decode_scale(sb ^ ((sb ^ 127u) & ~keep[i]));
            }
        };
        auto widen_bf16 = [&](int mm) {
            const int i = mm >> 2, d = mm & 3;
            const uint32_t w = wdw(wsrc, i, d) & keep[i];
            return __builtin_bit_cast(bf16x8, make_uint4(
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc[i], 0)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc[i], 1)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc[i], 2)),
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc[i], 3))));
        };
        if constexpr (FB) {
            // Weights outside the fp16 range (rare): each fp16 activation v as
            // the exact sum of two bf16 values, hi = v truncated to bf16 and
            // lo = v - hi (at most 3 significant bits), into the two
            // accumulators; one fragment at a time (few registers, no speed).
            lds_wait<0>();
            scales();
#pragma unroll
            for (int mm = 0; mm < 16; ++mm) {
                bf16x8 raw = lds_read16(xbase + (uint32_t)(s * kPlaneBytes) +
                                        (rbs ^ (uint32_t)((((mm >> 2) << 3) | (mm & 3)) << 4)));
                lds_wait<0>();
                asm volatile("" : "+v"(raw));
                const uint4 rw = __builtin_bit_cast(uint4, raw);
                const uint32_t r4[4] = {rw.x, rw.y, rw.z, rw.w};
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v0 = f16_bits_to_f32((uint16_t)r4[e]);
                    const float v1 = f16_bits_to_f32((uint16_t)(r4[e] >> 16));
                    const uint32_t b0 = __builtin_bit_cast(uint32_t, v0) & 0xFFFF0000u;
                    const uint32_t b1 = __builtin_bit_cast(uint32_t, v1) & 0xFFFF0000u;
                    const uint32_t l0 = __builtin_bit_cast(uint32_t, v0 - __builtin_bit_cast(float, b0));
                    const uint32_t l1 = __builtin_bit_cast(uint32_t, v1 - __builtin_bit_cast(float, b1));
                    hw[e] = (b0 >> 16) | b1;
                    lw[e] = (l0 >> 16) | (l1 & 0xFFFF0000u);
                }
                const bf16x8 aw = widen_bf16(mm);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    aw, __builtin_bit_cast(bf16x8, make_uint4(hw[0], hw[1], hw[2], hw[3])), acc, 0, 0, 0);
                acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    aw, __builtin_bit_cast(bf16x8, make_uint4(lw[0], lw[1], lw[2], lw[3])), acc1, 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
            return;
        }
        bf16x8 B[2][G][PL];
        read_group(0, B[0]);
        lds_wait<G * PL>();
        scales();
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            if (g + 1 < NG) read_group(g + 1, B[(g + 1) & 1]);
            if constexpr (F16IN) {
                // fp16 activations x weights widened to fp16 (exact for this
                // wave's scale bytes): one MFMA per fragment
                f16x8 A16[G];
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    const int mm = g * G + j, i = mm >> 2, d = mm & 3;
                    const uint32_t w = wdw(wsrc, i, d) & keep[i];
                    A16[j] = __builtin_bit_cast(f16x8, make_uint4(
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc[i], 0)),
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc[i], 1)),
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc[i], 2)),
                        __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc[i], 3))));
                }
                if (g + 1 < NG) lds_wait<G * PL>();
                else lds_wait<0>();
#pragma unroll
                for (int j = 0; j < G; ++j) asm volatile("" : "+v"(B[g & 1][j][0]));
#pragma unroll
                for (int j = 0; j < G; ++j) {
                    const f16x8 b16 = __builtin_bit_cast(f16x8, B[g & 1][j][0]);
                    if (j & 1)
                        acc1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(A16[j], b16, acc1, 0, 0, 0);
                    else
                        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(A16[j], b16, acc, 0, 0, 0);
                }
            } else {
                bf16x8 A[G];
#pragma unroll
                for (int j = 0; j < G; ++j) A[j] = widen_bf16(g * G + j);
                if (g + 1 < NG) lds_wait<G * PL>();
                else lds_wait<0>();
#pragma unroll
                for (int j = 0; j < G; ++j)
#pragma unroll
                    for (int p = 0; p < PL; ++p) asm volatile("" : "+v"(B[g & 1][j][p]));
#pragma unroll
                for (int j = 0; j < G; ++j) {
#pragma unroll
                    for (int p = 0; p < PL; ++p) {
                        if ((j * PL + p) & 1)
                            acc1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[j], B[g & 1][j][p], acc1, 0, 0, 0);
                        else
                            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[j], B[g & 1][j][p], acc, 0, 0, 0);
                    }
                }
            }
        }
    };

    // One step: issue chunk q+D-1 into the slot chunk q-1 left, multiply
    // chunk q, then wait for this wave's DMA of chunk q+1 and meet the other
    // waves (after which every row of chunk q+1 is in LDS and nobody reads
    // chunk q's buffer any more).
    const int nq = (nb + kKC - 1) / kKC;
    auto step = [&](int q, auto s_const, auto fb_const, auto guard_const) __attribute__((always_inline)) {
        constexpr int s = decltype(s_const)::value;
        constexpr int sn = (s + D - 1) % D;
        if constexpr (decltype(guard_const)::value)
            if (q >= nq) return;                      // uniform: past the last chunk
        if constexpr (decltype(fb_const)::value) {
            // The split body: the same staging and barrier as the other
            // waves, but this chunk's weights loaded here and every load
            // drained before the multiply (no weight ring held in registers).
            xload(sn, q + D - 1);
            __builtin_amdgcn_sched_barrier(0);
            u32x4v w1[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                w1[i] = kSwap ? *(g_u32x4v *)(wbase + ((i & 1) ? wrow1 : wrow0) +
                                              (uint32_t)min(q * kKC + 4 * (i >> 1) + 2 * (c & 1) + h, nb - 1) * 16u)
                              : *(g_u32x4v *)(wrow + (int64_t)min(q * kKC + 2 * i + h, nb - 1) * 16);
            wait_vmcnt<0>();
            multiply(q, s_const, fb_const, w1);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_sched_barrier(0);
            return;
        }
        // The counted wait below relies on a chunk's DMA being issued
        // before its weights: the scheduler may not swap them.
        xload(sn, q + D - 1);
        __builtin_amdgcn_sched_barrier(0);
        wload(sn, q + D - 1);
        __builtin_amdgcn_sched_barrier(0);
        multiply(q, s_const, fb_const, wq[s]);
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<kYounger>();
        // A bare barrier: a fenced one would also wait for every LDS-DMA in
        // flight.  Ordering is explicit here: the counted wait above for the
        // DMA, and lds_wait for this wave's reads.
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
    };

    // The loop runs over nq rounded up to the ring depth (the slot of a step
    // is a constant); steps past nq do nothing, and the chunks the last real
    // steps issued past nq are clamped reads that are never multiplied.  The
    // scale and bias copies are older than chunk 0's DMA, so the first
    // counted wait covers them too.
    const int nq_pad = (nq + D - 1) / D * D;
#pragma unroll
    for (int s = 0; s < D - 1; ++s) {
        xload(s, s);
        __builtin_amdgcn_sched_barrier(0);
        wload(s, s);
        __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<kYounger>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // The scales have landed.  A row that holds a 253 or 254 byte (e2m1 *
    // 2^126 or 2^127 would overflow bf16) has its staged bytes lowered by 2
    // (255 kept, 0 and 1 to 0) and its accumulator multiplied by 4 after the
    // K loop.  Lane half h takes the dwords j = h, h + 2, .. of row c's nb
    // bytes; bit r of rows_lowered is row r of the wave's 32.  Each wave
    // rewrites only its own rows (unclamped), before its own first read.
    uint32_t rows_lowered;
    bool f16ok;                                 // wave-uniform
    {
        const int lo = sshift + (wave * 32 + c) * nb;
        const int a0 = lo & ~3;
        const int ndw = (lo + nb - a0 + 3) >> 2;
        uint32_t big = 0, bad16 = 0;
        const bool row_real = f0 + wave * 32 + c < a.fdim;
        for (int j = h; j < ndw; j += 8) {
            uint32_t w4[4];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                w4[k] = lds_read4(sbase + (uint32_t)(a0 + 4 * min(j + 2 * k, ndw - 1)));
            lds_wait<0>();
#pragma unroll
            for (int k = 0; k < 4; ++k) asm volatile("" : "+v"(w4[k]));
#pragma unroll
            for (int k = 0; k < 4; ++k) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int idx = a0 + 4 * (j + 2 * k) + i;
                    const uint32_t b = (w4[k] >> (8 * i)) & 0xFFu;
                    const bool mine = idx >= lo && idx < lo + nb;
                    big |= (uint32_t)(mine && b - 253u <= 1u);
                    bad16 |= (uint32_t)(mine && row_real && (b < 104u || b > 140u));
                }
            }
        }
        const uint64_t m = __builtin_amdgcn_ballot_w64(big != 0u);
        rows_lowered = (uint32_t)m | (uint32_t)(m >> 32);
        f16ok = __builtin_amdgcn_ballot_w64(bad16 != 0u) == 0ull;
        if (rows_lowered != 0u) {                       // wave-uniform, and rare
            if ((rows_lowered >> c) & 1u) {
                for (int j = h; j < ndw; j += 2) {
                    uint32_t w = lds_read4(sbase + (uint32_t)(a0 + 4 * j));
                    lds_wait<0>();
                    asm volatile("" : "+v"(w));
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int idx = a0 + 4 * j + i;
                        const uint32_t b = (w >> (8 * i)) & 0xFFu;
                        if (idx >= lo && idx < lo + nb && b != 255u)
                            lds_write1(sbase + (uint32_t)idx, b >= 2u ? b - 2u : 0u);
                    }
                }
            }
            lds_wait<0>();
        }
    }
    // The K loop, with the fp16 body or, for a wave whose scales leave the
    // fp16 range, the split one: two copies of the loop rather than a branch
    // per chunk, so neither body's registers are held across the other.
    // Barriers match between the copies (one per step).
    // The common K sizes (12, 8 and 4 chunks, padded to the ring depth: hidden
    // or intermediate 2880, 2048, 768 ...) have their steps written out, the
    // guard only in the last ring-depth group: where a loop's back edge, or a
    // guard's skip path, meets the next step, the compiler's wait bookkeeping
    // no longer knows that a ring slot's last load was used a step ago, and
    // waits for nearly every load in flight before reusing the slot's
    // registers (the ring drains each step).  Other sizes take the loop.
    // (Written out only where it costs no register spill or stack: the
    // 4-wave 2-deep and 8-wave 4-deep shapes with one or two input planes,
    // and in the down GEMM only the fp16 body; the shapes held to fewer
    // registers and the rare split body keep the loop.)
    constexpr bool kWriteOutShape = PL <= 2 && ((W == 4 && D == 2) || (W == 8 && D == 4));
    auto kloop = [&](auto fb_const) {
        constexpr bool kWriteOut = kWriteOutShape && !decltype(fb_const)::value;
        auto written_out = [&](auto nc) {
            constexpr int N = decltype(nc)::value;
            Unroll<0, N>::run([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                step(q, std::integral_constant<int, q % D>{}, fb_const,
                     std::integral_constant<bool, (q >= N - D)>{});
            });
        };
        if (kWriteOut && nq_pad == 12) written_out(std::integral_constant<int, 12>{});
        else if (kWriteOut && nq_pad == 8) written_out(std::integral_constant<int, 8>{});
        else if (kWriteOut && nq_pad == 4) written_out(std::integral_constant<int, 4>{});
        else
            for (int q = 0; q < nq_pad; q += D)
                Unroll<0, D>::run(
                    [&](auto s_const) { step(q + decltype(s_const)::value, s_const, fb_const, std::true_type{}); });
    };
    if constexpr (F16IN) {
        if (f16ok) kloop(std::false_type{});
        else kloop(std::true_type{});
    } else {
        kloop(std::false_type{});
    }
    // Every DMA has landed (the padding chunks' too) and, after the barrier,
    // no wave reads the staging ring any more: it holds the output tile next.
    wait_vmcnt<0>();
    __syncthreads();
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int rl = 8 * (v >> 2) + 4 * h + (v & 3);
        acc[v] = (acc[v] + acc1[v]) * ((rows_lowered >> rl) & 1u ? 4.0f : 1.0f);
    }

    // Epilogue: lane holds entry column c, feature rows 8(v/4) + 4h + (v%4)
    // of the wave's 32; bias from the LDS tile.  The tile is written to LDS,
    // then stored as 16-byte rows per entry.
    float bv[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int rl = wave * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        bv[v] = a.bias_dt < 0 ? 0.0f
                : a.bias_dt == DT_F32 ? reinterpret_cast<const float *>(lds8 + lay.bias)[rl]
                : a.bias_dt == DT_BF16
                    ? bf16_bits_to_f32(reinterpret_cast<const uint16_t *>(lds8 + lay.bias)[rl])
                    : f16_bits_to_f32(reinterpret_cast<const uint16_t *>(lds8 + lay.bias)[rl]);
    }
    if constexpr (GATE_UP) {
        // [kPT entries][kF/2 activations] fp16: the reference rounds the
        // activation to fp16, and the down GEMM reads these bits.
        uint16_t *tile = reinterpret_cast<uint16_t *>(xring);
        constexpr int kCols = kF / 2;
#pragma unroll
        for (int v = 0; v < 16; v += 2) {
            const int rl = wave * 32 + 8 * (v >> 2) + 4 * h + (v & 3);   // even: gate, +1: up
            const float y = apply_activation(a.act_kind, acc[v] + bv[v], acc[v + 1] + bv[v + 1],
                                             a.limit, a.alpha);
            tile[c * kCols + (rl >> 1)] = f32_to_f16_bits(y);
        }
        __syncthreads();
        const int half = a.fdim >> 1;
        // kPT entries x kCols / 8 pieces = kThreads
        {
            const int idx = (int)threadIdx.x;
            const int t = idx / (kCols / 8), piece = idx % (kCols / 8);
            const int col0 = (f0 >> 1) + piece * 8;
            if (t < ntok && col0 + 8 <= half) {
                const uint4 v = *reinterpret_cast<const uint4 *>(tile + t * kCols + piece * 8);
                *reinterpret_cast<uint4 *>(a.act_out + (int64_t)ent[t] * half + col0) = v;
            }
        }
    } else {
        // [kPT entries][kF rows] fp32
        float *tile = reinterpret_cast<float *>(xring);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int rl = wave * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
            tile[c * kF + rl] = acc[v] + bv[v];
        }
        __syncthreads();
        const __amdgpu_buffer_rsrc_t yres =
            __builtin_amdgcn_make_buffer_rsrc(a.y_out, (short)0, (int)a.y_bytes, 0x00020000);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // kPT entries x kF / 4 pieces = 4 kThreads
            const int idx = (int)threadIdx.x + k * kThreads;
            const int t = idx / (8 * W), piece = idx % (8 * W);
            const int row0 = f0 + piece * 4;
            if (t < ntok && row0 + 4 <= a.fdim) {
                const float4 v = *reinterpret_cast<const float4 *>(tile + t * kF + piece * 4);
                const int64_t o = (int64_t)ent[t] * a.fdim + row0;
                if constexpr (COMB)   // write-through (sc1): read back by another workgroup
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4v, v), yres,
                                                           (int)(o * 4), 0, kCachePolicySc1);
                else
                    *reinterpret_cast<float4 *>(a.y_out + o) = v;
            }
        }
        if constexpr (COMB) {
            // Each thread waits for its own stores, then one relaxed count per
            // entry of the tile; the count that reaches K hands the token's
            // tile to this workgroup (and clears the counter for the next
            // launch: all K entries have counted).
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            int *todo = reinterpret_cast<int *>(xring + kPT * kF * 4);   // [kPT], then the count
            if (threadIdx.x == 0) todo[kPT] = 0;
            __syncthreads();
            const int K = a.comb_topk;
            if ((int)threadIdx.x < ntok) {
                const int tok = ent[threadIdx.x] / K;
                uint32_t *cnt = a.arrive + (int64_t)tok * nft + fidx;
                const uint32_t before =
                    __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (before == (uint32_t)(K - 1)) {
                    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    todo[atomicAdd(&todo[kPT], 1)] = tok;
                }
            }
            __syncthreads();
            const int ndo = todo[kPT];
            // out[tok, row] = sum_k w[tok, k] * y[tok*K + k, row], product and
            // sum rounded separately in router order (expert_accumulate), as
            // prefill_combine_kernel does; y read coherently (sc1).
            for (int idx = (int)threadIdx.x; idx < ndo * (kF / 4); idx += kThreads) {
                const int tok = todo[idx / (kF / 4)], row0 = f0 + (idx % (kF / 4)) * 4;
                if (row0 + 4 > a.fdim) continue;
                u32x4v yv[kMaxTopK];
#pragma unroll
                for (int k = 0; k < kMaxTopK; ++k)
                    if (k < K)
                        yv[k] = __builtin_amdgcn_raw_buffer_load_b128(
                            yres, (int)((((int64_t)tok * K + k) * a.fdim + row0) * 4), 0,
                            kCachePolicySc1);
                float d[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int k = 0; k < kMaxTopK; ++k) {
                    if (k < K) {
                        const float w = a.comb_w[(int64_t)tok * K + k];
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            d[i] = add_scaled_rn(d[i], __uint_as_float(yv[k][i]), w);
                    }
                }
                const int64_t o = (int64_t)tok * a.fdim + row0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float r = a.comb_residual ? a.comb_out[o + i] + d[i] : d[i];
                    a.comb_out[o + i] = r;
                    if (a.comb_out_bf16) a.comb_out_bf16[o + i] = f32_to_bf16_bits(r);
                }
            }
        }
    }
}

// Splits n fp16 or fp32 values into PL bf16 planes whose sum is exact.
template <int IN_DT, int PL>
__global__ __launch_bounds__(256) void prefill_split_kernel(const void *__restrict__ in,
                                                            int64_t n,
                                                            uint16_t *__restrict__ out)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        float r = IN_DT == DT_F32 ? static_cast<const float *>(in)[i]
                                  : f16_bits_to_f32(static_cast<const uint16_t *>(in)[i]);
#pragma unroll
        for (int p = 0; p < PL; ++p) {
            const uint16_t b = f32_to_bf16_bits(r);
            out[p * n + i] = b;
            r -= bf16_bits_to_f32(b);
        }
    }
}

// ---------------------------------------------------------------------------
// 5. Combine: out[t] = sum_k w[t,k] * y[t*K+k], product and sum rounded
// separately in router order (expert_accumulate), starting from zero; with
// `residual` the finished sum is added to out (the residual add after the
// block, TransformerLayer.swift:232-238).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(256) void prefill_combine_kernel(const float *__restrict__ y,
                                                              const float *__restrict__ w,
                                                              int T, int K, int H,
                                                              float *__restrict__ out,
                                                              uint16_t *__restrict__ out_bf16,
                                                              int residual)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * H) return;
    const int t = (int)(i / H), col = (int)(i - (int64_t)t * H);
    float dst = 0.0f;
    for (int k = 0; k < K; ++k)
        dst = add_scaled_rn(dst, y[((int64_t)t * K + k) * H + col], w[(int64_t)t * K + k]);
    if (residual) dst = out[i] + dst;
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

// The narrowest built workgroup: 4 waves of 32 feature rows.
constexpr int kMinFeatureRows = 128;
int64_t prefill_arrive_count(int T, int fdim) { return (int64_t)T * pdiv_up(fdim, kMinFeatureRows); }

bool prefill_routes_in_group(int T, int K) { return T <= kRouteGroupTokens && K <= kMaxTopK; }

bool prefill_self_groups(int T, int K, int E)
{
    return T >= 1 && T <= kSelfGroupTokens && K >= 1 && K <= kMaxTopK && E >= K &&
           E <= kPrefillMaxExperts;
}

hipError_t launch_prefill_group(const Launch &L, const float *logits, int T, int K, float *weights,
                                int32_t *ids, int E, int32_t *offsets, int32_t *order,
                                int32_t *tiles, int32_t *ntiles, int max_tiles)
{
    if (E > kPrefillMaxExperts || T <= 0 || K <= 0 || K > kMaxTopK) return hipErrorInvalidValue;
    if (logits && !prefill_routes_in_group(T, K)) return hipErrorInvalidValue;
    GW_LAUNCH(prefill_group_kernel, dim3(1), dim3(kGroupThreads), 0, L, logits, T, K, weights,
              ids, E, offsets, order, tiles, ntiles, max_tiles);
    return hipGetLastError();
}

int prefill_planes(int in_dt) { return in_dt == DT_BF16 ? 1 : in_dt == DT_F16 ? 2 : 3; }

int prefill_gemm_lds_bytes(int planes, int kdim, int waves, int depth)
{
    return prefill_lds(planes, depth, kdim / 32, waves).total;
}

// Workgroup shape of a grouped GEMM launch: W waves (256 or 384 features)
// and ring depth D.  The cost of a shape is the feature rows the busiest CU
// computes, ceil(units / CUs) x features per workgroup, times 8 — or times 7
// for the 8-wave, 2-deep form when two of its workgroups share a CU (LDS
// permitting, and more units than CUs): co-resident workgroups overlap each
// other's latencies (Qwen3 batch-8 down GEMM 25.9 -> 19 us, 512-token gate_up
// 426 -> 403 us), while one workgroup per CU runs better with a 4-deep ring
// (a 12-wave gate_up that fits the CUs in one round: 35 against 40 us).  The
// 4-wave, 2-deep form (one plane: 45 KB of LDS at K = 2880, three workgroups
// per CU) is priced at 6.6 where each CU takes at least six of its units and
// K spans at least eight chunks: three independent workgroups overlap one
// another's weight waits better still (512 tokens: gate_up 382 -> 365 us,
// down 208 -> 192 us; Qwen3 batch 32 gate_up 51.9 -> 49.8 us), but with
// fewer rounds (Qwen3 batch 8 gate_up: 34.3 against 33.4 us for 12x4) or
// short rows (Qwen3 down, K = 768: 36.3 against 34.8 us at batch 32) it
// loses.  Ties keep the earlier shape in the list.  `tiles_hint` bounds the
// work list.
struct PrefillShape { int waves, depth; };

static PrefillShape prefill_shape(int fdim, int kdim, int planes, int tiles_hint, int cus,
                                  bool twelve, bool four)
{
    const int c = cus > 0 ? cus : 1;
    const PrefillShape cand[4] = {{8, planes == 3 ? 2 : 4}, {12, planes == 3 ? 2 : 4}, {8, 2},
                                  {4, 2}};
    PrefillShape best = cand[0];
    int64_t best_cost = -1;
    for (int i = 0; i < 4; ++i) {
        const PrefillShape sh = cand[i];
        if (planes == 3 && i == 2) continue;          // 8x2 is cand[0] for three planes
        if (sh.waves == 12 && !twelve) continue;
        if (sh.waves == 4 && !four) continue;
        const int lds = prefill_gemm_lds_bytes(planes, kdim, sh.waves, sh.depth);
        if (lds > kPrefillLdsMax) continue;
        const int64_t units = (int64_t)tiles_hint * pdiv_up(fdim, 32 * sh.waves);
        const int64_t per_cu = (units + c - 1) / c;
        const bool shared = sh.waves == 8 && sh.depth == 2 && 2 * lds <= kPrefillLdsMax && per_cu >= 2;
        if (sh.waves == 4 && (3 * lds > kPrefillLdsMax || per_cu < 6 || kdim < 2048)) continue;
        // In tenths: 8, 7 for the shared 8x2 form, 6.6 for the 4-wave form.
        const int64_t cost = per_cu * 32 * sh.waves * (sh.waves == 4 ? 66 : shared ? 70 : 80);
        if (best_cost < 0 || cost < best_cost) {
            best = sh;
            best_cost = cost;
        }
    }
    return best;
}

bool prefill_down_four_wave(int fdim, int kdim, int tiles_hint, int max_tiles, int cus)
{
    const int hint = tiles_hint > 0 && tiles_hint < max_tiles ? tiles_hint : max_tiles;
    return prefill_shape(fdim, kdim, 1, hint, cus, false, true).waves == 4;
}

hipError_t launch_prefill_split(const Launch &L, const void *in, int in_dt, int64_t n,
                                uint16_t *out)
{
    if (n <= 0) return hipErrorInvalidValue;
    const dim3 grid((unsigned)std::min<int64_t>(pdiv_up(n, 256), 4096));
    if (in_dt == DT_F16)
        GW_LAUNCH((prefill_split_kernel<DT_F16, 2>), grid, dim3(256), 0, L, in, n, out);
    else if (in_dt == DT_F32)
        GW_LAUNCH((prefill_split_kernel<DT_F32, 3>), grid, dim3(256), 0, L, in, n, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_prefill_gemm(const Launch &L, bool gate_up, int planes, const PrefillGemm &g,
                               int max_tiles, int tiles_hint)
{
    // The staged rows are read 16 bytes at a time and the scale word 4 bytes
    // back from a row's end: K must be a multiple of 32 and at least 128.
    if (g.kdim % 32 != 0 || g.kdim < 128 || g.fdim <= 0 || max_tiles <= 0)
        return hipErrorInvalidValue;
    // gate_up: 1-3 bf16 planes of x; down: one plane of fp16 activations
    if (planes < 1 || planes > 3 || (!gate_up && planes != 1)) return hipErrorInvalidValue;
    // The output tile is stored 8 activations or 4 outputs at a time.
    if ((gate_up && g.fdim % 16 != 0) || (!gate_up && g.fdim % 4 != 0)) return hipErrorInvalidValue;
    GemmArgs a;
    a.tiles = g.tiles;
    a.ntiles = g.ntiles;
    a.offsets = g.offsets;
    a.order = g.order;
    a.in = g.in;
    a.in_plane = g.in_plane;
    if (g.in_plane <= 0 || (int64_t)planes * g.in_plane * 2 >= ((int64_t)1 << 31))
        return hipErrorInvalidValue;     // staged through 32-bit buffer offsets
    a.in_bytes = (uint32_t)(planes * g.in_plane * 2);
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
    a.sg_tokens = g.sg_tokens;
    a.sg_topk = g.sg_topk;
    a.sg_experts = g.sg_experts;
    a.sg_logits = g.sg_logits;
    a.sg_ids = g.sg_ids;
    a.sg_ids_out = g.sg_ids_out;
    a.sg_w_out = g.sg_w_out;
    a.arrive = nullptr;
    a.y_bytes = 0;
    a.comb_w = g.comb_w;
    a.comb_out = g.comb_out;
    a.comb_out_bf16 = g.comb_out_bf16;
    a.comb_topk = g.comb_topk;
    a.comb_residual = g.comb_residual;
    if (!gate_up) {
        // y is addressed through a 32-bit buffer range.
        if (g.y_bytes <= 0 || g.y_bytes >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
        a.y_bytes = (uint32_t)g.y_bytes;
        if (g.arrive) {
            if (!g.comb_w || !g.comb_out || g.comb_topk < 1 || g.comb_topk > kMaxTopK)
                return hipErrorInvalidValue;
            a.arrive = g.arrive;
        }
    }
    if (g.sg_tokens > 0) {
        // The workgroup routes or reads T*K <= 256 entries, one per thread,
        // and stages T*E <= 8192 logits in its staging ring.
        if (!prefill_self_groups(g.sg_tokens, g.sg_topk, g.sg_experts)) return hipErrorInvalidValue;
        if (gate_up ? (!g.sg_logits || !g.sg_ids_out || !g.sg_w_out) : !g.sg_ids)
            return hipErrorInvalidValue;
        if (max_tiles < std::min(g.sg_experts, g.sg_tokens * g.sg_topk)) return hipErrorInvalidValue;
    }
    // The down GEMM is built with 8 waves only: its two K-loop bodies (fp16
    // and split bf16) do not both fit the registers of 12 waves per CU.
    const bool twelve = gate_up;
    const bool four = planes == 1;                   // bf16 x (gate_up) or down
    PrefillShape sh = prefill_shape(
        g.fdim, g.kdim, planes, tiles_hint > 0 && tiles_hint < max_tiles ? tiles_hint : max_tiles,
        L.cus, twelve, four);
    if (g.force_waves == 4 && four) {
        const PrefillShape f = {4, 2};
        if (prefill_gemm_lds_bytes(planes, g.kdim, 4, 2) <= kPrefillLdsMax) sh = f;
    } else if (g.force_waves == 8 || (g.force_waves == 12 && twelve)) {
        // Built shapes: gate_up 8x4, 12x4 and 8x2 for one or two planes, 8x2
        // and 12x2 for three; down 8x4 and 8x2.
        const int d = planes == 3 ? 2 : g.force_waves == 12 ? 4 : g.force_depth == 2 ? 2 : 4;
        const PrefillShape f = {g.force_waves, d};
        if (prefill_gemm_lds_bytes(planes, g.kdim, f.waves, f.depth) <= kPrefillLdsMax) sh = f;
    }
    // One workgroup per (feature tile, tile) unit, rounded up to whole XCD
    // rounds; the kernel maps ids to units and retires the spare ones.
    // The fused combine counts each token's arrivals per feature tile of this
    // shape: the counters must cover comb_tokens x its tiles.
    if (!gate_up && g.arrive &&
        (g.comb_tokens < 1 ||
         (int64_t)g.comb_tokens * pdiv_up(g.fdim, 32 * sh.waves) > g.arrive_count))
        return hipErrorInvalidValue;
    const dim3 grid((pdiv_up(g.fdim, 32 * sh.waves) * max_tiles + 7) / 8 * 8);
    const int lds_bytes = prefill_gemm_lds_bytes(planes, g.kdim, sh.waves, sh.depth);
    if (lds_bytes > kPrefillLdsMax) return hipErrorInvalidValue;   // K too wide for the staging
    const size_t lds = (size_t)lds_bytes;
    hipError_t err = hipSuccess;
    auto go = [&](auto pl, auto gu) {
        constexpr int PL = decltype(pl)::value;
        constexpr bool GU = decltype(gu)::value;
        auto with_shape = [&](auto wc, auto dc) {
            constexpr int W = decltype(wc)::value;
            constexpr int D = decltype(dc)::value;
            auto with_comb = [&](auto cc) {
                constexpr bool C = decltype(cc)::value;
                // More than 64 KiB of dynamic LDS must be allowed explicitly,
                // once per instantiation.
                static bool lds_ok = false;
                if (!lds_ok) {
                    err = hipFuncSetAttribute(
                        reinterpret_cast<const void *>(&prefill_gemm_kernel<PL, GU, W, D, C>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kPrefillLdsMax);
                    if (err != hipSuccess) return;
                    lds_ok = true;
                }
                GW_LAUNCH((prefill_gemm_kernel<PL, GU, W, D, C>), grid, dim3(64 * W), lds, L, a);
            };
            // The fused combine is compiled into the down kernel only.
            if constexpr (!GU) {
                if (a.arrive) with_comb(std::true_type{});
                else with_comb(std::false_type{});
            } else {
                with_comb(std::false_type{});
            }
        };
        using I2 = std::integral_constant<int, 2>;
        using I4 = std::integral_constant<int, 4>;
        using I8 = std::integral_constant<int, 8>;
        using I12 = std::integral_constant<int, 12>;
        using IW4 = std::integral_constant<int, 4>;
        if constexpr (PL == 3) {
            if (sh.waves == 12) with_shape(I12{}, I2{});
            else with_shape(I8{}, I2{});
        } else {
            if constexpr (GU) {
                if (sh.waves == 12) {
                    with_shape(I12{}, I4{});
                    return;
                }
                if constexpr (PL == 1) {
                    if (sh.waves == 4) {
                        with_shape(IW4{}, I2{});
                        return;
                    }
                }
            } else {
                if (sh.waves == 4) {
                    with_shape(IW4{}, I2{});
                    return;
                }
            }
            if (sh.depth == 2) with_shape(I8{}, I2{});
            else with_shape(I8{}, I4{});
        }
    };
    using P1 = std::integral_constant<int, 1>;
    using P2 = std::integral_constant<int, 2>;
    using P3 = std::integral_constant<int, 3>;
    using Y = std::true_type;
    using N = std::false_type;
    if (gate_up) {
        if (planes == 1) go(P1{}, Y{});
        else if (planes == 2) go(P2{}, Y{});
        else go(P3{}, Y{});
    } else {
        go(P1{}, N{});
    }
    if (err != hipSuccess) return err;
    return hipGetLastError();
}

hipError_t launch_prefill_combine(const Launch &L, const float *y, const float *w, int T, int K,
                                  int H, float *out, uint16_t *out_bf16, int residual)
{
    GW_LAUNCH(prefill_combine_kernel, dim3(pdiv_up((int64_t)T * H, 256)), dim3(256), 0, L, y, w,
              T, K, H, out, out_bf16, residual);
    return hipGetLastError();
}

}  // namespace gw
