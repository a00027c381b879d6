// gw_decode.hip — the one-token MoE layer as ONE kernel (decode, batch 1).
//
// TransformerLayer.forward's MoE block for one token
// (Sources/Godwit/Runtime/TransformerLayer.swift:140-238): routing
// (Router.select, Runtime/Router.swift:78-98), the gate_up GEMV with bias and
// activation (Metal/MoE/expert.metal:311-368 then :82-102 or :380-393), the
// down GEMV with bias and the weighted combine (expert.metal:107-116), in one
// launch of one 512-thread workgroup per compute unit.
//
// At batch 1 the layer is two dependent streams of weights: k experts' gate_up
// rows (4 x 8.8 MB for GPT-OSS), then their down rows (4 x 4.4 MB), which
// need every activation of their expert.  The down rows' addresses are known
// as soon as the routing is.
//
// * routing: from the given logits, or, given the router weights instead
//   (bf16_gemv_bias, Metal/MoE/router.metal:18-34), from logits the grid
//   computes first: each workgroup dots one slice of one router row, the
//   partials go through their own exchange slot and every workgroup adds a
//   logit's partials in slice order (the standalone router's order too).
//
// * gate_up: waves 0-3 (one per SIMD) stream the workgroup's share of gate_up
//   rows through a ring of register stages and widen and dot each stage as it
//   lands; the share is a whole number of 4-feature quads, so the workgroup's
//   fp16 activations fill whole 8-byte exchange words.
// * down: every wave owns a fixed set of units (16 down rows x 4 MXFP4 blocks)
//   and copies exactly those rows' bytes into LDS by buffer LDS-DMA, in a
//   layout where the matrix-core operand reads are bank-conflict free.  Waves
//   4-7 issue theirs once the gate_up waves have queued their last stage (a
//   SIMD issues its older wave first, so the gate_up rows stay ahead); waves
//   0-3 once their activations are out.
// * exchange: a workgroup publishes its activations as 8-byte words of four
//   fp16 values (device-coherent stores) into the launch's slot; every word of
//   the slot was reset to an all-ones sentinel by the previous launch, so a
//   word differing from it is this launch's, whole (an aligned 8-byte store is
//   seen whole or not at all).  Each wave reads the activation blocks its own
//   units need straight into matrix-core operand registers, rereading words
//   still holding the sentinel past the L2 (a bounded spin: a wait that gives
//   up counts an error, read by gw_expert_runner_sync_errors, so no workgroup
//   ever waits unboundedly).  The grid must be co-resident (one workgroup per
//   CU; the host checks occupancy).
// * down products: v_mfma_f32_16x16x32_f16, weights widened to fp16 with the
//   block scale folded in (exact for scale bytes 104..140), the activation
//   columns one per selected expert; blocks with other scale bytes are dotted
//   on the VALU with the fp32 scale product instead.  Per-wave partial sums
//   meet in LDS and are summed in a fixed order, then biased and combined in
//   router order (expert_accumulate).
//
// The gate_up rows are computed exactly as in the two-kernel form
// (gate_up_kernel): the same widening, block dots, scale products, lane order
// and reductions, so the activations are the same bytes.  The down sums are
// accumulated in another order than the reference's sequential loop (products
// are exact, only the fp32 rounding of the sums differs); both hold the
// reference's tolerance.
#include <hip/hip_ext.h>

#include <type_traits>

#include "gw_device.h"
#include "gw_launch.h"
#include "gw_route.h"

namespace gw {

namespace {

constexpr int kDT = 512;          // threads per workgroup
constexpr int kDW = kDT / 64;     // waves per workgroup
// Waves 0..kGuWaves-1 (one per SIMD) stream and compute the gate_up rows.
constexpr int kGuWaves = 4;
constexpr int kChunk = 1024;      // bytes one wave-wide 16-byte LDS-DMA moves
constexpr int kRsrcWord3 = 0x00020000;   // raw (untyped) buffer access
constexpr int kNt = 2;                   // buffer cache policy: non-temporal (streamed once)
constexpr int kSc1 = 16;                 // buffer cache policy: device-coherent (past the L2)
constexpr uint32_t kOutOfRange = 0x80000000u;   // buffer offset past any layer (reads zero)
constexpr uint64_t kEmpty = ~0ull;       // an exchange word not written this launch

// Phase timeline (built only with -DGW_DECODE_TRACE, the library
// libgodwit_hip_trace.so of `build.py --trace`): lane 0 of every wave stores
// wall_clock64() (100 MHz) at 11 phase boundaries of the layer, one record
// per (launch % 4, workgroup, wave); gw_debug_decode_trace copies them out.
// 0 start, 1 routed, 2 gate_up stream queued (gate_up waves) / the gate_up
// wave's down pieces flagged (DMA waves), 3 exchange phase entered, 4 own
// pieces flagged and the workgroup's publication seen, 5 exchange reads
// issued, 6 down weights widened, 7 exchange complete, 8 products issued,
// 9 combine start, 10 end; 11 the exchange words' first check, 12 partial
// sums written.
#ifdef GW_DECODE_TRACE
constexpr int kTraceStamps = 16;
__device__ uint64_t g_decode_trace[4 * kDecodeMaxGrid * 8 * kTraceStamps];
// The wave's stamp row is addressed once (a scalar load of the array's
// address before every stamp would delay the code after it).
#define GW_TRACE_ROW()                                                                             \
    uint64_t *const gw_trace_row =                                                                 \
        g_decode_trace + (((epoch1 & 3u) * kDecodeMaxGrid + blockIdx.x) * 8 + (threadIdx.x >> 6)) * kTraceStamps
#define GW_TRACE(P)                                                                                \
    do {                                                                                           \
        if ((threadIdx.x & 63) == 0) gw_trace_row[(P)] = wall_clock64();                           \
    } while (0)
#else
#define GW_TRACE_ROW() \
    do {               \
    } while (0)
#define GW_TRACE(P) \
    do {            \
    } while (0)
#endif
// Ticks (10 ns) between publishing the router partial and the first read of
// the grid's partials (a read before the last publisher costs a round trip;
// measured on MI355X at the GPT-OSS-20B shape: 0: 22.8, 30: 21.1-21.4, 60:
// 21.1, 100: 21.3-21.5 us per layer with the layer's router).
constexpr int kRouterPollDelay = 60;
// Exchange slots: launches alternate between slots 0 and 1; slot 2 is never
// written (a host flag points the readers at it to exercise the give-up path).
constexpr int kXSlotWords = kDecodeXchgSlotBytes / 8;
static_assert(3 * kDecodeXchgSlotBytes <= kDecodeXchgBytes, "exchange buffer");

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void l_void;

template <int TPR_, int M_> struct DShape {
    static constexpr int TPR = TPR_;   // lanes per row
    static constexpr int M = M_;       // 16-byte blocks per lane (lane l: l, l+TPR, ...)
};

}  // namespace

// Byte layout of the kernel's LDS (host and device compute the same).
// pieces: 1 KiB pieces of the down rows (one per unit); scale_pieces: 1 KiB
// pieces of their scale bytes; parts: fp32 partial sums of the down rows
// (step groups x rows); rows_per_wg: gate_up rows a workgroup can hold (its
// fp16 activations take that many bytes at most); bx_pieces: 1 KiB pieces of
// the DMA waves' exchange words, read for them by the gate_up waves.
__host__ __device__ inline DecodeLds decode_lds(int hidden, int pieces, int scale_pieces, int parts,
                                               int rows_per_wg, int bx_pieces)
{
    DecodeLds l;
    const int hb = hidden / 32;
    l.route = 0;                                   // int32 ids[8], float w[8], counters
    l.xs = 256;                                    // x, 20 dwords per block
    l.actl = l.xs + hb * 80;                       // this workgroup's fp16 activations
    l.dma = (l.actl + rows_per_wg + 255) & ~255;   // down pieces (routing keys before them)
    l.scl = l.dma + (pieces > 1 ? pieces : 1) * kChunk;
    l.part = l.scl + scale_pieces * kChunk;
    l.bx = (l.part + parts * 4 + 15) & ~15;
    l.total = l.bx + bx_pieces * kChunk;
    return l;
}

namespace {

// The bias element of a row is read as the aligned dword containing it (one
// load whatever the dtype).
__device__ __forceinline__ float bias_of(uint32_t bw, int bshift, int bias_dt)
{
    if (bias_dt < 0) return 0.0f;
    if (bias_dt == DT_F32) return __uint_as_float(bw);
    const uint16_t b = (uint16_t)(bw >> bshift);
    return bias_dt == DT_BF16 ? bf16_bits_to_f32(b) : f16_bits_to_f32(b);
}

__device__ __forceinline__ void widen_v(const u32x4 &w, WBlock<DT_BF16> &o)
{ uint4 v; v.x = w.x; v.y = w.y; v.z = w.z; v.w = w.w; widen<DT_BF16>(v, o); }
__device__ __forceinline__ void widen_v(const u32x4 &w, WBlock<DT_F16> &o)
{ uint4 v; v.x = w.x; v.y = w.y; v.z = w.z; v.w = w.w; widen<DT_F16>(v, o); }

// The value of the up row of a gate/up pair, whose segment follows the gate
// row's segment in the wave: the next 16-lane row (permlane16 swap) or the
// other half of this 16-lane row (row rotate by 8), without going through LDS.
template <int TPR> __device__ __forceinline__ float next_segment(float v)
{
    if constexpr (TPR == 16) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v),
                                                        false, false);
        return __uint_as_float(p[1]);
    } else {
        static_assert(TPR == 8, "row segments are 8 or 16 lanes");
        return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                          0x128, 0xF, 0xF, false));
    }
}

// An LDS word read the compiler cannot see: after a wave has issued an
// LDS-DMA, the compiler makes every LDS access it can see wait for all of
// the wave's loads in flight.
__device__ __forceinline__ uint32_t lds_peek(const void *p)
{
    uint32_t v;
    const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
    return v;
}

// Four fp16 weights of a block (one packed dword) widened with the block's
// scale folded in: exact when the e8m0 byte lies in [104, 140].
__device__ __forceinline__ f16x8 widen_scaled(uint32_t w, float sc)
{
    return __builtin_bit_cast(
        f16x8, make_uint4(__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 0)),
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 1)),
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 2)),
                          __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp4(w, sc, 3))));
}

// 1 when either 8-byte word of a 16-byte read still holds the sentinel.
__device__ __forceinline__ uint32_t pair_empty(const u32x4 &v)
{
    return (uint32_t)((v.x & v.y) == ~0u) | (uint32_t)((v.z & v.w) == ~0u);
}

}  // namespace

// XK: x dtype (bf16 or fp16).  GS: gate_up row shape (hidden wide).  NSG:
// gate_up stages (of kGuWaves * 64 / TPR rows) a workgroup's share fills, GD
// of them in flight per wave.
// TD: 16-row tiles of down rows (the workgroup's rows of every selected
// expert, expert-major).  WT: tile groups the waves are split into (each
// wave takes TD / WT tiles); the kDW / WT step groups take SPW steps of four
// blocks each.  NSP: 1 KiB pieces of down scale bytes each DMA wave copies.  PD: ticks of the 100 MHz real-time counter between the
// workgroup publishing its activations and its first read of the exchange.
// PX: a gate_up wave reads its DMA partner's exchange words into LDS (else
// every wave reads its own).
template <int XK, class GS, int NSG, int GD, int TD, int WT, int SPW, int NSP, int PD, bool PX>
__global__ __launch_bounds__(kDT) void decode_layer_kernel(DecodeArgs a)
{
    constexpr int TPG = GS::TPR, MG = GS::M, SEGG = 64 / TPG, RGW = kGuWaves * SEGG;
    constexpr int BD = XL<XK>::kBlockDw;
    constexpr int TPW = TD / WT, WS = kDW / WT, UPW = TPW * SPW;
    static_assert(TD % WT == 0 && kDW % WT == 0, "wave split");
    extern __shared__ __align__(16) uint32_t lds[];
    uint8_t *lds8 = reinterpret_cast<uint8_t *>(lds);

    const int H = a.hidden, F = a.inter, K = a.top_k;
    const int hb = H >> 5, fb = F >> 5;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x;
    const int bsz = a.bias_dt == DT_F32 ? 4 : 2;
    int q0, q1;                          // gate_up: (expert, feature) quads [q0, q1)
    slice_of((K * F) >> 2, q0, q1);
    const int p0 = 4 * q0, p1 = 4 * q1;  // ... pairs [p0, p1)
    int r0, r1;                          // down: output rows [r0, r1) of every expert
    slice_of(H, r0, r1);
    const int nr = r1 - r0;
    const int nrows_dn = K * nr;         // down rows, expert-major: row k * nr + q
    const DecodeLds L = decode_lds(H, kDW * UPW, (kDW - kGuWaves) * NSP, WS * 16 * TD, RGW * NSG,
                                   PX ? (kDW - kGuWaves) * SPW * 4 : 0);
    int32_t *eid = reinterpret_cast<int32_t *>(lds8 + L.route);
    float *ew = reinterpret_cast<float *>(lds8 + L.route + 32);
    unsigned *gu_done = reinterpret_cast<unsigned *>(lds8 + L.route + 64);   // gate_up waves done
    unsigned *ready = reinterpret_cast<unsigned *>(lds8 + L.route + 112);    // [4] gate_up waves' units landed
    unsigned *t_pub = reinterpret_cast<unsigned *>(lds8 + L.route + 128);    // publish time (0: not yet)
    unsigned *scl_in = reinterpret_cast<unsigned *>(lds8 + L.route + 132);   // DMA waves' scale pieces landed
    unsigned *bx_in = reinterpret_cast<unsigned *>(lds8 + L.route + 144);    // [4] DMA waves' exchange words landed
    uint32_t *xs = reinterpret_cast<uint32_t *>(lds8 + L.xs);
    uint16_t *actl = reinterpret_cast<uint16_t *>(lds8 + L.actl);
    float *part = reinterpret_cast<float *>(lds8 + L.part);
    // Launches this workgroup has completed (written back at the end).
    const unsigned epoch1 = a.sync.epochs[b] + 1;
    GW_TRACE_ROW();
    GW_TRACE(0);

    // ---- 1. route while waves 1.. stage x -----------------------------------
    // Up to 128 experts: wave 0 writes the logits' order keys to LDS (0 for
    // NaN and for no expert), then every thread counts, for expert t / 4,
    // the keys greater than its own in quarter t % 4 of them.  When no logit
    // is NaN and no two experts share a selected rank's key, expert e's count
    // is its position in Router.select's result (the selection sort picks
    // the K largest in descending order whatever its permutation holds);
    // otherwise wave 0 runs the exact selection.  The softmax over the
    // selected logits is computed by a down-stream wave, off the gate_up
    // path.  More experts: wave 0 routes alone (select_one).
    const bool by_rank = a.experts <= 128;
    uint32_t *rkey = reinterpret_cast<uint32_t *>(lds8 + L.dma);   // keys [128]; the down
    float *rlogit = reinterpret_cast<float *>(lds8 + L.dma + 512);  // pieces come later
    // the experts placed at each rank, one byte a rank (at most 128 claims,
    // no carry), and a NaN flag: two LDS reads check the routing
    unsigned long long *rcnt = reinterpret_cast<unsigned long long *>(lds8 + L.route + 80);
    unsigned *rnan = reinterpret_cast<unsigned *>(lds8 + L.route + 88);
    bool route_fail = false;   // the router partials' exchange gave up
    // Router partial slots: every launch clears its word of the next launch's
    // slot, whether or not it computes the logits itself (that launch's slot
    // is then empty however the launches before it were made).
    uint64_t *pslots = a.xchg + 3 * (size_t)kXSlotWords;
    if (threadIdx.x == 0)
        __hip_atomic_store(pslots + (size_t)((epoch1 + 1) & 1u) * kDecodeMaxGrid + b, kEmpty,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wave == 0) {
        if (by_rank) {
            bool nan = false;
            float lv[2];
            if (a.rw) {
                // ---- 0. the router logits in the kernel: this workgroup's
                // partial out (a 64-bit word, never all ones), the next
                // launch's word cleared, every partial of the grid read back
                // (rereads past the L2 while a word is still empty), each
                // logit its partials in slice order plus the bias.
                const int S = a.rslices, Lw = H / S;
                const float p = router_partial_dt<XK>(a.rw, a.rw_dt, a.x, b / S, b % S, Lw, H, lane);
                float bias_e[2];
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int i = min(lane + 64 * r, a.experts - 1);
                    bias_e[r] = a.rb ? load_as_f32(a.rb, a.rb_dt, i) : 0.0f;
                }
                if (lane == 0)
                    __hip_atomic_store(pslots + (size_t)(epoch1 & 1u) * kDecodeMaxGrid + b,
                                       (uint64_t)__float_as_uint(p), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
                if constexpr (kRouterPollDelay > 0) {
                    const uint32_t t0 = (uint32_t)wall_clock64();
                    while ((uint32_t)wall_clock64() - t0 < (uint32_t)kRouterPollDelay)
                        __builtin_amdgcn_s_sleep(2);
                }
                const int pslot = a.poll_fault ? 2 : (int)(epoch1 & 1u);
                const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
                    pslots + (size_t)pslot * kDecodeMaxGrid, (short)0, (int)gridDim.x * 8, kRsrcWord3);
                constexpr int PW = kDecodeMaxGrid / 64;
                uint64_t pv[PW];
#pragma unroll
                for (int k = 0; k < PW; ++k)
                    pv[k] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                             pr, (uint32_t)(lane + 64 * k) * 8u, 0, 0));
                // words past the grid read zero (out of range), never empty
                unsigned spins = 0;
                uint32_t pend = 0;
#pragma unroll
                for (int k = 0; k < PW; ++k) pend |= (pv[k] == kEmpty ? 1u : 0u) << k;
                while (__ballot(pend != 0u) != 0ull) {
                    if (++spins > a.spin_limit) {
                        route_fail = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
#pragma unroll
                    for (int k = 0; k < PW; ++k)
                        if ((pend >> k) & 1u)
                            pv[k] = __builtin_bit_cast(uint64_t, __builtin_amdgcn_raw_buffer_load_b64(
                                                                     pr, (uint32_t)(lane + 64 * k) * 8u, 0, kSc1));
#pragma unroll
                    for (int k = 0; k < PW; ++k)
                        if (pv[k] != kEmpty) pend &= ~(1u << k);
                }
                float *rpart = reinterpret_cast<float *>(lds8 + L.dma + 1024);   // [grid]
#pragma unroll
                for (int k = 0; k < PW; ++k) rpart[lane + 64 * k] = __uint_as_float((uint32_t)pv[k]);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int r = 0; r < 2; ++r) {
                    const int i = min(lane + 64 * r, a.experts - 1);
                    float v = rpart[i * S];
                    for (int k = 1; k < S; ++k) v += rpart[i * S + k];
                    lv[r] = v + bias_e[r];
                }
            } else {
#pragma unroll
                for (int r = 0; r < 2; ++r) lv[r] = a.logits[min(lane + 64 * r, a.experts - 1)];
            }
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int i = lane + 64 * r;
                const float v = lv[r];
                const bool in = i < a.experts, isn = in && __builtin_isnan(v);
                nan |= isn;
                rkey[i] = in && !isn ? order_key(v) : 0u;
                rlogit[i] = v;
            }
            const bool any_nan = __ballot(nan) != 0ull;
            if (lane == 0) *rcnt = 0ull, *rnan = any_nan ? 1u : 0u;
            if (lane == 0) *gu_done = 0u, *t_pub = 0u, *scl_in = 0u;
            if (lane < 4) ready[lane] = 0u, bx_in[lane] = 0u;
        } else {
            if (lane == 0) *gu_done = 0u, *t_pub = 0u, *scl_in = 0u;
            if (lane < 4) ready[lane] = 0u, bx_in[lane] = 0u;
            int sid;
            float w;
            select_one<4>(a.logits, a.experts, K, sid, w);
            if (lane < K) {
                eid[lane] = sid;
                ew[lane] = w;
                if (b == 0 && a.ids_out) a.ids_out[lane] = sid;
                if (b == 0 && a.w_out) a.w_out[lane] = w;
            }
        }
    } else {
        stage_vector<XK>(xs, a.x, H, threadIdx.x - 64, kDT - 64);
    }
    __syncthreads();
    if (by_rank) {
        const int ie = threadIdx.x >> 2, qe = threadIdx.x & 3;
        const uint32_t mk = rkey[ie];
        const uint4 *kq = reinterpret_cast<const uint4 *>(rkey + 32 * qe);
        int gt0 = 0, gt1 = 0;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const uint4 k4 = kq[c];
            gt0 += (k4.x > mk ? 1 : 0) + (k4.y > mk ? 1 : 0);
            gt1 += (k4.z > mk ? 1 : 0) + (k4.w > mk ? 1 : 0);
        }
        int gt = gt0 + gt1;
        gt += __builtin_amdgcn_mov_dpp(gt, 0xB1, 0xF, 0xF, true);   // the element's 4 lanes
        gt += __builtin_amdgcn_mov_dpp(gt, 0x4E, 0xF, 0xF, true);
        if (qe == 0 && mk != 0u && gt < K) {
            eid[gt] = ie;
            ew[gt] = rlogit[ie];                  // the logit until the softmax below
            atomicAdd(rcnt, 1ull << (8 * gt));
        }
        __syncthreads();
        // exactly one expert at each of the K ranks and no NaN, else the
        // exact selection
        const bool exact = *rnan != 0u || *rcnt != (0x0101010101010101ull >> (8 * (kMaxTopK - K)));
        if (exact) {                              // uniform: NaN or a tie
            if (wave == 0) {
                int sid;
                float w;
                // the logits in LDS (rlogit holds all of them): with the
                // in-kernel router there is no logits array in memory
                select_one<2>(a.rw ? rlogit : a.logits, a.experts, K, sid, w);
                if (lane < K) {
                    eid[lane] = sid;
                    ew[lane] = w;
                    if (b == 0 && a.ids_out) a.ids_out[lane] = sid;
                    if (b == 0 && a.w_out) a.w_out[lane] = w;
                }
            }
            __syncthreads();
        } else if (wave == kGuWaves) {
            // ew is read at the combine, after the barriers that follow
            const float sv = ew[min(lane, K - 1)];
            const float w = softmax_ranked(sv, K);
            if (lane < K) {
                ew[lane] = w;
                if (b == 0 && a.ids_out) a.ids_out[lane] = eid[lane];
                if (b == 0 && a.w_out) a.w_out[lane] = w;
            }
        }
    }

    const int segg = lane / TPG, tlg = lane % TPG;
    GW_TRACE(1);
    const int nrows = 2 * (p1 - p0);
    const int two_f = 2 * F;
    const float inv_two_f = 1.0f / (float)two_f;
    const int64_t rbg = (int64_t)hb * 16;
    const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.base), (short)0, (int)a.base_bytes, kRsrcWord3);

    // ---- the down stream --------------------------------------------------------
    // The workgroup's down rows of every selected expert, expert-major (row
    // rho = k * nr + q is output row r0 + q of expert rank k), in tiles of 16
    // rows; a unit (t, s) is rows 16t..16t+15 x blocks 4s..4s+3.  The two
    // waves of SIMD d (gate_up wave d, DMA wave kGuWaves + d) share tiles
    // tg*TPW.. (tg = d % WT) and 2 * SPW steps from (d / WT) * 2 * SPW: the
    // gate_up wave takes the first SPW, the DMA wave the rest; a wave's unit
    // i = j * TPW + tt is tile tg*TPW + tt, the wave's j-th step.  The rows
    // come in 1 KiB pieces of 8 rows x 8 blocks (a chunk): row r8 at r8 * 128,
    // block b in slot b ^ r8, so a DMA lane group copies one whole 128-byte
    // line of a row and an operand read of eight lanes (rows 0..7 or 8..15 of
    // a tile, one block each) touches every LDS bank once.  DMA wave
    // kGuWaves + d copies its SIMD's pieces chunk by chunk, flags its gate_up
    // wave once that wave's chunks have landed, and widens its own units as
    // theirs land; every wave widens its units' weights to fp16 in registers
    // while the exchange is still in flight.
    constexpr int PPS = TPW * SPW * 2;   // pieces per SIMD: SPW chunks x TPW tiles x 2 row halves
    constexpr int CG = (SPW + 1) / 2;    // chunks holding the gate_up wave's steps
    const int rbd = fb * 16;
    const float inv_nr = 1.0f / (float)nr;
    const int simd = wave & 3, kind = wave >> 2;
    const int tg = simd % WT, sg = (simd / WT) * 2 + kind;   // tile group, step group
    const int sbase = (simd / WT) * 2 * SPW;                  // the SIMD's first step
    const int rr = lane & 15, gr = lane >> 4;
    // The scale bytes follow as one window per expert in LDS: nr * fb bytes
    // from a 16-byte aligned start, expert k's at k * sws.  This lane's
    // operand rows (one per tile): whether they exist and where their scale
    // bytes sit in the window.
    const int s0 = r0 * fb, shs = s0 & 15;
    const int sws = (nr * fb + shs + 15) & ~15;
    const float inv_sws = 1.0f / (float)sws;
    uint32_t srow[TPW];
    bool sok[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int rho = 16 * (tg * TPW + tt) + rr;
        sok[tt] = rho < nrows_dn;
        int k, q;
        divmod_small(sok[tt] ? rho : 0, nr, inv_nr, k, q);
        srow[tt] = (uint32_t)(L.scl + k * sws + shs + q * fb);
    }
    // Layer offset of DMA lane `lane`'s 16 bytes of this SIMD's piece
    // (chunk cl, tile tt, row half h).
    auto piece_off = [&](int cl, int tt, int h) -> uint32_t {
        const int t = tg * TPW + tt, c = sbase / 2 + cl;
        const int r8 = lane >> 3, blk = 8 * c + ((lane & 7) ^ r8);
        const int rho = 16 * t + 8 * h + r8;
        const bool ok = rho < nrows_dn && blk < fb;
        int k, q;
        divmod_small(ok ? rho : 0, nr, inv_nr, k, q);
        return ok ? (uint32_t)eid[k] * (uint32_t)a.stride + (uint32_t)a.sec.dn_blocks +
                        (uint32_t)((r0 + q) * rbd + blk * 16)
                  : kOutOfRange;
    };
    // The finishing lanes (wave kGuWaves, lane q < nr) read row q's bias of
    // every selected expert early, all loads in flight together (the dword
    // holding the element; decoded at the combine).
    uint32_t BW[kMaxTopK];
    int BSHF[kMaxTopK];
    auto read_bias = [&]() {
        uint32_t ba[kMaxTopK];
#pragma unroll
        for (int k = 0; k < kMaxTopK; ++k) {
            const bool use = k < K && lane < nr && a.bias_dt >= 0;
            ba[k] = use ? (uint32_t)eid[min(k, K - 1)] * (uint32_t)a.stride + (uint32_t)a.sec.dn_bias +
                              (uint32_t)((r0 + lane) * bsz)
                        : kOutOfRange;
            BSHF[k] = (int)(ba[k] & 2u) * 8;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int k = 0; k < kMaxTopK; ++k) BW[k] = __builtin_amdgcn_raw_buffer_load_b32(lr, ba[k] & ~3u, 0, 0);
    };

    if (wave >= kGuWaves) {
        // ---- 2a. waves kGuWaves..: clear this workgroup's share of the next
        // launch's exchange slot (its last readers finished with the previous
        // launch), then wait until the gate_up waves have queued their last
        // stage and queue this wave's down units behind them.
        if (wave == kGuWaves + 1) {
            uint64_t *nx = a.xchg + (size_t)((epoch1 + 1) & 1u) * kXSlotWords;
            const int words = (kMaxTopK * F) >> 2, per = (words + (int)gridDim.x - 1) / (int)gridDim.x;
            for (int i = lane; i < per; i += 64) {
                const int w = b * per + i;
                if (w < words) __hip_atomic_store(nx + w, kEmpty, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        if (wave == kGuWaves) read_bias();
        const int d = wave - kGuWaves;
        uint32_t va[PPS], vs[NSP];
#pragma unroll
        for (int cl = 0; cl < SPW; ++cl)
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
                for (int h = 0; h < 2; ++h) va[(cl * TPW + tt) * 2 + h] = piece_off(cl, tt, h);
#pragma unroll
        for (int pp = 0; pp < NSP; ++pp) {
            const int pos = (d + (kDW - kGuWaves) * pp) * kChunk + lane * 16;
            int k, o;
            divmod_small(pos, sws, inv_sws, k, o);
            const bool ok = k < K && o < shs + nr * fb;
            vs[pp] = ok ? (uint32_t)eid[min(k, K - 1)] * (uint32_t)a.stride + (uint32_t)a.sec.dn_scales +
                              (uint32_t)(s0 - shs + o)
                        : kOutOfRange;
        }
#pragma unroll
        for (int i = 0; i < PPS; ++i) asm volatile("" : "+v"(va[i]));
#pragma unroll
        for (int pp = 0; pp < NSP; ++pp) asm volatile("" : "+v"(vs[pp]));
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // (the builtin's operands as plain locals: with an array element among
        // them the host pass emitted no launch stub for the kernel)
#pragma unroll
        for (int pp = 0; pp < NSP; ++pp) {
            const uint32_t voff = vs[pp];
            uint8_t *dst = lds8 + L.scl + (d + (kDW - kGuWaves) * pp) * kChunk;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(lr, (l_void *)dst, 16, voff, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < PPS; ++i) {
            const uint32_t voff = va[i];
            uint8_t *dst = lds8 + L.dma + (simd * PPS + i) * kChunk;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(lr, (l_void *)dst, 16, voff, 0, 0, 0);
        }
        // the scale pieces have landed once only weight pieces are in flight,
        // the gate_up wave's chunks once only the later chunks are
        const uint32_t cnt_addr = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)scl_in;
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(PPS) : "memory");
        if (lane == 0) asm volatile("ds_add_u32 %0, %1" ::"v"(cnt_addr), "v"(1u) : "memory");
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((SPW - CG) * TPW * 2) : "memory");
        if (lane == 0)
            asm volatile("ds_write_b32 %0, %1" ::"v"((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)(ready + d)), "v"(1u) : "memory");
        GW_TRACE(2);
    } else {
        // ---- 2b. gate_up (waves 0..kGuWaves-1, one per SIMD): RGW rows a
        // stage, a ring of D stages in flight (stage s + D issued once stage s
        // is consumed), widened and dotted as they land.  Rows past the share
        // read zeros without a memory access (buffer loads over the layer).
        constexpr int D = NSG < GD ? NSG : GD;
        u32x4 W[D][MG];
        uint32_t SCG[D][MG];
        uint32_t BW[D];
        int BSH[D];
#define GW_ISSUE_STAGE(S)                                                                       \
    do {                                                                                        \
        constexpr int q_ = (S) % D;                                                             \
        const int i_ = (S) * RGW + wave * SEGG + segg;                                          \
        const bool live_ = i_ < nrows;                                                          \
        int k_, r_;                                                                             \
        divmod_small(2 * p0 + (live_ ? i_ : 0), two_f, inv_two_f, k_, r_);                     \
        const uint32_t eo_ = (uint32_t)eid[k_] * (uint32_t)a.stride;                            \
        const uint32_t row_ = eo_ + (uint32_t)a.sec.gu_blocks + (uint32_t)(r_ * rbg);           \
        const uint32_t srow_ = eo_ + (uint32_t)a.sec.gu_scales + (uint32_t)(r_ * hb);           \
        _Pragma("unroll") for (int m_ = 0; m_ < MG; ++m_) {                                     \
            const int cb_ = min(tlg + m_ * TPG, hb - 1);                                        \
            W[q_][m_] = __builtin_bit_cast(                                                     \
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(                                   \
                           lr, live_ ? row_ + (uint32_t)cb_ * 16 : kOutOfRange, 0, kNt));       \
            SCG[q_][m_] = __builtin_amdgcn_raw_buffer_load_b8(                                  \
                lr, live_ ? srow_ + (uint32_t)cb_ : kOutOfRange, 0, 0);                         \
        }                                                                                       \
        const uint32_t ba_ = a.bias_dt >= 0                                                     \
                                 ? eo_ + (uint32_t)a.sec.gu_bias + (uint32_t)(r_ * bsz)         \
                                 : srow_;                                                       \
        BSH[q_] = (int)(ba_ & 2u) * 8;                                                          \
        BW[q_] = __builtin_amdgcn_raw_buffer_load_b32(lr, live_ ? (ba_ & ~3u) : kOutOfRange,   \
                                                      0, 0);                                    \
    } while (0)
        Unroll<0, D>::run([&](auto sc) { GW_ISSUE_STAGE(decltype(sc)::value); });
        // This lane's activation blocks into registers, read with ds_read_b128
        // written out (the x stores happened before the barrier above).
        uint4 X[MG][4];
        {
            const uint32_t xa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)xs;
            u32x4 xv[MG][4];
#pragma unroll
            for (int m = 0; m < MG; ++m) {
                const int cb = tlg + m * TPG;
                const uint32_t addr = xa + (uint32_t)((cb < hb ? cb : 0) * BD * 4);
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(xv[m][q]) : "v"(addr), "i"(q * 16));
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int m = 0; m < MG; ++m)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    u32x4 v = xv[m][q];
                    asm volatile("" : "+v"(v));
                    X[m][q] = make_uint4(v.x, v.y, v.z, v.w);
                }
        }
        Unroll<0, NSG>::run([&](auto sc) {
            constexpr int s = decltype(sc)::value, q = s % D;
            const int i = s * RGW + wave * SEGG + segg;
            const bool valid = i < nrows;
            float acc = 0.0f;
#pragma unroll
            for (int m = 0; m < MG; ++m) {
                const int cb = tlg + m * TPG;
                const bool use = valid && cb < hb;
                WBlock<XK> wb;
                widen_v(W[q][m], wb);
                float dd = block_dot_r<XK>(wb, X[m]);
                dd *= decode_scale(SCG[q][m]);
                acc += use ? dd : 0.0f;
            }
            acc = seg_sum<TPG>(acc);
            const float up = next_segment<TPG>(acc);
            const float b_own = bias_of(BW[q], BSH[q], a.bias_dt);
            const float b_next = next_segment<TPG>(b_own);
            if (valid && (segg & 1) == 0 && tlg == 0) {
                const float v = apply_activation(a.act_kind, acc + b_own, up + b_next, a.limit,
                                                 a.alpha);
                actl[i >> 1] = f32_to_f16_bits(v);
            }
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (s + D < NSG) {
                GW_ISSUE_STAGE(s + D);
                __builtin_amdgcn_sched_barrier(0);
            }
            if constexpr (s == (NSG > D ? NSG - 1 - D : 0)) {
                // the last stage is queued (or all were up front): the other
                // waves may queue the down units behind it
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
            }
        });
#undef GW_ISSUE_STAGE
        GW_TRACE(2);
        // ---- 3. the activations out: the gate_up waves count themselves done
        // in LDS (their activations are written first); wave 0 waits for the
        // count and publishes the workgroup's words.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_fetch_add(gu_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (wave == 0) {
            while (__hip_atomic_load(gu_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <
                   (unsigned)kGuWaves)
                __builtin_amdgcn_s_sleep(1);
            uint64_t *xw = a.xchg + (size_t)(epoch1 & 1u) * kXSlotWords;
            if (lane < q1 - q0) {
                uint64_t v = *reinterpret_cast<const uint64_t *>(actl + 4 * lane);
                v = v == kEmpty ? v ^ 1ull : v;   // all-ones (four NaNs): another NaN
                __hip_atomic_store(xw + q0 + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            if (lane == 0) *t_pub = (uint32_t)wall_clock64() | 1u;
        }
    }

    GW_TRACE(3);
    // ---- 4. the exchange: this wave's activation blocks into operand registers
    // Lane (c, g) = lane c + 16 g holds, for each of the wave's steps s, the
    // block 4s + g of expert rank c (c < K; other lanes hold zeros): the B
    // operand of the unit's four MFMAs, one fp16 octet each.  A gate_up wave
    // reads its own once its units' pieces are flagged and PD ticks after this
    // workgroup published.  With PX, after widening its units, it reads its
    // DMA partner's into LDS (past this chip's L2, by LDS-DMA) and flags them
    // once they are in, so a DMA wave's words do not queue behind its own
    // down pieces (a wave's loads complete in order); else a DMA wave reads
    // its own at the same point as the gate_up wave, behind its pieces.
    // Waits on this workgroup's own waves (all resident with it) are bounded
    // by the fixed kDecodeSpinLimit, not the caller's exchange limit, and a
    // wait that ran out is counted like a failed exchange wait.
    bool local_fail = false;
    const bool dma_wave = wave >= kGuWaves;
    const bool own_reads = !PX || !dma_wave;
    if (!dma_wave) {
        unsigned spins = 0;
        while (lds_peek(ready + wave) == 0u) {
            if (++spins > kDecodeSpinLimit) { local_fail = true; break; }   // the DMA wave flags them
            __builtin_amdgcn_s_sleep(1);
        }
    }
    if (own_reads) {
        unsigned spins = 0, tp;
        while ((tp = lds_peek(t_pub)) == 0u) {
            if (++spins > kDecodeSpinLimit) { local_fail = true; break; }   // wave 0 publishes
            __builtin_amdgcn_s_sleep(1);
        }
        if constexpr (PD > 0)
            while ((uint32_t)wall_clock64() - tp < (uint32_t)PD) __builtin_amdgcn_s_sleep(2);
    }
    GW_TRACE(4);
    const int slot = a.poll_fault ? 2 : (int)(epoch1 & 1u);
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        a.xchg + (size_t)slot * kXSlotWords, (short)0, kDecodeXchgSlotBytes, kRsrcWord3);
    // the words of step group kind k's j-th step for this lane
    auto word_off = [&](int k, int j) -> uint32_t {
        const int blk = 4 * (sbase + k * SPW + j) + gr;
        const bool ok = (rr < K) & (blk < fb);   // a select, not a branch
        return ok ? (uint32_t)((rr * F + 32 * blk) * 2) : kOutOfRange;
    };
    uint32_t boff[SPW];
    u32x4 Bv[SPW][4];
#pragma unroll
    for (int j = 0; j < SPW; ++j) boff[j] = word_off(kind, j);
    if (own_reads) {
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int m = 0; m < 4; ++m)
                Bv[j][m] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, boff[j] + 16u * m, 0, 0));
    }
    // ---- 5. this wave's units widened to fp16 while the exchange is in flight
    // A DMA wave takes each of its own pieces as it lands (the vector-memory
    // counter completes in order: piece i is in once only the later pieces,
    // and its own exchange reads when it makes them, are outstanding); a
    // gate_up wave's are all in.
    // ds_read_b128 written out: the compiler would make each read wait for
    // every load in flight.
    GW_TRACE(5);
    f16x8 AH[UPW][4];
    uint32_t SC[UPW];                    // the units' scale bytes
    uint32_t oor = 0;                    // units whose block this lane dots on the VALU
    {
        // operand lane: row rr of the tile (piece half rr >> 3, row rr & 7),
        // block gr of the step's four (slot (4 (step & 1) + gr) ^ (rr & 7))
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)(lds8 + L.dma) +
                              (uint32_t)(simd * PPS * kChunk + (rr >> 3) * kChunk + (rr & 7) * 128);
        {
            unsigned spins = 0;
            while (lds_peek(scl_in) < (unsigned)(kDW - kGuWaves)) {
                if (++spins > kDecodeSpinLimit) { local_fail = true; break; }   // every DMA wave counts itself
                __builtin_amdgcn_s_sleep(1);
            }
        }
        // the unit's weights and scale byte: an address per lane, then the
        // widening (a gate_up wave reads all its units first, with one wait)
        auto unit_addr = [&](int j, int tt, uint32_t &wa, uint32_t &sa, bool &live) {
            const int sl = kind * SPW + j, blk = 4 * (sbase + sl) + gr;
            live = sok[tt] && blk < fb;
            wa = base + (uint32_t)(((sl >> 1) * TPW + tt) * 2 * kChunk + 16 * ((4 * (sl & 1) + gr) ^ (rr & 7)));
            sa = srow[tt] + (uint32_t)(live ? blk : 0);
        };
        auto widen_unit = [&](int i, int tt, u32x4 w, uint32_t sb, bool live) {
            SC[i] = sb;
            const bool inr = live && sb - 104u <= 36u;
            oor |= (uint32_t)(live && !inr) << i;
            const float scl = __uint_as_float((inr ? sb : 127u) << 23);
            const uint32_t msk = inr ? ~0u : 0u;
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                AH[i][m] = widen_scaled(w[m] & msk, scl);
                asm volatile("" : "+v"(AH[i][m]));   // widened now, not after the later waits
            }
        };
        if (dma_wave) {
            Unroll<0, UPW>::run([&](auto ic) {
                constexpr int i = decltype(ic)::value, j = i / TPW, tt = i % TPW;
                // a DMA wave's unit has landed once only later chunks' pieces
                // are in flight
                if constexpr (j == 0 || ((SPW + j) >> 1) != ((SPW + j - 1) >> 1)) {
                    constexpr int later = SPW - 1 - ((SPW + j) >> 1);
                    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(later * TPW * 2 + (PX ? 0 : 4 * SPW)) : "memory");
                }
                uint32_t wa, sa;
                bool live;
                unit_addr(j, tt, wa, sa, live);
                u32x4 w;
                uint32_t sb;
                asm volatile("ds_read_b128 %0, %2\n\tds_read_u8 %1, %3\n\ts_waitcnt lgkmcnt(0)"
                             : "=v"(w), "=v"(sb) : "v"(wa), "v"(sa) : "memory");
                widen_unit(i, tt, w, sb, live);
            });
        } else {
            u32x4 w[UPW];
            uint32_t sb[UPW];
            bool live[UPW];
#pragma unroll
            for (int i = 0; i < UPW; ++i) {
                uint32_t wa, sa;
                unit_addr(i / TPW, i % TPW, wa, sa, live[i]);
                u32x4 wv;
                uint32_t sv;
                asm volatile("ds_read_b128 %0, %2\n\tds_read_u8 %1, %3"
                             : "=v"(wv), "=v"(sv) : "v"(wa), "v"(sa) : "memory");
                w[i] = wv;
                sb[i] = sv;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int i = 0; i < UPW; ++i) {
                u32x4 wv = w[i];
                uint32_t sv = sb[i];
                asm volatile("" : "+v"(wv), "+v"(sv));   // loaded by the wait above
                widen_unit(i, i % TPW, wv, sv, live[i]);
            }
        }
    }
    GW_TRACE(6);
    if (PX && !dma_wave) {
        // the DMA partner's words into LDS past this chip's L2 (each lane's
        // 16-byte reads as in its own registers), flagged once all of this
        // wave's loads are in; its own words were read before the widening
        uint8_t *bxw = lds8 + L.bx + simd * SPW * 4 * kChunk;
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            const uint32_t po = word_off(1, j);
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const uint32_t voff = po + 16u * (uint32_t)m;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (l_void *)(bxw + (j * 4 + m) * kChunk), 16, voff, 0, 0,
                                                         kSc1);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (lane == 0)
            asm volatile("ds_write_b32 %0, %1"
                         ::"v"((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)(bx_in + simd)), "v"(1u)
                         : "memory");
    }
    uint32_t pend = 0;
    if (PX && dma_wave) {
        // this wave's words, read for it by its gate_up wave
        unsigned spins = 0;
        while (lds_peek(bx_in + simd) == 0u) {
            if (++spins > 4u * kDecodeSpinLimit) { local_fail = true; break; }   // the gate_up wave flags them
            __builtin_amdgcn_s_sleep(1);
        }
        const uint32_t bxa = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)(lds8 + L.bx) +
                             (uint32_t)(simd * SPW * 4 * kChunk + lane * 16);
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int m = 0; m < 4; ++m)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(Bv[j][m]) : "v"(bxa), "i"((j * 4 + m) * kChunk));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    // the reads are looked at only now, after the widening (the compiler
    // would hoist the check, and its wait for them, above it)
#pragma unroll
    for (int j = 0; j < SPW; ++j)
#pragma unroll
        for (int m = 0; m < 4; ++m) asm volatile("" : "+v"(Bv[j][m]));
    {
        // Words still empty are read again past this chip's L2 (the first
        // read may be served by an L2 line fetched before they were written).
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int m = 0; m < 4; ++m)
                pend |= pair_empty(Bv[j][m]) << (4 * j + m);
        GW_TRACE(11);
        unsigned spins = 0;
        bool gave_up = local_fail || route_fail;
        while (pend) {
            if (++spins > a.spin_limit) {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int j = 0; j < SPW; ++j)
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    if ((pend >> (4 * j + m)) & 1u)
                        Bv[j][m] = __builtin_bit_cast(
                            u32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, boff[j] + 16u * m, 0, kSc1));
#pragma unroll
            for (int j = 0; j < SPW; ++j)
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    if (!pair_empty(Bv[j][m])) pend &= ~(1u << (4 * j + m));
        }
        if (__ballot(gave_up) != 0ull && lane == 0) atomicAdd(a.sync.err, 1u);
    }
    GW_TRACE(7);
    // ---- 6. down products on the matrix cores -------------------------------
    f32x4 acc[TPW][2];
    float vf[TPW];
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        acc[tt][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        acc[tt][1] = acc[tt][0];
        vf[tt] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < SPW; ++j)
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt)
#pragma unroll
            for (int m = 0; m < 4; ++m)
                acc[tt][m & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    AH[j * TPW + tt][m], __builtin_bit_cast(f16x8, Bv[j][m]), acc[tt][m & 1], 0, 0, 0);
    GW_TRACE(8);
    const bool any_fb = __ballot(oor != 0u) != 0ull;
    if (any_fb) {
        // Scale bytes outside the fp16-exact range (rare): the block dotted on
        // the VALU with its activations fetched from the lane of this row's
        // expert, times the fp32 scale (referenceMXFP4's arithmetic).
        const uint8_t *pbase = lds8 + L.dma + simd * PPS * kChunk + (rr >> 3) * kChunk + (rr & 7) * 128;
#pragma unroll
        for (int j = 0; j < SPW; ++j)
#pragma unroll
            for (int tt = 0; tt < TPW; ++tt) {
                const int i = j * TPW + tt;
                if (__ballot((oor >> i) & 1u) == 0ull) continue;
                int k, q;
                divmod_small(16 * (tg * TPW + tt) + rr, nr, inv_nr, k, q);
                const int src = (min(k, 15) + 16 * gr) * 4;
                uint4 xa[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    xa[m].x = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)Bv[j][m].x);
                    xa[m].y = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)Bv[j][m].y);
                    xa[m].z = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)Bv[j][m].z);
                    xa[m].w = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)Bv[j][m].w);
                }
                const int sl = kind * SPW + j;
                WBlock<DT_F16> wb;
                widen_v(*reinterpret_cast<const u32x4 *>(pbase + ((sl >> 1) * TPW + tt) * 2 * kChunk +
                                                          16 * ((4 * (sl & 1) + gr) ^ (rr & 7))),
                        wb);
                const float d = block_dot_r<DT_F16>(wb, xa) * decode_scale(SC[i] & 0xFFu);
                vf[tt] += (oor >> i) & 1u ? d : 0.0f;
            }
    }
    // Partial sum of row rho = 16 t + r from its expert's column: lane l holds
    // D[4 (l >> 4) + v][l & 15], and column c is expert rank c, whose rows are
    // [c * nr, c * nr + nr) (two compares, no division).
    const int rlo = rr < K ? rr * nr : 0, rhi = rr < K ? rlo + nr : 0;
#pragma unroll
    for (int tt = 0; tt < TPW; ++tt) {
        const int t = tg * TPW + tt;
        const f32x4 dsum = acc[tt][0] + acc[tt][1];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int rho = 16 * t + 4 * gr + v;
            if (rho >= rlo && rho < rhi) part[sg * 16 * TD + rho] = dsum[v];
        }
    }
    if (any_fb) {
        // the VALU blocks' sums of each row (its four lanes), added in a fixed order
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            float v = vf[tt];
            v += __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 16) * 4, __float_as_int(v)));
            v += __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ 32) * 4, __float_as_int(v)));
            const int rho = 16 * (tg * TPW + tt) + rr;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (gr == 0 && rho < nrows_dn) part[sg * 16 * TD + rho] += v;
        }
    }
    GW_TRACE(12);
    __syncthreads();

    GW_TRACE(9);
    // ---- 7. bias and combine in router order: dst += out_k * w_k, the product
    // and the sum rounded separately (expert_accumulate).  accumulate: 0
    // overwrite; 1 add to out (applyAssignments); 2 out += the finished sum
    // (the residual add after the block, TransformerLayer.swift:232-238).
    if (wave == kGuWaves && lane < nr) {
        const int64_t o = r0 + lane;
        float dst = a.accumulate == 1 ? a.out[o] : 0.0f;
        // every partial and weight read at once (rank K - 1's again past K),
        // then summed in step-group and router order
        float pv[kMaxTopK][WS], wk[kMaxTopK];
#pragma unroll
        for (int k = 0; k < kMaxTopK; ++k) {
            const int kk = k < K ? k : K - 1, rho = kk * nr + lane;
#pragma unroll
            for (int g = 0; g < WS; ++g) pv[k][g] = part[g * 16 * TD + rho];
            wk[k] = ew[kk];
        }
#pragma unroll
        for (int k = 0; k < kMaxTopK; ++k) {
            float v = pv[k][0];
#pragma unroll
            for (int g = 1; g < WS; ++g) v += pv[k][g];
            const float nd = add_scaled_rn(dst, v + bias_of(BW[k], BSHF[k], a.bias_dt), wk[k]);
            dst = k < K ? nd : dst;
        }
        if (a.accumulate == 2) dst = a.out[o] + dst;
        a.out[o] = dst;
        if (a.out_bf16) a.out_bf16[o] = f32_to_bf16_bits(dst);
    }
    GW_TRACE(10);
    if (threadIdx.x == 0) a.sync.epochs[b] = epoch1;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

// Instantiations: GPT-OSS (hidden = intermediate = 2880: 90-block rows, up to
// top-4: 88 or 96 gate_up rows a workgroup on 256 CUs in six 16-row stages;
// 44 or 48 down rows in three tiles, 23 steps over eight step groups) and
// Qwen3-30B-A3B (2048 / 768: 64- and 24-block rows, up to top-8: 48 gate_up
// rows in three stages; 64 down rows in four tiles, each wave one tile and
// three of the six steps).
enum { kShapeGptOss = 0, kShapeQwen3 = 1 };
constexpr int kStagesG[2] = {6, 3};
constexpr int kRingG[2] = {2, 2};         // gate_up stages in flight per wave
constexpr int kRowsPerStage[2] = {kGuWaves * 64 / 16, kGuWaves * 64 / 16};
constexpr int kTiles[2] = {3, 4};
constexpr int kTileGroups[2] = {1, 4};
constexpr int kStepsPerWave[2] = {3, 3};
constexpr int kScalePieces[2] = {2, 1};   // per DMA wave
// The first read of the exchange waits at least this many ticks (10 ns)
// after the workgroup published (a read that comes before the slowest
// publisher costs a second round trip).  Measured on MI355X: GPT-OSS spans
// the same from 0 to 1 us (the reads queue behind the down pieces anyway);
// Qwen3 0.3 us is best.
constexpr int kPollDelay[2] = {60, 30};
// The gate_up waves read their DMA partners' exchange words (GPT-OSS: the
// DMA waves' reads would complete only behind their down pieces).
constexpr bool kPartnerReads[2] = {true, false};

int shape_of(int hidden, int inter)
{
    const int hb = hidden / 32, fb = inter / 32;
    if (hidden % 32 || inter % 32) return -1;
    if (hb > 64 && hb <= 96 && fb > 64 && fb <= 96) return kShapeGptOss;
    if (hb > 24 && hb <= 64 && fb > 8 && fb <= 24) return kShapeQwen3;
    return -1;
}

#define GW_DECODE_KERNEL(S, XD)                                                                 \
    decode_layer_kernel<XD, DShape<16, (S) == kShapeGptOss ? 6 : 4>, kStagesG[S], kRingG[S], kTiles[S], \
                        kTileGroups[S], kStepsPerWave[S], kScalePieces[S], kPollDelay[S], kPartnerReads[S]>

typedef void (*DecodeKernel)(DecodeArgs);

// The instantiation for (shape, x dtype).
DecodeKernel kernel_for(int shape, int x_dt)
{
    if (shape == kShapeGptOss)
        return x_dt == DT_BF16 ? &GW_DECODE_KERNEL(kShapeGptOss, DT_BF16)
                               : &GW_DECODE_KERNEL(kShapeGptOss, DT_F16);
    return x_dt == DT_BF16 ? &GW_DECODE_KERNEL(kShapeQwen3, DT_BF16)
                           : &GW_DECODE_KERNEL(kShapeQwen3, DT_F16);
}

}  // namespace
#undef GW_DECODE_KERNEL

int decode_layer_plan(const Launch &L, int hidden, int inter, int x_dt, int top_k, int experts,
                      int64_t stride, int bias_dt, DecodeArgs *args, size_t *lds_bytes)
{
    (void)bias_dt;
    const int shape = shape_of(hidden, inter);
    if (shape < 0 || (x_dt != DT_BF16 && x_dt != DT_F16)) return 0;
    if (top_k < 1 || top_k > kMaxTopK || experts > 256 || experts < top_k) return 0;
    if ((int64_t)experts * stride >= (int64_t)kOutOfRange) return 0;   // 32-bit buffer offsets
    const int G = L.cus;
    if (G <= 0 || G > kDecodeMaxGrid) return 0;
    // A slot holds every word a launch of this width can publish.
    if ((int64_t)kMaxTopK * inter * 2 > kDecodeXchgSlotBytes) return 0;
    // Every workgroup's gate_up share (whole quads) must fit the register stages.
    const int quads = (int)(((int64_t)top_k * inter / 4 + G - 1) / G);
    if (8 * quads > kStagesG[shape] * kRowsPerStage[shape]) return 0;
    // The down rows of every selected expert fit the tiles, the blocks the steps.
    const int nrmax = (hidden + G - 1) / G;
    if (top_k * nrmax > 16 * kTiles[shape]) return 0;
    const int wt = kTileGroups[shape], spw = kStepsPerWave[shape];
    const int fb = inter / 32;
    if ((fb + 3) / 4 > (8 / wt) * spw) return 0;
    // every expert's scale window (from a 16-byte aligned start) fits the pieces
    if (top_k * ((nrmax * fb + 15 + 15) & ~15) > (8 - kGuWaves) * kScalePieces[shape] * kChunk) return 0;
    const DecodeLds l = decode_lds(hidden, 8 * (kTiles[shape] / wt) * spw, (8 - kGuWaves) * kScalePieces[shape],
                                   (8 / wt) * 16 * kTiles[shape], kStagesG[shape] * kRowsPerStage[shape],
                                   kPartnerReads[shape] ? (8 - kGuWaves) * spw * 4 : 0);
    if (l.total > kDecodeLdsMax) return 0;
    // The exchange needs the whole grid resident: one workgroup per CU.
    const void *fn = reinterpret_cast<const void *>(kernel_for(shape, x_dt));
    static const void *attr_done[4] = {};
    int slot = -1;
    for (int i = 0; i < 4; ++i)
        if (attr_done[i] == fn || attr_done[i] == nullptr) { slot = i; break; }
    if (slot < 0) return 0;
    if (attr_done[slot] != fn) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kDecodeLdsMax) !=
            hipSuccess)
            return 0;
        attr_done[slot] = fn;
    }
    int occ = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fn, kDT, (size_t)l.total) != hipSuccess ||
        occ < 1)
        return 0;
    if (args) {
        args->nrmax = nrmax;
        args->base_bytes = (uint32_t)((int64_t)experts * stride);
    }
    if (lds_bytes) *lds_bytes = (size_t)l.total;
    return G;
}

hipError_t launch_decode_layer(const Launch &L, int grid, size_t lds, int x_dt, const DecodeArgs &a)
{
    const int shape = shape_of(a.hidden, a.inter);
    if (shape < 0 || grid <= 0) return hipErrorInvalidValue;
    const DecodeKernel kernel = kernel_for(shape, x_dt);
    if (L.coop && !L.ev_start) {
        DecodeArgs copy = a;
        void *args[] = {&copy};
        return hipLaunchCooperativeKernel(reinterpret_cast<const void *>(kernel), dim3(grid), dim3(kDT),
                                          args, (unsigned)lds, L.stream);
    }
    GW_LAUNCH(kernel, dim3(grid), dim3(kDT), lds, L, a);
    return hipGetLastError();
}

#ifdef GW_DECODE_TRACE
extern "C" __attribute__((visibility("default"))) int gw_debug_decode_trace(uint64_t *dst)
{
    return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_decode_trace), sizeof(g_decode_trace));
}
#endif

}  // namespace gw
