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
// as soon as the routing is.  Each SIMD runs one gate_up wave and one DMA
// wave: the gate_up waves stream their rows through a ring of register stages
// and widen and dot them as they land; the DMA waves, released once the last
// gate_up stage is queued, copy the workgroup's down rows with their scales
// and biases straight into LDS by buffer LDS-DMA (no registers held).  A SIMD
// lets its older wave issue first, so the gate_up rows are queued ahead of
// the down stream.  The activations are exchanged across the grid while the
// down rows are still streaming in, and the down products are computed from
// LDS once both are there.
//
// The exchange: a workgroup stores its activations with their launch tag in
// 8-byte words (device-coherent stores, no wait); the gate_up waves of every
// workgroup, which hold no down stream of their own, poll all words until
// each carries the current tag (a bounded spin: a wait that gives
// up sets an error word, read by gw_expert_runner_sync_errors, so no
// workgroup ever waits unboundedly) and stages the activations in LDS.  The
// grid must be co-resident (one workgroup per CU; the host checks occupancy).
//
// The gate_up rows are computed exactly as in the two-kernel form
// (gate_up_kernel): the same widening, block dots, scale products, lane order
// and reductions, so the activations are the same bytes.  The down rows are
// split over the lanes differently (see step 6), so their fp32 sums may round
// differently; both forms hold the reference's tolerance.
#include <hip/hip_ext.h>

#include <type_traits>

#include "gw_device.h"
#include "gw_launch.h"
#include "gw_route.h"

namespace gw {

namespace {

constexpr int kDT = 512;          // threads per workgroup
constexpr int kDW = kDT / 64;     // waves per workgroup
// Waves 0..kGuWaves-1 (one per SIMD) stream and compute the gate_up rows and
// then poll the exchange; the others issue the down stream's LDS-DMA.
constexpr int kGuWaves = 4;
constexpr int kDmaWaves = kDW - kGuWaves;
constexpr int kChunk = 1024;      // bytes one wave-wide 16-byte LDS-DMA moves
constexpr int kRsrcWord3 = 0x00020000;   // raw (untyped) buffer access
constexpr int kNt = 2;                   // buffer cache policy: non-temporal (streamed once)
constexpr uint32_t kOutOfRange = 0x80000000u;   // buffer offset past any layer (reads zero)
constexpr int kXWords = 16;              // exchange words per workgroup at most (3 activations each)
constexpr int kXSlotWords = kDecodeMaxGrid * kXWords;   // one launch's words
static_assert(kXSlotWords * 8 * kDecodeXchgSlots <= kDecodeXchgBytes, "exchange buffer");
constexpr unsigned kSpinLimit = 1u << 18;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void l_void;

template <int TPR_, int M_> struct DShape {
    static constexpr int TPR = TPR_;   // lanes per row
    static constexpr int M = M_;       // 16-byte blocks per lane (lane l: l, l+TPR, ...)
};

}  // namespace

// Byte layout of the kernel's LDS (host and device compute the same).
__host__ __device__ inline DecodeLds decode_lds(int hidden, int inter, int top_k, int nrmax,
                                               int sw_total, int rows_per_wg)
{
    DecodeLds l;
    const int hb = hidden / 32, fb = inter / 32;
    l.route = 0;                                   // int32 ids[8], float w[8], done count, rank counts
    l.xs = 128;                                    // x, 20 dwords per block
    l.actl = l.xs + hb * 80;                       // this workgroup's fp16 activations
    l.dma = (l.actl + rows_per_wg + 255) & ~255;   // the down stream (+ one spare chunk)
    const int dma_bytes = (top_k * sw_total + kChunk - 1) / kChunk * kChunk + kChunk;
    l.as = l.dma + dma_bytes;                      // all activations, fp16 [top_k][inter]
    // (the routing keys and logits, 1 KiB, use the same area before the exchange)
    l.vals = l.as + max(top_k * fb * 64, 1024);    // down outputs [top_k][nrmax]
    l.total = l.vals + top_k * nrmax * 4;
    return l;
}

// Per-expert windows of the down stream in LDS: the workgroup's down rows,
// their scale bytes and their biases, each from a 16-byte aligned start.
__host__ __device__ inline void decode_windows(int hidden, int inter, int nrmax, int bias_bytes,
                                               int &sww, int &sws, int &swb)
{
    (void)hidden;
    const int fb = inter / 32;
    sww = nrmax * fb * 16;
    sws = (nrmax * fb + 15 + 15) & ~15;
    swb = bias_bytes > 0 ? (nrmax * bias_bytes + 15 + 15) & ~15 : 0;
}

namespace {

// The bias element of a gate_up row is read with the stage as the aligned
// dword containing it (one load whatever the dtype).
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

}  // namespace

// XK: x dtype (bf16 or fp16).  GS / DS: row shapes of gate_up (hidden wide)
// and down (intermediate wide) rows.  NSG: gate_up stages (of kGuWaves * 64 /
// TPR rows) a workgroup's share fills.  NDMA: 1 KiB LDS-DMA pieces each DMA
// wave issues for the down stream.  PD: ticks of the 100 MHz real-time
// counter between publishing and the first poll of the exchange.  XW: words
// of a workgroup's exchange slot (a power of two, at most kXWords).
template <int XK, class GS, int NSG, class DS, int NDMA, int PD, int XW>
__global__ __launch_bounds__(kDT) void decode_layer_kernel(DecodeArgs a)
{
    constexpr int TPG = GS::TPR, MG = GS::M, SEGG = 64 / TPG, RGW = kGuWaves * SEGG;
    constexpr int TPD = DS::TPR, MD = DS::M, SEGD = 64 / TPD;
    constexpr int BD = XL<XK>::kBlockDw;
    extern __shared__ __align__(16) uint32_t lds[];
    uint8_t *lds8 = reinterpret_cast<uint8_t *>(lds);

    const int H = a.hidden, F = a.inter, K = a.top_k;
    const int hb = H >> 5, fb = F >> 5;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int b = blockIdx.x;
    const int bsz = a.bias_dt == DT_F32 ? 4 : 2;
    int sww, sws, swb;
    decode_windows(H, F, a.nrmax, a.bias_dt >= 0 ? bsz : 0, sww, sws, swb);
    const int swt = sww + sws + swb;
    int p0, p1;                          // gate_up: (expert, feature) pairs [p0, p1)
    slice_of(K * F, p0, p1);
    int r0, r1;                          // down: output rows [r0, r1) of every expert
    slice_of(H, r0, r1);
    const int nr = r1 - r0;
    const DecodeLds L = decode_lds(H, F, K, a.nrmax, swt, RGW * NSG);
    int32_t *eid = reinterpret_cast<int32_t *>(lds8 + L.route);
    float *ew = reinterpret_cast<float *>(lds8 + L.route + 32);
    unsigned *gu_done = reinterpret_cast<unsigned *>(lds8 + L.route + 64);   // gate_up waves done
    uint32_t *xs = reinterpret_cast<uint32_t *>(lds8 + L.xs);
    uint16_t *actl = reinterpret_cast<uint16_t *>(lds8 + L.actl);
    uint32_t *as = reinterpret_cast<uint32_t *>(lds8 + L.as);
    float *vals = reinterpret_cast<float *>(lds8 + L.vals);
    // Launches this workgroup has completed (written back at the end).
    const unsigned epoch1 = a.sync.epochs[b] + 1;

    // ---- 1. route while waves 1.. stage x -----------------------------------
    // Up to 128 experts: wave 0 writes the logits' order keys to LDS (0 for
    // NaN and for no expert), then every thread counts, for expert t / 4,
    // the keys greater than its own in quarter t % 4 of them.  When no logit
    // is NaN and no two experts share a selected rank's key, expert e's count
    // is its position in Router.select's result (the selection sort picks
    // the K largest in descending order whatever its permutation holds);
    // otherwise wave 0 runs the exact selection.  The softmax over the
    // selected logits is computed by a DMA wave, off the gate_up path.  More
    // experts: wave 0 routes alone (select_one).
    const bool by_rank = a.experts <= 128;
    uint32_t *rkey = reinterpret_cast<uint32_t *>(lds8 + L.as);   // keys [128]; the
    float *rlogit = reinterpret_cast<float *>(lds8 + L.as + 512);  // exchange area is free
    unsigned *rcount = reinterpret_cast<unsigned *>(lds8 + L.route + 68);   // [kMaxTopK + 1]
    if (wave == 0) {
        if (by_rank) {
            bool nan = false;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int i = lane + 64 * r;
                const float v = a.logits[min(i, a.experts - 1)];
                const bool in = i < a.experts, isn = in && __builtin_isnan(v);
                nan |= isn;
                rkey[i] = in && !isn ? order_key(v) : 0u;
                rlogit[i] = v;
            }
            // rcount[0..K) count the experts placed at each rank; rcount[K]
            // flags a NaN
            const bool any_nan = __ballot(nan) != 0ull;
            if (lane <= K) rcount[lane] = lane == K && any_nan ? 1u : 0u;
            if (lane == 0) *gu_done = 0u;
        } else {
            if (lane == 0) *gu_done = 0u;
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
            atomicAdd(rcount + gt, 1u);
        }
        __syncthreads();
        bool exact = rcount[K] != 0u;
        for (int r = 0; r < K; ++r) exact |= rcount[r] != 1u;
        if (exact) {                              // uniform: NaN or a tie
            if (wave == 0) {
                int sid;
                float w;
                select_one<2>(a.logits, a.experts, K, sid, w);
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
    const int nrows = 2 * (p1 - p0);
    const int two_f = 2 * F;
    const float inv_two_f = 1.0f / (float)two_f;
    const int64_t rbg = (int64_t)hb * 16;
    const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(a.base), (short)0, (int)a.base_bytes, kRsrcWord3);

    if (wave >= kGuWaves) {
        // ---- 3a. the down stream (waves kGuWaves..): the workgroup's down
        // rows, their scale bytes and biases straight into LDS by LDS-DMA.
        // Piece c of DMA wave d is packed position (d + kDmaWaves*c) KiB of
        // the per-expert windows [rows | scale bytes | biases] x top_k; pieces
        // past the end read zeros into the spare chunk without a memory
        // access.  These waves share each SIMD with a gate_up wave, which
        // takes precedence in issuing, so the gate_up rows are queued first.
        const int d = wave - kGuWaves;
        const int total = K * swt;
        const int nchunks = (total + kChunk - 1) / kChunk;
        const int rbd = fb * 16;
        const int s0 = r0 * fb, b0 = r0 * bsz;
        const int s0a = s0 & ~15, b0a = b0 & ~15;
        const int lim_w = nr * rbd, lim_s = (s0 - s0a) + nr * fb;
        const int lim_b = a.bias_dt >= 0 ? (b0 - b0a) + nr * bsz : 0;
        const uint32_t rel_w = (uint32_t)(a.sec.dn_blocks + (int64_t)r0 * rbd);
        const uint32_t rel_s = (uint32_t)(a.sec.dn_scales + s0a) - (uint32_t)sww;
        const uint32_t rel_b = (uint32_t)(a.sec.dn_bias + b0a) - (uint32_t)(sww + sws);
        const float inv_swt = 1.0f / (float)swt;
        // Wait until the gate_up waves have queued their last stage.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < NDMA; ++c) {
            const int chunk = d + kDmaWaves * c;
            const int pos = chunk * kChunk + lane * 16;
            int k, o;
            divmod_small(pos, swt, inv_swt, k, o);
            const uint32_t eo = (uint32_t)eid[min(k, K - 1)] * (uint32_t)a.stride;
            const bool is_w = o < sww, is_s = !is_w && o < sww + sws;
            const int lim = is_w ? lim_w : is_s ? lim_s + sww : lim_b + sww + sws;
            const uint32_t rel = is_w ? rel_w : is_s ? rel_s : rel_b;
            const bool ok = pos < total && o < lim;
            const uint32_t voff = ok ? eo + rel + (uint32_t)o : kOutOfRange;
            uint8_t *dst = lds8 + L.dma + (chunk < nchunks ? chunk : nchunks) * kChunk;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(lr, (l_void *)dst, 16, voff, 0, 0, 0);
        }
    } else {
        // ---- 3b. gate_up (waves 0..kGuWaves-1, one per SIMD): RGW rows a
        // stage, a ring of D stages in flight (stage s + D issued once stage s
        // is consumed), widened and dotted as they land.  Rows past the share
        // read zeros without a memory access (buffer loads over the layer).
        constexpr int D = NSG < 2 ? NSG : 2;
        u32x4 W[D][MG];
        uint32_t SC[D][MG];
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
            SC[q_][m_] = __builtin_amdgcn_raw_buffer_load_b8(                                   \
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
        // written out: the compiler would make an LDS read after an LDS-DMA
        // wait for every load in flight; x was stored before the barrier above.
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
                dd *= decode_scale(SC[q][m]);
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
                // the last stage is queued (or all were up front): the DMA
                // waves may queue the down stream behind it
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
            }
        });
#undef GW_ISSUE_STAGE
    }
    // The gate_up waves count themselves done in LDS (their activations are
    // written first); the publishing wave waits for the count instead of a
    // barrier, which would also wait for the DMA waves still queuing the
    // down stream.
    if (wave < kGuWaves) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_fetch_add(gu_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (wave == 0) {
            while (__hip_atomic_load(gu_done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) <
                   (unsigned)kGuWaves)
                __builtin_amdgcn_s_sleep(1);
        }
    }

    // ---- 5. exchange ---------------------------------------------------------
    // Workgroup b publishes its activations as XW 8-byte words, three
    // fp16 values and the 16-bit launch tag each, with device-coherent stores;
    // an aligned 8-byte store is seen whole or not at all, so the tag marks
    // the word valid and no separate flag, wait or counter is needed.  The
    // gate_up waves (no down stream of their own, so their loads are not
    // queued behind it) then read all words, keeping those carrying this
    // launch's tag and polling the rest (a bounded spin), and place the
    // activations in LDS while the down stream still lands; the DMA waves
    // wait for their part of it.  Every workgroup completes every launch, so
    // all agree on the tag.
    const int G = gridDim.x;
    const int npair = K * F;
    const unsigned pq = (unsigned)npair / (unsigned)G, pr = (unsigned)npair - pq * (unsigned)G;
    const uint64_t tag = (uint64_t)(epoch1 & 0xFFFFu);
    uint64_t *xw = a.xchg + (epoch1 % kDecodeXchgSlots) * kXSlotWords;
    if (wave == 0 && 3 * lane < p1 - p0) {
        uint64_t v = tag << 48;
#pragma unroll
        for (int e = 0; e < 3; ++e) {
            const int j = 3 * lane + e;
            v |= (uint64_t)(j < p1 - p0 ? actl[j] : 0) << (16 * e);
        }
        __hip_atomic_store(xw + b * XW + lane, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wave >= kGuWaves) {
        __builtin_amdgcn_s_waitcnt(0);            // this wave's part of the down stream is in LDS
    } else {
        // Thread t reads word j = t % XW of workgroups t / XW +
        // u * kPbStep.  The first round's loads are all issued before any
        // LDS address is formed, so that work overlaps their latency.
        constexpr int kPollT = kGuWaves * 64;
        static_assert(XW <= kXWords && (XW & (XW - 1)) == 0, "slot words");
        constexpr int WPT = kDecodeMaxGrid * XW / kPollT;        // words per thread
        constexpr int kPbStep = kPollT / XW;
        static_assert(WPT <= 32, "pending mask");
        const int t = (int)threadIdx.x;
        const int j = t % XW, pb0 = t / XW;
        uint32_t pending = 0;
#pragma unroll
        for (int u = 0; u < WPT; ++u) {
            const int pb = pb0 + u * kPbStep;
            const int np = (int)pq + (pb < (int)pr ? 1 : 0);
            pending |= (uint32_t)((pb < G) & (3 * j < np)) << u;
        }
        {
            const uint64_t t_pub = wall_clock64();
            while (wall_clock64() - t_pub < (uint64_t)PD) __builtin_amdgcn_s_sleep(2);
        }
        // The first round may be served by this chip's L2 (the first of its
        // compute units to read a line fetches it once for all); a word
        // found stale there is read again past the L2.
        uint64_t v[WPT];
#pragma unroll
        for (int u = 0; u < WPT; ++u)
            v[u] = (pending >> u) & 1u
                       ? __hip_atomic_load(xw + t + u * kPollT, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WAVEFRONT)
                       : 0ull;
        __builtin_amdgcn_sched_barrier(0);
        // Word (pb, j) holds pairs pb * pq + min(pb, pr) + 3j .. +2 of the
        // linear fp16 [top_k][inter] layout; they are written with ds_write
        // written out, which waits only for this word's load.
        const uint32_t as_addr = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)(lds8 + L.as);
        unsigned spins = 0;
        for (;;) {
#pragma unroll
            for (int u = 0; u < WPT; ++u) {
                if (((pending >> u) & 1u) && (v[u] >> 48) == tag) {
                    pending &= ~(1u << u);
                    const int pb = pb0 + u * kPbStep;
                    const int nv = (int)pq + (pb < (int)pr ? 1 : 0) - 3 * j;   // >= 1
                    const uint32_t pair = __umul24((uint32_t)pb, pq) + (uint32_t)min(pb, (int)pr) +
                                          (uint32_t)(3 * j);
                    const uint32_t addr = as_addr + 2 * pair;
                    const uint32_t lo = (uint32_t)v[u], hi = (uint32_t)(v[u] >> 32);
                    asm volatile("ds_write_b16 %0, %1" ::"v"(addr), "v"(lo) : "memory");
                    if (nv > 1) asm volatile("ds_write_b16_d16_hi %0, %1 offset:2" ::"v"(addr), "v"(lo) : "memory");
                    if (nv > 2) asm volatile("ds_write_b16 %0, %1 offset:4" ::"v"(addr), "v"(hi) : "memory");
                }
            }
            if (!pending) break;
            if (++spins > kSpinLimit) {
                atomicOr(a.sync.err, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
#pragma unroll
            for (int u = 0; u < WPT; ++u)
                v[u] = (pending >> u) & 1u
                           ? __hip_atomic_load(xw + t + u * kPollT, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT)
                           : 0ull;
        }
    }
    __syncthreads();

    // ---- 6. down from LDS -------------------------------------------------------
    // Groups of RPW rows (one per TPD-lane segment of a wave) of one expert;
    // each wave takes a contiguous run of groups, so the blocks of its
    // expert's activations that its lanes need are read from LDS into
    // registers once per expert, not once per block.
    {
        constexpr int RPW = SEGD;
        const int segd = lane / TPD, tld = lane % TPD;
        const int rbd = fb * 16;
        const int shs = (r0 * fb) & 15, shb = (r0 * bsz) & 15;
        const int gpk = (nr + RPW - 1) / RPW;            // groups per expert
        const int ngroups = K * gpk;
        const int gpw = (ngroups + kDW - 1) / kDW;       // groups per wave
        const int g0 = wave * gpw, g1 = min(g0 + gpw, ngroups);
        int kx = -1;
        uint4 A[MD][4];
        // (k, group within expert) advanced per group: no division in the loop
        int k = g0 / gpk, qg = g0 - k * gpk;
        for (int g = g0; g < g1; ++g) {
            const int q = qg * RPW + segd;
            const bool valid = q < nr;
            const int qc = valid ? q : 0;
            const uint8_t *wrow = lds8 + L.dma + k * swt + qc * rbd;
            const uint8_t *srow = lds8 + L.dma + k * swt + sww + shs + qc * fb;
            // this group's weight blocks and scale bytes, all read before use
            u32x4 wv[MD];
            uint32_t sv[MD];
#pragma unroll
            for (int m = 0; m < MD; ++m) {
                const int cb = tld + m * TPD;
                const int cbc = valid && cb < fb ? cb : 0;
                wv[m] = *reinterpret_cast<const u32x4 *>(wrow + cbc * 16);
                sv[m] = srow[cbc];
            }
            if (k != kx) {                                // wave-uniform
                const uint32_t *xk = as + k * fb * 16;
#pragma unroll
                for (int m = 0; m < MD; ++m) {
                    const int cb = tld + m * TPD;
                    const uint4 *xv = reinterpret_cast<const uint4 *>(xk + (cb < fb ? cb : 0) * 16);
#pragma unroll
                    for (int qq = 0; qq < 4; ++qq) A[m][qq] = xv[qq];
                }
                kx = k;
            }
            float acc = 0.0f;
#pragma unroll
            for (int m = 0; m < MD; ++m) {
                const int cb = tld + m * TPD;
                const bool use = valid && cb < fb;
                WBlock<DT_F16> wb;
                widen_v(wv[m], wb);
                const float d = block_dot_r<DT_F16>(wb, A[m]) * decode_scale(sv[m]);
                acc += use ? d : 0.0f;
            }
            acc = seg_sum<TPD>(acc);
            if (valid && tld == 0) {
                float bias = 0.0f;
                if (a.bias_dt >= 0) {
                    const uint8_t *bp = lds8 + L.dma + k * swt + sww + sws + shb + q * bsz;
                    bias = a.bias_dt == DT_F32 ? *reinterpret_cast<const float *>(bp)
                                               : load_as_f32(bp, a.bias_dt, 0);
                }
                vals[k * a.nrmax + q] = acc + bias;
            }
            if (++qg == gpk) {
                qg = 0;
                ++k;
            }
        }
    }
    __syncthreads();

    // Combine in router order: dst += out_k * w_k, the product and the sum
    // rounded separately (expert_accumulate).  accumulate: 0 overwrite; 1 add
    // to out (applyAssignments); 2 out += the finished sum (the residual add
    // after the block, TransformerLayer.swift:232-238).
    for (int q = threadIdx.x; q < nr; q += kDT) {
        const int64_t o = r0 + q;
        float dst = a.accumulate == 1 ? a.out[o] : 0.0f;
        for (int k = 0; k < K; ++k) dst = add_scaled_rn(dst, vals[k * a.nrmax + q], ew[k]);
        if (a.accumulate == 2) dst = a.out[o] + dst;
        a.out[o] = dst;
        if (a.out_bf16) a.out_bf16[o] = f32_to_bf16_bits(dst);
    }
    if (threadIdx.x == 0) a.sync.epochs[b] = epoch1;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

namespace {

// Instantiations: GPT-OSS (hidden = intermediate = 2880: 90-block rows, up to
// top-4: 90 gate_up rows a workgroup on 256 CUs, three 32-row stages) and
// Qwen3-30B-A3B (2048 / 768: 64- and 24-block rows, up to top-8).
enum { kShapeGptOss = 0, kShapeQwen3 = 1 };
constexpr int kNdma[2] = {20, 10};   // 1 KiB pieces per DMA wave
// The first poll of the exchange waits this many ticks (10 ns) after the
// workgroup published, measured best on MI355X: about the spread of the
// grid's publish times (a round that comes too early costs a second memory
// round trip), and for GPT-OSS also the time its own down stream, queued
// ahead of the poll's loads, still takes to land.
constexpr int kPollDelay[2] = {140, 40};
// Words of a workgroup's exchange slot: GPT-OSS publishes up to 15 (45
// activations at top-4 on 256 CUs), Qwen3 8 (24 at top-8), so two Qwen3
// slots share a 128-byte line.  A poll's time follows the lines each compute
// unit reads, so the slots are packed to the power of two that holds them.
constexpr int kSlotWords[2] = {16, 8};
constexpr int kStagesG[2] = {6, 3};
constexpr int kRowsPerStage[2] = {kGuWaves * 64 / 16, kGuWaves * 64 / 16};

int shape_of(int hidden, int inter)
{
    const int hb = hidden / 32, fb = inter / 32;
    if (hidden % 32 || inter % 32) return -1;
    if (hb > 64 && hb <= 96 && fb > 64 && fb <= 96) return kShapeGptOss;
    if (hb > 24 && hb <= 64 && fb > 8 && fb <= 24) return kShapeQwen3;
    return -1;
}

// Calls f(kernel) with the instantiation for (shape, x dtype).
template <class F> void with_kernel(int shape, int x_dt, F &&f)
{
    if (shape == kShapeGptOss) {
        if (x_dt == DT_BF16) f(decode_layer_kernel<DT_BF16, DShape<16, 6>, kStagesG[kShapeGptOss], DShape<32, 3>, kNdma[kShapeGptOss], kPollDelay[kShapeGptOss], kSlotWords[kShapeGptOss]>);
        else f(decode_layer_kernel<DT_F16, DShape<16, 6>, kStagesG[kShapeGptOss], DShape<32, 3>, kNdma[kShapeGptOss], kPollDelay[kShapeGptOss], kSlotWords[kShapeGptOss]>);
    } else {
        if (x_dt == DT_BF16) f(decode_layer_kernel<DT_BF16, DShape<16, 4>, kStagesG[kShapeQwen3], DShape<8, 3>, kNdma[kShapeQwen3], kPollDelay[kShapeQwen3], kSlotWords[kShapeQwen3]>);
        else f(decode_layer_kernel<DT_F16, DShape<16, 4>, kStagesG[kShapeQwen3], DShape<8, 3>, kNdma[kShapeQwen3], kPollDelay[kShapeQwen3], kSlotWords[kShapeQwen3]>);
    }
}

}  // namespace

int decode_layer_plan(const Launch &L, int hidden, int inter, int x_dt, int top_k, int experts,
                      int64_t stride, int bias_dt, DecodeArgs *args, size_t *lds_bytes)
{
    const int shape = shape_of(hidden, inter);
    if (shape < 0 || (x_dt != DT_BF16 && x_dt != DT_F16)) return 0;
    if (top_k < 1 || top_k > kMaxTopK || experts > 256 || experts < top_k) return 0;
    if ((int64_t)experts * stride >= (int64_t)kOutOfRange) return 0;   // 32-bit buffer offsets
    const int G = L.cus;
    if (G <= 0 || G > kDecodeMaxGrid) return 0;
    // Each workgroup publishes at most 3 * XW activations.
    if (((int64_t)top_k * inter + G - 1) / G > 3 * kSlotWords[shape]) return 0;
    // Every workgroup's gate_up share must fit the register stages.
    const int rows_g = 2 * (int)(((int64_t)top_k * inter + G - 1) / G);
    if (rows_g > kStagesG[shape] * kRowsPerStage[shape]) return 0;
    const int nrmax = (hidden + G - 1) / G;
    const int bsz = bias_dt == DT_F32 ? 4 : bias_dt >= 0 ? 2 : 0;
    int sww, sws, swb;
    decode_windows(hidden, inter, nrmax, bsz, sww, sws, swb);
    const int swt = sww + sws + swb;
    const int chunks = (top_k * swt + kChunk - 1) / kChunk;
    if (chunks > kDmaWaves * kNdma[shape]) return 0;
    const DecodeLds l = decode_lds(hidden, inter, top_k, nrmax, swt,
                                   kStagesG[shape] * kRowsPerStage[shape]);
    if (l.total > kDecodeLdsMax) return 0;
    // The exchange needs the whole grid resident: one workgroup per CU.
    const void *fn = nullptr;
    with_kernel(shape, x_dt, [&](auto k) { fn = reinterpret_cast<const void *>(k); });
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
    with_kernel(shape, x_dt, [&](auto kernel) { GW_LAUNCH(kernel, dim3(grid), dim3(kDT), lds, L, a); });
    return hipGetLastError();
}

}  // namespace gw
