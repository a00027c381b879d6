// gw_route.h — wave-level routing (Router.select, Router.swift:78-98, and the
// demand map of TransformerLayer.swift:175-181) shared by the decode and
// prefill kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gw_device.h"
#include "gw_plan.h"

namespace gw {

// ---------------------------------------------------------------------------
// Routing by one wave (Router.select, Router.swift:78-98, plus the demand map
// of TransformerLayer.swift:175-181), register resident.
//
// select_exact follows the selection sort's permutation in registers: lane l
// holds elements l, l+64, ... (R per lane) with their current positions.  At
// position p the reference keeps the first position >= p holding the largest
// logit (strict `>` scan), or p itself when logits[order[p]] is NaN; positions
// are swapped exactly as `order.swapAt(p, best)` does, so ties resolve as in
// the reference.  select_fast gives the same result in far fewer instructions
// when there is no NaN and no tie among the ranks it picks, and hands over to
// select_exact otherwise.
// ---------------------------------------------------------------------------

// Float -> unsigned key with the same order; 0 is reserved for "no candidate"
// (NaN and out-of-range positions never win, as `>` never picks them).
__device__ __forceinline__ uint32_t order_key(float v)
{
    const uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);   // -0 and +0 compare equal
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave-wide max / min left in every lane, entirely in VALU: DPP-combined
// steps inside each 16-lane row, then v_permlane16_swap / v_permlane32_swap
// exchange rows and halves (gfx950), so no value goes through an SGPR.
#define GW_DPPC(x, ctrl) ((uint32_t)__builtin_amdgcn_mov_dpp((int)(x), (ctrl), 0xF, 0xF, true))
__device__ __forceinline__ uint32_t wave_allmax_u32(uint32_t x)
{
    x = max(x, GW_DPPC(x, 0xB1));
    x = max(x, GW_DPPC(x, 0x4E));
    x = max(x, GW_DPPC(x, 0x141));
    x = max(x, GW_DPPC(x, 0x140));
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = max(p[0], p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return max(q[0], q[1]);
}
__device__ __forceinline__ uint32_t wave_allmin_u32(uint32_t x)
{
    x = min(x, GW_DPPC(x, 0xB1));
    x = min(x, GW_DPPC(x, 0x4E));
    x = min(x, GW_DPPC(x, 0x141));
    x = min(x, GW_DPPC(x, 0x140));
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = min(p[0], p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return min(q[0], q[1]);
}
#undef GW_DPPC

__device__ __forceinline__ float lane_value(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}


// Routing of ONE token by one wave, branch-free: Router.select's selection
// sort (Router.swift:78-98) tracked per element instead of per position.
// Lane l holds elements l, l+64, ... (R per lane) with their current position
// in the sort's permutation.  Step p picks the largest logit among unselected
// elements, the smallest current position among ties (the strict `>` scan
// from p keeps the first), or the element at p itself when its logit is NaN
// (nothing compares greater than NaN); then it swaps positions exactly as
// `order.swapAt(p, best)`.  The plan is the single-token demand map: group,
// slot and rank k are the k-th selected expert.
// On return lane k < K holds the expert of rank k in sid_out and its logit in
// sv_out (lanes >= K hold unspecified values).
template <int R>
__device__ __forceinline__ void select_exact(const float *__restrict__ logits, int E, int K,
                                             int &sid_out, float &sv_out)
{
    const int lane = threadIdx.x & 63;
    float v[R];
    uint32_t cp[R];
    bool sel[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = lane + 64 * r;
        v[r] = logits[min(i, E - 1)];
        cp[r] = (uint32_t)i;
        sel[r] = i >= E;            // elements past E never take part
    }
    int sid = 0;                    // lane k < K: expert of rank k
    float sv = 0.0f;                // and its logit
    for (int pos = 0; pos < K; ++pos) {
        uint32_t key[R];
        uint32_t km = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            key[r] = (sel[r] || __builtin_isnan(v[r])) ? 0u : order_key(v[r]);
            km = max(km, key[r]);
        }
        const uint32_t kmax = wave_allmax_u32(km);
        int nhit = 0;
        uint32_t hcp = 0;
        bool nan_here = false;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool hit = kmax != 0u && key[r] == kmax;
            nhit += hit ? 1 : 0;
            hcp = hit ? cp[r] : hcp;
            nan_here |= !sel[r] && cp[r] == (uint32_t)pos && __builtin_isnan(v[r]);
        }
        // Usually one element holds the maximum: its position is read from its
        // lane.  Ties (several holders) take the smallest current position.
        const unsigned long long hits = __ballot(nhit != 0);
        const bool tie = __popcll(hits) > 1 || __ballot(nhit > 1) != 0ull;
        uint32_t pmin = 0xFFFFFFFFu;
        if (hits != 0ull && !tie) {
            pmin = (uint32_t)__builtin_amdgcn_readlane((int)hcp, (int)__builtin_ctzll(hits));
        } else if (tie) {
            uint32_t pm = 0xFFFFFFFFu;
#pragma unroll
            for (int r = 0; r < R; ++r) pm = (kmax != 0u && key[r] == kmax) ? min(pm, cp[r]) : pm;
            pmin = wave_allmin_u32(pm);
        }
        const bool nan_at_pos = __ballot(nan_here) != 0ull;
        const uint32_t best = (pmin == 0xFFFFFFFFu || nan_at_pos) ? (uint32_t)pos : pmin;
        int my_id = 0;
        float my_v = 0.0f;
        bool mine = false;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool at_best = !sel[r] && cp[r] == best;
            const bool at_pos = !sel[r] && cp[r] == (uint32_t)pos;
            my_id = at_best ? lane + 64 * r : my_id;
            my_v = at_best ? v[r] : my_v;
            mine |= at_best;
            cp[r] = at_best ? (uint32_t)pos : (at_pos ? best : cp[r]);
            sel[r] = sel[r] || at_best;
        }
        const int src = (int)__builtin_ctzll(__ballot(mine));
        const int id = __builtin_amdgcn_readlane(my_id, src);
        const float val = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), src));
        sid = lane == pos ? id : sid;
        sv = lane == pos ? val : sv;
    }
    sid_out = sid;
    sv_out = sv;
}

// The common case in a few instructions per rank: when no logit is NaN and
// each of the K largest keys is held by one element only, the selection sort
// picks those elements in descending order whatever its permutation holds, so
// K wave-wide maxima give exactly its result.  A NaN, or a rank whose maximum
// two elements share (a tie, -0 and +0 included), returns false and the
// caller runs select_exact instead.  Same outputs as select_exact for the
// first `npass` ranks (npass <= K; lanes >= npass hold unspecified values).
template <int R>
__device__ __forceinline__ bool select_fast(const float *__restrict__ logits, int E, int npass,
                                            int &sid_out, float &sv_out)
{
    const int lane = threadIdx.x & 63;
    float v[R];
    uint32_t key[R];
    bool nan = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = lane + 64 * r;
        v[r] = logits[min(i, E - 1)];
        const bool in = i < E;
        nan |= in && __builtin_isnan(v[r]);
        key[r] = in && !__builtin_isnan(v[r]) ? order_key(v[r]) : 0u;
    }
    if (__ballot(nan) != 0ull) return false;
    int sid = 0;
    float sv = 0.0f;
    for (int pos = 0; pos < npass; ++pos) {
        uint32_t km = key[0];
#pragma unroll
        for (int r = 1; r < R; ++r) km = max(km, key[r]);
        const uint32_t kmax = wave_allmax_u32(km);
        int count = 0, id = -1;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const unsigned long long b = __ballot(key[r] == kmax);
            count += __popcll(b);
            if (id < 0 && b != 0ull) id = 64 * r + (int)__builtin_ctzll(b);
        }
        if (count != 1 || kmax == 0u) return false;
        const int src = id & 63, rs = id >> 6;
        float val = lane_value(v[0], src);
#pragma unroll
        for (int r = 1; r < R; ++r) val = rs == r ? lane_value(v[r], src) : val;
#pragma unroll
        for (int r = 0; r < R; ++r) key[r] = lane + 64 * r == id ? 0u : key[r];
        sid = lane == pos ? id : sid;
        sv = lane == pos ? val : sv;
    }
    sid_out = sid;
    sv_out = sv;
    return true;
}

// Softmax over the K selected logits held by lanes 0..K-1 in rank order
// (Router.swift:92-96): the peak subtracted, exponentials summed in rank
// order.  Returns lane k's weight (lanes >= K: unspecified).
__device__ __forceinline__ float softmax_ranked(float sv, int K)
{
    float peak = lane_value(sv, 0);
    for (int i = 1; i < K; ++i) {
        const float x = lane_value(sv, i);
        peak = x > peak ? x : peak;
    }
    const float ex = expf(sv - peak);
    float total = 0.0f;
    for (int i = 0; i < K; ++i) total += lane_value(ex, i);
    return ex / total;
}

// Top-K of one token's logits by one wave, then the softmax over the K
// selected (Router.select, Router.swift:78-98).  On return lane k < K holds
// the expert of rank k in sid_out and its softmax weight in w_out (lanes >= K
// hold unspecified values).
template <int R>
__device__ __forceinline__ void select_one(const float *__restrict__ logits, int E, int K,
                                           int &sid_out, float &w_out)
{
    int sid;
    float sv;
    if (!select_fast<R>(logits, E, K, sid, sv)) select_exact<R>(logits, E, K, sid, sv);
    sid_out = sid;
    w_out = softmax_ranked(sv, K);
}

// Routing of T tokens by one wave (select_one per token) and the demand map
// of TransformerLayer.swift:175-181: entries grouped by expert in order of
// first appearance, each group's tokens in token order.
template <int R>
__device__ __forceinline__ void route_wave(const float *__restrict__ logits, int E, int K,
                                           int T, const uint8_t *experts_base, int64_t stride,
                                           Plan *plan, int32_t *ids_out, float *w_out)
{
    const int lane = threadIdx.x & 63;
    int my_e = -1;
    float my_w = 0.0f;
    for (int t = 0; t < T; ++t) {
        int sid;
        float w;
        select_one<R>(logits + (int64_t)t * E, E, K, sid, w);
        const int src = lane - t * K;
        const bool mine = src >= 0 && src < K;
        int e_src = 0;
        float w_src = 0.0f;
        for (int i = 0; i < K; ++i) {   // entry (t, i) moves to lane t*K + i
            const int ei = __builtin_amdgcn_readlane(sid, i);
            const float wi = lane_value(w, i);
            if (src == i) {
                e_src = ei;
                w_src = wi;
            }
        }
        if (mine) {
            my_e = e_src;
            my_w = w_src;
        }
        if (ids_out && lane < K) ids_out[(int64_t)t * K + lane] = sid;
        if (w_out && lane < K) w_out[(int64_t)t * K + lane] = w;
    }

    // Expert-major grouping of the T*K (token, rank) entries by first appearance.
    const int n = T * K;
    int first = -1, before = 0, same = 0;
    for (int j = 0; j < n; ++j) {
        const int ej = __builtin_amdgcn_readlane(my_e, j);
        if (lane < n && ej == my_e) {
            if (first < 0) first = j;
            if (j < lane) ++before;
            ++same;
        }
    }
    const bool leader = lane < n && first == lane;
    const unsigned long long leaders = __ballot(leader);
    int slot0 = 0;
    for (int j = 0; j < n; ++j) {
        const int fj = __builtin_amdgcn_readlane(first, j);
        if (lane < n && fj < first) ++slot0;
    }
    if (lane < n) {
        const int gi = __popcll(leaders & ((1ull << first) - 1ull));
        const int slot = slot0 + before;
        const int t = lane / K, r = lane - (lane / K) * K;
        plan->slot_token[slot] = t;
        plan->slot_group[slot] = gi;
        plan->slot_weight[slot] = my_w;
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

// One token's plan.  `need` ranks are enough for a caller that only streams
// the rows of experts of rank < need (a gate_up workgroup's slice): it stops
// the selection there and skips the softmax, and the plan's other ranks and
// weights stay unspecified.  need >= K gives the whole plan with weights.
template <int R>
__device__ __forceinline__ void route_one(const float *__restrict__ logits, int E, int K,
                                          const uint8_t *experts_base, int64_t stride,
                                          Plan *plan, int32_t *ids_out, float *w_out,
                                          int need = 1 << 30)
{
    const int lane = threadIdx.x & 63;
    int sid;
    float w = 0.0f;
    if (need >= K) {
        select_one<R>(logits, E, K, sid, w);
    } else {
        float sv;
        if (!select_fast<R>(logits, E, need, sid, sv)) select_exact<R>(logits, E, K, sid, sv);
    }
    if (lane < K) {
        if (ids_out) ids_out[lane] = sid;
        if (w_out) w_out[lane] = w;
        plan->group_base[lane] = experts_base + (int64_t)sid * stride;
        plan->group_slot0[lane] = lane;
        plan->group_ntok[lane] = 1;
        plan->slot_token[lane] = 0;
        plan->slot_group[lane] = lane;
        plan->slot_weight[lane] = w;
        plan->tok_slots[0][lane] = lane;
    }
    if (lane == 0) {
        plan->tok_global[0] = 0;
        plan->tok_nslots[0] = K;
        plan->ngroups = K;
        plan->nslots = K;
        plan->ntokens = 1;
        plan->pad0 = 0;
    }
}


}  // namespace gw
