// gw_plan.h — the routing plan shared by host code and the decode kernels.
//
// A plan is the device-side form of TransformerLayer's demand map
// (Sources/Godwit/Runtime/TransformerLayer.swift:175-181): the unique experts
// of one call ("groups", in first-appearance order), the (group, token) pairs
// that need them ("slots", numbered group-major), and for each token the
// ordered list of its slots, which fixes the order of the weighted combine
// (dst += out * w, expert.metal:107-116).
#pragma once
#include <stdint.h>

namespace gw {

constexpr int kMaxTokens = 8;               // decode tokens per plan
constexpr int kMaxTopK = 8;                 // slots per token per plan
constexpr int kMaxSlots = kMaxTokens * kMaxTopK;

struct Plan {
    int32_t ngroups;
    int32_t nslots;
    int32_t ntokens;
    int32_t pad0;
    int32_t tok_global[kMaxTokens];         // row of inputs/outputs for local token t
    int32_t tok_nslots[kMaxTokens];
    int32_t tok_slots[kMaxTokens][kMaxTopK];
    const uint8_t *group_base[kMaxSlots];   // expert stride base (sections at runner offsets)
    int32_t group_slot0[kMaxSlots];
    int32_t group_ntok[kMaxSlots];
    int32_t slot_token[kMaxSlots];          // local token of each slot
    int32_t slot_group[kMaxSlots];
    float slot_weight[kMaxSlots];
};

// Section byte offsets within an expert stride, passed by value to kernels.
struct Sections {
    int64_t gu_blocks, gu_scales, dn_blocks, dn_scales, gu_bias, dn_bias;
};

// Router logits of one token by slices (router_partial in gw_device.h).
constexpr int kRouterUnits = 4;        // 8-element units a lane, per slice
constexpr int kRouterMaxSlices = 16;   // a standalone workgroup's waves

// S for E experts of width H over `waves` waves (waves / E when that divides
// evenly, into at most 16 slices of whole 8-element units, at most
// kRouterUnits a lane), else 0.
#if defined(__HIPCC__)
__host__ __device__
#endif
inline int router_slices(int experts, int hidden, int waves)
{
    if (experts <= 0 || waves % experts != 0) return 0;
    const int S = waves / experts;
    if (S < 1 || S > kRouterMaxSlices || hidden % S != 0) return 0;
    const int L = hidden / S;
    return L % 8 == 0 && L <= 64 * 8 * kRouterUnits ? S : 0;
}

}  // namespace gw
