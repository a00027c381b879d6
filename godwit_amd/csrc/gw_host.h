// gw_host.h — host-only pieces of the library in plain C++ (gw_host.cpp):
// the .gwt manifest reader and the decode plan builder, kept free of HIP so
// that they also build and run under the host sanitizers.
#pragma once
#include <stdint.h>

#include <string>

#include "../../include/godwit_hip.h"
#include "gw_plan.h"

namespace gw {

// Manifest bounds: far above any real install, low enough that every derived
// size (stride x experts, one file handle per layer) is representable.
constexpr int64_t kMaxLayers = 4096;
constexpr int64_t kMaxExpertsPerLayer = 1 << 20;
constexpr int64_t kMaxExpertStride = (int64_t)1 << 40;

// Parses manifest.json text into `info`; GW_OK, or an error status with the
// message recorded for gw_last_error().
int parse_manifest(const std::string &text, gw_model_info &info);

// A host-built plan: expert-major groups over assignments, in order.
struct HostPlan {
    Plan p;
    const gw_expert_weights *group_w[kMaxSlots];
    int max_group_tokens = 0;
    void clear()
    {
        p = Plan();
        max_group_tokens = 0;
    }
};

bool same_weights(const gw_expert_weights *a, const gw_expert_weights *b);
// Adds (weights, token, weight) to the plan; false when it does not fit (the
// caller runs the plan and starts an empty one).  merge: an assignment joins
// an existing group of the same weights that does not yet hold its token.
bool plan_add(HostPlan &hp, const gw_expert_weights *w, int32_t token, float weight,
              bool merge);
// The plan with its slots renumbered group-major, as the kernels read it.
void plan_regroup(const HostPlan &hp, Plan &q);

}  // namespace gw
