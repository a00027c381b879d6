// Host-side fuzz driver for the library's plain-C++ logic (gw_host.cpp): the
// .gwt manifest reader and the decode plan builder.  Built with g++ under
// -fsanitize=address,undefined by tests/test_host_sanitize.py; any memory
// error, leak, undefined behaviour or broken invariant ends the run with a
// non-zero status.  No GPU, no HIP.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "gw_host.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint32_t next_u32()
{
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return (uint32_t)(g_state >> 11);
}

#define REQUIRE(c)                                                                   \
    do {                                                                             \
        if (!(c)) {                                                                  \
            fprintf(stderr, "invariant failed at %s:%d: %s\n", __FILE__, __LINE__, #c); \
            exit(3);                                                                 \
        }                                                                            \
    } while (0)

static const char *kValid =
    "{\"formatVersion\": 2, \"layerCount\": 36, \"expertCount\": 128,"
    " \"expertStride\": 13287424,"
    " \"expertSections\": {"
    "  \"gate_up_blocks\": {\"offset\": 0, \"length\": 8294400},"
    "  \"gate_up_scales\": {\"offset\": 8306688, \"length\": 518400},"
    "  \"down_blocks\": {\"offset\": 8830976, \"length\": 4147200},"
    "  \"down_scales\": {\"offset\": 12984320, \"length\": 259200},"
    "  \"gate_up_bias\": {\"offset\": 13254656, \"length\": 11520},"
    "  \"down_bias\": {\"offset\": 13271040, \"length\": 5760}},"
    " \"spec\": {\"hiddenSize\": 2880, \"intermediateSize\": 2880,"
    "  \"rmsNormEpsilon\": 1e-05, \"activation\": \"gptOssClampedGLU\","
    "  \"activationLimit\": 7.0, \"activationAlpha\": 1.702, \"expertBias\": true,"
    "  \"layers\": [{\"expertsPerToken\": 4}, {\"expertsPerToken\": 4}],"
    "  \"name\": \"caf\\u00e9 \\\"quoted\\\" \\\\ \\/\"}}";

static int parse(const std::string &text)
{
    gw_model_info info;
    const int rc = gw::parse_manifest(text, info);
    REQUIRE(rc >= GW_OK && rc <= GW_ERR_UNSUPPORTED);
    REQUIRE(rc != GW_OK || (info.layer_count <= gw::kMaxLayers &&
                            info.expert_count <= gw::kMaxExpertsPerLayer &&
                            info.expert_stride > 0 && info.expert_stride <= gw::kMaxExpertStride));
    if (rc == GW_OK)
        for (int s = 0; s < GW_SECTION_COUNT; ++s)
            REQUIRE(info.section_offset[s] + info.section_length[s] <= info.expert_stride);
    return rc;
}

static void fuzz_manifest()
{
    const std::string valid = kValid;
    {
        gw_model_info info;
        REQUIRE(gw::parse_manifest(valid, info) == GW_OK);
        REQUIRE(info.layer_count == 36 && info.expert_count == 128 && info.hidden_size == 2880);
        REQUIRE(info.experts_per_token == 4 && info.expert_bias == 1);
    }
    // Every truncation is malformed.
    for (size_t n = 0; n < valid.size(); ++n) REQUIRE(parse(valid.substr(0, n)) != GW_OK);
    // Seeded mutations: byte flips, insertions, deletions, digit bursts.
    const char alphabet[] = "{}[]\":,-+.eE0123456789 \\u\ttruefalsenull";
    for (int it = 0; it < 20000; ++it) {
        std::string t = valid;
        const int edits = 1 + (int)(next_u32() % 8);
        for (int e = 0; e < edits && !t.empty(); ++e) {
            const size_t at = next_u32() % t.size();
            switch (next_u32() % 5) {
            case 0: t[at] = (char)(next_u32() & 0xFF); break;
            case 1: t.insert(at, 1, alphabet[next_u32() % (sizeof(alphabet) - 1)]); break;
            case 2: t.erase(at, 1 + next_u32() % 16); break;
            case 3: t.insert(at, std::string(1 + next_u32() % 40, '9')); break;
            default: t.insert(at, "1e999"); break;
            }
        }
        parse(t);
    }
    // Structural extremes.
    REQUIRE(parse(std::string(200000, '[')) != GW_OK);          // nesting past the depth bound
    REQUIRE(parse(std::string(200000, '{')) != GW_OK);
    REQUIRE(parse("\"" + std::string(100000, 'a')) != GW_OK);   // unterminated string
    REQUIRE(parse("{\"a\": \"\\u12") != GW_OK);                 // escape cut short
    REQUIRE(parse("{\"a\": \"\\") != GW_OK);
    REQUIRE(parse(std::string("{\"formatVersion\": 2\0}", 21)) != GW_OK);
    const char *subs[][2] = {
        {"\"layerCount\": 36", "\"layerCount\": 1e300"},
        {"\"layerCount\": 36", "\"layerCount\": 100000"},
        {"\"layerCount\": 36", "\"layerCount\": -1"},
        {"\"expertCount\": 128", "\"expertCount\": 9007199254740991"},
        {"\"expertStride\": 13287424", "\"expertStride\": 0"},
        {"\"expertStride\": 13287424", "\"expertStride\": 1.5"},
        {"\"expertStride\": 13287424", "\"expertStride\": 8999999999999999"},
        {"\"length\": 5760}", "\"length\": 8999999999999999}"},
        {"\"rmsNormEpsilon\": 1e-05", "\"rmsNormEpsilon\": 1e300"},
        {"\"activationLimit\": 7.0", "\"activationLimit\": -1e39"},
        {"\"activationAlpha\": 1.702", "\"activationAlpha\": nan"},
        {"\"formatVersion\": 2", "\"formatVersion\": 3"},
        {"\"gptOssClampedGLU\"", "\"gelu\""},
        {"\"layers\": [", "\"layers\": [1, \"x\", null, "},
    };
    for (auto &sub : subs) {
        std::string t = valid;
        const size_t at = t.find(sub[0]);
        REQUIRE(at != std::string::npos);
        t.replace(at, strlen(sub[0]), sub[1]);
        const int rc = parse(t);
        // only the malformed `layers` entries are tolerated (they are skipped)
        REQUIRE((rc == GW_OK) == (strcmp(sub[0], "\"layers\": [") == 0));
    }
}

static void fuzz_plans()
{
    static uint8_t pool[8][64];
    gw_expert_weights w[8];
    for (int i = 0; i < 8; ++i) {
        w[i].buffer = pool[i];
        for (int s = 0; s < GW_SECTION_COUNT; ++s) w[i].offsets[s] = 16 * s * (1 + (i & 1));
    }
    for (int it = 0; it < 20000; ++it) {
        gw::HostPlan hp;
        hp.clear();
        const bool merge = next_u32() & 1;
        const int n = (int)(next_u32() % 200);
        int added = 0;
        for (int i = 0; i < n; ++i) {
            const gw_expert_weights *x = &w[next_u32() % 8];
            const int32_t token = (int32_t)(next_u32() % 12);
            if (!gw::plan_add(hp, x, token, 0.25f, merge)) break;
            ++added;
        }
        const gw::Plan &p = hp.p;
        REQUIRE(p.nslots == added && p.nslots <= gw::kMaxSlots);
        REQUIRE(p.ntokens <= gw::kMaxTokens && p.ngroups <= p.nslots);
        gw::Plan q;
        gw::plan_regroup(hp, q);
        int total = 0;
        for (int g = 0; g < q.ngroups; ++g) {
            REQUIRE(q.group_slot0[g] == total);
            for (int k = 0; k < q.group_ntok[g]; ++k) REQUIRE(q.slot_group[total + k] == g);
            total += q.group_ntok[g];
            REQUIRE(q.group_base[g] != nullptr);
        }
        REQUIRE(total == q.nslots);
        for (int t = 0; t < q.ntokens; ++t) {
            REQUIRE(q.tok_nslots[t] <= gw::kMaxTopK);
            for (int k = 0; k < q.tok_nslots[t]; ++k) {
                const int s = q.tok_slots[t][k];
                REQUIRE(s >= 0 && s < q.nslots && q.slot_token[s] == t);
            }
        }
    }
}

int main()
{
    fuzz_manifest();
    fuzz_plans();
    printf("host fuzz: ok\n");
    return 0;
}
