// gw_host.cpp — the library's host-only logic, plain C++ (no HIP): the
// error record, the .gwt manifest reader and the decode plan builder.  Kept
// apart from the HIP sources so that it also builds with g++ under the
// address and undefined-behaviour sanitizers (tests/test_host_sanitize.py).
#include "gw_host.h"

#include <cfloat>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "gw_error.h"

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------

static thread_local std::string g_error;

int gw::set_error(int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

extern "C" const char *gw_last_error(void) { return g_error.c_str(); }

namespace gw {

namespace {

// ---------------------------------------------------------------------------
// A small JSON reader: enough for manifest.json (objects, arrays, strings,
// numbers, true/false/null; \uXXXX escapes kept as '?').
// ---------------------------------------------------------------------------

struct Json {
    enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
    bool b = false;
    double num = 0.0;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;

    const Json *get(const char *key) const
    {
        if (kind != Obj) return nullptr;
        for (const auto &kv : obj)
            if (kv.first == key) return &kv.second;
        return nullptr;
    }
};

class JsonParser {
  public:
    JsonParser(const char *p, const char *end) : p_(p), end_(end) {}

    bool parse(Json &out)
    {
        if (!value(out, 0)) return false;
        ws();
        return p_ == end_;
    }
    const char *where() const { return p_; }

  private:
    const char *p_, *end_;

    void ws()
    {
        while (p_ < end_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
    }
    bool lit(const char *s)
    {
        const size_t n = strlen(s);
        if ((size_t)(end_ - p_) < n || strncmp(p_, s, n) != 0) return false;
        p_ += n;
        return true;
    }
    bool string(std::string &out)
    {
        if (p_ >= end_ || *p_ != '"') return false;
        ++p_;
        while (p_ < end_ && *p_ != '"') {
            if (*p_ == '\\') {
                if (++p_ >= end_) return false;
                const char c = *p_++;
                switch (c) {
                case 'n': out += '\n'; break;
                case 't': out += '\t'; break;
                case 'r': out += '\r'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'u':
                    if (end_ - p_ < 4) return false;
                    p_ += 4;
                    out += '?';
                    break;
                default: out += c; break;   // \" \\ \/
                }
            } else {
                out += *p_++;
            }
        }
        if (p_ >= end_) return false;
        ++p_;
        return true;
    }
    bool value(Json &v, int depth)
    {
        if (depth > 64) return false;
        ws();
        if (p_ >= end_) return false;
        const char c = *p_;
        if (c == '{') {
            v.kind = Json::Obj;
            ++p_;
            ws();
            if (p_ < end_ && *p_ == '}') { ++p_; return true; }
            for (;;) {
                ws();
                std::string key;
                if (!string(key)) return false;
                ws();
                if (p_ >= end_ || *p_ != ':') return false;
                ++p_;
                Json child;
                if (!value(child, depth + 1)) return false;
                v.obj.emplace_back(std::move(key), std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == '}') { ++p_; return true; }
                return false;
            }
        }
        if (c == '[') {
            v.kind = Json::Arr;
            ++p_;
            ws();
            if (p_ < end_ && *p_ == ']') { ++p_; return true; }
            for (;;) {
                Json child;
                if (!value(child, depth + 1)) return false;
                v.arr.push_back(std::move(child));
                ws();
                if (p_ < end_ && *p_ == ',') { ++p_; continue; }
                if (p_ < end_ && *p_ == ']') { ++p_; return true; }
                return false;
            }
        }
        if (c == '"') { v.kind = Json::Str; return string(v.str); }
        if (lit("true")) { v.kind = Json::Bool; v.b = true; return true; }
        if (lit("false")) { v.kind = Json::Bool; v.b = false; return true; }
        if (lit("null")) { v.kind = Json::Null; return true; }
        char *stop = nullptr;
        const std::string tok(p_, (size_t)std::min<ptrdiff_t>(end_ - p_, 64));
        v.num = strtod(tok.c_str(), &stop);
        if (stop == tok.c_str()) return false;
        v.kind = Json::Num;
        p_ += stop - tok.c_str();
        return true;
    }
};

const char *const kSectionNames[GW_SECTION_COUNT] = {"gate_up_blocks", "gate_up_scales",
                                                     "down_blocks",    "down_scales",
                                                     "gate_up_bias",   "down_bias"};

bool number_of(const Json &o, const char *key, double &out)
{
    const Json *v = o.get(key);
    if (!v || v->kind != Json::Num) return false;
    out = v->num;
    return true;
}

bool integer_of(const Json &o, const char *key, int64_t &out)
{
    double d;
    if (!number_of(o, key, d) || d != std::floor(d) || d < 0 || d > 9.0e15) return false;
    out = (int64_t)d;
    return true;
}

bool bool_or(const Json &o, const char *key, bool dflt)
{
    const Json *v = o.get(key);
    return v && v->kind == Json::Bool ? v->b : dflt;
}

bool finite_float(double d) { return std::fabs(d) <= (double)FLT_MAX; }   // false for NaN


}  // namespace

// Parses manifest.json (GodwitManifest, decoded as ModelReader.init does,
// ModelReader.swift:17-37): format version 2, layer/expert counts, the expert
// stride and sections, and the spec fields the MoE path needs (with the
// decoder's defaults for fields older installs lack, ArchitectureSpec.swift:
// 176-205).
int parse_manifest(const std::string &text, gw_model_info &info)
{
    Json root;
    JsonParser parser(text.data(), text.data() + text.size());
    if (!parser.parse(root) || root.kind != Json::Obj)
        return gw::set_error(GW_ERR_ARG, "manifest.json is not valid JSON (near byte %ld)",
                             (long)(parser.where() - text.data()));
    memset(&info, 0, sizeof(info));
    if (!integer_of(root, "formatVersion", info.format_version))
        return gw::set_error(GW_ERR_ARG, "manifest.json has no formatVersion");
    if (info.format_version != GW_GWT_FORMAT_VERSION)
        return gw::set_error(GW_ERR_ARG, "format v%lld, runtime expects v%d",
                             (long long)info.format_version, GW_GWT_FORMAT_VERSION);
    if (!integer_of(root, "layerCount", info.layer_count) ||
        !integer_of(root, "expertCount", info.expert_count) ||
        !integer_of(root, "expertStride", info.expert_stride) || info.expert_stride <= 0)
        return gw::set_error(GW_ERR_ARG,
                             "manifest.json lacks layerCount, expertCount or expertStride");
    // Bounds that keep every derived size (stride x experts, per-layer file
    // handles) representable: far above any real install.
    if (info.layer_count > kMaxLayers || info.expert_count > kMaxExpertsPerLayer ||
        info.expert_stride > kMaxExpertStride)
        return gw::set_error(GW_ERR_ARG,
                             "manifest.json counts out of range (layers %lld, experts %lld, "
                             "stride %lld)", (long long)info.layer_count,
                             (long long)info.expert_count, (long long)info.expert_stride);
    const Json *secs = root.get("expertSections");
    if (!secs || secs->kind != Json::Obj)
        return gw::set_error(GW_ERR_ARG, "manifest.json has no expertSections");
    for (int s = 0; s < GW_SECTION_COUNT; ++s) {
        const Json *span = secs->get(kSectionNames[s]);
        if (!span || !integer_of(*span, "offset", info.section_offset[s]) ||
            !integer_of(*span, "length", info.section_length[s]))
            return gw::set_error(GW_ERR_ARG, "manifest has no section '%s'", kSectionNames[s]);
        if (info.section_offset[s] + info.section_length[s] > info.expert_stride)
            return gw::set_error(GW_ERR_ARG, "section '%s' ends past the expert stride",
                                 kSectionNames[s]);
    }
    const Json *spec = root.get("spec");
    if (!spec || spec->kind != Json::Obj)
        return gw::set_error(GW_ERR_ARG, "manifest.json has no spec");
    double eps = 0.0;
    if (!integer_of(*spec, "hiddenSize", info.hidden_size) ||
        !integer_of(*spec, "intermediateSize", info.intermediate_size) ||
        !number_of(*spec, "rmsNormEpsilon", eps))
        return gw::set_error(GW_ERR_ARG, "spec lacks hiddenSize, intermediateSize or rmsNormEpsilon");
    if (!finite_float(eps))
        return gw::set_error(GW_ERR_ARG, "spec rmsNormEpsilon is not a finite fp32 value");
    info.rms_norm_epsilon = (float)eps;
    const Json *act = spec->get("activation");
    if (!act || act->kind != Json::Str)
        return gw::set_error(GW_ERR_ARG, "spec has no activation");
    if (act->str == "gptOssClampedGLU") info.activation = GW_ACT_GPTOSS_CLAMPED_GLU;
    else if (act->str == "silu") info.activation = GW_ACT_SILU;
    else return gw::set_error(GW_ERR_SHAPE, "expert activation '%s' is not supported", act->str.c_str());
    double lim = 7.0, alpha = 1.702;
    number_of(*spec, "activationLimit", lim);
    number_of(*spec, "activationAlpha", alpha);
    if (!finite_float(lim) || !finite_float(alpha))
        return gw::set_error(GW_ERR_ARG, "spec activationLimit / activationAlpha out of range");
    info.activation_limit = (float)lim;
    info.activation_alpha = (float)alpha;
    info.expert_bias = bool_or(*spec, "expertBias", false) ? 1 : 0;
    info.router_bias = bool_or(*spec, "routerBias", false) ? 1 : 0;
    info.experts_per_token = 0;
    if (const Json *layers = spec->get("layers"); layers && layers->kind == Json::Arr)
        for (const Json &l : layers->arr) {
            int64_t k = 0;
            if (integer_of(l, "expertsPerToken", k) && k > info.experts_per_token)
                info.experts_per_token = k;
        }
    return GW_OK;
}


// ---------------------------------------------------------------------------
// decode plans
// ---------------------------------------------------------------------------

bool same_weights(const gw_expert_weights *a, const gw_expert_weights *b)
{
    if (a->buffer != b->buffer) return false;
    for (int s = 0; s < GW_SECTION_COUNT; ++s)
        if (a->offsets[s] != b->offsets[s]) return false;
    return true;
}

// Adds (weights, token, w) to the plan being built; returns false if it does
// not fit (the caller flushes and retries on an empty plan).
bool plan_add(HostPlan &hp, const gw_expert_weights *w, int32_t token, float weight,
                     bool merge)
{
    Plan &p = hp.p;
    if (p.nslots >= kMaxSlots) return false;
    int local = -1;
    for (int t = 0; t < p.ntokens; ++t)
        if (p.tok_global[t] == token) local = t;
    if (local < 0) {
        if (p.ntokens >= kMaxTokens) return false;
        local = p.ntokens;
        p.tok_global[local] = token;
        p.tok_nslots[local] = 0;
        p.ntokens += 1;
    }
    if (p.tok_nslots[local] >= kMaxTopK) return false;
    int g = -1;
    if (merge) {
        for (int k = 0; k < p.ngroups; ++k) {
            if (!same_weights(hp.group_w[k], w)) continue;
            bool has = false;   // a group holds each token at most once
            for (int s = 0; s < p.nslots; ++s)
                if (p.slot_group[s] == k && p.slot_token[s] == local) has = true;
            if (!has) { g = k; break; }
        }
    }
    if (g < 0) {
        g = p.ngroups++;
        hp.group_w[g] = w;
        p.group_ntok[g] = 0;
    }
    const int s = p.nslots++;
    p.slot_token[s] = local;
    p.slot_group[s] = g;
    p.slot_weight[s] = weight;
    p.group_ntok[g] += 1;
    if (p.group_ntok[g] > hp.max_group_tokens) hp.max_group_tokens = p.group_ntok[g];
    p.tok_slots[local][p.tok_nslots[local]++] = s;
    return true;
}

// Renumbers a built plan's slots group-major (the kernels' convention): slots
// were appended in assignment order; each group's slots become contiguous,
// and every token's slot list follows them.
void plan_regroup(const HostPlan &hp, Plan &q)
{
    const Plan &p = hp.p;
    q = p;
    int next = 0;
    int remap[kMaxSlots];
    for (int g = 0; g < p.ngroups; ++g) {
        q.group_slot0[g] = next;
        int k = 0;
        for (int s = 0; s < p.nslots; ++s) {
            if (p.slot_group[s] != g) continue;
            remap[s] = next;
            q.slot_token[next] = p.slot_token[s];
            q.slot_group[next] = g;
            q.slot_weight[next] = p.slot_weight[s];
            ++next;
            ++k;
        }
        q.group_ntok[g] = k;
    }
    for (int t = 0; t < p.ntokens; ++t)
        for (int k = 0; k < p.tok_nslots[t]; ++k) q.tok_slots[t][k] = remap[p.tok_slots[t][k]];
    for (int g = 0; g < p.ngroups; ++g) q.group_base[g] = hp.group_w[g]->buffer;
}

}  // namespace gw
