// gw_model.hip — a .gwt installation read into HBM: the manifest
// (GodwitManifest, Install/GodwitManifest.swift:8-105) and the expert layer
// files (ModelReader, Runtime/ModelReader.swift:11-111), without Metal's
// shared-memory buffers: files are read with pread into pinned staging
// buffers and copied to device memory by the context's stream, two buffers
// alternating so the next read overlaps the previous copy.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fcntl.h>
#include <string>
#include <sys/stat.h>
#include <unistd.h>
#include <utility>
#include <vector>

#include "../../include/godwit_hip.h"
#include "gw_error.h"
#include "gw_host.h"


struct gw_model {
    std::string dir;
    gw_model_info info;
    std::vector<int> fds;   // per layer, opened on first use (-1: not yet)
    // Two pinned staging buffers of kStageBytes for read_to_device, allocated
    // on the first load and kept until gw_model_close (pinning is slow).
    void *stage[2] = {nullptr, nullptr};
};

static constexpr size_t kStageBytes = (size_t)32 << 20;

static std::string layer_path(const gw_model *m, int layer)
{
    char name[32];
    snprintf(name, sizeof(name), "layer_%02d.bin", layer);
    return m->dir + "/experts/" + name;
}

extern "C" int gw_model_open(const char *directory, gw_model **out)
{
    if (!directory || !out) return gw::set_error(GW_ERR_ARG, "null argument");
    *out = nullptr;
    const std::string dir = directory;
    const std::string mpath = dir + "/manifest.json";
    struct stat st;
    if (stat(mpath.c_str(), &st) != 0) {
        if (stat(directory, &st) == 0)
            return gw::set_error(GW_ERR_ARG,
                                 "%s has no manifest.json — not a .gwt install, or an install "
                                 "that did not finish", directory);
        return gw::set_error(GW_ERR_ARG, "no such directory: %s", directory);
    }
    FILE *f = fopen(mpath.c_str(), "rb");
    if (!f) return gw::set_error(GW_ERR_ARG, "could not open %s: %s", mpath.c_str(), strerror(errno));
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), f)) > 0) text.append(buf, n);
    fclose(f);
    gw_model *m = new gw_model;
    m->dir = dir;
    const int rc = gw::parse_manifest(text, m->info);
    if (rc != GW_OK) {
        delete m;
        return rc;
    }
    m->fds.assign((size_t)m->info.layer_count, -1);
    *out = m;
    return GW_OK;
}

extern "C" int gw_model_close(gw_model *m)
{
    if (!m) return GW_OK;
    for (int fd : m->fds)
        if (fd >= 0) close(fd);
    for (void *p : m->stage)
        if (p) (void)hipHostFree(p);
    delete m;
    return GW_OK;
}

extern "C" int gw_model_info_get(const gw_model *m, gw_model_info *info)
{
    if (!m || !info) return gw::set_error(GW_ERR_ARG, "null argument");
    *info = m->info;
    return GW_OK;
}

// GodwitManifest.validate (GodwitManifest.swift:79-104): every layer file is
// exactly expertStride * expertCount bytes.
extern "C" int gw_model_validate(const gw_model *m)
{
    if (!m) return gw::set_error(GW_ERR_ARG, "null argument");
    const int64_t expected = m->info.expert_stride * m->info.expert_count;
    for (int l = 0; l < (int)m->info.layer_count; ++l) {
        struct stat st;
        const std::string p = layer_path(m, l);
        if (stat(p.c_str(), &st) != 0)
            return gw::set_error(GW_ERR_ARG, "layer %d file is unreadable", l);
        if ((int64_t)st.st_size != expected)
            return gw::set_error(GW_ERR_ARG, "layer %d is %lld bytes, expected %lld", l,
                                 (long long)st.st_size, (long long)expected);
    }
    return GW_OK;
}

static int layer_fd(gw_model *m, int layer, int &fd)
{
    if (layer < 0 || layer >= (int)m->info.layer_count)
        return gw::set_error(GW_ERR_ARG, "layer %d out of range (install has %lld)", layer,
                             (long long)m->info.layer_count);
    if (m->fds[(size_t)layer] < 0) {
        const std::string p = layer_path(m, layer);
        const int d = open(p.c_str(), O_RDONLY);
        if (d < 0)
            return gw::set_error(GW_ERR_ARG, "could not open %s: %s", p.c_str(), strerror(errno));
        m->fds[(size_t)layer] = d;
    }
    fd = m->fds[(size_t)layer];
    return GW_OK;
}

// Reads [offset, offset + length) of a layer file into device memory: pread
// into two pinned staging buffers in turn, each copied by the context stream
// while the other fills (ModelReader.read, ModelReader.swift:78-110, with the
// same short-read and error reporting).  Returns when the bytes are on the
// device.
static int read_to_device(gw_context *ctx, gw_model *m, int layer, int64_t offset,
                          int64_t length, void *dst)
{
    constexpr size_t kChunk = kStageBytes;
    int fd = -1;
    int rc = layer_fd(m, layer, fd);
    if (rc != GW_OK) return rc;
    hipStream_t stream = static_cast<hipStream_t>(gw_context_stream(ctx));
    void **stage = m->stage;
    hipEvent_t done[2] = {nullptr, nullptr};
    bool pending[2] = {false, false};
    hipError_t e = hipSuccess;
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        if (!stage[i]) e = hipHostMalloc(&stage[i], kChunk, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
    }
    int64_t filled = 0;
    int which = 0;
    while (e == hipSuccess && rc == GW_OK && filled < length) {
        if (pending[which]) {
            e = hipEventSynchronize(done[which]);
            pending[which] = false;
            if (e != hipSuccess) break;
        }
        const size_t want = (size_t)std::min<int64_t>((int64_t)kChunk, length - filled);
        size_t got = 0;
        while (got < want) {
            const ssize_t r = pread(fd, static_cast<char *>(stage[which]) + got, want - got,
                                    (off_t)(offset + filled + (int64_t)got));
            if (r < 0) {
                if (errno == EINTR) continue;
                rc = gw::set_error(GW_ERR_ARG, "reading layer %d failed: %s", layer, strerror(errno));
                break;
            }
            if (r == 0) {
                rc = gw::set_error(GW_ERR_ARG, "reading layer %d returned %lld of %lld bytes",
                                   layer, (long long)(filled + (int64_t)got), (long long)length);
                break;
            }
            got += (size_t)r;
        }
        if (rc != GW_OK) break;
        e = hipMemcpyAsync(static_cast<char *>(dst) + filled, stage[which], want,
                           hipMemcpyHostToDevice, stream);
        if (e == hipSuccess) e = hipEventRecord(done[which], stream);
        if (e == hipSuccess) pending[which] = true;
        filled += (int64_t)want;
        which ^= 1;
    }
    for (int i = 0; i < 2; ++i)
        if (pending[i]) {
            const hipError_t w = hipEventSynchronize(done[i]);
            if (e == hipSuccess) e = w;
        }
    for (int i = 0; i < 2; ++i)
        if (done[i]) (void)hipEventDestroy(done[i]);
    if (rc != GW_OK) return rc;
    if (e != hipSuccess)
        return gw::set_error(e == hipErrorOutOfMemory ? GW_ERR_OOM : GW_ERR_HIP,
                             "loading layer %d: %s", layer, hipGetErrorString(e));
    return GW_OK;
}

extern "C" int gw_model_load_layer(gw_context *ctx, gw_model *m, int32_t layer, void *dst,
                                   size_t capacity)
{
    if (!ctx || !m || !dst) return gw::set_error(GW_ERR_ARG, "null argument");
    const int64_t bytes = m->info.expert_stride * m->info.expert_count;
    if ((int64_t)capacity < bytes)
        return gw::set_error(GW_ERR_ARG, "destination holds %zu bytes, layer needs %lld",
                             capacity, (long long)bytes);
    if ((reinterpret_cast<uintptr_t>(dst) & 15u) != 0)
        return gw::set_error(GW_ERR_ARG, "destination must be 16-byte aligned");
    return read_to_device(ctx, m, layer, 0, bytes, dst);
}

extern "C" int gw_model_load_expert(gw_context *ctx, gw_model *m, int32_t layer, int32_t expert,
                                    void *dst)
{
    if (!ctx || !m || !dst) return gw::set_error(GW_ERR_ARG, "null argument");
    if (expert < 0 || expert >= (int)m->info.expert_count)
        return gw::set_error(GW_ERR_ARG, "expert %d out of range (layer has %lld)", expert,
                             (long long)m->info.expert_count);
    return read_to_device(ctx, m, layer, (int64_t)expert * m->info.expert_stride,
                          m->info.expert_stride, dst);
}
