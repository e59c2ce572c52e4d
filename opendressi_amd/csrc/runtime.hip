// runtime.hip -- context, errors, memory and host-side scene builders of the
// C ABI (include/dressi_hip.h).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>

#include "internal.h"

namespace dressi {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

void clear_error() { g_last_error.clear(); }

int ctx_workspace_zeroed(dressi_ctx* ctx, int slot, size_t bytes, void** out) {
    const bool grow = (int)ctx->ws_ptr.size() <= slot || ctx->ws_size[slot] < bytes;
    if (int rc = ctx_workspace(ctx, slot, bytes, out)) {
        return rc;
    }
    if (grow) {
        DRESSI_TRY_HIP(hipMemsetAsync(*out, 0, ctx->ws_size[slot], ctx->stream));
    }
    return DRESSI_OK;
}

int ctx_workspace(dressi_ctx* ctx, int slot, size_t bytes, void** out) {
    if ((int)ctx->ws_ptr.size() <= slot) {
        ctx->ws_ptr.resize(slot + 1, nullptr);
        ctx->ws_size.resize(slot + 1, 0);
        ctx->ws_stream.resize(slot + 1, nullptr);
        ctx->ws_event.resize(slot + 1, nullptr);
    }
    hipStream_t cur = ctx->stream;
    if (ctx->ws_ptr[slot] && ctx->ws_stream[slot] != cur) {
        // the slot's last user ran on another stream: order this stream after it
        if (!ctx->ws_event[slot]) {
            DRESSI_TRY_HIP(hipEventCreateWithFlags(&ctx->ws_event[slot], hipEventDisableTiming));
        }
        DRESSI_TRY_HIP(hipEventRecord(ctx->ws_event[slot], ctx->ws_stream[slot]));
        DRESSI_TRY_HIP(hipStreamWaitEvent(cur, ctx->ws_event[slot], 0));
    }
    ctx->ws_stream[slot] = cur;
    if (ctx->ws_size[slot] < bytes) {
        if (ctx->ws_ptr[slot]) {
            // earlier work may still use the old buffer: every earlier user is
            // ordered before `cur` (above), so draining `cur` drains them all
            DRESSI_TRY_HIP(hipStreamSynchronize(cur));
            DRESSI_TRY_HIP(hipFree(ctx->ws_ptr[slot]));
            ctx->ws_ptr[slot] = nullptr;
            ctx->ws_size[slot] = 0;
            ctx->ws_generation++;
        }
        size_t sz = bytes < 256 ? 256 : bytes;
        DRESSI_TRY_HIP(hipMalloc(&ctx->ws_ptr[slot], sz));
        ctx->ws_size[slot] = sz;
    }
    *out = ctx->ws_ptr[slot];
    return DRESSI_OK;
}

__global__ __launch_bounds__(256) void k_zero_words(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x) {
        p[i] = 0u;
    }
}

int launch_zero(hipStream_t s, void* p, size_t bytes) {
    const size_t n = bytes / 4;
    if (n == 0) {
        return DRESSI_OK;
    }
    const uint32_t blocks = (uint32_t)std::min<size_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_zero_words, dim3(blocks), dim3(256), 0, s, (uint32_t*)p, n);
    DRESSI_CHECK_LAUNCH();
    return DRESSI_OK;
}

}  // namespace dressi

using namespace dressi;

extern "C" {

const char* dressi_last_error(void) { return g_last_error.c_str(); }

const char* dressi_version(void) { return "dressi-hip 0.1 (gfx950)"; }

int dressi_ctx_create(int device, dressi_ctx** out) {
    DRESSI_REQUIRE(out != nullptr, "dressi_ctx_create: out is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) {
        set_error("no HIP device available (%s)", hipGetErrorString(e));
        return DRESSI_ERR_NO_DEVICE;
    }
    DRESSI_REQUIRE(device >= 0 && device < n, "device %d out of range (%d devices)", device, n);
    DRESSI_TRY_HIP(hipSetDevice(device));
    dressi_ctx* c = new dressi_ctx();
    c->device = device;
    hipError_t se = hipStreamCreateWithFlags(&c->own_stream, hipStreamNonBlocking);
    if (se != hipSuccess) {
        delete c;
        set_error("hipStreamCreate failed: %s", hipGetErrorString(se));
        return DRESSI_ERR_HIP;
    }
    c->stream = c->own_stream;
    se = hipMalloc(&c->d_err, sizeof(uint32_t));
    if (se == hipSuccess) {
        se = hipMemset(c->d_err, 0, sizeof(uint32_t));
    }
    if (se != hipSuccess) {
        hipStreamDestroy(c->own_stream);
        delete c;
        set_error("context allocation failed: %s", hipGetErrorString(se));
        return DRESSI_ERR_HIP;
    }
    *out = c;
    return DRESSI_OK;
}

int dressi_ctx_destroy(dressi_ctx* ctx) {
    if (!ctx) {
        return DRESSI_OK;
    }
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    for (size_t i = 0; i < ctx->ws_ptr.size(); ++i) {
        if (ctx->ws_ptr[i]) {
            hipStreamSynchronize(ctx->ws_stream[i]);
            hipFree(ctx->ws_ptr[i]);
        }
        if (ctx->ws_event[i]) {
            hipEventDestroy(ctx->ws_event[i]);
        }
    }
    if (ctx->d_err) {
        hipFree(ctx->d_err);
    }
    if (ctx->own_stream) {
        hipStreamDestroy(ctx->own_stream);
    }
    delete ctx;
    return DRESSI_OK;
}

int dressi_ctx_set_stream(dressi_ctx* ctx, void* stream) {
    DRESSI_REQUIRE(ctx, "NULL context");
    // NULL is the device's null stream: torch's default stream has handle 0
    ctx->stream = (hipStream_t)stream;
    return DRESSI_OK;
}

int dressi_ctx_reset_stream(dressi_ctx* ctx) {
    DRESSI_REQUIRE(ctx, "NULL context");
    ctx->stream = ctx->own_stream;
    return DRESSI_OK;
}

void* dressi_ctx_stream(dressi_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

uint64_t dressi_ctx_workspace_generation(dressi_ctx* ctx) { return ctx ? ctx->ws_generation : 0; }

int dressi_ctx_synchronize(dressi_ctx* ctx) {
    DRESSI_REQUIRE(ctx, "NULL context");
    DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
    uint32_t err = 0;
    DRESSI_TRY_HIP(hipMemcpy(&err, ctx->d_err, sizeof(err), hipMemcpyDeviceToHost));
    if (err) {
        DRESSI_TRY_HIP(hipMemset(ctx->d_err, 0, sizeof(uint32_t)));
        if (err & 0x100u) {
            set_error("fixed-point gradient term out of range (clamped; error bits 0x%x)", err);
        } else {
            set_error("index out of range in a kernel input (error bits 0x%x)", err);
        }
        return DRESSI_ERR_INVALID;
    }
    return DRESSI_OK;
}

int dressi_ctx_device_name(dressi_ctx* ctx, char* buf, size_t len) {
    DRESSI_REQUIRE(ctx && buf && len > 0, "bad arguments");
    hipDeviceProp_t p;
    DRESSI_TRY_HIP(hipGetDeviceProperties(&p, ctx->device));
    snprintf(buf, len, "%s (%s)", p.name, p.gcnArchName);
    return DRESSI_OK;
}

int dressi_malloc(dressi_ctx* ctx, void** ptr, size_t bytes) {
    DRESSI_REQUIRE(ctx && ptr, "bad arguments");
    DRESSI_TRY_HIP(hipSetDevice(ctx->device));
    DRESSI_TRY_HIP(hipMalloc(ptr, bytes ? bytes : 4));
    return DRESSI_OK;
}

int dressi_free(dressi_ctx* ctx, void* ptr) {
    DRESSI_REQUIRE(ctx, "NULL context");
    if (ptr) {
        DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
        DRESSI_TRY_HIP(hipFree(ptr));
    }
    return DRESSI_OK;
}

int dressi_memcpy_h2d(dressi_ctx* ctx, void* dst, const void* src, size_t bytes) {
    DRESSI_REQUIRE(ctx && dst && src, "bad arguments");
    DRESSI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
    return DRESSI_OK;
}

int dressi_memcpy_d2h(dressi_ctx* ctx, void* dst, const void* src, size_t bytes) {
    DRESSI_REQUIRE(ctx && dst && src, "bad arguments");
    DRESSI_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    DRESSI_TRY_HIP(hipStreamSynchronize(ctx->stream));
    return DRESSI_OK;
}

int dressi_memset(dressi_ctx* ctx, void* dst, int value, size_t bytes) {
    DRESSI_REQUIRE(ctx && dst, "bad arguments");
    DRESSI_TRY_HIP(hipMemsetAsync(dst, value, bytes, ctx->stream));
    return DRESSI_OK;
}

// ---------------------------------------------------------------------------
// Host-side scene builders
// ---------------------------------------------------------------------------

namespace {

struct V3 {
    float x, y, z;
};

// examples/common/geometry_utils.cpp:17-20 (Normalized)
V3 unit(V3 v) {
    const float len = std::sqrt(v.x * v.x + v.y * v.y + v.z * v.z);
    return {v.x / len, v.y / len, v.z / len};
}

}  // namespace

// examples/common/geometry_utils.cpp:24-84: golden-rectangle icosahedron,
// `level` midpoint subdivisions (midpoints appended on first use; children
// {v0,a,c},{v1,b,a},{v2,c,b},{a,b,c}).
int dressi_icosphere(uint32_t level, uint32_t* n_verts, uint32_t* n_faces, float* pos,
                     float* faces) {
    DRESSI_REQUIRE(n_verts && n_faces, "bad arguments");
    DRESSI_REQUIRE(level <= 9, "icosphere level %u too large", level);
    uint32_t nv = 12, nf = 20;
    for (uint32_t l = 0; l < level; l++) {
        nv += nf * 3 / 2;
        nf *= 4;
    }
    *n_verts = nv;
    *n_faces = nf;
    if (!pos && !faces) {
        return DRESSI_OK;
    }
    const float g = (1.f + std::sqrt(5.f)) / 2.f;
    std::vector<V3> verts = {{-1, g, 0}, {1, g, 0},  {-1, -g, 0}, {1, -g, 0},
                             {0, -1, g}, {0, 1, g},  {0, -1, -g}, {0, 1, -g},
                             {g, 0, -1}, {g, 0, 1},  {-g, 0, -1}, {-g, 0, 1}};
    for (V3& v : verts) {
        v = unit(v);
    }
    std::vector<uint32_t> tri = {0, 11, 5, 0, 5,  1,  0,  1, 7, 0, 7, 10, 0, 10, 11,
                                 1, 5,  9, 5, 11, 4,  11, 10, 2, 10, 7, 6, 7, 1,  8,
                                 3, 9,  4, 3, 4,  2,  3,  2, 6, 3, 6, 8,  3, 8,  9,
                                 4, 9,  5, 2, 4,  11, 6,  2, 10, 8, 6, 7, 9, 8, 1};
    for (uint32_t l = 0; l < level; l++) {
        std::map<uint64_t, uint32_t> mid_of;
        auto mid = [&](uint32_t a, uint32_t b) {
            const uint64_t key = a < b ? ((uint64_t)a << 32 | b) : ((uint64_t)b << 32 | a);
            auto it = mid_of.find(key);
            if (it != mid_of.end()) {
                return it->second;
            }
            verts.push_back(unit({(verts[a].x + verts[b].x) * 0.5f,
                                  (verts[a].y + verts[b].y) * 0.5f,
                                  (verts[a].z + verts[b].z) * 0.5f}));
            const uint32_t id = (uint32_t)verts.size() - 1;
            mid_of.emplace(key, id);
            return id;
        };
        std::vector<uint32_t> next;
        next.reserve(tri.size() * 4);
        for (size_t f = 0; f < tri.size(); f += 3) {
            const uint32_t v0 = tri[f], v1 = tri[f + 1], v2 = tri[f + 2];
            const uint32_t a = mid(v0, v1);
            const uint32_t b = mid(v1, v2);
            const uint32_t c = mid(v2, v0);
            const uint32_t kids[12] = {v0, a, c, v1, b, a, v2, c, b, a, b, c};
            next.insert(next.end(), kids, kids + 12);
        }
        tri.swap(next);
    }
    if (pos) {
        for (size_t i = 0; i < verts.size(); i++) {
            pos[i * 3 + 0] = verts[i].x;
            pos[i * 3 + 1] = verts[i].y;
            pos[i * 3 + 2] = verts[i].z;
        }
    }
    if (faces) {
        for (size_t i = 0; i < tri.size(); i++) {
            faces[i] = (float)tri[i];
        }
    }
    return DRESSI_OK;
}

// src/core/mesh_utils.cpp:53-71 (VertexFacesTex)
int dressi_vertex_faces_tex(const float* faces, uint32_t n_faces, uint32_t n_verts,
                            uint32_t* max_deg, float* out, size_t cap) {
    DRESSI_REQUIRE(faces && max_deg, "bad arguments");
    std::vector<std::vector<uint32_t>> vf(n_verts);
    for (uint32_t f = 0; f < n_faces; f++) {
        for (int k = 0; k < 3; k++) {
            const float fv = faces[(size_t)f * 3 + k];
            DRESSI_REQUIRE(fv >= 0.f && (uint32_t)fv < n_verts, "face %u index out of range", f);
            vf[(uint32_t)fv].push_back(f);
        }
    }
    uint32_t deg = 1;
    for (const auto& l : vf) {
        deg = l.size() > deg ? (uint32_t)l.size() : deg;
    }
    *max_deg = deg;
    if (out && cap >= (size_t)deg * n_verts) {
        for (size_t i = 0; i < (size_t)deg * n_verts; i++) {
            out[i] = -1.f;
        }
        for (uint32_t v = 0; v < n_verts; v++) {
            for (size_t d = 0; d < vf[v].size(); d++) {
                out[d * n_verts + v] = (float)vf[v][d];
            }
        }
    }
    return DRESSI_OK;
}

// examples/common/asset_utils.cpp:733-755 (LookAt; Normalize3/Cross3/Dot3
// :161-174)
void dressi_look_at(const float eye[3], const float center[3], const float up[3], float m[16]) {
    auto norm = [](const float v[3], float r[3]) {
        const float len = std::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
        r[0] = v[0] / len;
        r[1] = v[1] / len;
        r[2] = v[2] / len;
    };
    auto cross = [](const float a[3], const float b[3], float r[3]) {
        r[0] = a[1] * b[2] - a[2] * b[1];
        r[1] = a[2] * b[0] - a[0] * b[2];
        r[2] = a[0] * b[1] - a[1] * b[0];
    };
    auto dot = [](const float a[3], const float b[3]) {
        return a[0] * b[0] + a[1] * b[1] + a[2] * b[2];
    };
    const float fwd[3] = {center[0] - eye[0], center[1] - eye[1], center[2] - eye[2]};
    float f[3], s0[3], s[3], u[3];
    norm(fwd, f);
    cross(f, up, s0);
    norm(s0, s);
    cross(s, f, u);
    std::memset(m, 0, sizeof(float) * 16);
    m[0] = s[0];
    m[4] = s[1];
    m[8] = s[2];
    m[1] = u[0];
    m[5] = u[1];
    m[9] = u[2];
    m[2] = -f[0];
    m[6] = -f[1];
    m[10] = -f[2];
    m[12] = -dot(s, eye);
    m[13] = -dot(u, eye);
    m[14] = dot(f, eye);
    m[15] = 1.f;
}

// examples/common/asset_utils.cpp:757-766 (PerspectiveVk: y down, z in [0,1])
void dressi_perspective_vk(float fovy_rad, float aspect, float z_near, float z_far,
                           float m[16]) {
    const float t = 1.f / std::tan(fovy_rad * 0.5f);
    std::memset(m, 0, sizeof(float) * 16);
    m[0] = t / aspect;
    m[5] = -t;
    m[10] = z_far / (z_near - z_far);
    m[11] = -1.f;
    m[14] = z_near * z_far / (z_near - z_far);
}

float dressi_expf(float x) { return libc_expf(x); }

// examples/common/asset_utils.cpp:719-731 (Mul, column-major)
void dressi_mat4_mul(const float a[16], const float b[16], float r[16]) {
    float t[16];
    for (int col = 0; col < 4; col++) {
        for (int row = 0; row < 4; row++) {
            float acc = 0.f;
            for (int k = 0; k < 4; k++) {
                acc += a[k * 4 + row] * b[col * 4 + k];
            }
            t[col * 4 + row] = acc;
        }
    }
    std::memcpy(r, t, sizeof(t));
}

}  // extern "C"
