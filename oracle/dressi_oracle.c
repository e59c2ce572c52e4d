/*
 * dressi_oracle.c -- CPU restatement ("oracle") of the reference's
 * HardSoftRas silhouette hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the HIP product
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg load liboracle.so. It is never linked into, loaded by or called from
 * the product library.
 *
 * Every function restates one reference function and cites it (paths are
 * relative to the reference checkout). Floating-point expressions keep the
 * reference's operation order and are compiled with -ffp-contract=off so the
 * results are bit-identical to the reference CPU evaluator wherever the same
 * libm routine is used (sqrtf/division are correctly rounded; expf/powf come
 * from the same glibc). Pinning: tests/test_oracle_vs_reference.py checks
 * each function against the reference's own CPU build (oracle/_ref) through
 * the committed golden fixtures, plus closed forms and invariants.
 *
 * The reference evaluates whole images op by op; this restatement evaluates
 * the same op chain per pixel (identical values: every op is elementwise).
 * Gradient contributions are summed in the order the reference's
 * BuildBackward sums them: contributions are listed in descending node
 * creation order (src/core/build_backward.cpp:79-137) and reduced by a
 * tree of <=4-ary sequential sums (build_backward.cpp:41-58). Node creation
 * order follows the example's C++ expressions evaluated right-to-left (the
 * reference's g++ build evaluates overloaded-operator and call arguments
 * right-to-left).
 */
#define _GNU_SOURCE
#include "dressi_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* small helpers                                                            */
/* ------------------------------------------------------------------------ */

/* std::min / std::max semantics: min(a,b) = (b < a) ? b : a */
static inline float smin(float a, float b) { return (b < a) ? b : a; }
static inline float smax(float a, float b) { return (a < b) ? b : a; }
/* F::Step(edge, x): x < edge ? 0 : 1 (src/core/f_ops.cpp:530-537) */
static inline float step_f(float edge, float x) { return x < edge ? 0.f : 1.f; }
/* uint32_t(int64_t(v + 0.5f)): the reference's float-id decode */
static inline uint32_t fid_u(float v) { return (uint32_t)(int64_t)(v + 0.5f); }

/* ------------------------------------------------------------------------ */
/* scene generation                                                         */
/* ------------------------------------------------------------------------ */

typedef struct { float x, y, z; } v3;

/* examples/common/geometry_utils.cpp:17-20 (Normalized) */
static v3 normalized(v3 v) {
    const float len = sqrtf(v.x * v.x + v.y * v.y + v.z * v.z);
    v3 r = {v.x / len, v.y / len, v.z / len};
    return r;
}

/* examples/common/geometry_utils.cpp:24-84 (GenerateIcosphere): the
 * icosahedron from three golden rectangles, `level` midpoint subdivisions,
 * new vertices appended in first-use order, child faces
 * {f0,a,c},{f1,b,a},{f2,c,b},{a,b,c}. */
int or_icosphere(uint32_t level, uint32_t* n_verts, uint32_t* n_faces,
                 float* pos, float* faces) {
    uint32_t nv = 12, nf = 20;
    for (uint32_t l = 0; l < level; l++) {
        nv += nf * 3 / 2;
        nf *= 4;
    }
    *n_verts = nv;
    *n_faces = nf;
    if (!pos && !faces) {
        return 0;
    }
    const float t = (1.f + sqrtf(5.f)) / 2.f;
    v3* verts = (v3*)malloc(sizeof(v3) * nv);
    uint32_t* fa = (uint32_t*)malloc(sizeof(uint32_t) * 3 * nf);
    uint32_t* fb = (uint32_t*)malloc(sizeof(uint32_t) * 3 * nf);
    const float base[12][3] = {{-1, t, 0}, {1, t, 0},  {-1, -t, 0}, {1, -t, 0},
                               {0, -1, t}, {0, 1, t},  {0, -1, -t}, {0, 1, -t},
                               {t, 0, -1}, {t, 0, 1},  {-t, 0, -1}, {-t, 0, 1}};
    const uint32_t base_f[20][3] = {
            {0, 11, 5}, {0, 5, 1},  {0, 1, 7},   {0, 7, 10}, {0, 10, 11},
            {1, 5, 9},  {5, 11, 4}, {11, 10, 2}, {10, 7, 6}, {7, 1, 8},
            {3, 9, 4},  {3, 4, 2},  {3, 2, 6},   {3, 6, 8},  {3, 8, 9},
            {4, 9, 5},  {2, 4, 11}, {6, 2, 10},  {8, 6, 7},  {9, 8, 1}};
    for (int i = 0; i < 12; i++) {
        v3 v = {base[i][0], base[i][1], base[i][2]};
        verts[i] = normalized(v);
    }
    memcpy(fa, base_f, sizeof(base_f));
    uint32_t cur_v = 12, cur_f = 20;
    /* midpoint cache: per vertex up to 8 (neighbor, midpoint) pairs */
    enum { KCAP = 8 };
    for (uint32_t l = 0; l < level; l++) {
        uint32_t* nb = (uint32_t*)malloc(sizeof(uint32_t) * nv * KCAP * 2);
        uint8_t* cnt = (uint8_t*)calloc(nv, 1);
        uint32_t out_f = 0;
        for (uint32_t f = 0; f < cur_f; f++) {
            uint32_t m3[3];
            for (int e = 0; e < 3; e++) {
                uint32_t a = fa[f * 3 + e], b = fa[f * 3 + (e + 1) % 3];
                uint32_t lo = a < b ? a : b, hi = a < b ? b : a;
                uint32_t found = UINT32_MAX;
                for (uint32_t i = 0; i < cnt[lo]; i++) {
                    if (nb[(lo * KCAP + i) * 2] == hi) {
                        found = nb[(lo * KCAP + i) * 2 + 1];
                    }
                }
                if (found == UINT32_MAX) {
                    v3 m = {(verts[a].x + verts[b].x) * 0.5f,
                            (verts[a].y + verts[b].y) * 0.5f,
                            (verts[a].z + verts[b].z) * 0.5f};
                    verts[cur_v] = normalized(m);
                    found = cur_v++;
                    nb[(lo * KCAP + cnt[lo]) * 2] = hi;
                    nb[(lo * KCAP + cnt[lo]) * 2 + 1] = found;
                    cnt[lo]++;
                }
                m3[e] = found;
            }
            const uint32_t f0 = fa[f * 3], f1 = fa[f * 3 + 1], f2 = fa[f * 3 + 2];
            const uint32_t a = m3[0], b = m3[1], c = m3[2];
            const uint32_t kids[4][3] = {{f0, a, c}, {f1, b, a}, {f2, c, b}, {a, b, c}};
            memcpy(&fb[out_f * 3], kids, sizeof(kids));
            out_f += 4;
        }
        free(nb);
        free(cnt);
        uint32_t* tmp = fa;
        fa = fb;
        fb = tmp;
        cur_f = out_f;
    }
    if (pos) {
        for (uint32_t i = 0; i < nv; i++) {
            pos[i * 3 + 0] = verts[i].x;
            pos[i * 3 + 1] = verts[i].y;
            pos[i * 3 + 2] = verts[i].z;
        }
    }
    if (faces) {
        for (uint32_t i = 0; i < 3 * nf; i++) {
            faces[i] = (float)fa[i];
        }
    }
    free(verts);
    free(fa);
    free(fb);
    return 0;
}

/* examples/common/asset_utils.cpp:719-731 (Mul): column-major r = a*b */
void or_mat4_mul(const float a[16], const float b[16], float r[16]) {
    for (int col = 0; col < 4; col++) {
        for (int row = 0; row < 4; row++) {
            float acc = 0.f;
            for (int k = 0; k < 4; k++) {
                acc += a[k * 4 + row] * b[col * 4 + k];
            }
            r[col * 4 + row] = acc;
        }
    }
}

/* examples/common/asset_utils.cpp:161-174 (Normalize3, Cross3, Dot3) */
static void normalize3(const float v[3], float r[3]) {
    const float len = sqrtf(v[0] * v[0] + v[1] * v[1] + v[2] * v[2]);
    r[0] = v[0] / len;
    r[1] = v[1] / len;
    r[2] = v[2] / len;
}
static void cross3(const float a[3], const float b[3], float r[3]) {
    r[0] = a[1] * b[2] - a[2] * b[1];
    r[1] = a[2] * b[0] - a[0] * b[2];
    r[2] = a[0] * b[1] - a[1] * b[0];
}
static float dot3(const float a[3], const float b[3]) {
    return a[0] * b[0] + a[1] * b[1] + a[2] * b[2];
}

/* examples/common/asset_utils.cpp:733-755 (LookAt) */
void or_look_at(const float eye[3], const float center[3], const float up[3],
                float m[16]) {
    const float fd[3] = {center[0] - eye[0], center[1] - eye[1],
                         center[2] - eye[2]};
    float f[3], sc[3], s[3], u[3];
    normalize3(fd, f);
    cross3(f, up, sc);
    normalize3(sc, s);
    cross3(s, f, u);
    memset(m, 0, sizeof(float) * 16);
    m[0] = s[0];
    m[4] = s[1];
    m[8] = s[2];
    m[1] = u[0];
    m[5] = u[1];
    m[9] = u[2];
    m[2] = -f[0];
    m[6] = -f[1];
    m[10] = -f[2];
    m[12] = -dot3(s, eye);
    m[13] = -dot3(u, eye);
    m[14] = dot3(f, eye);
    m[15] = 1.f;
}

/* examples/common/asset_utils.cpp:757-766 (PerspectiveVk) */
void or_perspective_vk(float fovy_rad, float aspect, float z_near,
                       float z_far, float m[16]) {
    const float t = 1.f / tanf(fovy_rad * 0.5f);
    memset(m, 0, sizeof(float) * 16);
    m[0] = t / aspect;
    m[5] = -t;
    m[10] = z_far / (z_near - z_far);
    m[11] = -1.f;
    m[14] = z_near * z_far / (z_near - z_far);
}

static uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* Seeded standard normals: SplitMix64 uniforms in (0,1) -> Box-Muller
 * (cosine branch), computed in double and rounded once to float. */
void or_randn(uint64_t seed, uint32_t n, float* out) {
    uint64_t s = seed;
    for (uint32_t i = 0; i < n; i++) {
        const double u1 = ((double)(splitmix64(&s) >> 11) + 0.5) * 0x1.0p-53;
        const double u2 = ((double)(splitmix64(&s) >> 11) + 0.5) * 0x1.0p-53;
        out[i] = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
    }
}

/* examples/common/asset_utils.cpp:768-782 (TransformToClip). The graph form
 * used for the optimized mesh (geometry_utils.cpp:391-402) evaluates
 * ((x*m0 + y*m4) + z*m8) + m12 per row, which is the same float sequence. */
void or_transform_to_clip(const float* pos, uint32_t n_verts,
                          const float mvp[16], float* clip) {
    for (uint32_t i = 0; i < n_verts; i++) {
        const float p[4] = {pos[i * 3 + 0], pos[i * 3 + 1], pos[i * 3 + 2], 1.f};
        for (int row = 0; row < 4; row++) {
            float acc = 0.f;
            for (int k = 0; k < 4; k++) {
                acc += mvp[k * 4 + row] * p[k];
            }
            clip[(size_t)i * 4 + row] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* mesh topology                                                            */
/* ------------------------------------------------------------------------ */

/* src/core/mesh_utils.cpp:53-71 (VertexFacesTex): incident faces in
 * ascending face order, {V, max_deg} row-major d*V + v, -1 padding. */
uint32_t or_vertex_faces_tex(const float* faces, uint32_t n_faces,
                             uint32_t n_verts, float* out, uint32_t cap) {
    uint32_t* deg = (uint32_t*)calloc(n_verts, sizeof(uint32_t));
    for (uint32_t f = 0; f < n_faces; f++) {
        for (int k = 0; k < 3; k++) {
            deg[(uint32_t)faces[f * 3 + k]]++;
        }
    }
    uint32_t max_deg = 1;
    for (uint32_t v = 0; v < n_verts; v++) {
        if (deg[v] > max_deg) {
            max_deg = deg[v];
        }
    }
    if (out && cap >= max_deg * n_verts) {
        for (size_t i = 0; i < (size_t)max_deg * n_verts; i++) {
            out[i] = -1.f;
        }
        memset(deg, 0, sizeof(uint32_t) * n_verts);
        for (uint32_t f = 0; f < n_faces; f++) {
            for (int k = 0; k < 3; k++) {
                const uint32_t v = (uint32_t)faces[f * 3 + k];
                out[(size_t)deg[v] * n_verts + v] = (float)f;
                deg[v]++;
            }
        }
    }
    free(deg);
    return max_deg;
}

/* ------------------------------------------------------------------------ */
/* screen-space helpers (src/core/cpu_raster.cpp)                           */
/* ------------------------------------------------------------------------ */

#define K_W_EPS 1e-6f
#define K_DIST_EPS 1e-6f

typedef struct {
    float x, y, z, inv_w;
} screen_vert;

/* cpu_raster.cpp:19-27 (ProjectToScreen) */
static screen_vert project_to_screen(const float* clip, uint32_t w, uint32_t h) {
    const float inv_w = 1.f / clip[3];
    screen_vert v;
    v.x = (clip[0] * inv_w * 0.5f + 0.5f) * (float)w;
    v.y = (clip[1] * inv_w * 0.5f + 0.5f) * (float)h;
    v.z = clip[2] * inv_w;
    v.inv_w = inv_w;
    return v;
}

/* cpu_raster.cpp:227-239 (ProjectClipToScreen) */
static int project_clip_to_screen(const float clip[4], uint32_t w, uint32_t h,
                                  float s_xy[2], float* z_ndc) {
    if (fabsf(clip[3]) <= K_W_EPS || clip[3] < 0.f) {
        return 0;
    }
    const screen_vert v = project_to_screen(clip, w, h);
    s_xy[0] = v.x;
    s_xy[1] = v.y;
    if (z_ndc) {
        *z_ndc = v.z;
    }
    return 1;
}

typedef struct {
    float dist;
    int edge;
    float t;
} tri_dist;

/* cpu_raster.cpp:114-151 (SignedDistToTri): >= 0 inside, winding-agnostic */
static tri_dist signed_dist_to_tri(const float p[2], float s[3][2]) {
    tri_dist best;
    best.dist = 0.f;
    best.edge = 0;
    best.t = 0.f;
    float best_d2 = -1.f;
    int n_pos = 0, n_neg = 0;
    for (int k = 0; k < 3; k++) {
        const float* a = s[k];
        const float* b = s[(k + 1) % 3];
        const float ex = b[0] - a[0];
        const float ey = b[1] - a[1];
        const float len2 = ex * ex + ey * ey;
        float t = 0.f;
        if (len2 > K_DIST_EPS * K_DIST_EPS) {
            t = ((p[0] - a[0]) * ex + (p[1] - a[1]) * ey) / len2;
            t = smin(smax(t, 0.f), 1.f);
        }
        const float qx = a[0] + t * ex;
        const float qy = a[1] + t * ey;
        const float dx = p[0] - qx;
        const float dy = p[1] - qy;
        const float d2 = dx * dx + dy * dy;
        if (best_d2 < 0.f || d2 < best_d2) {
            best_d2 = d2;
            best.edge = k;
            best.t = t;
        }
        const float cr = ex * (p[1] - a[1]) - ey * (p[0] - a[0]);
        n_pos += (cr >= 0.f);
        n_neg += (cr <= 0.f);
    }
    const float sgn = (n_pos == 3 || n_neg == 3) ? 1.f : -1.f;
    best.dist = sgn * sqrtf(smax(best_d2, 0.f));
    return best;
}

/* cpu_raster.cpp:177-193 (ScreenBarycentric) */
static int screen_barycentric(const float p[2], float s[3][2], float lambda[3]) {
    const float area = (s[1][0] - s[0][0]) * (s[2][1] - s[0][1]) -
                       (s[1][1] - s[0][1]) * (s[2][0] - s[0][0]);
    if (fabsf(area) < K_DIST_EPS) {
        return 0;
    }
    const float inv_area = 1.f / area;
    lambda[0] = ((s[1][0] - p[0]) * (s[2][1] - p[1]) -
                 (s[1][1] - p[1]) * (s[2][0] - p[0])) *
                inv_area;
    lambda[1] = ((s[2][0] - p[0]) * (s[0][1] - p[1]) -
                 (s[2][1] - p[1]) * (s[0][0] - p[0])) *
                inv_area;
    lambda[2] = 1.f - lambda[0] - lambda[1];
    return 1;
}

/* ------------------------------------------------------------------------ */
/* ops                                                                      */
/* ------------------------------------------------------------------------ */

/* src/core/f_ops.cpp:1915-1979 (SoftClip CPU kernel): unweld each face and
 * enlarge it about its screen centroid by k = min(1 + r / max(d_min, 1e-3), 8)
 * where d_min is the centroid's distance to the nearest edge line; faces
 * with a corner at w <= 1e-6 pass through unchanged. */
void or_soft_clip(const float* clip, uint32_t n_verts, const float* faces,
                  uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                  float* out) {
    (void)n_verts;
    for (uint32_t f = 0; f < n_faces; f++) {
        float s[3][2];
        const float* c[3];
        int valid = 1;
        for (int k = 0; k < 3; k++) {
            const uint32_t idx = fid_u(faces[f * 3 + k]);
            c[k] = &clip[(size_t)idx * 4];
            if (c[k][3] <= 1e-6f || !project_clip_to_screen(c[k], w, h, s[k], NULL)) {
                valid = 0;
            }
        }
        float scale = 1.f, cx = 0.f, cy = 0.f;
        if (valid) {
            cx = (s[0][0] + s[1][0] + s[2][0]) / 3.f;
            cy = (s[0][1] + s[1][1] + s[2][1]) / 3.f;
            float d_min = 1e30f;
            for (int k = 0; k < 3; k++) {
                const int k2 = (k + 1) % 3;
                const float ex = s[k2][0] - s[k][0];
                const float ey = s[k2][1] - s[k][1];
                const float len = sqrtf(ex * ex + ey * ey);
                if (len < 1e-6f) {
                    continue;
                }
                d_min = smin(d_min, fabsf(ex * (cy - s[k][1]) - ey * (cx - s[k][0])) / len);
            }
            scale = d_min < 1e29f ? smin(1.f + radius / smax(d_min, 1e-3f), 8.f) : 1.f;
        }
        for (int k = 0; k < 3; k++) {
            float* dst = &out[((size_t)f * 3 + (size_t)k) * 4];
            for (int j = 0; j < 4; j++) {
                dst[j] = c[k][j];
            }
            if (valid) {
                const float sx = cx + (s[k][0] - cx) * scale;
                const float sy = cy + (s[k][1] - cy) * scale;
                dst[0] = (sx / (float)w * 2.f - 1.f) * c[k][3];
                dst[1] = (sy / (float)h * 2.f - 1.f) * c[k][3];
            }
        }
    }
}

/* src/core/cpu_raster.cpp:241-355 (RasterizeSoftCpu): rasterize the soft
 * triangles (inclusive barycentric test, soft z in [0,1]), signed distance
 * to the hard face, hard z by unclamped screen barycentrics, Eq.3 depth shift,
 * optional peel reject, depth test with later faces winning ties. */
void or_rasterize_soft(const float* soft_clip, const float* face_id,
                       const float* faces_soft, const float* hard_clip,
                       uint32_t n_verts, const float* faces_tex,
                       uint32_t n_faces, uint32_t w, uint32_t h, float radius,
                       const float* prev, float* out) {
    (void)n_verts;
    const size_t npx = (size_t)w * h;
    memset(out, 0, sizeof(float) * npx * 4);
    float* zbuf = (float*)malloc(sizeof(float) * npx);
    for (size_t i = 0; i < npx; i++) {
        zbuf[i] = 1.f;
    }
    for (uint32_t f = 0; f < n_faces; f++) {
        float ss[3][2], sz[3], fid = 0.f;
        int valid = 1;
        for (int k = 0; k < 3; k++) {
            const uint32_t vi = (uint32_t)(int64_t)faces_soft[f * 3 + k];
            if (!project_clip_to_screen(&soft_clip[(size_t)vi * 4], w, h, ss[k], &sz[k])) {
                valid = 0;
                break;
            }
            fid = face_id[vi];
        }
        if (!valid) {
            continue;
        }
        const uint32_t hf = fid_u(fid);
        float hs[3][2], hz[3];
        for (int k = 0; k < 3; k++) {
            const uint32_t vi = fid_u(faces_tex[(size_t)hf * 3 + k]);
            if (!project_clip_to_screen(&hard_clip[(size_t)vi * 4], w, h, hs[k], &hz[k])) {
                valid = 0;
                break;
            }
        }
        if (!valid) {
            continue;
        }
        const float min_x = smin(smin(ss[0][0], ss[1][0]), ss[2][0]);
        const float max_x = smax(smax(ss[0][0], ss[1][0]), ss[2][0]);
        const float min_y = smin(smin(ss[0][1], ss[1][1]), ss[2][1]);
        const float max_y = smax(smax(ss[0][1], ss[1][1]), ss[2][1]);
        int x0 = (int)floorf(min_x - 0.5f);
        x0 = x0 > 0 ? x0 : 0;
        int x1 = (int)ceilf(max_x - 0.5f);
        x1 = x1 < (int)w - 1 ? x1 : (int)w - 1;
        int y0 = (int)floorf(min_y - 0.5f);
        y0 = y0 > 0 ? y0 : 0;
        int y1 = (int)ceilf(max_y - 0.5f);
        y1 = y1 < (int)h - 1 ? y1 : (int)h - 1;
        for (int y = y0; y <= y1; y++) {
            for (int x = x0; x <= x1; x++) {
                const float p[2] = {(float)x + 0.5f, (float)y + 0.5f};
                float sl[3];
                if (!screen_barycentric(p, ss, sl) || sl[0] < 0.f || sl[1] < 0.f ||
                    sl[2] < 0.f) {
                    continue;
                }
                const float soft_z = sl[0] * sz[0] + sl[1] * sz[1] + sl[2] * sz[2];
                if (soft_z < 0.f || soft_z > 1.f) {
                    continue;
                }
                const tri_dist td = signed_dist_to_tri(p, hs);
                float hl[3];
                float hard_z = 0.5f;
                if (screen_barycentric(p, hs, hl)) {
                    hard_z = hl[0] * hz[0] + hl[1] * hz[1] + hl[2] * hz[2];
                }
                const float depth = td.dist >= 0.f
                                            ? 0.5f * smin(smax(hard_z, 0.f), 1.f)
                                            : 0.5f + 0.5f * smin(-td.dist / radius, 1.f);
                const size_t o = (size_t)y * w + (size_t)x;
                if (prev && depth <= prev[o] + 1e-4f) {
                    continue;
                }
                if (depth > zbuf[o]) {
                    continue;
                }
                zbuf[o] = depth;
                out[o * 4 + 0] = td.dist;
                out[o * 4 + 1] = fid;
                out[o * 4 + 2] = hard_z;
                out[o * 4 + 3] = 1.f;
            }
        }
    }
    free(zbuf);
}

/* src/core/cpu_raster.cpp:31-110 (RasterizeCore): faces with any corner at
 * |w| <= 1e-6 or w < 0 skipped, |area| < 1e-6 skipped, inclusive
 * barycentric coverage, NDC z in [0,1], LessOrEqual depth test against 1.
 * mode 0: perspective-correct attribute (RasterizeHardCpu :195-225),
 * mode 1: float(f) + 1 (RasterizeFaceIdCpu :357-369). */
static void raster_core(const float* clip, const float* attr, uint32_t n_comp,
                        const float* faces, uint32_t n_faces, uint32_t w,
                        uint32_t h, int mode, float* out) {
    const size_t npx = (size_t)w * h;
    memset(out, 0, sizeof(float) * npx * n_comp);
    float* zbuf = (float*)malloc(sizeof(float) * npx);
    for (size_t i = 0; i < npx; i++) {
        zbuf[i] = 1.f;
    }
    for (uint32_t f = 0; f < n_faces; f++) {
        uint32_t idx[3];
        screen_vert sv[3];
        int skip = 0;
        for (int k = 0; k < 3; k++) {
            idx[k] = (uint32_t)(int64_t)faces[f * 3 + k];
            const float* c = &clip[(size_t)idx[k] * 4];
            if (fabsf(c[3]) <= K_W_EPS || c[3] < 0.f) {
                skip = 1;
                break;
            }
            sv[k] = project_to_screen(c, w, h);
        }
        if (skip) {
            continue;
        }
        const float area = (sv[1].x - sv[0].x) * (sv[2].y - sv[0].y) -
                           (sv[1].y - sv[0].y) * (sv[2].x - sv[0].x);
        if (fabsf(area) < K_DIST_EPS) {
            continue;
        }
        const float inv_area = 1.f / area;
        const float min_xf = smin(smin(sv[0].x, sv[1].x), sv[2].x);
        const float max_xf = smax(smax(sv[0].x, sv[1].x), sv[2].x);
        const float min_yf = smin(smin(sv[0].y, sv[1].y), sv[2].y);
        const float max_yf = smax(smax(sv[0].y, sv[1].y), sv[2].y);
        int min_x = (int)floorf(min_xf - 0.5f);
        min_x = min_x > 0 ? min_x : 0;
        int max_x = (int)ceilf(max_xf - 0.5f);
        max_x = max_x < (int)w - 1 ? max_x : (int)w - 1;
        int min_y = (int)floorf(min_yf - 0.5f);
        min_y = min_y > 0 ? min_y : 0;
        int max_y = (int)ceilf(max_yf - 0.5f);
        max_y = max_y < (int)h - 1 ? max_y : (int)h - 1;
        for (int y = min_y; y <= max_y; y++) {
            for (int x = min_x; x <= max_x; x++) {
                const float px = (float)x + 0.5f;
                const float py = (float)y + 0.5f;
                const float l0 = ((sv[1].x - px) * (sv[2].y - py) -
                                  (sv[1].y - py) * (sv[2].x - px)) *
                                 inv_area;
                const float l1 = ((sv[2].x - px) * (sv[0].y - py) -
                                  (sv[2].y - py) * (sv[0].x - px)) *
                                 inv_area;
                const float l2 = 1.f - l0 - l1;
                if (l0 < 0.f || l1 < 0.f || l2 < 0.f) {
                    continue;
                }
                const float z = l0 * sv[0].z + l1 * sv[1].z + l2 * sv[2].z;
                if (z < 0.f || z > 1.f) {
                    continue;
                }
                const size_t o = (size_t)y * w + (size_t)x;
                if (z > zbuf[o]) {
                    continue;
                }
                zbuf[o] = z;
                if (mode == 1) {
                    out[o] = (float)f + 1.f;
                    continue;
                }
                const float lambda[3] = {l0, l1, l2};
                const float denom = lambda[0] * sv[0].inv_w + lambda[1] * sv[1].inv_w +
                                    lambda[2] * sv[2].inv_w;
                for (uint32_t c = 0; c < n_comp; c++) {
                    float num = 0.f;
                    for (int k = 0; k < 3; k++) {
                        num += lambda[k] * sv[k].inv_w * attr[(size_t)idx[k] * n_comp + c];
                    }
                    out[o * n_comp + c] = num / denom;
                }
            }
        }
    }
    free(zbuf);
}

void or_rasterize(const float* clip, uint32_t n_verts, const float* attr,
                  uint32_t n_comp, const float* faces, uint32_t n_faces,
                  uint32_t w, uint32_t h, float* out) {
    (void)n_verts;
    raster_core(clip, attr, n_comp, faces, n_faces, w, h, 0, out);
}

void or_rasterize_face_id(const float* clip, uint32_t n_verts,
                          const float* faces, uint32_t n_faces, uint32_t w,
                          uint32_t h, float* out) {
    (void)n_verts;
    raster_core(clip, NULL, 1, faces, n_faces, w, h, 1, out);
}

/* src/core/f_ops.cpp:1594-1615 (LookupFaces CPU kernel) */
void or_lookup_faces(const float* attr, uint32_t n_comp, const float* faces,
                     uint32_t n_faces, uint32_t corner, float* out) {
    for (uint32_t f = 0; f < n_faces; f++) {
        const uint32_t vi = fid_u(faces[f * 3 + corner]);
        for (uint32_t c = 0; c < n_comp; c++) {
            out[(size_t)f * n_comp + c] = attr[(size_t)vi * n_comp + c];
        }
    }
}

/* src/core/f_ops.cpp:1532-1562 (LookupFacesBwd CPU kernel): per vertex, sum
 * the incident faces' gradients (rows d = 0..max_deg-1 in order) whose
 * corner `corner` is this vertex. */
void or_lookup_faces_bwd(const float* gy, uint32_t n_comp, const float* faces,
                         uint32_t n_faces, const float* vtx_faces,
                         uint32_t n_verts, uint32_t max_deg, uint32_t corner,
                         float* out) {
    (void)n_faces;
    memset(out, 0, sizeof(float) * n_verts * n_comp);
    for (uint32_t v = 0; v < n_verts; v++) {
        for (uint32_t d = 0; d < max_deg; d++) {
            const float fv = vtx_faces[(size_t)d * n_verts + v];
            if (fv < -0.5f) {
                continue;
            }
            const uint32_t f = fid_u(fv);
            const uint32_t vi = fid_u(faces[(size_t)f * 3 + corner]);
            if (vi != v) {
                continue;
            }
            for (uint32_t c = 0; c < n_comp; c++) {
                out[(size_t)v * n_comp + c] += gy[(size_t)f * n_comp + c];
            }
        }
    }
}

/* src/core/f_ops.cpp:1782-1797 (FaceFetch CPU kernel) */
void or_face_fetch(const float* attr, uint32_t n_comp, uint32_t n_faces,
                   const float* idx, uint32_t w, uint32_t h, float* out) {
    const size_t npx = (size_t)w * h;
    memset(out, 0, sizeof(float) * npx * n_comp);
    for (size_t p = 0; p < npx; p++) {
        const int f = (int)(idx[p] + 0.5f) - 1;
        if (f < 0 || (uint32_t)f >= n_faces) {
            continue;
        }
        for (uint32_t c = 0; c < n_comp; c++) {
            out[p * n_comp + c] = attr[(size_t)f * n_comp + c];
        }
    }
}

/* src/core/f_ops.cpp:1473-1487 (WangHash, HashToUnit) */
uint32_t or_wang_hash(uint32_t x) {
    x = (x ^ 61u) ^ (x >> 16);
    x *= 9u;
    x ^= x >> 4;
    x *= 0x27d4eb2du;
    x ^= x >> 15;
    return x;
}

float or_hash_to_unit(uint32_t f, uint32_t s, uint32_t seed, uint32_t salt) {
    const uint32_t hh = or_wang_hash(f * 9781u ^ s * 6151u ^ seed * 26699u ^ salt * 42589u);
    return (float)(hh & 0xFFFFFFu) / 16777216.f;
}

/* src/core/f_ops.cpp:1646-1729 (FaceFetchBwd CPU kernel). n_samples > 0:
 * per face, sample s on hard edge s % 3 at u = H(f,s,seed,0) along it and
 * offset o = (2 H(f,s,seed,1) - 1) r along its normal; gather gy at the
 * sample's pixel iff the ID buffer shows face f there. n_samples == 0: exact
 * sum over the face's screen bbox +-1 px. */
void or_face_fetch_bwd(const float* gy, uint32_t n_comp, const float* idx,
                       uint32_t w, uint32_t h, const float* prj0,
                       const float* prj1, const float* prj2, uint32_t n_faces,
                       float seed, float radius, uint32_t n_samples,
                       float* out) {
    const float* prj[3] = {prj0, prj1, prj2};
    const uint32_t seed_u = (uint32_t)(int64_t)(seed + 0.5f);
    memset(out, 0, sizeof(float) * n_faces * n_comp);
    for (uint32_t f = 0; f < n_faces; f++) {
        float s[3][2];
        int ok = 1;
        for (int k = 0; k < 3; k++) {
            const float* c = &prj[k][(size_t)f * 4];
            if (c[3] <= 1e-6f) {
                ok = 0;
                break;
            }
            s[k][0] = (c[0] / c[3] * 0.5f + 0.5f) * (float)w;
            s[k][1] = (c[1] / c[3] * 0.5f + 0.5f) * (float)h;
        }
        if (!ok) {
            continue;
        }
        float* dst = &out[(size_t)f * n_comp];
        if (n_samples == 0) {
            const float lo_x = smin(smin(s[0][0], s[1][0]), s[2][0]);
            const float hi_x = smax(smax(s[0][0], s[1][0]), s[2][0]);
            const float lo_y = smin(smin(s[0][1], s[1][1]), s[2][1]);
            const float hi_y = smax(smax(s[0][1], s[1][1]), s[2][1]);
            int x0 = (int)floorf(lo_x - 1.f);
            x0 = x0 > 0 ? x0 : 0;
            int x1 = (int)ceilf(hi_x + 1.f);
            x1 = x1 < (int)w - 1 ? x1 : (int)w - 1;
            int y0 = (int)floorf(lo_y - 1.f);
            y0 = y0 > 0 ? y0 : 0;
            int y1 = (int)ceilf(hi_y + 1.f);
            y1 = y1 < (int)h - 1 ? y1 : (int)h - 1;
            for (int iy = y0; iy <= y1; iy++) {
                for (int ix = x0; ix <= x1; ix++) {
                    const size_t p = (size_t)iy * w + (size_t)ix;
                    if (fid_u(idx[p]) != f + 1) {
                        continue;
                    }
                    for (uint32_t c = 0; c < n_comp; c++) {
                        dst[c] += gy[p * n_comp + c];
                    }
                }
            }
            continue;
        }
        for (uint32_t smp = 0; smp < n_samples; smp++) {
            const int e = (int)(smp % 3);
            const float* a = s[e];
            const float* b = s[(e + 1) % 3];
            const float ex = b[0] - a[0];
            const float ey = b[1] - a[1];
            const float len = sqrtf(ex * ex + ey * ey);
            if (len < 1e-6f) {
                continue;
            }
            const float u = or_hash_to_unit(f, smp, seed_u, 0);
            const float o = (or_hash_to_unit(f, smp, seed_u, 1) * 2.f - 1.f) * radius;
            const float px = a[0] + u * ex - o * (ey / len);
            const float py = a[1] + u * ey + o * (ex / len);
            const int ix = (int)floorf(px);
            const int iy = (int)floorf(py);
            if (ix < 0 || iy < 0 || ix >= (int)w || iy >= (int)h) {
                continue;
            }
            const size_t p = (size_t)iy * w + (size_t)ix;
            if (fid_u(idx[p]) != f + 1) {
                continue;
            }
            for (uint32_t c = 0; c < n_comp; c++) {
                dst[c] += gy[p * n_comp + c];
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* HardSoftRas soft-probability chain (per pixel)                            */
/* ------------------------------------------------------------------------ */

/* Forward intermediates of one edge_dist(a, b) of the example
 * (examples/silhouette_optimization/run.cpp:270-278) */
typedef struct {
    float e[2], pa[2], num, den, q, t, dd[2], d;
} edge_fw;

static void edge_dist_fw(const float a[2], const float b[2], const float pc[2],
                         edge_fw* r) {
    r->e[0] = b[0] - a[0];
    r->e[1] = b[1] - a[1];
    r->pa[0] = pc[0] - a[0];
    r->pa[1] = pc[1] - a[1];
    r->num = r->pa[0] * r->e[0] + r->pa[1] * r->e[1];      /* F::Dot */
    const float ee = r->e[0] * r->e[0] + r->e[1] * r->e[1];
    r->den = ee + 1e-12f;
    r->q = r->num / r->den;
    r->t = smin(smax(r->q, 0.f), 1.f);                      /* F::Clamp */
    const float ate0 = a[0] + r->t * r->e[0];
    const float ate1 = a[1] + r->t * r->e[1];
    r->dd[0] = pc[0] - ate0;
    r->dd[1] = pc[1] - ate1;
    const float dd2 = r->dd[0] * r->dd[0] + r->dd[1] * r->dd[1];
    r->d = sqrtf(dd2 + 1e-12f);
}

/* Backward of edge_dist given g_d. Writes the contributions to a (three, in
 * the reference's summation order: Add(a,te), Sub(pc,a), Sub(b,a)) and to b
 * (one: Sub(b,a)). */
static void edge_dist_bw(const edge_fw* r, float g_d, float ga[3][2],
                         float gb[2]) {
    const float g_s = g_d * (0.5f / r->d);                  /* Sqrt bwd */
    /* Dot(dd,dd): two equal contributions, summed (0 + A) + A */
    float g_dd[2];
    for (int c = 0; c < 2; c++) {
        const float A = g_s * r->dd[c];
        g_dd[c] = A + A;
    }
    const float g_ate[2] = {-g_dd[0], -g_dd[1]};           /* Sub(pc, ate) */
    const float g_te[2] = {g_ate[0], g_ate[1]};             /* Add(a, te) */
    /* Mul(t, e): t gets CompSum(g_te * e), e gets g_te * t */
    const float g_t = g_te[0] * r->e[0] + g_te[1] * r->e[1];
    /* Clamp(q, 0, 1): inclusive pass-through */
    const float inside = step_f(0.f, r->q) * step_f(r->q, 1.f);
    const float g_q = g_t * inside;
    /* Div(num, den) */
    const float g_num = g_q / r->den;
    const float g_den = -((g_q * r->num) / (r->den * r->den));
    const float g_ee = g_den;                               /* Add(ee, eps) */
    /* e contributions in descending creation order:
     * Mul(t,e), Dot(pa,e), Dot(e,e) x2 */
    float g_e[2], g_pa[2];
    for (int c = 0; c < 2; c++) {
        const float c0 = g_te[c] * r->t;
        const float c1 = g_num * r->pa[c];
        const float c2 = g_ee * r->e[c];
        float acc = 0.f;
        acc += c0;
        acc += c1;
        acc += c2;
        acc += c2;
        g_e[c] = acc;
        g_pa[c] = g_num * r->e[c];
    }
    for (int c = 0; c < 2; c++) {
        ga[0][c] = g_ate[c];     /* Add(a, te) */
        ga[1][c] = -g_pa[c];     /* Sub(pc, a) */
        ga[2][c] = -g_e[c];      /* Sub(b, a) */
        gb[c] = g_e[c];          /* Sub(b, a) */
    }
}

/* Forward state of the soft-probability chain at one pixel */
typedef struct {
    float mask, w[3], s[3][2];
    edge_fw ed[3]; /* 0: (s0,s1), 1: (s1,s2), 2: (s2,s0) */
    float m01, dmin, inside, dist, sig, D, soft_sil, hard, pred;
} hsr_px;

/* examples/silhouette_optimization/run.cpp:253-300, 320-342: the example's
 * image-space signed distance over the FaceFetch'd corners, the soft
 * probability D = mask * sigmoid(dist * 7 / r), Eq.6 with K = 1 and the
 * Max(hard, soft) composition. `c[k]` are the fetched corner clips. */
static void hsr_px_fw(const float c[3][4], float mask, float dist_c, float cov,
                      const float pc[2], uint32_t w, uint32_t h, float radius,
                      hsr_px* st) {
    st->mask = mask;
    const float om = 1.f - mask;
    for (int k = 0; k < 3; k++) {
        st->w[k] = c[k][3] + om;
        st->s[k][0] = ((c[k][0] / st->w[k]) * 0.5f + 0.5f) * (float)w;
        st->s[k][1] = ((c[k][1] / st->w[k]) * 0.5f + 0.5f) * (float)h;
    }
    edge_dist_fw(st->s[0], st->s[1], pc, &st->ed[0]);
    edge_dist_fw(st->s[1], st->s[2], pc, &st->ed[1]);
    edge_dist_fw(st->s[2], st->s[0], pc, &st->ed[2]);
    st->m01 = smin(st->ed[0].d, st->ed[1].d);
    st->dmin = smin(st->m01, st->ed[2].d);
    float cr[3];
    for (int k = 0; k < 3; k++) {
        const float* a = st->s[k];
        const float* b = st->s[(k + 1) % 3];
        const float ex = b[0] - a[0];
        const float ey = b[1] - a[1];
        cr[k] = ex * (pc[1] - a[1]) - ey * (pc[0] - a[0]);
    }
    const float P = step_f(0.f, cr[0]) * step_f(0.f, cr[1]) * step_f(0.f, cr[2]);
    const float Q = step_f(0.f, -cr[0]) * step_f(0.f, -cr[1]) * step_f(0.f, -cr[2]);
    st->inside = smin(P + Q, 1.f);
    st->dist = (st->inside * 2.f - 1.f) * st->dmin;
    const float sigma_scale = 7.f / radius;
    const float z = st->dist * sigma_scale;
    st->sig = 1.f / (1.f + expf(-z));
    st->D = mask * st->sig;
    const float one_minus = 1.f * (1.f - st->D);
    st->soft_sil = 1.f - one_minus;
    st->hard = cov * step_f(0.f, dist_c);
    st->pred = smax(st->hard, st->soft_sil);
}

/* Backward of hsr_px_fw for the L2 term diff = target - pred scaled by
 * inv_px (run.cpp:382-393), seeded with 1 per pixel: writes the VEC4
 * gradients reaching FaceFetch(tri_k). */
static void hsr_px_bw(const hsr_px* st, const float c[3][4], float target,
                      float inv_px, uint32_t w, uint32_t h, float radius,
                      float g_c[3][4]) {
    const float diff = target - st->pred;
    const float cd = inv_px * diff;           /* Mul(gy=c, diff) */
    const float g_diff = cd + cd;             /* Mul(diff, diff): two terms */
    const float g_pred = -g_diff;             /* Sub(target, pred) */
    const float mk = step_f(st->soft_sil, st->hard);  /* Max bwd mask */
    const float g_soft = g_pred * (1.f - mk);
    const float g_one_minus = -g_soft;        /* Sub(1, one_minus) */
    const float g_om2 = g_one_minus * 1.f;    /* Mul(one, 1 - D) */
    const float g_D = -g_om2;                 /* Sub(1, D) */
    const float g_sig = g_D * st->mask;       /* Mul(mask, sig) */
    const float g_z = g_sig * (st->sig * (1.f - st->sig));
    const float sigma_scale = 7.f / radius;
    const float g_dist = g_z * sigma_scale;
    const float g_dmin = g_dist * (st->inside * 2.f - 1.f);
    /* Min(m01, d20), Min(d01, d12) */
    const float mk1 = step_f(st->m01, st->ed[2].d);
    const float g_m01 = g_dmin * mk1;
    const float g_d20 = g_dmin * (1.f - mk1);
    const float mk2 = step_f(st->ed[0].d, st->ed[1].d);
    const float g_d01 = g_m01 * mk2;
    const float g_d12 = g_m01 * (1.f - mk2);
    float ga01[3][2], gb01[2], ga12[3][2], gb12[2], ga20[3][2], gb20[2];
    edge_dist_bw(&st->ed[0], g_d01, ga01, gb01);
    edge_dist_bw(&st->ed[1], g_d12, ga12, gb12);
    edge_dist_bw(&st->ed[2], g_d20, ga20, gb20);
    /* s_k contributions in descending creation order. The edge_dist nodes
     * were created ed20, ed12, ed01 (right-to-left argument evaluation), so
     * ed01's consumers come first. One 4-ary sequential sum each. */
    float g_s[3][2];
    for (int cc = 0; cc < 2; cc++) {
        float acc;
        acc = 0.f;
        acc += ga01[0][cc];
        acc += ga01[1][cc];
        acc += ga01[2][cc];
        acc += gb20[cc];
        g_s[0][cc] = acc;
        acc = 0.f;
        acc += gb01[cc];
        acc += ga12[0][cc];
        acc += ga12[1][cc];
        acc += ga12[2][cc];
        g_s[1][cc] = acc;
        acc = 0.f;
        acc += gb12[cc];
        acc += ga20[0][cc];
        acc += ga20[1][cc];
        acc += ga20[2][cc];
        g_s[2][cc] = acc;
    }
    /* screen_of backward: s = ((c.xy / w) * 0.5 + 0.5) * (W, H),
     * w = c.w + (1 - mask) */
    for (int k = 0; k < 3; k++) {
        const float g_ax = g_s[k][0] * (float)w;
        const float g_xw = g_ax * 0.5f;
        const float g_ay = g_s[k][1] * (float)h;
        const float g_yw = g_ay * 0.5f;
        const float wk = st->w[k];
        const float g_cx = g_xw / wk;
        const float g_cy = g_yw / wk;
        const float gw_x = -((g_xw * c[k][0]) / (wk * wk));
        const float gw_y = -((g_yw * c[k][1]) / (wk * wk));
        g_c[k][0] = g_cx;
        g_c[k][1] = g_cy;
        g_c[k][2] = 0.f;
        g_c[k][3] = gw_y + gw_x;
    }
}

static void fetch_corners(const float* rs_px, const float* tri0,
                          const float* tri1, const float* tri2,
                          uint32_t n_faces, float c[3][4], float* mask) {
    const float idx = (rs_px[1] + 1.f) * rs_px[3];
    *mask = idx > 0.5f ? 1.f : 0.f;
    const int f = (int)(idx + 0.5f) - 1;
    const float* tri[3] = {tri0, tri1, tri2};
    for (int k = 0; k < 3; k++) {
        for (int j = 0; j < 4; j++) {
            c[k][j] = (f < 0 || (uint32_t)f >= n_faces) ? 0.f : tri[k][(size_t)f * 4 + j];
        }
    }
}

void or_hsr_forward(const float* rs, const float* tri0, const float* tri1,
                    const float* tri2, uint32_t n_faces, const float* target,
                    uint32_t w, uint32_t h, float radius, float* pred,
                    float* view_loss) {
    const float inv_px = 1.f / (float)(w * h);
    for (uint32_t y = 0; y < h; y++) {
        for (uint32_t x = 0; x < w; x++) {
            const size_t o = (size_t)y * w + x;
            float c[3][4], mask;
            fetch_corners(&rs[o * 4], tri0, tri1, tri2, n_faces, c, &mask);
            const float pc[2] = {(float)x + 0.5f, (float)y + 0.5f};
            hsr_px st;
            hsr_px_fw(c, mask, rs[o * 4 + 0], rs[o * 4 + 3], pc, w, h, radius, &st);
            if (pred) {
                pred[o] = st.pred;
            }
            if (view_loss) {
                const float diff = target[o] - st.pred;
                view_loss[o] = diff * diff * inv_px;
            }
        }
    }
}

void or_hsr_backward(const float* rs, const float* tri0, const float* tri1,
                     const float* tri2, uint32_t n_faces, const float* target,
                     uint32_t w, uint32_t h, float radius, float* gy0,
                     float* gy1, float* gy2) {
    const float inv_px = 1.f / (float)(w * h);
    float* gy[3] = {gy0, gy1, gy2};
    for (uint32_t y = 0; y < h; y++) {
        for (uint32_t x = 0; x < w; x++) {
            const size_t o = (size_t)y * w + x;
            float c[3][4], mask;
            fetch_corners(&rs[o * 4], tri0, tri1, tri2, n_faces, c, &mask);
            const float pc[2] = {(float)x + 0.5f, (float)y + 0.5f};
            hsr_px st;
            hsr_px_fw(c, mask, rs[o * 4 + 0], rs[o * 4 + 3], pc, w, h, radius, &st);
            float g_c[3][4];
            hsr_px_bw(&st, c, target[o], inv_px, w, h, radius, g_c);
            for (int k = 0; k < 3; k++) {
                for (int j = 0; j < 4; j++) {
                    gy[k][o * 4 + j] = g_c[k][j];
                }
            }
        }
    }
}

/* SumContribs / SumPixelWise tree (src/core/build_backward.cpp:41-58,
 * src/core/f_ops.cpp:893-948): levels of <=4-ary sequential sums. Reduces
 * `n` vectors of `dim` floats stored consecutively in `v` in place; result
 * in v[0..dim). */
static void sum_tree(float* v, uint32_t n, uint32_t dim) {
    while (n > 1) {
        uint32_t out = 0;
        for (uint32_t i = 0; i < n; i += 4) {
            const uint32_t cnt = (n - i) < 4 ? (n - i) : 4;
            for (uint32_t c = 0; c < dim; c++) {
                float acc;
                if (cnt == 1) {
                    acc = v[(size_t)i * dim + c];
                } else {
                    acc = 0.f;
                    for (uint32_t j = 0; j < cnt; j++) {
                        acc += v[(size_t)(i + j) * dim + c];
                    }
                }
                v[(size_t)out * dim + c] = acc;
            }
            out++;
        }
        n = out;
    }
}

/* One iteration of the example's graph for one view: RasterizeSoft output,
 * pred, view loss, and the clip-space vertex gradient {V,4}. */
static void hsr_view(const float* pos, uint32_t n_verts, const float* faces,
                     uint32_t n_faces, const float* vtx_faces, uint32_t max_deg,
                     const float* mvp, const float* target, uint32_t s,
                     float radius, uint32_t samples, float seed, float* rs,
                     float* pred, float* view_loss, float* g_clip) {
    const size_t npx = (size_t)s * s;
    float* clip = (float*)malloc(sizeof(float) * 4 * n_verts);
    float* soft = (float*)malloc(sizeof(float) * 12 * n_faces);
    float* fid = (float*)malloc(sizeof(float) * 3 * n_faces);
    float* fsoft = (float*)malloc(sizeof(float) * 3 * n_faces);
    float* tri[3];
    float* gy[3];
    float* gtri[3];
    for (int k = 0; k < 3; k++) {
        tri[k] = (float*)malloc(sizeof(float) * 4 * n_faces);
        gy[k] = (float*)malloc(sizeof(float) * 4 * npx);
        gtri[k] = (float*)malloc(sizeof(float) * 4 * n_faces);
    }
    float* lfb = (float*)malloc(sizeof(float) * 12 * n_verts);
    or_transform_to_clip(pos, n_verts, mvp, clip);
    or_soft_clip(clip, n_verts, faces, n_faces, s, s, radius, soft);
    for (uint32_t f = 0; f < n_faces; f++) {
        for (uint32_t k = 0; k < 3; k++) {
            fid[f * 3 + k] = (float)f;
            fsoft[f * 3 + k] = (float)(f * 3 + k);
        }
    }
    or_rasterize_soft(soft, fid, fsoft, clip, n_verts, faces, n_faces, s, s, radius, NULL, rs);
    for (int k = 0; k < 3; k++) {
        or_lookup_faces(clip, 4, faces, n_faces, (uint32_t)k, tri[k]);
    }
    or_hsr_forward(rs, tri[0], tri[1], tri[2], n_faces, target, s, s, radius, pred, view_loss);
    or_hsr_backward(rs, tri[0], tri[1], tri[2], n_faces, target, s, s, radius, gy[0], gy[1], gy[2]);
    /* idx image = (fid + 1) * cov */
    float* idx = (float*)malloc(sizeof(float) * npx);
    for (size_t p = 0; p < npx; p++) {
        idx[p] = (rs[p * 4 + 1] + 1.f) * rs[p * 4 + 3];
    }
    for (int k = 0; k < 3; k++) {
        or_face_fetch_bwd(gy[k], 4, idx, s, s, tri[0], tri[1], tri[2], n_faces, seed, radius,
                          samples, gtri[k]);
        or_lookup_faces_bwd(gtri[k], 4, faces, n_faces, vtx_faces, n_verts, max_deg,
                            (uint32_t)k, lfb + (size_t)k * 4 * n_verts);
    }
    /* clip_v gradient: contributions LookupFaces k = 2, 1, 0 (descending
     * creation), one 3-ary sum */
    for (size_t i = 0; i < (size_t)4 * n_verts; i++) {
        float acc = 0.f;
        acc += lfb[(size_t)2 * 4 * n_verts + i];
        acc += lfb[(size_t)1 * 4 * n_verts + i];
        acc += lfb[i];
        g_clip[i] = acc;
    }
    free(idx);
    free(lfb);
    for (int k = 0; k < 3; k++) {
        free(tri[k]);
        free(gy[k]);
        free(gtri[k]);
    }
    free(clip);
    free(soft);
    free(fid);
    free(fsoft);
}

/* The pos gradient from per-view clip gradients through the example's
 * TransformToClipVar (examples/common/geometry_utils.cpp:391-402): per view
 * x/y/z get one 4-ary sum over rows 0..3 (Mul(x, m) nodes of row 0 are the
 * newest), pos gets the GetZ, GetY, GetX contributions of view N-1 .. 0
 * (newest first) through the <=4-ary SumContribs tree. */
static void pos_grad(const float* g_clip_views, const float* mvps,
                     uint32_t n_views, uint32_t n_verts, float* g_pos) {
    float* contrib = (float*)malloc(sizeof(float) * 3 * 3 * n_views);
    for (uint32_t i = 0; i < n_verts; i++) {
        uint32_t n = 0;
        for (int v = (int)n_views - 1; v >= 0; v--) {
            const float* m = mvps + 16 * v;
            const float* gc = g_clip_views + ((size_t)v * n_verts + i) * 4;
            float gxyz[3];
            for (int comp = 0; comp < 3; comp++) {
                float acc = 0.f;
                for (int r = 0; r < 4; r++) {
                    acc += gc[r] * m[comp * 4 + r];
                }
                gxyz[comp] = acc;
            }
            /* GetZ, GetY, GetX contributions, each a zero-padded VEC3 */
            for (int comp = 2; comp >= 0; comp--) {
                float* dst = contrib + (size_t)n * 3;
                dst[0] = dst[1] = dst[2] = 0.f;
                dst[comp] = gxyz[comp];
                n++;
            }
        }
        sum_tree(contrib, n, 3);
        g_pos[(size_t)i * 3 + 0] = contrib[0];
        g_pos[(size_t)i * 3 + 1] = contrib[1];
        g_pos[(size_t)i * 3 + 2] = contrib[2];
    }
    free(contrib);
}

/* examples/silhouette_optimization/run.cpp:421-436 (in-graph Adam) */
static void adam_step(float* pos, float* m, float* v, float* t, const float* g,
                      uint32_t n, float lr) {
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const float t_new = *t + 1.f;
    const float bc1 = 1.f - powf(b1, t_new);
    const float bc2 = 1.f - powf(b2, t_new);
    const float cb1 = 1.f - b1, cb2 = 1.f - b2;
    for (uint32_t i = 0; i < n; i++) {
        const float m_new = m[i] * b1 + g[i] * cb1;
        const float v_new = v[i] * b2 + g[i] * g[i] * cb2;
        const float step = (m_new / bc1) / (sqrtf(v_new / bc2) + eps) * lr;
        pos[i] = pos[i] - step;
        m[i] = m_new;
        v[i] = v_new;
    }
    *t = t_new;
}

int or_hsr_fit(const float* pos0, uint32_t n_verts, const float* faces,
               uint32_t n_faces, const float* tgt_pos, uint32_t n_tverts,
               const float* tgt_faces, uint32_t n_tfaces, const float* mvps,
               uint32_t n_views, uint32_t screen_px, float radius_px,
               uint32_t samples, float lr, uint32_t iters, float* out_pos,
               float* out_m, float* out_v, float* out_t, float* out_loss,
               float* out_grad0, float* out_pred0, float* out_target,
               float* out_rs0, float* out_lossimg0) {
    const uint32_t s = screen_px;
    const size_t npx = (size_t)s * s;
    const uint32_t max_deg = or_vertex_faces_tex(faces, n_faces, n_verts, NULL, 0);
    float* vf = (float*)malloc(sizeof(float) * max_deg * n_verts);
    or_vertex_faces_tex(faces, n_faces, n_verts, vf, max_deg * n_verts);
    /* static targets: StopGradient(Rasterize(tgt_clip, ones, tgt_faces)) */
    float* targets = (float*)malloc(sizeof(float) * npx * n_views);
    float* tclip = (float*)malloc(sizeof(float) * 4 * n_tverts);
    float* ones = (float*)malloc(sizeof(float) * n_tverts);
    for (uint32_t i = 0; i < n_tverts; i++) {
        ones[i] = 1.f;
    }
    for (uint32_t v = 0; v < n_views; v++) {
        or_transform_to_clip(tgt_pos, n_tverts, mvps + 16 * v, tclip);
        or_rasterize(tclip, n_tverts, ones, 1, tgt_faces, n_tfaces, s, s, targets + v * npx);
    }
    free(tclip);
    free(ones);
    float* pos = (float*)malloc(sizeof(float) * 3 * n_verts);
    float* m = (float*)calloc(3 * (size_t)n_verts, sizeof(float));
    float* vv = (float*)calloc(3 * (size_t)n_verts, sizeof(float));
    float t = 0.f;
    memcpy(pos, pos0, sizeof(float) * 3 * n_verts);
    float* rs = (float*)malloc(sizeof(float) * 4 * npx);
    float* pred = (float*)malloc(sizeof(float) * npx);
    float* vloss = (float*)malloc(sizeof(float) * npx * n_views);
    float* loss = (float*)malloc(sizeof(float) * npx);
    float* gclip = (float*)malloc(sizeof(float) * 4 * n_verts * n_views);
    float* gpos = (float*)malloc(sizeof(float) * 3 * n_verts);
    float* lacc = (float*)malloc(sizeof(float) * n_views);
    for (uint32_t it = 0; it < iters; it++) {
        for (uint32_t v = 0; v < n_views; v++) {
            hsr_view(pos, n_verts, faces, n_faces, vf, max_deg, mvps + 16 * v,
                     targets + v * npx, s, radius_px, samples, t, rs, pred,
                     vloss + v * npx, gclip + (size_t)v * 4 * n_verts);
            if (it == 0) {
                if (out_pred0) {
                    memcpy(out_pred0 + v * npx, pred, sizeof(float) * npx);
                }
                if (out_rs0) {
                    memcpy(out_rs0 + v * npx * 4, rs, sizeof(float) * 4 * npx);
                }
            }
        }
        /* loss image: SumPixelWise over views (<=4-ary tree) */
        for (size_t p = 0; p < npx; p++) {
            for (uint32_t v = 0; v < n_views; v++) {
                lacc[v] = vloss[v * npx + p];
            }
            sum_tree(lacc, n_views, 1);
            loss[p] = lacc[0];
        }
        if (out_loss) {
            double acc = 0.0;
            for (size_t p = 0; p < npx; p++) {
                acc += loss[p];
            }
            out_loss[it] = (float)acc;
        }
        pos_grad(gclip, mvps, n_views, n_verts, gpos);
        if (it == 0) {
            if (out_lossimg0) {
                memcpy(out_lossimg0, loss, sizeof(float) * npx);
            }
            if (out_grad0) {
                memcpy(out_grad0, gpos, sizeof(float) * 3 * n_verts);
            }
        }
        adam_step(pos, m, vv, &t, gpos, 3 * n_verts, lr);
    }
    if (out_target) {
        memcpy(out_target, targets, sizeof(float) * npx * n_views);
    }
    if (out_pos) memcpy(out_pos, pos, sizeof(float) * 3 * n_verts);
    if (out_m) memcpy(out_m, m, sizeof(float) * 3 * n_verts);
    if (out_v) memcpy(out_v, vv, sizeof(float) * 3 * n_verts);
    if (out_t) *out_t = t;
    free(vf);
    free(targets);
    free(pos);
    free(m);
    free(vv);
    free(rs);
    free(pred);
    free(vloss);
    free(loss);
    free(gclip);
    free(gpos);
    free(lacc);
    return 0;
}

/* ===================================================================== */
/* Screen-space antialiasing (Dr.Hair-style AA, technique "aa")           */
/* ===================================================================== */

/* f_ops.cpp:2213-2214 (kAaOffs) */
static const int k_aa_offs[8][2] = {{-1, -1}, {0, -1}, {1, -1}, {-1, 0},
                                    {1, 0},   {-1, 1}, {0, 1},  {1, 1}};

/* src/core/cpu_raster.cpp:371-454 (EvalAaPair). `tri` holds float(face)+1
 * (0 = background); `faces` float VEC3. Owner preference: the neighbour's
 * triangle first (the edge crossed walking s -> n; max crossing parameter),
 * then s's own (min crossing parameter). */
int or_eval_aa_pair(const float* tri, const float* clip, uint32_t n_verts,
                    const float* faces, uint32_t n_faces, uint32_t w, uint32_t h,
                    int sx, int sy, int nx, int ny, or_aa_pair* out) {
    const int its = (int)(tri[(size_t)sy * w + sx] + 0.5f);
    const int itn = (int)(tri[(size_t)ny * w + nx] + 0.5f);
    if (its == itn) {
        return 0;
    }
    const float ps[2] = {(float)sx + 0.5f, (float)sy + 0.5f};
    const float pn[2] = {(float)nx + 0.5f, (float)ny + 0.5f};
    for (int o = 0; o < 2; o++) {
        const int owner = o == 0 ? itn : its;
        if (owner == 0) {
            continue;
        }
        const uint32_t f = (uint32_t)(owner - 1);
        if (f >= n_faces) {
            continue;
        }
        uint32_t vi[3];
        float q[3][2];
        int ok = 1;
        for (int k = 0; k < 3; k++) {
            vi[k] = (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
            if (vi[k] >= n_verts ||
                !project_clip_to_screen(&clip[(size_t)vi[k] * 4], w, h, q[k], NULL)) {
                ok = 0;
                break;
            }
        }
        if (!ok) {
            continue;
        }
        int best_j = -1;
        float best_t = 0.f;
        for (int j = 0; j < 3; j++) {
            const float* a = q[j];
            const float* b = q[(j + 1) % 3];
            const float es = (b[0] - a[0]) * (ps[1] - a[1]) - (b[1] - a[1]) * (ps[0] - a[0]);
            const float en = (b[0] - a[0]) * (pn[1] - a[1]) - (b[1] - a[1]) * (pn[0] - a[0]);
            if (es * en >= 0.f) {
                continue;
            }
            const float t = es / (es - en);
            if (best_j < 0 || (o == 0 ? t > best_t : t < best_t)) {
                best_t = t;
                best_j = j;
            }
        }
        if (best_j < 0) {
            continue;
        }
        const float* a = q[best_j];
        const float* b = q[(best_j + 1) % 3];
        const float ex = b[0] - a[0];
        const float ey = b[1] - a[1];
        const float len = sqrtf(ex * ex + ey * ey);
        if (len < 1e-6f) {
            continue;
        }
        const float es = ex * (ps[1] - a[1]) - ey * (ps[0] - a[0]);
        out->r = smin(fabsf(es) / len, 1.f);
        out->ia = vi[best_j];
        out->ib = vi[(best_j + 1) % 3];
        out->qa[0] = a[0];
        out->qa[1] = a[1];
        out->qb[0] = b[0];
        out->qb[1] = b[1];
        out->es = es;
        out->len = len;
        return 1;
    }
    return 0;
}

static int aa_in(int x, int y, uint32_t w, uint32_t h) {
    return !(x < 0 || y < 0 || x >= (int)w || y >= (int)h);
}

/* f_ops.cpp:2544-2576 (AntiAlias CPU): c_aa = (c + sum_k [r c + (1-r) c_n]) / 9,
 * inactive or off-screen neighbours add c. */
void or_antialias(const float* img, uint32_t n_comp, const float* tri,
                  const float* clip, uint32_t n_verts, const float* faces,
                  uint32_t n_faces, uint32_t w, uint32_t h, float* out) {
    for (int y = 0; y < (int)h; y++) {
        for (int x = 0; x < (int)w; x++) {
            const size_t so = ((size_t)y * w + x) * n_comp;
            const float* cs = &img[so];
            float* dst = &out[so];
            for (uint32_t c = 0; c < n_comp; c++) {
                dst[c] = cs[c];
            }
            for (int k = 0; k < 8; k++) {
                const int nx = x + k_aa_offs[k][0];
                const int ny = y + k_aa_offs[k][1];
                or_aa_pair pr;
                if (!aa_in(nx, ny, w, h) ||
                    !or_eval_aa_pair(tri, clip, n_verts, faces, n_faces, w, h, x, y, nx, ny, &pr)) {
                    for (uint32_t c = 0; c < n_comp; c++) {
                        dst[c] += cs[c];
                    }
                    continue;
                }
                const float* cn = &img[((size_t)ny * w + nx) * n_comp];
                for (uint32_t c = 0; c < n_comp; c++) {
                    dst[c] += pr.r * cs[c] + (1.f - pr.r) * cn[c];
                }
            }
            for (uint32_t c = 0; c < n_comp; c++) {
                dst[c] /= 9.f;
            }
        }
    }
}

/* f_ops.cpp:2231-2275 (AntiAliasBwdImg CPU) */
void or_antialias_bwd_img(const float* gy, uint32_t n_comp, const float* tri,
                          const float* clip, uint32_t n_verts, const float* faces,
                          uint32_t n_faces, uint32_t w, uint32_t h, float* out) {
    memset(out, 0, sizeof(float) * (size_t)w * h * n_comp);
    for (int y = 0; y < (int)h; y++) {
        for (int x = 0; x < (int)w; x++) {
            const size_t so = ((size_t)y * w + x) * n_comp;
            float alpha_sum = 0.f;
            float* dst = &out[so];
            for (int k = 0; k < 8; k++) {
                const int nx = x + k_aa_offs[k][0];
                const int ny = y + k_aa_offs[k][1];
                if (!aa_in(nx, ny, w, h)) {
                    alpha_sum += 1.f;
                    continue;
                }
                or_aa_pair pr;
                alpha_sum += or_eval_aa_pair(tri, clip, n_verts, faces, n_faces, w, h, x, y, nx,
                                             ny, &pr)
                                     ? pr.r
                                     : 1.f;
                or_aa_pair pr2;
                if (or_eval_aa_pair(tri, clip, n_verts, faces, n_faces, w, h, nx, ny, x, y, &pr2)) {
                    const size_t no = ((size_t)ny * w + nx) * n_comp;
                    for (uint32_t c = 0; c < n_comp; c++) {
                        dst[c] += (1.f - pr2.r) * gy[no + c];
                    }
                }
            }
            for (uint32_t c = 0; c < n_comp; c++) {
                dst[c] += gy[so + c] * (1.f + alpha_sum);
                dst[c] /= 9.f;
            }
        }
    }
}

/* One active pair's contribution (f_ops.cpp:2345-2386): (1/9) dot(gy(s),
 * c(s) - c(n)) times d r / d q_a, d r / d q_b through the screen -> clip
 * Jacobian (x: 0.5 W / w, y: 0.5 H / w, w: -(..)/w^2, z: 0). `only_v`:
 * add only endpoint `v` into dst_v, else scatter to both endpoints' rows. */
static void aa_accumulate(const float* gy, const float* img, uint32_t n_comp,
                          const float* clip, uint32_t w, uint32_t h, uint32_t v,
                          int x, int y, int nx, int ny, const or_aa_pair* pr,
                          int only_v, float* dst_v, float* out) {
    const size_t so = ((size_t)y * w + x) * n_comp;
    const size_t no = ((size_t)ny * w + nx) * n_comp;
    float gr = 0.f;
    for (uint32_t c = 0; c < n_comp; c++) {
        gr += gy[so + c] * (img[so + c] - img[no + c]);
    }
    gr /= 9.f;
    if (gr == 0.f) {
        return;
    }
    const float ps[2] = {(float)x + 0.5f, (float)y + 0.5f};
    const float sgn = pr->es >= 0.f ? 1.f : -1.f;
    const float inv_l = 1.f / pr->len;
    const float l3 = fabsf(pr->es) * inv_l * inv_l * inv_l;
    const float ex = pr->qb[0] - pr->qa[0];
    const float ey = pr->qb[1] - pr->qa[1];
    const float dqa[2] = {sgn * inv_l * (pr->qb[1] - ps[1]) + l3 * ex,
                          sgn * inv_l * (ps[0] - pr->qb[0]) + l3 * ey};
    const float dqb[2] = {sgn * inv_l * (ps[1] - pr->qa[1]) - l3 * ex,
                          sgn * inv_l * (pr->qa[0] - ps[0]) - l3 * ey};
    const uint32_t ids[2] = {pr->ia, pr->ib};
    const float* dqs[2] = {dqa, dqb};
    const float w_scr = (float)w, h_scr = (float)h;
    for (int e = 0; e < 2; e++) {
        if (only_v && ids[e] != v) {
            continue;
        }
        const float gqx = gr * dqs[e][0];
        const float gqy = gr * dqs[e][1];
        const float* c = &clip[(size_t)ids[e] * 4];
        float* dst = only_v ? dst_v : &out[(size_t)ids[e] * 4];
        dst[0] += gqx * 0.5f * w_scr / c[3];
        dst[1] += gqy * 0.5f * h_scr / c[3];
        dst[3] += -(gqx * 0.5f * w_scr * c[0] + gqy * 0.5f * h_scr * c[1]) / (c[3] * c[3]);
    }
}

/* f_ops.cpp:2321-2474 (AntiAliasBwdVtx CPU). n_samples = 0: exact scatter
 * over every active pair with r < 1, out {V,1} VEC4. n_samples > 0: per
 * (vertex v, incident face slot d), n jittered samples along the face's
 * edges (salts 2 and 3, +-2 px band), accumulated into row (d, v) of out
 * {V, max_deg} VEC4 when `wide`, else into row v. */
void or_antialias_bwd_vtx(const float* gy, const float* img, uint32_t n_comp,
                          const float* tri, const float* clip, uint32_t n_verts,
                          const float* faces, uint32_t n_faces, const float* vtx_faces,
                          uint32_t max_deg, float seed, uint32_t n_samples, int wide,
                          uint32_t w, uint32_t h, float* out) {
    const size_t rows = wide ? max_deg : 1;
    memset(out, 0, sizeof(float) * 4 * (size_t)n_verts * rows);
    if (n_samples == 0) {
        for (int y = 0; y < (int)h; y++) {
            for (int x = 0; x < (int)w; x++) {
                for (int k = 0; k < 8; k++) {
                    const int nx = x + k_aa_offs[k][0];
                    const int ny = y + k_aa_offs[k][1];
                    if (!aa_in(nx, ny, w, h)) {
                        continue;
                    }
                    or_aa_pair pr;
                    if (!or_eval_aa_pair(tri, clip, n_verts, faces, n_faces, w, h, x, y, nx, ny,
                                         &pr) ||
                        pr.r >= 1.f) {
                        continue;
                    }
                    aa_accumulate(gy, img, n_comp, clip, w, h, 0, x, y, nx, ny, &pr, 0, NULL,
                                  out);
                }
            }
        }
        return;
    }
    const uint32_t seed_u = (uint32_t)(int64_t)(seed + 0.5f);
    const float w_scr = (float)w, h_scr = (float)h;
    for (uint32_t v = 0; v < n_verts; v++) {
        for (uint32_t d = 0; d < max_deg; d++) {
            float* dst_v = wide ? &out[((size_t)d * n_verts + v) * 4] : &out[(size_t)v * 4];
            const float fv = vtx_faces[(size_t)d * n_verts + v];
            if (fv < -0.5f) {
                continue;
            }
            const uint32_t f = (uint32_t)(int64_t)(fv + 0.5f);
            float s3[3][2];
            int ok = 1;
            for (int k = 0; k < 3; k++) {
                const uint32_t vi = (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
                const float* c = &clip[(size_t)vi * 4];
                if (c[3] <= 1e-6f) {
                    ok = 0;
                    break;
                }
                s3[k][0] = (c[0] / c[3] * 0.5f + 0.5f) * w_scr;
                s3[k][1] = (c[1] / c[3] * 0.5f + 0.5f) * h_scr;
            }
            if (!ok) {
                continue;
            }
            for (uint32_t smp = 0; smp < n_samples; smp++) {
                const int e = (int)(smp % 3);
                const float* a = s3[e];
                const float* b = s3[(e + 1) % 3];
                const float ex = b[0] - a[0];
                const float ey = b[1] - a[1];
                const float len = sqrtf(ex * ex + ey * ey);
                if (len < 1e-6f) {
                    continue;
                }
                const float u = or_hash_to_unit(f, smp, seed_u, 2);
                const float o = (or_hash_to_unit(f, smp, seed_u, 3) * 2.f - 1.f) * 2.f;
                const int x = (int)floorf(a[0] + u * ex - o * (ey / len));
                const int y = (int)floorf(a[1] + u * ey + o * (ex / len));
                if (!aa_in(x, y, w, h)) {
                    continue;
                }
                for (int k = 0; k < 8; k++) {
                    const int nx = x + k_aa_offs[k][0];
                    const int ny = y + k_aa_offs[k][1];
                    if (!aa_in(nx, ny, w, h)) {
                        continue;
                    }
                    or_aa_pair pr;
                    if (!or_eval_aa_pair(tri, clip, n_verts, faces, n_faces, w, h, x, y, nx, ny,
                                         &pr) ||
                        pr.r >= 1.f) {
                        continue;
                    }
                    if (pr.ia != v && pr.ib != v) {
                        continue;
                    }
                    aa_accumulate(gy, img, n_comp, clip, w, h, v, x, y, nx, ny, &pr, 1, dst_v,
                                  NULL);
                }
            }
        }
    }
}

/* f_ops.cpp:1227-1244 (ColSum CPU): per column, rows summed in order */
void or_col_sum(const float* x, uint32_t n_comp, uint32_t w, uint32_t h, float* out) {
    memset(out, 0, sizeof(float) * (size_t)w * n_comp);
    for (uint32_t r = 0; r < h; r++) {
        for (uint32_t xw = 0; xw < w; xw++) {
            for (uint32_t c = 0; c < n_comp; c++) {
                out[(size_t)xw * n_comp + c] += x[((size_t)r * w + xw) * n_comp + c];
            }
        }
    }
}

/* The AA silhouette fit of the reference example (technique aa, no
 * regularizers; run.cpp:229-238, 346-357, 382-437): per view
 * pred = AntiAlias(Rasterize(clip, 1), RasterizeFaceId(clip), clip, faces,
 * vtx_faces, t, samples), target = StopGradient(AntiAlias(Rasterize(tgt),
 * RasterizeFaceId(tgt), tgt_clip, tgt_faces, tgt_vtx_faces, 0, 0)), L2 loss
 * image summed over views; backward: d loss / d pred -> AntiAliasBwdVtx
 * (wide) -> ColSum -> TransformToClipVar -> pos; in-graph Adam.
 * Outputs (nullable): as or_hsr_fit, with out_tri0 {N,S,S} the face-id
 * images of iteration 0. */
int or_aa_fit(const float* pos0, uint32_t n_verts, const float* faces, uint32_t n_faces,
              const float* tgt_pos, uint32_t n_tverts, const float* tgt_faces,
              uint32_t n_tfaces, const float* mvps, uint32_t n_views, uint32_t screen_px,
              uint32_t samples, float lr, uint32_t iters, float* out_pos, float* out_m,
              float* out_v, float* out_t, float* out_loss, float* out_grad0,
              float* out_pred0, float* out_target, float* out_tri0, float* out_lossimg0) {
    const uint32_t s = screen_px;
    const size_t npx = (size_t)s * s;
    const float inv_px = 1.f / (float)(s * s);
    const uint32_t max_deg = or_vertex_faces_tex(faces, n_faces, n_verts, NULL, 0);
    float* vf = (float*)malloc(sizeof(float) * max_deg * n_verts);
    or_vertex_faces_tex(faces, n_faces, n_verts, vf, max_deg * n_verts);
    float* targets = (float*)malloc(sizeof(float) * npx * n_views);
    float* img = (float*)malloc(sizeof(float) * npx);
    float* tri = (float*)malloc(sizeof(float) * npx);
    {
        float* tclip = (float*)malloc(sizeof(float) * 4 * n_tverts);
        float* ones = (float*)malloc(sizeof(float) * n_tverts);
        for (uint32_t i = 0; i < n_tverts; i++) {
            ones[i] = 1.f;
        }
        for (uint32_t v = 0; v < n_views; v++) {
            or_transform_to_clip(tgt_pos, n_tverts, mvps + 16 * v, tclip);
            or_rasterize(tclip, n_tverts, ones, 1, tgt_faces, n_tfaces, s, s, img);
            or_rasterize_face_id(tclip, n_tverts, tgt_faces, n_tfaces, s, s, tri);
            or_antialias(img, 1, tri, tclip, n_tverts, tgt_faces, n_tfaces, s, s,
                         targets + v * npx);
        }
        free(tclip);
        free(ones);
    }
    float* ones = (float*)malloc(sizeof(float) * n_verts);
    for (uint32_t i = 0; i < n_verts; i++) {
        ones[i] = 1.f;
    }
    float* pos = (float*)malloc(sizeof(float) * 3 * n_verts);
    float* m = (float*)calloc(3 * (size_t)n_verts, sizeof(float));
    float* vv = (float*)calloc(3 * (size_t)n_verts, sizeof(float));
    float t = 0.f;
    memcpy(pos, pos0, sizeof(float) * 3 * n_verts);
    float* clip = (float*)malloc(sizeof(float) * 4 * n_verts);
    float* pred = (float*)malloc(sizeof(float) * npx);
    float* gy = (float*)malloc(sizeof(float) * npx);
    float* vloss = (float*)malloc(sizeof(float) * npx * n_views);
    float* loss = (float*)malloc(sizeof(float) * npx);
    float* wide = (float*)malloc(sizeof(float) * 4 * (size_t)n_verts * max_deg);
    float* gclip = (float*)malloc(sizeof(float) * 4 * n_verts * n_views);
    float* gpos = (float*)malloc(sizeof(float) * 3 * n_verts);
    float* lacc = (float*)malloc(sizeof(float) * n_views);
    for (uint32_t it = 0; it < iters; it++) {
        for (uint32_t v = 0; v < n_views; v++) {
            const float* target = targets + v * npx;
            or_transform_to_clip(pos, n_verts, mvps + 16 * v, clip);
            or_rasterize(clip, n_verts, ones, 1, faces, n_faces, s, s, img);
            or_rasterize_face_id(clip, n_verts, faces, n_faces, s, s, tri);
            or_antialias(img, 1, tri, clip, n_verts, faces, n_faces, s, s, pred);
            for (size_t p = 0; p < npx; p++) {
                const float diff = target[p] - pred[p];
                vloss[v * npx + p] = diff * diff * inv_px;
                const float cd = inv_px * diff; /* Mul(gy = c, diff) */
                gy[p] = -(cd + cd);             /* Mul(diff, diff), Sub(target, pred) */
            }
            or_antialias_bwd_vtx(gy, img, 1, tri, clip, n_verts, faces, n_faces, vf, max_deg, t,
                                 samples, 1, s, s, wide);
            or_col_sum(wide, 4, n_verts, max_deg, gclip + (size_t)v * 4 * n_verts);
            if (it == 0) {
                if (out_pred0) {
                    memcpy(out_pred0 + v * npx, pred, sizeof(float) * npx);
                }
                if (out_tri0) {
                    memcpy(out_tri0 + v * npx, tri, sizeof(float) * npx);
                }
            }
        }
        for (size_t p = 0; p < npx; p++) {
            for (uint32_t v = 0; v < n_views; v++) {
                lacc[v] = vloss[v * npx + p];
            }
            sum_tree(lacc, n_views, 1);
            loss[p] = lacc[0];
        }
        if (out_loss) {
            double acc = 0.0;
            for (size_t p = 0; p < npx; p++) {
                acc += loss[p];
            }
            out_loss[it] = (float)acc;
        }
        pos_grad(gclip, mvps, n_views, n_verts, gpos);
        if (it == 0) {
            if (out_lossimg0) {
                memcpy(out_lossimg0, loss, sizeof(float) * npx);
            }
            if (out_grad0) {
                memcpy(out_grad0, gpos, sizeof(float) * 3 * n_verts);
            }
        }
        adam_step(pos, m, vv, &t, gpos, 3 * n_verts, lr);
    }
    if (out_target) memcpy(out_target, targets, sizeof(float) * npx * n_views);
    if (out_pos) memcpy(out_pos, pos, sizeof(float) * 3 * n_verts);
    if (out_m) memcpy(out_m, m, sizeof(float) * 3 * n_verts);
    if (out_v) memcpy(out_v, vv, sizeof(float) * 3 * n_verts);
    if (out_t) *out_t = t;
    free(vf);
    free(targets);
    free(img);
    free(tri);
    free(ones);
    free(pos);
    free(m);
    free(vv);
    free(clip);
    free(pred);
    free(gy);
    free(vloss);
    free(loss);
    free(wide);
    free(gclip);
    free(gpos);
    free(lacc);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Texture path (C3)                                                        */
/* ------------------------------------------------------------------------ */

/* examples/common/geometry_utils.cpp:86-131 (GenerateUvSphere): (stacks + 1)
 * rows of slices + 1 vertices (seam column duplicated), pole triangles
 * skipped. Counts only when an output is NULL. */
int or_uv_sphere(uint32_t stacks, uint32_t slices, uint32_t* n_verts, uint32_t* n_faces,
                 float* pos, float* uv, float* faces) {
    if (stacks < 2) stacks = 2;
    if (slices < 3) slices = 3;
    const uint32_t cols = slices + 1;
    const uint32_t nv = cols * (stacks + 1);
    const uint32_t nf = 2 * stacks * slices - 2 * slices;
    if (n_verts) *n_verts = nv;
    if (n_faces) *n_faces = nf;
    if (!pos || !uv || !faces) {
        return 0;
    }
    const float k_pi = 3.14159265358979323846f;
    for (uint32_t i = 0; i <= stacks; i++) {
        const float theta = k_pi * (float)i / (float)stacks;
        const float st = sinf(theta), ct = cosf(theta);
        for (uint32_t j = 0; j <= slices; j++) {
            const float phi = 2.f * k_pi * (float)j / (float)slices;
            const uint32_t v = i * cols + j;
            pos[v * 3 + 0] = st * cosf(phi);
            pos[v * 3 + 1] = ct;
            pos[v * 3 + 2] = st * sinf(phi);
            uv[v * 2 + 0] = (float)j / (float)slices;
            uv[v * 2 + 1] = (float)i / (float)stacks;
        }
    }
    uint32_t f = 0;
    for (uint32_t i = 0; i < stacks; i++) {
        for (uint32_t j = 0; j < slices; j++) {
            const uint32_t tl = i * cols + j, tr = i * cols + j + 1;
            const uint32_t bl = (i + 1) * cols + j, br = (i + 1) * cols + j + 1;
            if (i != stacks - 1) {
                faces[f * 3 + 0] = (float)tl;
                faces[f * 3 + 1] = (float)br;
                faces[f * 3 + 2] = (float)bl;
                f++;
            }
            if (i != 0) {
                faces[f * 3 + 0] = (float)tl;
                faces[f * 3 + 1] = (float)tr;
                faces[f * 3 + 2] = (float)br;
                f++;
            }
        }
    }
    return 0;
}

/* src/core/mesh_utils.cpp:180-189 (UvAsClip) */
void or_uv_as_clip(const float* uv, uint32_t n_verts, float* clip) {
    for (uint32_t i = 0; i < n_verts; i++) {
        clip[i * 4 + 0] = uv[i * 2 + 0] * 2.f - 1.f;
        clip[i * 4 + 1] = uv[i * 2 + 1] * 2.f - 1.f;
        clip[i * 4 + 2] = 0.5f;
        clip[i * 4 + 3] = 1.f;
    }
}

/* src/core/mesh_utils.cpp:191-203 (ScreenAttr) */
void or_screen_attr(const float* clip, uint32_t n_verts, uint32_t w, uint32_t h, float* attr) {
    for (uint32_t i = 0; i < n_verts; i++) {
        const float cw = clip[i * 4 + 3];
        const float ndc_x = clip[i * 4 + 0] / cw;
        const float ndc_y = clip[i * 4 + 1] / cw;
        attr[i * 4 + 0] = (ndc_x * 0.5f + 0.5f) * (float)w;
        attr[i * 4 + 1] = (ndc_y * 0.5f + 0.5f) * (float)h;
        attr[i * 4 + 2] = 1.f;
        attr[i * 4 + 3] = 0.f;
    }
}

/* src/core/ibl_math.h:91-115 (BilerpClamp) */
static void bilerp_clamp(const float* data, uint32_t w, uint32_t h, uint32_t n, float u, float v,
                         float* out) {
    const float sx = u * (float)w - 0.5f;
    const float sy = v * (float)h - 0.5f;
    const int ix = (int)floorf(sx);
    const int iy = (int)floorf(sy);
    const float fx = sx - (float)ix;
    const float fy = sy - (float)iy;
    for (uint32_t c = 0; c < n; c++) {
        out[c] = 0.f;
    }
    for (int dy = 0; dy <= 1; dy++) {
        for (int dx = 0; dx <= 1; dx++) {
            int x = ix + dx, y = iy + dy;
            x = x < 0 ? 0 : (x > (int)w - 1 ? (int)w - 1 : x);
            y = y < 0 ? 0 : (y > (int)h - 1 ? (int)h - 1 : y);
            const float wgt = (dx == 0 ? 1.f - fx : fx) * (dy == 0 ? 1.f - fy : fy);
            const float* p = data + ((size_t)y * w + (size_t)x) * n;
            for (uint32_t c = 0; c < n; c++) {
                out[c] += wgt * p[c];
            }
        }
    }
}

/* src/core/f_ops.cpp:2764-2778 (TextureBilinear CPU kernel): tex {tw,th} x
 * n_comp sampled at uv {n_px} VEC2 */
void or_texture_bilinear(const float* tex, uint32_t tw, uint32_t th, uint32_t n_comp,
                         const float* uv, size_t n_px, float* out) {
    for (size_t p = 0; p < n_px; p++) {
        bilerp_clamp(tex, tw, th, n_comp, uv[p * 2 + 0], uv[p * 2 + 1], out + p * n_comp);
    }
}

/* src/core/f_ops.cpp:2605-2639 (F::Texture forward): GLSL texture() through
 * the nearest, clamp-to-edge sampler the executor binds
 * (src/vk/executor.cpp:192-202): texel (clamp(floor(u tw), 0, tw - 1),
 * clamp(floor(v th), 0, th - 1)). */
static int nearest_index(float u, uint32_t n) {
    const float f = floorf(u * (float)n);
    if (!(f > 0.f)) {
        return 0;
    }
    return f >= (float)(n - 1) ? (int)n - 1 : (int)f;
}

void or_texture_nearest(const float* tex, uint32_t tw, uint32_t th, uint32_t n_comp,
                        const float* uv, size_t n_px, float* out) {
    for (size_t p = 0; p < n_px; p++) {
        const int ix = nearest_index(uv[p * 2 + 0], tw);
        const int iy = nearest_index(uv[p * 2 + 1], th);
        const float* t = tex + ((size_t)iy * tw + (size_t)ix) * n_comp;
        for (uint32_t c = 0; c < n_comp; c++) {
            out[p * n_comp + c] = t[c];
        }
    }
}

/* GLSL int(x) of the gather's texel test: truncation toward zero, kept
 * defined for out-of-range x */
static int trunc_i32(float x) {
    if (x != x) {
        return 0;
    }
    if (x >= 2147483520.f) {
        return 2147483647;
    }
    if (x <= -2147483648.f) {
        return (-2147483647 - 1);
    }
    return (int)x;
}

/* GatherByInverseUV (src/core/f_ops.cpp:2586-2601; its GLSL,
 * src/codegen/glsl_codegen.cpp:658-703): per texel, the inverse-UV anchor
 * (its own entry, or the first covered entry of the +-4 dilation in row
 * order), then the first pixel of the 7 x 7 window around the anchor's
 * truncated screen position, rows then columns, whose uv truncates to this
 * texel; the texel takes that pixel's gradient, zero when none matches. */
void or_gather_inv_uv(const float* gy, uint32_t n_comp, uint32_t sw, uint32_t sh,
                      const float* inv_uv, uint32_t tw, uint32_t th, const float* uv,
                      float* out) {
    memset(out, 0, sizeof(float) * (size_t)tw * th * n_comp);
    for (int ty = 0; ty < (int)th; ty++) {
        for (int tx = 0; tx < (int)tw; tx++) {
            const float* iv0 = &inv_uv[((size_t)ty * tw + tx) * 4];
            float iv[4] = {iv0[0], iv0[1], iv0[2], iv0[3]};
            for (int ny = -4; ny <= 4 && iv[2] < 0.5f; ny++) {
                for (int nx = -4; nx <= 4; nx++) {
                    const int px = tx + nx, py = ty + ny;
                    if (px < 0 || py < 0 || px >= (int)tw || py >= (int)th) {
                        continue;
                    }
                    const float* q = &inv_uv[((size_t)py * tw + px) * 4];
                    iv[0] = q[0];
                    iv[1] = q[1];
                    iv[2] = q[2];
                    iv[3] = q[3];
                    if (iv[2] > 0.5f) {
                        break;
                    }
                }
            }
            if (!(iv[2] > 0.5f)) {
                continue;
            }
            const int scx = trunc_i32(iv[0]), scy = trunc_i32(iv[1]);
            float* o = &out[((size_t)ty * tw + tx) * n_comp];
            int found = 0;
            for (int dy = -3; dy <= 3 && !found; dy++) {
                for (int dx = -3; dx <= 3; dx++) {
                    const long spx = (long)scx + dx, spy = (long)scy + dy;
                    if (spx < 0 || spy < 0 || spx >= (long)sw || spy >= (long)sh) {
                        continue;
                    }
                    const float* suv = &uv[((size_t)spy * sw + (size_t)spx) * 2];
                    if (trunc_i32(suv[0] * (float)tw) == tx &&
                        trunc_i32(suv[1] * (float)th) == ty) {
                        const float* g = &gy[((size_t)spy * sw + (size_t)spx) * n_comp];
                        for (uint32_t c = 0; c < n_comp; c++) {
                            o[c] = g[c];
                        }
                        found = 1;
                        break;
                    }
                }
            }
        }
    }
}

/* src/core/f_ops.cpp:2665-2731 (GatherByInverseUVBilinear CPU kernel): per
 * texel, the inverse-UV anchor (its own entry, or the first covered entry of
 * the +-4 dilation in row order), then the tent-weighted gradient of the
 * 7 x 7 screen pixels around it, rows then columns. */
void or_gather_inv_uv_bilinear(const float* gy, uint32_t n_comp, uint32_t sw, uint32_t sh,
                               const float* inv_uv, uint32_t tw, uint32_t th, const float* uv,
                               float* out) {
    memset(out, 0, sizeof(float) * (size_t)tw * th * n_comp);
    for (int ty = 0; ty < (int)th; ty++) {
        for (int tx = 0; tx < (int)tw; tx++) {
            const float* iv0 = &inv_uv[((size_t)ty * tw + tx) * 4];
            float iv[4] = {iv0[0], iv0[1], iv0[2], iv0[3]};
            for (int ny = -4; ny <= 4 && iv[2] < 0.5f; ny++) {
                for (int nx = -4; nx <= 4; nx++) {
                    const int px = tx + nx, py = ty + ny;
                    if (px < 0 || py < 0 || px >= (int)tw || py >= (int)th) {
                        continue;
                    }
                    const float* q = &inv_uv[((size_t)py * tw + px) * 4];
                    iv[0] = q[0];
                    iv[1] = q[1];
                    iv[2] = q[2];
                    iv[3] = q[3];
                    if (iv[2] > 0.5f) {
                        break;
                    }
                }
            }
            if (iv[2] <= 0.5f) {
                continue;
            }
            const int scx = (int)iv[0], scy = (int)iv[1];
            float* o = &out[((size_t)ty * tw + tx) * n_comp];
            for (int dy = -3; dy <= 3; dy++) {
                for (int dx = -3; dx <= 3; dx++) {
                    const int spx = scx + dx, spy = scy + dy;
                    if (spx < 0 || spy < 0 || spx >= (int)sw || spy >= (int)sh) {
                        continue;
                    }
                    const float* suv = &uv[((size_t)spy * sw + spx) * 2];
                    const float stx = suv[0] * (float)tw - 0.5f;
                    const float sty = suv[1] * (float)th - 0.5f;
                    const float a = 1.f - fabsf(stx - (float)tx);
                    const float b = 1.f - fabsf(sty - (float)ty);
                    const float w = (a > 0.f ? a : 0.f) * (b > 0.f ? b : 0.f);
                    if (w > 0.f) {
                        const float* g = &gy[((size_t)spy * sw + spx) * n_comp];
                        for (uint32_t c = 0; c < n_comp; c++) {
                            o[c] += g[c] * w;
                        }
                    }
                }
            }
        }
    }
}

/* The C3 texture fit (the graph of examples/texture_optimization/run.cpp:
 * 112-145 with TextureBilinear, an RGBA texture and in-graph Adam as in
 * examples/silhouette_optimization/run.cpp:404-437). Per iteration `it` and
 * view v the cameras are mvps[(it % n_sets) * n_views + v]; the host sends
 * clip = TransformToClip(pos, mvp) and inv_uv_attr = ScreenAttr(clip):
 *   g_uv   = Rasterize(clip, uv, faces, S)      g_mask = Rasterize(clip, 1, faces, S)
 *   inv_uv = Rasterize(UvAsClip(uv), inv_uv_attr, faces, T)
 *   target = g_mask * TextureBilinear(gt_tex, g_uv, inv_uv)
 *   pred   = g_mask * TextureBilinear(tex, g_uv, inv_uv)
 *   diff   = StopGradient(target) - pred
 *   loss   = SumPixelWise_v(diff * diff * Vec4(c, c, c, 0)),  c = 1 / S^2
 * Backward (image loss seeded with 1): d diff = (0 + c diff) + c diff,
 * d pred = -d diff, d sample = d pred * g_mask, the texel gradient of each
 * view by GatherByInverseUVBilinear, summed over the views newest first
 * through the <=4-ary tree; Adam on the texture. */
int or_tex_fit(const float* pos, uint32_t n_verts, const float* uv, const float* faces,
               uint32_t n_faces, const float* mvps, uint32_t n_sets, uint32_t n_views,
               uint32_t screen_px, uint32_t tex_w, uint32_t tex_h, const float* gt_tex,
               const float* tex0, float lr, uint32_t iters, float* out_tex, float* out_m,
               float* out_v, float* out_t, float* out_loss, float* out_grad0, float* out_pred0,
               float* out_target0, float* out_lossimg0, float* out_uv0, float* out_invuv0) {
    const uint32_t s = screen_px;
    const size_t npx = (size_t)s * s;
    const size_t ntx = (size_t)tex_w * tex_h;
    const float c = 1.f / (float)(s * s);
    const float kw[4] = {c, c, c, 0.f};
    float* clip = (float*)malloc(sizeof(float) * 4 * n_verts);
    float* attr = (float*)malloc(sizeof(float) * 4 * n_verts);
    float* uv_clip = (float*)malloc(sizeof(float) * 4 * n_verts);
    float* ones = (float*)malloc(sizeof(float) * n_verts);
    float* g_uv = (float*)malloc(sizeof(float) * 2 * npx);
    float* g_mask = (float*)malloc(sizeof(float) * npx);
    float* inv_uv = (float*)malloc(sizeof(float) * 4 * ntx);
    float* smp_t = (float*)malloc(sizeof(float) * 4 * npx);
    float* smp_p = (float*)malloc(sizeof(float) * 4 * npx);
    float* gsmp = (float*)malloc(sizeof(float) * 4 * npx);
    float* vloss = (float*)malloc(sizeof(float) * 4 * npx * n_views);
    float* gview = (float*)malloc(sizeof(float) * 4 * ntx * n_views);
    float* gtex = (float*)malloc(sizeof(float) * 4 * ntx);
    float* lacc = (float*)malloc(sizeof(float) * 4 * n_views);
    float* gacc = (float*)malloc(sizeof(float) * 4 * n_views);
    float* tex = (float*)malloc(sizeof(float) * 4 * ntx);
    float* m = (float*)calloc(4 * ntx, sizeof(float));
    float* vv = (float*)calloc(4 * ntx, sizeof(float));
    float t = 0.f;
    memcpy(tex, tex0, sizeof(float) * 4 * ntx);
    or_uv_as_clip(uv, n_verts, uv_clip);
    for (uint32_t i = 0; i < n_verts; i++) {
        ones[i] = 1.f;
    }
    for (uint32_t it = 0; it < iters; it++) {
        const float* set = mvps + (size_t)(it % n_sets) * n_views * 16;
        for (uint32_t v = 0; v < n_views; v++) {
            or_transform_to_clip(pos, n_verts, set + 16 * v, clip);
            or_screen_attr(clip, n_verts, s, s, attr);
            or_rasterize(clip, n_verts, uv, 2, faces, n_faces, s, s, g_uv);
            or_rasterize(clip, n_verts, ones, 1, faces, n_faces, s, s, g_mask);
            or_rasterize(uv_clip, n_verts, attr, 4, faces, n_faces, tex_w, tex_h, inv_uv);
            or_texture_bilinear(gt_tex, tex_w, tex_h, 4, g_uv, npx, smp_t);
            or_texture_bilinear(tex, tex_w, tex_h, 4, g_uv, npx, smp_p);
            for (size_t p = 0; p < npx; p++) {
                for (int k = 0; k < 4; k++) {
                    const float target = g_mask[p] * smp_t[p * 4 + k];
                    const float pred = g_mask[p] * smp_p[p * 4 + k];
                    const float diff = target - pred;
                    vloss[(v * npx + p) * 4 + k] = diff * diff * kw[k];
                    const float cd = kw[k] * diff;
                    float gd = 0.f;
                    gd += cd;
                    gd += cd;
                    gsmp[p * 4 + k] = -gd * g_mask[p];
                    if (it == 0) {
                        if (out_pred0) out_pred0[(v * npx + p) * 4 + k] = pred;
                        if (out_target0) out_target0[(v * npx + p) * 4 + k] = target;
                    }
                }
            }
            or_gather_inv_uv_bilinear(gsmp, 4, s, s, inv_uv, tex_w, tex_h, g_uv,
                                      gview + (size_t)v * 4 * ntx);
            if (it == 0) {
                if (out_uv0) memcpy(out_uv0 + v * 2 * npx, g_uv, sizeof(float) * 2 * npx);
                if (out_invuv0) memcpy(out_invuv0 + v * 4 * ntx, inv_uv, sizeof(float) * 4 * ntx);
            }
        }
        /* loss image: SumPixelWise over views (view order) */
        double ltot = 0.0;
        for (size_t p = 0; p < npx; p++) {
            for (uint32_t v = 0; v < n_views; v++) {
                memcpy(lacc + v * 4, vloss + (v * npx + p) * 4, sizeof(float) * 4);
            }
            sum_tree(lacc, n_views, 4);
            for (int k = 0; k < 4; k++) {
                ltot += lacc[k];
            }
            if (it == 0 && out_lossimg0) {
                memcpy(out_lossimg0 + p * 4, lacc, sizeof(float) * 4);
            }
        }
        if (out_loss) {
            out_loss[it] = (float)ltot;
        }
        /* texel gradient: views newest first */
        for (size_t q = 0; q < ntx; q++) {
            for (uint32_t v = 0; v < n_views; v++) {
                memcpy(gacc + v * 4, gview + ((size_t)(n_views - 1 - v) * ntx + q) * 4,
                       sizeof(float) * 4);
            }
            sum_tree(gacc, n_views, 4);
            memcpy(gtex + q * 4, gacc, sizeof(float) * 4);
        }
        if (it == 0 && out_grad0) {
            memcpy(out_grad0, gtex, sizeof(float) * 4 * ntx);
        }
        adam_step(tex, m, vv, &t, gtex, (uint32_t)(4 * ntx), lr);
    }
    if (out_tex) memcpy(out_tex, tex, sizeof(float) * 4 * ntx);
    if (out_m) memcpy(out_m, m, sizeof(float) * 4 * ntx);
    if (out_v) memcpy(out_v, vv, sizeof(float) * 4 * ntx);
    if (out_t) *out_t = t;
    free(clip);
    free(attr);
    free(uv_clip);
    free(ones);
    free(g_uv);
    free(g_mask);
    free(inv_uv);
    free(smp_t);
    free(smp_p);
    free(gsmp);
    free(vloss);
    free(gview);
    free(gtex);
    free(lacc);
    free(gacc);
    free(tex);
    free(m);
    free(vv);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* GatherDistGrad (exact backward of RasterizeSoft's dist channel)          */
/* ------------------------------------------------------------------------ */

/* cpu_raster.cpp:153-175 (SignedDistGradToTri): d dist / d s for the argmin
 * edge with t held fixed (envelope theorem); 0 on the boundary. */
static void signed_dist_grad(const float p[2], float s[3][2], tri_dist td, float g_s[3][2]) {
    for (int k = 0; k < 3; k++) {
        g_s[k][0] = 0.f;
        g_s[k][1] = 0.f;
    }
    const float d = fabsf(td.dist);
    if (d < K_DIST_EPS) {
        return;
    }
    const int ia = td.edge;
    const int ib = (td.edge + 1) % 3;
    const float qx = s[ia][0] + td.t * (s[ib][0] - s[ia][0]);
    const float qy = s[ia][1] + td.t * (s[ib][1] - s[ia][1]);
    const float sgn = td.dist >= 0.f ? 1.f : -1.f;
    const float nx = (p[0] - qx) / d;
    const float ny = (p[1] - qy) / d;
    g_s[ia][0] = -sgn * (1.f - td.t) * nx;
    g_s[ia][1] = -sgn * (1.f - td.t) * ny;
    g_s[ib][0] = -sgn * td.t * nx;
    g_s[ib][1] = -sgn * td.t * ny;
}

/* src/core/f_ops.cpp:1281-1355 (GatherDistGrad CPU kernel): for every
 * covered pixel (raster order) with gy.x != 0, the dist gradient of its
 * face's projected corners through the screen -> clip Jacobian (x: 0.5 W /
 * w, y: 0.5 H / w, w: -(gx 0.5 W c.x + gy 0.5 H c.y) / w^2, z untouched).
 * wide: the contribution of face f to vertex u lands in u's adjacency row
 * holding f, out {max_deg, V, 4}; else out {V, 4}. gy, ro {h, w, 4}. */
void or_gather_dist_grad(const float* gy, const float* ro, const float* clip, uint32_t n_verts,
                         const float* faces, uint32_t n_faces, const float* vtx_faces,
                         uint32_t max_deg, int wide, uint32_t w, uint32_t h, float* out) {
    (void)n_faces;
    const size_t rows = wide ? max_deg : 1;
    memset(out, 0, sizeof(float) * 4 * rows * n_verts);
    const float ws = (float)w, hs = (float)h;
    for (uint32_t y = 0; y < h; y++) {
        for (uint32_t x = 0; x < w; x++) {
            const size_t o = ((size_t)y * w + x) * 4;
            if (ro[o + 3] < 0.5f) {
                continue;
            }
            const float g = gy[o + 0];
            if (g == 0.f) {
                continue;
            }
            const uint32_t f = (uint32_t)(int64_t)(ro[o + 1] + 0.5f);
            uint32_t idx[3];
            float s[3][2];
            int valid = 1;
            for (int k = 0; k < 3; k++) {
                idx[k] = (uint32_t)(int64_t)(faces[(size_t)f * 3 + k] + 0.5f);
                const float* c = &clip[(size_t)idx[k] * 4];
                if (fabsf(c[3]) <= K_W_EPS || c[3] < 0.f) {
                    valid = 0;
                    break;
                }
                const screen_vert v = project_to_screen(c, w, h);
                s[k][0] = v.x;
                s[k][1] = v.y;
            }
            if (!valid) {
                continue;
            }
            const float p[2] = {(float)x + 0.5f, (float)y + 0.5f};
            const tri_dist td = signed_dist_to_tri(p, s);
            float g_s[3][2];
            signed_dist_grad(p, s, td, g_s);
            for (int k = 0; k < 3; k++) {
                const float gsx = g * g_s[k][0];
                const float gsy = g * g_s[k][1];
                if (gsx == 0.f && gsy == 0.f) {
                    continue;
                }
                const float* c = &clip[(size_t)idx[k] * 4];
                size_t row = 0;
                if (wide) {
                    for (uint32_t d = 0; d < max_deg; d++) {
                        const float fv = vtx_faces[(size_t)d * n_verts + idx[k]];
                        if (fv >= -0.5f && (uint32_t)(int64_t)(fv + 0.5f) == f) {
                            row = d;
                            break;
                        }
                    }
                }
                float* dst = &out[(row * n_verts + idx[k]) * 4];
                dst[0] += gsx * 0.5f * ws / c[3];
                dst[1] += gsy * 0.5f * hs / c[3];
                dst[3] += -(gsx * 0.5f * ws * c[0] + gsy * 0.5f * hs * c[1]) / (c[3] * c[3]);
            }
        }
    }
}
