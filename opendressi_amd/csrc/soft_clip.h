// soft_clip.h -- HardSoftRas soft geometry of one face.
#pragma once

#include "dressi_math.h"

namespace dressi {

// src/core/f_ops.cpp:1915-1979 (SoftClip CPU kernel): unweld the face and
// enlarge it about its screen centroid by k = min(1 + r / max(d_min, 1e-3), 8),
// d_min = centroid distance to the nearest edge line (edges shorter than 1e-6
// ignored). Faces with a corner at w <= 1e-6 (or failing the projection)
// pass through unchanged.
__host__ __device__ __forceinline__ void soft_clip_face(const float4 c[3], uint32_t w,
                                                        uint32_t h, float radius,
                                                        float4 out[3]) {
    const float W = (float)w, H = (float)h;
    float sx[3], sy[3];
    bool valid = true;
    for (int k = 0; k < 3; k++) {
        if (c[k].w <= 1e-6f || !clip_w_valid(c[k].w)) {
            valid = false;
            sx[k] = sy[k] = 0.f;
        } else {
            const ScreenVert v = project_to_screen(c[k].x, c[k].y, c[k].z, c[k].w, W, H);
            sx[k] = v.x;
            sy[k] = v.y;
        }
    }
    float scale = 1.f, cx = 0.f, cy = 0.f;
    if (valid) {
        cx = (sx[0] + sx[1] + sx[2]) / 3.f;
        cy = (sy[0] + sy[1] + sy[2]) / 3.f;
        float d_min = 1e30f;
        for (int k = 0; k < 3; k++) {
            const int k2 = (k + 1) % 3;
            const float ex = sx[k2] - sx[k];
            const float ey = sy[k2] - sy[k];
            const float len = sqrtf(ex * ex + ey * ey);
            if (len < 1e-6f) {
                continue;
            }
            d_min = smin(d_min, fabsf(ex * (cy - sy[k]) - ey * (cx - sx[k])) / len);
        }
        scale = d_min < 1e29f ? smin(1.f + radius / smax(d_min, 1e-3f), 8.f) : 1.f;
    }
    for (int k = 0; k < 3; k++) {
        out[k] = c[k];
        if (valid) {
            const float px = cx + (sx[k] - cx) * scale;
            const float py = cy + (sy[k] - cy) * scale;
            out[k].x = (px / W * 2.f - 1.f) * c[k].w;
            out[k].y = (py / H * 2.f - 1.f) * c[k].w;
        }
    }
}

}  // namespace dressi
