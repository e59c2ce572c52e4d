"""Writes the golden fixtures under tests/golden/ from the reference's own CPU
build (oracle/_ref/libdressi_ref.so, compiled from the reference sources by
oracle/Makefile). Inputs are generated with the oracle's seeded scene helpers
and stored next to the outputs, so the fixtures are self-contained data.

    python tests/golden/make_golden.py

Each .npz holds `in_*` arrays (inputs) and `out_*` arrays (reference outputs).
"""
from __future__ import annotations

import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.pyoracle import Oracle, Reference, build  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def clip_of_screen(sx, sy, z, screen, w=1.0):
    """Clip position whose projection lands on screen pixel coords (sx, sy)
    (the reference tests' ClipOfScreen helper convention, tests/softras_scene.h)."""
    return [(sx / screen * 2 - 1) * w, (sy / screen * 2 - 1) * w, z * w, w]


def orbit_mvps(o, n, dist=3.0, pitch_deg=15.0, fov_deg=45.0):
    proj = o.perspective_vk(fov_deg * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    out = []
    for v in range(n):
        yaw = math.radians(360.0 * v / n)
        pitch = math.radians(pitch_deg)
        eye = [dist * math.cos(pitch) * math.sin(yaw), dist * math.sin(pitch),
               dist * math.cos(pitch) * math.cos(yaw)]
        out.append(o.mat4_mul(proj, o.look_at(eye)))
    return np.stack(out).astype(np.float32)


def front_mvp(o, dist=3.0, fov_deg=45.0):
    proj = o.perspective_vk(fov_deg * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    return o.mat4_mul(proj, o.look_at([0.0, 0.0, dist]))[None].astype(np.float32)


def fit_fixture(o, r, name, level, noise, seed, mvps, screen, iters, lr, images):
    pos, faces = o.icosphere(level)
    tgt = (pos * (1.0 + noise * o.randn(seed, len(pos)))[:, None]).astype(np.float32)
    res = r.hsr_fit(pos, faces, tgt, faces, mvps, screen, lr=lr, iters=iters, want_images=images)
    arrs = dict(in_pos=pos, in_faces=faces, in_tgt_pos=tgt, in_mvps=mvps,
                in_cfg=np.array([screen, iters, 3.0, 8, lr], np.float64))
    for k, v in res.items():
        if k == "rs0":
            # keep the ID/coverage channels exactly plus dist / hard_z
            arrs["out_rs0"] = v
        else:
            arrs["out_" + k] = v
    np.savez_compressed(os.path.join(OUT, name), **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items()})


def op_fixtures(o, r):
    s = 16
    # SoftRas.ForwardDistProfile / DepthShiftNearWins scenes (tests/test_softras.cpp)
    scenes = {
        "profile": ([clip_of_screen(4, 4, 0.5, s), clip_of_screen(12, 4, 0.5, s),
                     clip_of_screen(4, 12, 0.5, s)], [[0, 1, 2]]),
        "depth": ([clip_of_screen(4, 4, 0.2, s), clip_of_screen(12, 4, 0.2, s),
                   clip_of_screen(4, 12, 0.2, s), clip_of_screen(4, 4, 0.8, s),
                   clip_of_screen(12, 4, 0.8, s), clip_of_screen(4, 12, 0.8, s)],
                  [[3, 4, 5], [0, 1, 2]]),
        "generic": ([clip_of_screen(4.3, 3.8, 0.5, s), clip_of_screen(12.4, 5.2, 0.5, s, 1.3),
                     clip_of_screen(5.1, 12.6, 0.5, s), clip_of_screen(11.2, 12.1, 0.5, s)],
                    [[0, 1, 2], [1, 3, 2]]),
    }
    arrs = {}
    for name, (clip, faces) in scenes.items():
        clip = np.array(clip, np.float32)
        faces = np.array(faces, np.float32)
        nf = len(faces)
        soft = r.soft_clip(clip, faces, s, s, 3.0)
        fid = np.repeat(np.arange(nf, dtype=np.float32), 3)
        fsoft = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
        vf = r.vertex_faces_tex(faces, len(clip))
        rs = r.rasterize_soft(soft, fid, fsoft, clip, faces, s, s, 3.0, vtx_faces=vf)
        hard = r.rasterize(clip, np.ones((len(clip), 1), np.float32), faces, s, s)
        ids = r.rasterize_face_id(clip, faces, s, s)
        arrs[f"in_{name}_clip"] = clip
        arrs[f"in_{name}_faces"] = faces
        arrs[f"out_{name}_soft_clip"] = soft
        arrs[f"out_{name}_rasterize_soft"] = rs
        arrs[f"out_{name}_rasterize"] = hard
        arrs[f"out_{name}_face_id"] = ids
    # Stochastic FaceFetchBwd parity scene (tests/test_softras_gpu.cpp:164-224:
    # seed 7, n = 8) plus the exact mode and LookupFacesBwd
    clip = arrs["in_generic_clip"]
    faces = arrs["in_generic_faces"]
    ids = arrs["out_generic_face_id"]
    rng = np.random.default_rng(5)
    tri = [o.lookup_faces(clip, faces, k) for k in range(3)]
    gy = rng.standard_normal((s, s, 4)).astype(np.float32)
    vf = r.vertex_faces_tex(faces, len(clip))
    arrs["in_ffb_gy"] = gy
    arrs["out_ffb_n8_seed7"] = r.face_fetch_bwd(gy, ids, tri[0], tri[1], tri[2], 7.0, 3.0, 8)
    arrs["out_ffb_n0"] = r.face_fetch_bwd(gy, ids, tri[0], tri[1], tri[2], 7.0, 3.0, 0)
    gtri = rng.standard_normal((len(faces), 4)).astype(np.float32)
    arrs["in_lfb_gy"] = gtri
    for k in range(3):
        arrs[f"out_lfb_k{k}"] = r.lookup_faces_bwd(gtri, faces, vf, k)
    arrs["out_face_fetch"] = r.face_fetch(tri[1], ids)
    np.savez_compressed(os.path.join(OUT, "ops_unit.npz"), **arrs)
    print("wrote ops_unit.npz", len(arrs), "arrays")


def aa_fixtures(o, r):
    """AntiAlias fwd / bwd scenes of tests/test_antialias.cpp:153-273 (16x16):
    the generic-position triangle, the same with one w = 1.3 vertex, and the
    occlusion scene (full-screen back triangle, shaded front triangle)."""
    s = 16
    scenes = {
        "generic": ([clip_of_screen(4.3, 3.8, 0.5, s), clip_of_screen(12.4, 5.2, 0.5, s),
                     clip_of_screen(5.1, 12.6, 0.5, s)], [[0, 1, 2]], None),
        "w13": ([clip_of_screen(4.3, 3.8, 0.5, s), clip_of_screen(12.4, 5.2, 0.5, s, 1.3),
                 clip_of_screen(5.1, 12.6, 0.5, s)], [[0, 1, 2]], None),
        "occlusion": ([clip_of_screen(-40, -40, 0.8, s), clip_of_screen(100, -40, 0.8, s),
                       clip_of_screen(-40, 100, 0.8, s), clip_of_screen(5.2, 4.7, 0.2, s),
                       clip_of_screen(11.6, 6.3, 0.2, s), clip_of_screen(6.4, 11.8, 0.2, s)],
                      [[0, 1, 2], [3, 4, 5]], [0.2, 0.2, 0.2, 0.9, 0.9, 0.9]),
    }
    rng = np.random.default_rng(11)
    arrs = {}
    for name, (clip, faces, shade) in scenes.items():
        clip = np.array(clip, np.float32)
        faces = np.array(faces, np.float32)
        attr = np.ones(len(clip), np.float32) if shade is None else np.array(shade, np.float32)
        img = r.rasterize(clip, attr, faces, s, s)[..., 0]
        tri = r.rasterize_face_id(clip, faces, s, s)
        vf = r.vertex_faces_tex(faces, len(clip))
        gy = rng.standard_normal((s, s)).astype(np.float32)
        g_img, wide, g_vtx = r.antialias_bwd(gy, img, tri, clip, faces, vf, 7.0, 8)
        _, _, g_vtx0 = r.antialias_bwd(gy, img, tri, clip, faces, vf, 7.0, 0)
        arrs.update({f"in_{name}_clip": clip, f"in_{name}_faces": faces,
                     f"in_{name}_img": img, f"in_{name}_tri": tri, f"in_{name}_vf": vf,
                     f"in_{name}_gy": gy,
                     f"out_{name}_aa": r.antialias(img, tri, clip, faces, vf),
                     f"out_{name}_bwd_img": g_img, f"out_{name}_bwd_vtx_wide_n8_seed7": wide,
                     f"out_{name}_bwd_vtx_n8_seed7": g_vtx, f"out_{name}_bwd_vtx_n0": g_vtx0})
    np.savez_compressed(os.path.join(OUT, "aa_unit.npz"), **arrs)
    print("wrote aa_unit.npz", len(arrs), "arrays")


def aa_fit_fixture(o, r, name, level, noise, seed, mvps, screen, iters, lr, images):
    pos, faces = o.icosphere(level)
    tgt = (pos * (1.0 + noise * o.randn(seed, len(pos)))[:, None]).astype(np.float32)
    res = r.aa_fit(pos, faces, tgt, faces, mvps, screen, lr=lr, iters=iters, want_images=images)
    arrs = dict(in_pos=pos, in_faces=faces, in_tgt_pos=tgt, in_mvps=mvps,
                in_cfg=np.array([screen, iters, 8, lr], np.float64))
    arrs.update({"out_" + k: v for k, v in res.items()})
    np.savez_compressed(os.path.join(OUT, name), **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items()})


def main():
    build(ref=True)
    o, r = Oracle(), Reference()
    op_fixtures(o, r)
    aa_fixtures(o, r)
    aa_fit_fixture(o, r, "aa_ico3_64px_5it.npz", 3, 0.05, 1, front_mvp(o), 64, 5, 1e-3, True)
    aa_fit_fixture(o, r, "aa_ico4_4view_128px_3it.npz", 4, 0.05, 2, orbit_mvps(o, 4), 128, 3,
                   1e-3, True)
    aa_fit_fixture(o, r, "aa_c1_256px_50it.npz", 3, 0.05, 1, front_mvp(o), 256, 50, 1e-3, False)
    # C1-shaped fits: ico3 front camera. Small screens keep the files small;
    # the 256^2 x 50-iteration run stores only the parameter trajectory.
    fit_fixture(o, r, "hsr_ico3_64px_5it.npz", 3, 0.05, 1, front_mvp(o), 64, 5, 1e-3, True)
    fit_fixture(o, r, "hsr_c1_256px_50it.npz", 3, 0.05, 1, front_mvp(o), 256, 50, 1e-3, False)
    # C2-shaped: ico4, 4-view orbit (pitch 15 deg), reduced screen / iterations
    fit_fixture(o, r, "hsr_ico4_4view_128px_3it.npz", 4, 0.05, 2, orbit_mvps(o, 4), 128, 3,
                1e-3, True)


if __name__ == "__main__":
    main()
