"""Writes the golden fixtures under tests/golden/ from the reference's own CPU
build (oracle/_ref/libdressi_ref.so, compiled from the reference sources by
oracle/Makefile). Inputs are generated with the oracle's seeded scene helpers
and stored next to the outputs, so the fixtures are self-contained data.

    python tests/golden/make_golden.py            # every fixture
    python tests/golden/make_golden.py texture    # the texture path's only
    python tests/golden/make_golden.py dist       # GatherDistGrad's only
    python tests/golden/make_golden.py pbr        # the PBR / IBL path's only
    python tests/golden/make_golden.py peels      # the depth-peeled fits' only

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


def random_orbit_sets(o, n_sets, n_views, seed, dist=3.0):
    """{n_sets, n_views, 16} MVPs of random orbit cameras (inputs only)."""
    rng = np.random.default_rng(seed)
    proj = o.perspective_vk(45.0 * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    out = np.zeros((n_sets, n_views, 16), np.float32)
    for s in range(n_sets):
        for v in range(n_views):
            yaw, pitch = rng.random() * 2 * math.pi, (rng.random() - 0.5) * 2.0
            eye = [dist * math.cos(pitch) * math.sin(yaw), dist * math.sin(pitch),
                   dist * math.cos(pitch) * math.cos(yaw)]
            out[s, v] = o.mat4_mul(proj, o.look_at(eye))
    return out


def tex_fixtures(o, r):
    """Per-op texture scenes: TextureBilinear (in and out of the clamp
    region, 1 / 3 / 4 components), GatherByInverseUVBilinear (covered and
    uncovered inverse-UV entries, anchors near and off the screen edges) and
    the UV-sphere generator."""
    rng = np.random.default_rng(11)
    arrs = {}
    for nc in (1, 3, 4):
        tex = rng.random((5, 7, nc)).astype(np.float32)
        uv = (rng.random((9, 11, 2)) * 1.4 - 0.2).astype(np.float32)
        arrs[f"in_bl{nc}_tex"], arrs[f"in_bl{nc}_uv"] = tex, uv
        arrs[f"out_bl{nc}"] = r.texture_bilinear(tex, uv)
    for name, (sh, sw, th, tw, cov) in {"g_small": (12, 10, 6, 8, 0.7),
                                        "g_sparse": (20, 24, 16, 12, 0.15)}.items():
        gy = rng.standard_normal((sh, sw, 4)).astype(np.float32)
        iv = np.zeros((th, tw, 4), np.float32)
        iv[..., 0] = rng.random((th, tw)) * (sw + 4) - 2
        iv[..., 1] = rng.random((th, tw)) * (sh + 4) - 2
        iv[..., 2] = (rng.random((th, tw)) < cov).astype(np.float32)
        uv = rng.random((sh, sw, 2)).astype(np.float32)
        arrs[f"in_{name}_gy"], arrs[f"in_{name}_iv"], arrs[f"in_{name}_uv"] = gy, iv, uv
        arrs[f"out_{name}"] = r.gather_inv_uv_bilinear(gy, iv, uv)
    pos, uv, faces = r.uv_sphere(16, 8)
    arrs.update(out_uvs16_pos=pos, out_uvs16_uv=uv, out_uvs16_faces=faces)
    p2, _, f2 = r.uv_sphere(128, 64)
    arrs["out_uvs128_counts"] = np.array([len(p2), len(f2)], np.int64)
    np.savez_compressed(os.path.join(OUT, "tex_unit.npz"), **arrs)
    print("wrote tex_unit.npz", len(arrs), "arrays")


def tex_fit_fixture(o, r, name, stacks, slices, screen, tex, views, sets, iters, seed, images):
    pos, uv, faces = o.uv_sphere(stacks, slices)
    mvps = random_orbit_sets(o, sets, views, seed)
    rng = np.random.default_rng(seed + 100)
    gt = rng.random((tex, tex, 4)).astype(np.float32)
    tex0 = np.full((tex, tex, 4), 0.5, np.float32)
    res = r.tex_fit(pos, uv, faces, mvps, screen, gt, tex0, lr=1e-2, iters=iters,
                    want_images=images)
    arrs = dict(in_pos=pos, in_uv=uv, in_faces=faces, in_mvps=mvps, in_gt=gt, in_tex0=tex0,
                in_cfg=np.array([screen, iters, 1e-2], np.float64))
    arrs.update({"out_" + k: v for k, v in res.items()})
    np.savez_compressed(os.path.join(OUT, name), **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items()})


def ds_fixtures(o, r):
    """GatherDistGrad (RasterizeSoft's backward w.r.t. the hard clips) on an
    icosphere L2 at 48^2 for three cameras, gy with some zero pixels."""
    rng = np.random.default_rng(21)
    pos, faces = o.icosphere(2)
    proj = o.perspective_vk(45.0 * 3.14159265 / 180.0, 1.0, 0.1, 10.0)
    s = 48
    nf = len(faces)
    fid = np.repeat(np.arange(nf, dtype=np.float32), 3)[:, None]
    fs = np.arange(3 * nf, dtype=np.float32).reshape(nf, 3)
    vf = r.vertex_faces_tex(faces, len(pos))
    arrs = dict(in_faces=faces, in_vf=vf, in_cfg=np.array([s, 3.0], np.float64))
    for i in range(3):
        eye = [rng.standard_normal() * 0.5, rng.standard_normal() * 0.5, 2.6 + 0.4 * i]
        clip = o.transform_to_clip(pos, o.mat4_mul(proj, o.look_at(eye)))
        soft = r.soft_clip(clip, faces, s, s, 3.0)
        rs = r.rasterize_soft(soft, fid, fs, clip, faces, s, s, 3.0, vtx_faces=vf)
        gy = rng.standard_normal((s, s, 4)).astype(np.float32)
        gy[rng.random((s, s)) < 0.2, 0] = 0.0
        wide, g = r.rasterize_soft_bwd(soft, fid, fs, clip, faces, vf, s, s, 3.0, gy)
        arrs.update({f"in_clip{i}": clip, f"in_rs{i}": rs, f"in_gy{i}": gy,
                     f"out_wide{i}": wide, f"out_g{i}": g})
    np.savez_compressed(os.path.join(OUT, "ds_unit.npz"), **arrs)
    print("wrote ds_unit.npz", len(arrs), "arrays")


def texture_main(o, r):
    tex_fixtures(o, r)
    tex_fit_fixture(o, r, "tex_uvs16_64px_3view_3it.npz", 16, 8, 64, 32, 3, 2, 3, 5, True)
    tex_fit_fixture(o, r, "tex_uvs32_8view_128px_3it.npz", 32, 16, 128, 64, 8, 3, 3, 6, False)
    tex_fit_fixture(o, r, "tex_uvs16_64px_20it.npz", 16, 8, 64, 32, 2, 20, 20, 7, False)


def ibl_fixtures(o, r):
    """Per-op IBL scenes: EquirectSample and its map VJP (1 / 3 / 4
    components; zero-length, pole and seam directions), AvgPool2x2 and its
    VJP (odd sizes), IrradianceConv / PrefilterConv (roughness 0, 0.5, 1) and
    their transposes, PrefilterEnv and the BRDF LUT."""
    rng = np.random.default_rng(31)
    arrs = {}
    for nc in (1, 3, 4):
        m = rng.random((8, 16, nc)).astype(np.float32)
        d = rng.standard_normal((9, 11, 3)).astype(np.float32)
        d[0, 0] = 0.0
        d[0, 1] = [0.0, 1.0, 0.0]
        d[0, 2] = [0.0, -2.0, 0.0]
        d[0, 3] = [-1.0, 0.3, 0.0]
        d[0, 4] = [-1.0, 0.0, -1e-7]
        gy = rng.standard_normal((9, 11, nc)).astype(np.float32)
        arrs.update({f"in_eq{nc}_map": m, f"in_eq{nc}_dir": d, f"in_eq{nc}_gy": gy,
                     f"out_eq{nc}": r.equirect_sample(m, d),
                     f"out_eq{nc}_bwd": r.equirect_sample(m, d, gy)})
    for name, (h, w) in {"pool_odd": (5, 7), "pool_even": (16, 32)}.items():
        x = rng.random((h, w, 3)).astype(np.float32)
        g = rng.standard_normal(((h + 1) // 2, (w + 1) // 2, 3)).astype(np.float32)
        arrs.update({f"in_{name}_x": x, f"in_{name}_gy": g, f"out_{name}": r.avg_pool2x2(x),
                     f"out_{name}_bwd": r.avg_pool2x2(x, g)})
    env = rng.random((8, 16, 3)).astype(np.float32)
    g84 = rng.standard_normal((4, 8, 3)).astype(np.float32)
    g168 = rng.standard_normal((8, 16, 3)).astype(np.float32)
    arrs.update(in_env=env, in_g84=g84, in_g168=g168,
                out_irr=r.irradiance_conv(env, 8, 4), out_irr_bwd=r.irradiance_conv(env, 8, 4, g84))
    for i, rough in enumerate((0.0, 0.5, 1.0)):
        arrs[f"out_pref{i}_16"] = r.prefilter_conv(env, 16, 8, rough)
        arrs[f"out_pref{i}_8"] = r.prefilter_conv(env, 8, 4, rough)
        arrs[f"out_pref{i}_16_bwd"] = r.prefilter_conv(env, 16, 8, rough, g168)
        arrs[f"out_pref{i}_8_bwd"] = r.prefilter_conv(env, 8, 4, rough, g84)
    arrs["out_prefenv"] = r.prefilter_env(env, 8, 4, 0.5, 64)
    arrs["out_lut16"] = r.brdf_lut(16, 16, 64)
    arrs["out_lut64"] = r.brdf_lut(64, 64, 512)
    np.savez_compressed(os.path.join(OUT, "ibl_unit.npz"), **arrs)
    print("wrote ibl_unit.npz", len(arrs), "arrays")


def pbr_scene(o, level, screen, views, tex, ew, eh, seed):
    """A C5-style scene (the layout of opendressi_amd.pbr.make_pbr_scene):
    unit icosphere with equirect uv, the material example's camera ring,
    U[0.05, 0.95] materials, a smooth log-normal env with 3 lobes."""
    pos, faces = o.icosphere(level)
    d = pos.astype(np.float64) / np.linalg.norm(pos, axis=1, keepdims=True)
    uv = np.stack([np.arctan2(d[:, 2], d[:, 0]) / (2 * math.pi) + 0.5,
                   np.arccos(np.clip(d[:, 1], -1, 1)) / math.pi], 1).astype(np.float32)
    fov = np.float32(45.0 * 3.14159265 / 180.0)
    th = np.float32(math.tan(float(fov) * 0.5))
    proj = o.perspective_vk(float(fov), 1.0, 0.1, 10.0)
    mvps = np.zeros((views, 16), np.float32)
    frames = np.zeros((views, 12), np.float32)
    for i in range(views):
        ang = np.float32(2.0 * 3.14159265 * i / views)
        eye = np.array([2.2 * math.sin(ang) * 0.92, 0.85, 2.2 * math.cos(ang) * 0.92], np.float32)
        vm = o.look_at(eye)
        mvps[i] = o.mat4_mul(proj, vm)
        frames[i] = np.concatenate([eye, [-vm[2], -vm[6], -vm[10]],
                                    np.array([vm[0], vm[4], vm[8]], np.float32) * th,
                                    np.array([vm[1], vm[5], vm[9]], np.float32) * th])
    rng = np.random.default_rng(seed)
    gt_albedo = (0.05 + 0.9 * rng.random((tex, tex, 3))).astype(np.float32)
    gt_mr = np.zeros((tex, tex, 3), np.float32)
    gt_mr[..., 1:] = 0.05 + 0.9 * rng.random((tex, tex, 2))
    yy, xx = np.meshgrid((np.arange(eh) + 0.5) / eh, (np.arange(ew) + 0.5) / ew, indexing="ij")
    env = 0.3 * np.exp(0.6 * (np.sin(2 * math.pi * (2 * xx + 0.3)) * np.sin(math.pi * yy * 3)))
    env = env[..., None] * np.ones(3)
    dirs = np.stack([np.sin(math.pi * yy) * np.cos((xx - 0.5) * 2 * math.pi),
                     np.cos(math.pi * yy),
                     np.sin(math.pi * yy) * np.sin((xx - 0.5) * 2 * math.pi)], -1)
    for k in range(3):
        mu = rng.standard_normal(3)
        mu /= np.linalg.norm(mu)
        ang = np.arccos(np.clip(dirs @ mu, -1, 1))
        sig = 0.15 + 0.2 * rng.random()
        env = env + np.exp(-ang ** 2 / (2 * sig * sig))[..., None] * (4 + 12 * rng.random(3))
    return dict(pos=pos, normal=pos.copy(), uv=uv, faces=faces, mvps=mvps, frames=frames,
                light=np.array([2, 2, 2, 20, 20, 20], np.float32), screen=screen, levels=6,
                lr=1e-2, gt_albedo=gt_albedo, gt_mr=gt_mr, gt_env=env.astype(np.float32),
                albedo0=np.full((tex, tex, 3), 0.5, np.float32),
                mr0=np.full((tex, tex, 3), 0.5, np.float32),
                env0=np.full((eh, ew, 3), 0.3, np.float32))


def pbr_fit_fixture(o, r, name, level, screen, views, tex, ew, eh, iters, seed, images):
    sc = pbr_scene(o, level, screen, views, tex, ew, eh, seed)
    res = r.pbr_fit(sc, iters=iters, want_images=images)
    arrs = {"in_" + k: (v if isinstance(v, np.ndarray) else np.array(v)) for k, v in sc.items()}
    arrs.update({"out_" + k: v for k, v in res.items()})
    np.savez_compressed(os.path.join(OUT, name), **arrs)
    print("wrote", name, {k: v.shape for k, v in arrs.items()})


def peel_main(o, r):
    """HardSoftRas fits with K = 2 and 3 depth peels (the example's --peels,
    examples/silhouette_optimization/run.cpp:302-343): ico3, 2 orbit views,
    96 px, 3 iterations, from the reference build with the peel loop."""
    import ctypes as C
    for k in (2, 3):
        r.fn("set_peels")(C.c_uint32(k))
        try:
            fit_fixture(o, r, f"hsr_peel{k}_ico3_2view_96px_3it.npz", 3, 0.05, 3,
                        orbit_mvps(o, 2), 96, 3, 1e-3, True)
        finally:
            r.fn("set_peels")(C.c_uint32(1))


def pbr_main(o, r):
    ibl_fixtures(o, r)
    pbr_fit_fixture(o, r, "pbr_ico2_48px_2view_3it.npz", 2, 48, 2, 16, 64, 32, 3, 41, True)
    pbr_fit_fixture(o, r, "pbr_ico3_96px_3view_2it.npz", 3, 96, 3, 64, 256, 128, 2, 42, False)


def main():
    build(ref=True)
    o, r = Oracle(), Reference()
    if sys.argv[1:] == ["texture"]:
        texture_main(o, r)
        return
    if sys.argv[1:] == ["pbr"]:
        pbr_main(o, r)
        return
    if sys.argv[1:] == ["dist"]:
        ds_fixtures(o, r)
        return
    if sys.argv[1:] == ["peels"]:
        peel_main(o, r)
        return
    ds_fixtures(o, r)
    peel_main(o, r)
    pbr_main(o, r)
    texture_main(o, r)
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
