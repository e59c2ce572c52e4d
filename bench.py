"""Benchmark of the fused silhouette-fit iteration (fwd + bwd + Adam) on one
MI355X.

    python bench.py [--steps K] [--warmup W] [--workload c4_hsr|c4|c5|c3|c2|c1]

A step is one iteration of the silhouette fit. HardSoftRas (c4_hsr, c2, c1):
per view clip transform, SoftClip, tile-binned RasterizeSoft, the per-pixel
soft-probability chain and L2 loss image, the stochastic FaceFetchBwd gather
fused with the chain's backward, LookupFacesBwd + clip->pos chain, Adam. AA
(c4): clip transform, tile-binned hard raster of face ids, AntiAlias of the
mask + L2 loss image, the stochastic AntiAliasBwdVtx gather, ColSum +
clip->pos chain, Adam. Texture (c3): per view clip transform + ScreenAttr,
hard raster of face ids, g_uv / g_mask interpolation and bilinear samples of
the texture and the target texture + RGB L2 loss image, then per texel the
inverse-UV gather of every view and Adam. PBR / IBL (c5): the env's pooling
chain, IrradianceConv + 6 PrefilterConv levels, per pixel the split-sum
shading forward + L1 loss + backward with the map gradients scattered in
fixed point, the convolutions' transposes, the static texture gather list,
Adam on albedo / mr / env. One hipGraph launch per step. Inputs (mesh, Adam
state, target images) are resident in HBM before the timed region. Prints
ONE JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "fwd+bwd+Adam iterations/sec at 512²/2048² silhouette; achieved HBM GB/s"
HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s


def iteration_bytes_aa(n_views: int, s: int, n_faces: int, n_verts: int) -> float:
    """Compulsory bytes of one AA-technique iteration (per pixel and view:
    target read, 8-byte visibility write and read; per view: clip, faces,
    adjacency, per-vertex gradient; loss image; Adam state)."""
    return n_views * (20.0 * s * s + 12.0 * n_faces + 88.0 * n_verts) + 4.0 * s * s + 72.0 * n_verts


def kernel_bytes_aa(n_views: int, s: int, n_faces: int, n_verts: int, samples: int = 8) -> dict:
    """Algorithmic bytes per launch of the AA-technique kernels.

    setup:   positions (12 B/vertex) and faces in, clip (16 B/vertex) and the
             screen triangles (36 B/face) out, per view
    raster:  screen triangles in, 4-byte face-id image out, per view
    fwd:     face-id + target in, pred out per view, loss image out
    face_bwd: corner clips (48 B) in, corner gradients (48 B) out, and a
             face-id + pred + target read (12 B) per sample, per face and view
    vertex_adam: as the HardSoftRas vertex kernel
    """
    n, S2, F, V = n_views, float(s) * s, float(n_faces), float(n_verts)
    return {
        "k_aa_setup": n * (28.0 * V + 48.0 * F),
        "k_aa_raster": n * (4.0 * S2 + 36.0 * F),
        "k_aa_fwd": n * 12.0 * S2 + 4.0 * S2,
        "k_aa_face_bwd": n * F * (96.0 + 12.0 * samples),
        "k_aa_vertex_adam": n * 120.0 * V + 72.0 * V,
    }


def iteration_bytes_tex(n_views: int, s: int, n_faces: int, n_verts: int, texels: int) -> float:
    """Compulsory bytes of one texture iteration (per pixel and view: 8-byte
    visibility write and read; per view: faces, clip, uv, screen attribute;
    the loss image; per texel: texture read, target texture read, gradient
    write + read, Adam state 3 reads + 3 writes, 16 B each)."""
    return (n_views * (16.0 * s * s + 12.0 * n_faces + 40.0 * n_verts) + 4.0 * s * s
            + 160.0 * texels)


def kernel_bytes_tex(n_views: int, s: int, n_faces: int, n_verts: int, texels: int) -> dict:
    """Compulsory bytes per launch of the texture-plan kernels, the
    iteration's compulsory traffic (iteration_bytes_tex) split over the
    kernels that need it; the plan's own intermediates (per-pixel g_uv and
    d loss / d sample) are not counted.

    clip:     positions and uv in, clip (16 B) and screen attribute (8 B) out,
              per vertex and view
    setup:    clip in, faces in, per view
    raster:   the 8-byte visibility word (depth | id) written per pixel and
              view
    fwd:      the visibility word read per pixel and view, the loss image
              out, the texture and the target texture read (16 B + 16 B per
              texel)
    bwd_adam: the texel gradient written and read (32 B per texel, as the
              iteration model counts it; here it stays in registers) and
              texture / m / v read and written (96 B per texel)
    The shares add up to iteration_bytes_tex.
    """
    n, S2, F, V, T = n_views, float(s) * s, float(n_faces), float(n_verts), float(texels)
    return {
        "k_tex_clip": n * 32.0 * V,
        "k_aa_setup": n * (8.0 * V + 12.0 * F),
        "k_aa_raster": n * 8.0 * S2,
        "k_tex_fwd": n * 8.0 * S2 + 4.0 * S2 + 32.0 * T,
        "k_tex_bwd_adam": 128.0 * T,
    }


def iteration_bytes_pbr(n_views: int, s: int, n_faces: int, n_verts: int, texels: int,
                        env_texels: int) -> float:
    """Compulsory bytes of one PBR / IBL iteration (per pixel and view: the
    precomputed target RGB, the G-buffer and the material gradient; the loss;
    per material texel: albedo + mr read and written, their Adam state and
    gradient; per env texel: env, Adam state, gradient)."""
    return (n_views * (28.0 * s * s + 12.0 * n_faces + 76.0 * n_verts) + 4.0 * s * s
            + 200.0 * texels + 120.0 * env_texels)


def kernel_bytes_pbr(n_views: int, s: int, texels: int, env_texels: int, pooled: int,
                     map_texels: int, gather_maps: list) -> dict:
    """Algorithmic bytes per launch of the PBR-plan kernels.

    pool:       env read (12 B/texel), pooled sources written (12 B/texel)
    conv_fwd:   pooled sources read, irradiance + prefilter maps written
    shade:      per pixel and view the target RGB (12 B) and the G-buffer the
                shading needs (material uv, normal, position: 16 B packed):
                28 B; its per-pixel material gradient is counted in tex_adam
    map_gather: per pixel and view its two uv pairs (16 B) and its two
                map-gradient seeds (32 B) read; per (map, view, band, texel)
                one 16 B partial written
    tile_sum:   per map with bands > 1: the band partials read, one 16 B
                sum per (view, texel) written
    view_sum:   per map texel the views' sums read, one 16 B gradient written
    conv_bwd:   map gradients read, source gradients written
    env_adam:   background gradient, source gradients, env + m + v in and out
    tex_adam:   per-pixel material gradients (20 B/pixel) gathered once,
                albedo + mr with their Adam state in and out (96 B/texel)
    loss:       one partial per workgroup
    """
    n, S2, T, E = n_views, float(s) * s, float(texels), float(env_texels)
    band_texels = sum(float(w * h * k) for w, h, k in gather_maps)
    split_texels = sum(float(w * h * k) for w, h, k in gather_maps if k > 1)
    split_maps = sum(float(w * h) for w, h, k in gather_maps if k > 1)
    all_maps = sum(float(w * h) for w, h, _ in gather_maps)
    return {
        "k_pbr_pool": 12.0 * E + 12.0 * pooled,
        "k_pbr_conv_fwd": 12.0 * pooled + 12.0 * map_texels,
        "k_pbr_shade": n * 28.0 * S2,
        "k_pbr_map_gather": n * 48.0 * S2 + 16.0 * n * band_texels,
        "k_pbr_tile_sum": 16.0 * n * (split_texels + split_maps),
        "k_pbr_view_sum": 16.0 * (n + 1) * all_maps,
        "k_pbr_conv_bwd": 12.0 * map_texels + 12.0 * pooled,
        "k_pbr_env_adam": 24.0 * E + 72.0 * E,
        "k_pbr_tex_adam": n * 20.0 * S2 + 96.0 * T,
        "k_pbr_loss_blocks": 16.0 * n * S2 / 256.0,
        "k_pbr_loss": 16.0 * n * S2 / 65536.0,
    }


# FP32 operations (add, sub, mul, div, abs) per pixel of k_pbr_shade, counted
# from the shading arithmetic of one pixel:
#   foreground: forward 349 (material bilinear weights 12 + albedo / mr taps
#     48 + ao 8; irradiance weights and taps 36; two active prefilter levels
#     2 x 45; LUT weights and taps 28; GGX D / G / denominators 27; per
#     channel Fresnel, diffuse, specular, ambient 3 x 31; lod 1; tone map 6),
#     L1 loss and d loss / d hdr 30, backward to albedo / metallic /
#     roughness 205, map-gradient VJP of the irradiance and two prefilter tap
#     sets 78 (12 weighted taps and their accumulation each, + 6)
#   background with env: env weights and taps 36, tone map 6, loss 30, env
#     map-gradient VJP 24
#   neither: tone map of zero 6, loss 30
SHADE_FLOPS = {"fg": 662.0, "env": 96.0, "none": 36.0}
# per (output texel, source texel) pair of the dense IBL convolutions: the
# direction dot product, the GGX (or cosine) weight, the weighted RGB sum
CONV_FLOPS_PER_PAIR = 30.0
VALU_PEAK = 157.3e12  # MI355X dense FP32 vector, FLOP/s


def kernel_flops_pbr(pixel_classes: dict, conv_pairs: float) -> dict:
    """Algorithmic FP32 operations per launch of the PBR plan's VALU-bound
    kernels: the shading kernel per pixel class, each convolution per
    (output, source) pair (irradiance + every prefilter level)."""
    shade = sum(SHADE_FLOPS[k] * float(n) for k, n in pixel_classes.items())
    return {"k_pbr_shade": shade,
            "k_pbr_conv_fwd": CONV_FLOPS_PER_PAIR * conv_pairs,
            "k_pbr_conv_bwd": CONV_FLOPS_PER_PAIR * conv_pairs}


def iteration_bytes(n_views: int, s: int, n_faces: int, n_verts: int) -> float:
    """Compulsory bytes of one HSR iteration (per pixel and view: target read,
    8-byte visibility write and read; per view: clip, soft clip, corner clips,
    per-face corner gradients, faces, adjacency, per-vertex gradient; the loss
    image; Adam pos/m/v read + write)."""
    return n_views * (20.0 * s * s + 300.0 * n_faces + 88.0 * n_verts) + 4.0 * s * s + 72.0 * n_verts


def kernel_bytes(n_views: int, s: int, n_faces: int, n_verts: int, samples: int = 8) -> dict:
    """Algorithmic bytes per launch of each kernel of the iteration.

    setup:      positions (12 B/vertex) and faces (12 B/face) in, soft + hard
                corner clips (96 B/face) out, per view
    raster:     soft + hard corner clips in, 4-byte face-id image out, per view
    loss:       face-id + target image in per view, loss image out
    face_bwd:   corner clips (48 B) in, corner gradients (48 B) out, and a
                face-id + target read (8 B) per sample, per face and view
    vertex_adam: adjacency (24 B) + corner gradients (96 B) per vertex and
                view, Adam pos/m/v read + write (72 B/vertex)
    """
    n, S2, F, V = n_views, float(s) * s, float(n_faces), float(n_verts)
    return {
        "k_hsr_setup": n * (12.0 * V + 12.0 * F + 96.0 * F),
        "k_hsr_raster": n * (4.0 * S2 + 96.0 * F),
        "k_hsr_loss": n * 8.0 * S2 + 4.0 * S2,
        "k_hsr_face_bwd": n * F * (96.0 + 8.0 * samples),
        "k_hsr_vertex_adam": n * 120.0 * V + 72.0 * V,
    }


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summaries (profiles/traffic.json, per workload: FETCH_SIZE + WRITE_SIZE
    per dispatch, scaled by the counters' reading for a plain copy of known
    size), or None when no summary covers that kernel and workload."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as fh:
            rec = json.load(fh).get("workloads", {}).get(workload, {})
    except (OSError, ValueError, AttributeError):
        return None
    for k in rec.get("kernels", []):
        if k.get("kernel") == kernel:
            return k["fetch_bytes"] + k["write_bytes"]
    return None


def cpu_info() -> str:
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True).stdout
        for line in out.splitlines():
            if line.startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return platform.processor() or "unknown"


def cpu_baseline_tex(workload) -> dict:
    """The oracle's texture fit (single thread) on a bounded sample: one
    iteration with ONE of the workload's views at full resolution, scaled to
    iterations/s of all views (the views are independent until the texel
    gradient; Adam is negligible)."""
    import opendressi_amd as od
    from oracle.pyoracle import ORACLE_SO, Oracle, build
    if not os.path.exists(ORACLE_SO):
        build()
    pos, uv, faces, mvps, gt, tex0 = od.make_tex_scene(workload)
    o = Oracle()
    t0 = time.perf_counter()
    o.tex_fit(pos, uv, faces, mvps[:1, :1], workload.screen, gt, tex0, lr=workload.lr, iters=1,
              want_images=False)
    dt = time.perf_counter() - t0
    n = mvps.shape[1]
    return {"value": 1.0 / (dt * n), "unit": "iterations/s", "cores": 1, "kind": "port",
            "sample": (f"1 iteration of 1 of {n} views at {workload.screen}^2 with the "
                       f"{workload.tex}^2 texture, {dt:.2f} s, scaled x{n}; host CPU: "
                       f"{cpu_info()}, nproc {os.cpu_count()}")}


def cpu_baseline_pbr(workload) -> dict:
    """The oracle's PBR / IBL fit (single thread) on a bounded sample: ONE of
    the workload's views at full resolution with the full maps, timed for 1
    and for 2 iterations; the difference is one iteration of that view
    (set-up excluded), scaled to all views (this counts the view-independent
    env convolutions once per view, so it understates the CPU rate)."""
    from opendressi_amd.pbr import workload_scene
    from oracle.pyoracle import ORACLE_SO, Oracle, build
    if not os.path.exists(ORACLE_SO):
        build()
    sc = workload_scene(workload)
    sc1 = dict(sc, mvps=sc["mvps"][:1], frames=sc["frames"][:1])
    o = Oracle()
    times = []
    for iters in (1, 2):
        t0 = time.perf_counter()
        o.pbr_fit(sc1, iters=iters, want_images=False)
        times.append(time.perf_counter() - t0)
    dt = max(times[1] - times[0], 1e-9)
    n = len(sc["mvps"])
    return {"value": 1.0 / (dt * n), "unit": "iterations/s", "cores": 1, "kind": "port",
            "sample": (f"1 of {n} views at {workload.screen}^2, {workload.tex}^2 textures, "
                       f"{workload.env_w}x{workload.env_h} env: 1 and 2 iterations "
                       f"({times[0]:.1f} s, {times[1]:.1f} s), difference scaled x{n}; host "
                       f"CPU: {cpu_info()}, nproc {os.cpu_count()}")}


def cpu_baseline(workload) -> dict:
    """The oracle (C restatement of the reference CPU evaluator, single
    thread) on a bounded sample: ONE of the workload's views at full
    resolution, timed for 1 and for 2 iterations; the difference is one
    steady-state iteration of that view (the static target raster, which
    the reference prunes after its warm-up, and the set-up drop out),
    scaled to iterations/s of all views (views are independent until the
    per-vertex gradient; the Adam step is negligible)."""
    import opendressi_amd as od
    from oracle.pyoracle import ORACLE_SO, Oracle, build
    if not os.path.exists(ORACLE_SO):
        build()
    pos, faces, tgt, mvps = od.make_scene(workload)
    o = Oracle()
    fit = o.aa_fit if workload.technique == "aa" else o.hsr_fit
    times = []
    for iters in (1, 2):
        t0 = time.perf_counter()
        fit(pos, faces, tgt, faces, mvps[:1], workload.screen, lr=workload.lr, iters=iters,
            want_images=False)
        times.append(time.perf_counter() - t0)
    dt = max(times[1] - times[0], 1e-9)
    n = len(mvps)
    return {"value": 1.0 / (dt * n), "unit": "iterations/s", "cores": 1, "kind": "port",
            "sample": (f"1 of {n} views at {workload.screen}^2: 1 and 2 iterations "
                       f"({times[0]:.2f} s, {times[1]:.2f} s), the difference (one iteration "
                       f"without the static target raster) scaled x{n}; host CPU: "
                       f"{cpu_info()}, nproc {os.cpu_count()}")}


BENCH_KEYS = ("example", "device", "platform", "os", "cpu", "cpu_cores", "ram_gb", "funcs",
              "substages", "stages", "technique", "screen", "views", "iters", "samples", "peels",
              "single_view", "median_ms_per_iter", "warmup_excluded", "warmup_ms",
              "first_build_ms", "mean_iou", "loss_drop")
# decimals of the record's fixed-notation reals (BenchRecord::add(key, double,
# precision), default 4: examples/common/bench.h:33, run.cpp:686-703)
BENCH_DECIMALS = {"ram_gb": 1, "median_ms_per_iter": 4, "warmup_ms": 1, "first_build_ms": 1,
                  "mean_iou": 4, "loss_drop": 1}


def median_upper(samples) -> float:
    """The reference's MedianMs (examples/common/bench.cpp:145-151): the
    element at n / 2 of the sorted samples (the upper median), 0 if none."""
    s = sorted(samples)
    return float(s[len(s) // 2]) if s else 0.0


def bench_fields(device: str, cpu: str, cores: int, ram_gb: float, kernels: int,
                 technique: str, screen: int, views: int, iters: int, iter_ms,
                 mean_iou: float, first_loss: float, last_loss: float) -> dict:
    """The silhouette example's bench.json record
    (examples/silhouette_optimization/run.cpp:573-587, 676-702;
    examples/common/bench.cpp:145-209) from per-execStep wall times
    `iter_ms` of the whole run: the first min(20, iters / 2) are the warm-up
    (the first of them is first_build_ms), the median of the rest is the
    upper median. The packing counts describe this executor: `funcs` and
    `substages` are the fused kernels of one iteration, `stages` the one
    hipGraph launch per iteration."""
    warm_n = min(20, iters // 2)
    warm, steady = list(iter_ms[:warm_n]), list(iter_ms[warm_n:])
    median = median_upper(steady)
    warm_ms = max(0.0, sum(warm) - median * len(warm))
    fields = {
        "example": "silhouette_optimization", "device": device, "platform": "linux",
        "os": f"{platform.system()} {platform.release()}", "cpu": cpu, "cpu_cores": int(cores),
        "ram_gb": float(ram_gb), "funcs": int(kernels), "substages": int(kernels),
        "stages": 1, "technique": technique, "screen": int(screen), "views": int(views),
        "iters": int(iters), "samples": 8, "peels": 1, "single_view": views == 1,
        "median_ms_per_iter": float(median), "warmup_excluded": int(warm_n),
        "warmup_ms": float(warm_ms), "first_build_ms": float(warm[0] if warm else 0.0),
        "mean_iou": float(mean_iou),
        "loss_drop": float(first_loss / max(last_loss, 1e-12)),
    }
    assert tuple(fields) == BENCH_KEYS
    return fields


def bench_json_text(fields: dict) -> str:
    """The record as the reference writes it (examples/common/bench.cpp:
    187-209): one object, no spaces, strings quoted as given, integers plain,
    booleans true / false, reals in fixed notation with their key's
    decimals."""
    parts = []
    for k, v in fields.items():
        if isinstance(v, bool):
            val = "true" if v else "false"
        elif isinstance(v, int):
            val = str(v)
        elif isinstance(v, float):
            val = f"{v:.{BENCH_DECIMALS[k]}f}"
        else:
            val = f'"{v}"'
        parts.append(f'"{k}":{val}')
    return "{" + ",".join(parts) + "}\n"


def bench_record(workload: str, path: str) -> None:
    """The reference example's bench.json record for a silhouette workload:
    the fit run from its start for the workload's iteration count, each
    execStep timed to a host synchronisation; after the loop one more
    execStep, then the mean IoU of the predictions and the target masks
    (> 0.5) over the views and the last loss (run.cpp:640-662)."""
    import opendressi_amd as od
    from opendressi_amd import _lib
    w = od.WORKLOADS[workload]
    ctx = od.Context(0)
    fit = od.SilhouetteFit.from_workload(ctx, workload, keep_pred=True)
    iter_ms = []
    first_loss = None
    for i in range(w.iters):
        t = time.perf_counter()
        fit.step(1)
        fit.synchronize()
        iter_ms.append((time.perf_counter() - t) * 1e3)
        if i == 0:
            first_loss = fit.loss()
    fit.step(1)
    fit.synchronize()
    last_loss = fit.loss()
    pred, tgt = fit.read(_lib.BUF_PRED) > 0.5, fit.read(_lib.BUF_TARGET) > 0.5
    ious = [float((p & t).sum()) / max(float((p | t).sum()), 1.0) for p, t in zip(pred, tgt)]
    try:
        ram_gb = os.sysconf("SC_PAGE_SIZE") * os.sysconf("SC_PHYS_PAGES") / 2**30
    except (ValueError, OSError):
        ram_gb = 0.0
    fields = bench_fields(ctx.device_name, cpu_info(), os.cpu_count() or 0, ram_gb,
                          len(fit.profile(1)), "hardsoftras" if w.technique == "hsr" else "aa",
                          w.screen, w.views, w.iters, iter_ms, float(np.mean(ious)), first_loss,
                          last_loss)
    with open(path, "w") as fh:
        fh.write(bench_json_text(fields))
    fit.close()
    ctx.close()


def metric_point(name: str, steps: int, warmup: int) -> dict:
    """Iterations/s of another workload (graph replays, inputs resident):
    the metric's other resolution points (c1, c2, c4) and the texture (c3)
    and PBR / IBL (c5) fits, each with its iteration's fraction of the HBM
    roofline; c5 adds its shading kernel's FP32 VALU fraction (from a short
    eager profile, HIP events between the kernels)."""
    import opendressi_amd as od
    ctx = od.Context(0)
    extra = {}
    if name in od.TEX_WORKLOADS:
        w = od.TEX_WORKLOADS[name]
        fit = od.TextureFit.from_workload(ctx, name)
        nb = iteration_bytes_tex(fit.n_views, fit.screen, fit.n_faces, fit.n_verts,
                                 fit.tex_w * fit.tex_h)
        desc = (f"{name}: texture {w.screen}^2 x {w.views} views, UV sphere "
                f"{w.stacks}x{w.slices}, {w.tex}^2 RGBA")
    elif name in od.PBR_WORKLOADS:
        w = od.PBR_WORKLOADS[name]
        fit = od.PbrFit.from_workload(ctx, name)
        nb = iteration_bytes_pbr(fit.n_views, fit.screen, fit.n_faces, fit.n_verts,
                                 fit.tex_w * fit.tex_h, fit.env_w * fit.env_h)
        desc = (f"{name}: PBR/IBL {w.screen}^2 x {w.views} views, icosphere L{w.level}, "
                f"{fit.tex_w}^2 materials, {fit.env_w}x{fit.env_h} env")
    else:
        w = od.WORKLOADS[name]
        fit = od.SilhouetteFit.from_workload(ctx, name)
        nb = (iteration_bytes_aa if w.technique == "aa" else iteration_bytes)(
            fit.n_views, fit.screen, fit.n_faces, fit.n_verts)
        desc = (f"{name}: {'AA' if w.technique == 'aa' else 'HardSoftRas'} "
                f"{w.screen}^2 x {w.views} views, icosphere L{w.level}")
    fit.step(warmup)
    ctx.synchronize()
    t0 = time.perf_counter()
    fit.step(steps)
    ctx.synchronize()
    dt = time.perf_counter() - t0
    its = steps / dt
    if name in od.PBR_WORKLOADS:
        prof = fit.profile(5)
        g = fit.read(od._lib.PBR_GBUF0)
        fg = g[..., 2] >= 0.0
        env = ~fg & (g[..., 0] >= 0.0)
        classes = {"fg": int(fg.sum()), "env": int(env.sum()),
                   "none": int(g[..., 0].size - fg.sum() - env.sum())}
        flops = kernel_flops_pbr(classes, 0.0)["k_pbr_shade"]
        extra = {"k_pbr_shade_us": prof["k_pbr_shade"],
                 "k_pbr_shade_valu_frac": flops / (prof["k_pbr_shade"] * 1e-6) / VALU_PEAK}
    nviews, screen = fit.n_views, fit.screen
    fit.close()
    ctx.close()
    return {"workload": desc, "value": its, "unit": "iterations/s", "ms_per_step": 1e3 / its,
            "steps": steps, "mpixels_per_s": nviews * screen * screen * its / 1e6,
            "iteration_frac_of_hbm_peak": nb * its / HBM_PEAK, **extra}


def dressi_ad_point(name: str, naive: bool, steps: int, warmup: int) -> dict:
    """Iterations/s of the texture fit driven through the DressiAD graph API
    (tests/graph_tex.cpp: the example's graph written with F:: ops; every
    step sends each view's clip and ScreenAttr images and runs execStep,
    which synchronises, as the reference example's loop does). RSP packing
    runs it on the fused texture plan (the route), Naive on the generic
    per-op executor."""
    import tempfile
    import opendressi_amd as od
    w = od.TEX_WORKLOADS[name]
    pos, uv, faces, mvps, gt, tex0 = od.make_tex_scene(w)
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "_bin", "graph_tex")
    if not os.path.exists(exe):
        return {"error": "tests/_bin/graph_tex is not built"}
    hdr = np.array([len(pos), len(faces), w.views, w.screen, w.tex, w.tex, steps, w.sets,
                    1 if naive else 0], np.uint32)
    with tempfile.TemporaryDirectory() as d:
        inp, out = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        with open(inp, "wb") as f:
            f.write(hdr.tobytes())
            f.write(np.float32(w.lr).tobytes())
            for a in (pos, uv, faces, mvps, gt, tex0):
                f.write(np.ascontiguousarray(a, np.float32).tobytes())
        res = subprocess.run([exe, inp, out, str(warmup)], capture_output=True, text=True,
                             timeout=900)
    if res.returncode != 0:
        return {"error": res.stderr.strip()[-400:]}
    info = dict(kv.split("=", 1) for kv in res.stdout.split() if "=" in kv)
    ms = float(info["ms_per_step"])
    return {"workload": f"{name}: texture {w.screen}^2 x {w.views} views through DressiAD "
                        f"({'Naive' if naive else 'RSP'} packing)",
            "plan": info.get("plan"), "stages": int(info.get("stages", 0)),
            "value": 1e3 / ms, "unit": "iterations/s", "ms_per_step": ms, "steps": steps}


def peel_point(name: str, peels: int, iters: int, skip: int) -> dict:
    """Median execStep wall time of the silhouette fit driven through the
    DressiAD graph API (tests/graph_c1.cpp: the example's graph with `peels`
    RasterizeSoft layers, run.cpp:302-343; each step uploads the clip images,
    runs, and downloads the loss, as the reference example's loop does).
    K = 1 runs on the fused plan (the route), K > 1 on the generic executor;
    the reference reports K = 1 against K = 3 (docs/benchmarks.md:150-156)."""
    import tempfile
    import opendressi_amd as od
    w = od.WORKLOADS[name]
    pos, faces, tgt, mvps = od.make_scene(w)
    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests", "_bin", "graph_c1")
    if not os.path.exists(exe):
        return {"error": "tests/_bin/graph_c1 is not built"}
    nv, nf, n = len(pos), len(faces), len(mvps)
    hdr = np.array([nv, nf, len(tgt), nf, n, w.screen, 8, iters, 0, 0, 0, peels, 0, 0],
                   np.uint32)
    with tempfile.TemporaryDirectory() as d:
        inp, out = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        with open(inp, "wb") as f:
            f.write(hdr.tobytes())
            f.write(np.array([3.0, w.lr, 0.0, 0.0], np.float32).tobytes())
            for a in (pos, faces, tgt, faces, mvps):
                f.write(np.ascontiguousarray(a, np.float32).tobytes())
        res = subprocess.run([exe, inp, out], capture_output=True, text=True, timeout=900)
        if res.returncode != 0:
            return {"error": res.stderr.strip()[-400:]}
        ms = np.fromfile(out, np.float32)[-iters:]
    info = dict(kv.split("=", 1) for kv in res.stdout.split() if "=" in kv)
    med = float(np.median(ms[skip:]))
    return {"workload": f"{name}: HardSoftRas K={peels} {w.screen}^2 x {w.views} views through "
                        "DressiAD (median execStep, uploads included)",
            "plan": info.get("plan"), "stages": int(info.get("stages", 0)),
            "value": 1e3 / med, "unit": "iterations/s", "ms_per_step": med,
            "steps": iters - skip}


def reference_cpu_c1() -> dict:
    """The reference's own CPU evaluator (oracle/_ref: the reference's
    src/core built in place, BuildBackward + CpuEvaluator with DressiAD's
    copy-back; single-threaded, as the reference's evaluator is) on the whole
    C1 fit: 256^2, 1 view, icosphere L3, 50 iterations. None when the
    reference build is absent."""
    import opendressi_amd as od
    from oracle.pyoracle import REF_SO, Reference
    if not os.path.exists(REF_SO):
        return None
    w = od.WORKLOADS["c1"]
    pos, faces, tgt, mvps = od.make_scene(w)
    t0 = time.perf_counter()
    Reference().hsr_fit(pos, faces, tgt, faces, mvps, w.screen, lr=w.lr, iters=w.iters,
                        want_images=False)
    dt = time.perf_counter() - t0
    return {"value": w.iters / dt, "unit": "iterations/s", "cores": 1, "kind": "reference",
            "sample": (f"the whole c1 fit: {w.screen}^2 x 1 view, icosphere L{w.level}, "
                       f"{w.iters} iterations in {dt:.1f} s (the static target raster "
                       f"included); host CPU: {cpu_info()}, nproc {os.cpu_count()}")}


def torch_surface(views: int = 8, screen: int = 256, level: int = 3, steps: int = 50,
                  warmup: int = 5) -> dict:
    """Iterations/s of the silhouette fit written against the
    nvdiffrast-compatible torch surface (the loop of the reference's
    examples/python/silhouette_optimization.py, technique aa, without its
    regularisers): per iteration rasterize + antialias of the N views' masks,
    the L2 loss against fixed target masks, autograd backward and
    torch.optim.Adam on the vertex positions. The ops loop over the batch
    items on the device (no host round trip)."""
    import numpy as np
    import torch

    import opendressi_amd as od
    import opendressi_amd.torch as dr
    dev = torch.device("cuda", 0)
    pos0, faces = od.icosphere(level)
    w = od.Workload("torch", level, screen, views, 0.05, 0.1, 1e-3, steps, 3, "aa")
    _, _, tgt, mvps = od.make_scene(w)
    tri = torch.as_tensor(faces.astype(np.int32), device=dev)
    # the column-major MVPs read row-major are M^T: clip rows = (x, y, z, 1) M^T
    m = torch.as_tensor(np.asarray(mvps, np.float32).reshape(-1, 4, 4), device=dev)
    ctx = dr.RasterizeHipContext(device=dev)

    def clips(p):
        ph = torch.cat([p, torch.ones_like(p[:, :1])], 1)
        return torch.matmul(ph.unsqueeze(0), m)

    def render(p):
        c = clips(p)
        rast, _ = dr.rasterize(ctx, c, tri, resolution=[screen, screen])
        mask = (rast[..., 3:4] > 0).float()
        return dr.antialias(mask, rast, c, tri)

    with torch.no_grad():
        target = render(torch.as_tensor(tgt, device=dev)).detach()
    pos = torch.as_tensor(pos0, device=dev).clone().requires_grad_(True)
    opt = torch.optim.Adam([pos], lr=1e-3)

    def step():
        opt.zero_grad(set_to_none=True)
        loss = ((render(pos) - target) ** 2).mean()
        loss.backward()
        opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(steps):
        loss = step()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t
    return {"workload": f"torch surface silhouette fit (aa): {screen}x{screen} x {views} views, "
                        f"icosphere L{level} ({len(pos0)} v / {len(faces)} f), torch Adam",
            "value": steps / dt, "unit": "iterations/s", "ms_per_step": 1e3 * dt / steps,
            "steps": steps, "loss_after": float(loss)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="c4_hsr")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-points", action="store_true",
                    help="skip the metric's other points (c2 at 512^2, c4 AA at 2048^2)")
    ap.add_argument("--profile-iters", type=int, default=20)
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="after the JSON line, run a plain device copy of this many MiB "
                         "(the reference kernel for scaling rocprofv3 FETCH/WRITE_SIZE)")
    ap.add_argument("--torch-surface", action="store_true",
                    help="also time the silhouette fit written against opendressi_amd.torch "
                         "(rasterize + antialias + autograd + torch Adam) as `torch_surface`")
    ap.add_argument("--bench-json", default=None,
                    help="after the JSON line, run the silhouette workload's whole fit and write "
                         "the reference example's bench.json record to this path")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; the multi-GPU path "
                          "(views sharded over ranks + one gradient all-reduce) is design-only",
                          "n_gpus": args.gpus}))
        return 2

    import opendressi_amd as od
    ctx = od.Context(0)
    tex = args.workload in od.TEX_WORKLOADS
    pbr = args.workload in od.PBR_WORKLOADS
    if tex:
        w = od.TEX_WORKLOADS[args.workload]
        fit = od.TextureFit.from_workload(ctx, args.workload)
    elif pbr:
        w = od.PBR_WORKLOADS[args.workload]
        fit = od.PbrFit.from_workload(ctx, args.workload)
    else:
        w = od.WORKLOADS[args.workload]
        fit = od.SilhouetteFit.from_workload(ctx, args.workload)
    nv, nf, nviews, s = fit.n_verts, fit.n_faces, fit.n_views, fit.screen

    fit.step(args.warmup)
    ctx.synchronize()
    t0 = time.perf_counter()
    fit.step(args.steps)
    ctx.synchronize()
    dt = time.perf_counter() - t0
    its = args.steps / dt
    loss_end = fit.loss()

    # per-kernel durations: eager iterations with HIP events between kernels
    prof = fit.profile(args.profile_iters)
    dom = max(prof, key=prof.get)
    dom_us = prof[dom]
    if pbr:
        texels, envt = fit.tex_w * fit.tex_h, fit.env_w * fit.env_h
        kbytes = kernel_bytes_pbr(nviews, s, texels, envt, fit.pooled_texels, fit.map_texels,
                                  fit.gather_maps)
        ibytes = iteration_bytes_pbr(nviews, s, nf, nv, texels, envt)
        desc = (f"{w.name}: PBR/IBL material + env fit, {s}x{s} x {nviews} views, icosphere "
                f"L{w.level} ({nv} v / {nf} f) with equirect uv, {fit.tex_w}x{fit.tex_h} albedo "
                f"+ metallic-roughness, {fit.env_w}x{fit.env_h} env, {fit.levels} prefilter "
                f"levels, LUT 256^2, L1, Adam lr {w.lr}")
    elif tex:
        texels = fit.tex_w * fit.tex_h
        kbytes = kernel_bytes_tex(nviews, s, nf, nv, texels)
        ibytes = iteration_bytes_tex(nviews, s, nf, nv, texels)
        desc = (f"{w.name}: texture fit, {s}x{s} x {nviews} random orbit views per iteration, "
                f"UV sphere {w.stacks}x{w.slices} ({nv} v / {nf} f), {fit.tex_w}x{fit.tex_h} "
                f"RGBA texture, bilinear, Adam lr {w.lr}")
    else:
        aa = w.technique == "aa"
        kbytes = (kernel_bytes_aa if aa else kernel_bytes)(nviews, s, nf, nv)
        ibytes = (iteration_bytes_aa if aa else iteration_bytes)(nviews, s, nf, nv)
        desc = (f"{w.name}: {'AA' if aa else 'HardSoftRas'} silhouette fit, "
                f"{s}x{s} x {nviews} views, icosphere L{w.level} "
                f"({nv} v / {nf} f), {'' if aa else 'r=3 px, '}8 samples, Adam lr {w.lr}")
    dbytes = kbytes[dom]
    achieved = dbytes / (dom_us * 1e-6)
    traffic = measured_traffic(dom, args.workload)
    valu = None
    if pbr:
        # pixel classes from the static G-buffer (n.v < 0: background; its
        # u < 0: no env behind it); convolution pairs from the map sizes
        g = fit.read(od._lib.PBR_GBUF0)
        fg = g[..., 2] >= 0.0
        env = ~fg & (g[..., 0] >= 0.0)
        classes = {"fg": int(fg.sum()), "env": int(env.sum()), "none": int(g[..., 0].size
                                                                            - fg.sum() - env.sum())}
        psw, psh = fit.prefilter_source
        isw, ish = fit.irradiance_source
        pairs = (fit.map_texels - 32 * 16) * psw * psh + 32 * 16 * isw * ish
        kfl = kernel_flops_pbr(classes, pairs)
        valu = {k: {"achieved": f / (prof[k] * 1e-6) / 1e12, "frac": f / (prof[k] * 1e-6) / VALU_PEAK,
                    "algorithmic_flops_per_launch": f, "avg_launch_us": prof[k]}
                for k, f in kfl.items() if k in prof}
        valu["pixel_classes"] = classes
        valu["conv_pairs"] = pairs
    fit.close()

    line = {
        "metric": METRIC,
        "value": its,
        "unit": "iterations/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": 1000.0 * dt / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": desc, "screen": s, "views": nviews, "verts": nv, "faces": nf},
        "roofline": ({"bound": "hbm", "kernel": dom,
                      "achieved": achieved / 1e9,
                      "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                      "frac": achieved / HBM_PEAK,
                      "traffic": traffic,
                      "algorithmic_bytes_per_launch": dbytes,
                      "avg_launch_us": dom_us}
                     if valu is None or dom not in valu else
                     {"bound": "valu", "kernel": dom,
                      "achieved": valu[dom]["achieved"],
                      "peak": VALU_PEAK / 1e12, "unit": "TFLOP/s",
                      "frac": valu[dom]["frac"],
                      "traffic": traffic,
                      "algorithmic_flops_per_launch": valu[dom]["algorithmic_flops_per_launch"],
                      "algorithmic_bytes_per_launch": dbytes,
                      "hbm_frac": achieved / HBM_PEAK,
                      "avg_launch_us": dom_us}),
        "iteration_roofline": {"algorithmic_bytes": ibytes,
                               "achieved_GBps": ibytes * its / 1e9,
                               "frac": ibytes * its / HBM_PEAK},
        "mpixels_per_s": nviews * s * s * its / 1e6,
        "kernel_us": prof,
        "loss_after": loss_end,
    }
    if valu is not None:
        line["valu_rooflines"] = valu
    if args.workload == "c4_hsr" and not args.no_points:
        # the metric's 512^2 point and the AA technique at 2048^2
        line["metric_points"] = {"c1": metric_point("c1", 400, 20),
                                 "c2": metric_point("c2", 400, 20),
                                 "c3": metric_point("c3", 100, 10),
                                 "c4": metric_point("c4", 100, 10),
                                 "c5": metric_point("c5", 50, 5),
                                 "c3_dressi_ad": dressi_ad_point("c3", False, 30, 5),
                                 "c3_dressi_ad_generic": dressi_ad_point("c3", True, 3, 2),
                                 "c2_dressi_ad_k1": peel_point("c2", 1, 60, 10),
                                 "c2_dressi_ad_k3": peel_point("c2", 3, 30, 10)}
    if args.torch_surface:
        line["torch_surface"] = torch_surface()
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = (cpu_baseline_pbr(w) if pbr else
                                cpu_baseline_tex(w) if tex else cpu_baseline(w))
        if not (tex or pbr):
            try:
                ref = reference_cpu_c1()
            except Exception as exc:  # the reference build is a baseline, not the product
                ref = {"error": str(exc)}
            if ref is not None:
                line["cpu_baseline"]["reference_c1"] = ref
    print(json.dumps(line), flush=True)
    ctx.close()
    if args.bench_json:
        if tex or pbr:
            print("--bench-json: the record covers the silhouette workloads", file=sys.stderr)
        else:
            bench_record(args.workload, args.bench_json)
    if args.copy_mb > 0:
        import torch
        n = args.copy_mb * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
