"""Writes the final-parameter fixtures of every benchmark workload: the
oracle's fit (oracle/liboracle.so, whose restatement the unit and
trajectory fixtures pin to the reference's own CPU build) run at the
workload's full size for its full iteration count.

    python tests/golden/make_final_params.py              # every workload
    python tests/golden/make_final_params.py c2 c4_hsr    # the named ones

`final_c5_first.npz` holds C5's first two iterations (images and gradients
of the first, parameters after the second) at full size, sampled.

The reference example stops after a fixed iteration count and reports the
optimised parameters (examples/silhouette_optimization/run.cpp:574-637,
examples/texture_optimization/run.cpp:205-250,
examples/pbr_material_optimization/run.cpp); these files hold those
parameters. Each `final_<workload>.npz` stores:

  in_sha_*     SHA-256 of every input array the fit starts from (the scene
               generators are seeded; the GPU test regenerates the scene and
               checks these first)
  out_loss     the loss of every iteration
  out_sha_*    SHA-256 of every final parameter array (bit-exact check)
  out_<p>      the final parameter array when small (silhouette positions),
  out_idx_<p>, out_smp_<p>
               otherwise a seeded sample of 16384 rows and their values
  out_sum_<p>  float64 sum of |p| (a whole-array check for the sampled ones)
"""
from __future__ import annotations

import hashlib
import os
import sys
import time
from concurrent.futures import ProcessPoolExecutor

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
OUT = os.path.dirname(os.path.abspath(__file__))
SAMPLE_ROWS = 16384


def sha(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    return np.frombuffer(hashlib.sha256(a.tobytes()).digest(), np.uint8).copy()


def sample_rows(n_rows: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return np.sort(rng.choice(n_rows, size=min(SAMPLE_ROWS, n_rows), replace=False)).astype(
        np.int64)


def put_param(arrs: dict, name: str, a: np.ndarray, full: bool, seed: int) -> None:
    arrs["out_sha_" + name] = sha(a)
    arrs["out_sum_" + name] = np.array([np.abs(a.astype(np.float64)).sum()])
    if full:
        arrs["out_" + name] = a
    else:
        rows = a.reshape(-1, a.shape[-1])
        idx = sample_rows(len(rows), seed)
        arrs["out_idx_" + name] = idx
        arrs["out_smp_" + name] = rows[idx]


def silhouette(name: str) -> dict:
    import opendressi_amd as od
    from oracle.pyoracle import Oracle
    w = od.WORKLOADS[name]
    pos, faces, tgt, mvps = od.make_scene(w)
    fit = Oracle().aa_fit if w.technique == "aa" else Oracle().hsr_fit
    r = fit(pos, faces, tgt, faces, mvps, w.screen, lr=w.lr, iters=w.iters, want_images=False)
    arrs = {"in_sha_pos": sha(pos), "in_sha_faces": sha(faces), "in_sha_tgt": sha(tgt),
            "in_sha_mvps": sha(mvps), "out_loss": r["loss"], "out_t": r["t"],
            "in_cfg": np.array([w.screen, w.views, w.iters, w.lr], np.float64)}
    put_param(arrs, "pos", r["pos"], True, 1)
    put_param(arrs, "m", r["m"], False, 2)
    put_param(arrs, "v", r["v"], False, 3)
    return arrs


def texture(name: str) -> dict:
    import opendressi_amd as od
    from oracle.pyoracle import Oracle
    w = od.TEX_WORKLOADS[name]
    pos, uv, faces, mvps, gt, tex0 = od.make_tex_scene(w)
    r = Oracle().tex_fit(pos, uv, faces, mvps, w.screen, gt, tex0, lr=w.lr, iters=w.iters,
                         want_images=False)
    arrs = {"in_sha_pos": sha(pos), "in_sha_uv": sha(uv), "in_sha_faces": sha(faces),
            "in_sha_mvps": sha(mvps), "in_sha_gt": sha(gt), "in_sha_tex0": sha(tex0),
            "out_loss": r["loss"], "out_t": r["t"],
            "in_cfg": np.array([w.screen, w.views, w.iters, w.lr], np.float64)}
    put_param(arrs, "tex", r["tex"], False, 4)
    put_param(arrs, "m", r["m"], False, 5)
    put_param(arrs, "v", r["v"], False, 6)
    return arrs


def pbr(name: str) -> dict:
    import opendressi_amd as od
    from opendressi_amd.pbr import workload_scene
    from oracle.pyoracle import Oracle
    w = od.PBR_WORKLOADS[name]
    sc = workload_scene(w)
    r = Oracle().pbr_fit(sc, iters=w.iters, want_images=False)
    arrs = {"in_sha_" + k: sha(v) for k, v in sc.items() if isinstance(v, np.ndarray)}
    arrs.update(out_loss=r["loss"],
                in_cfg=np.array([w.screen, w.views, w.iters, w.lr], np.float64))
    put_param(arrs, "albedo", r["albedo"], False, 7)
    put_param(arrs, "mr", r["mr"], False, 8)
    put_param(arrs, "env", r["env"], False, 9)
    return arrs


def pbr_first(name: str) -> dict:
    """C5's first iterations at full size: the first iteration's target and
    prediction images and parameter gradients, the parameters after two
    iterations (sampled: the images alone are 75 MB each)."""
    import opendressi_amd as od
    from opendressi_amd.pbr import workload_scene
    from oracle.pyoracle import Oracle
    w = od.PBR_WORKLOADS[name.split("_")[0]]
    sc = workload_scene(w)
    r = Oracle().pbr_fit(sc, iters=2, want_images=True)
    arrs = {"in_sha_" + k: sha(v) for k, v in sc.items() if isinstance(v, np.ndarray)}
    arrs.update(out_loss=r["loss"])
    for i, k in enumerate(("pred0", "target0", "mask0", "g_albedo0", "g_mr0", "g_env0",
                           "albedo", "mr", "env")):
        a = r[k] if r[k].ndim == 4 or k != "mask0" else r[k][..., None]
        put_param(arrs, k, a, False, 20 + i)
        arrs["out_max_" + k] = np.array([np.abs(a).max()], np.float64)
    return arrs


KINDS = {"c2": silhouette, "c4_hsr": silhouette, "c4": silhouette, "c3": texture, "c5": pbr,
         "c5_first": pbr_first}


def run(name: str) -> str:
    t0 = time.perf_counter()
    arrs = KINDS[name](name)
    path = os.path.join(OUT, f"final_{name}.npz")
    np.savez_compressed(path, **arrs)
    return f"wrote {path} in {time.perf_counter() - t0:.0f} s (loss {arrs['out_loss'][0]:.6g} -> " \
           f"{arrs['out_loss'][-1]:.6g})"


def main() -> None:
    names = sys.argv[1:] or list(KINDS)
    for n in names:
        if n not in KINDS:
            raise SystemExit(f"unknown workload {n!r}; known: {sorted(KINDS)}")
    with ProcessPoolExecutor(max_workers=min(len(names), 5)) as ex:
        for msg in ex.map(run, names):
            print(msg, flush=True)


if __name__ == "__main__":
    main()
