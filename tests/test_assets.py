"""The examples' asset and geometry helpers (include/dressi_examples/*.h,
the reference's examples/common/asset_utils.cpp and geometry_utils.cpp),
driven through tests/_bin/assets_cli on the CPU.

The reference reads these formats through libraries that are not part of
its sources (tinyobjloader v2.0.0rc13, tinygltf v2.9.5, tinyexr v1.0.9, stb
at c9064e3) and ships no asset file, so the files here are written by the
tests themselves from the format specifications (OBJ text, glTF 2.0 JSON /
GLB, OpenEXR 2 scanline files, PNG), and the expected values come from what
the formats fix plus the reference's own post-processing (unwelding, the v
flip, the normalisation), evaluated in float32 with numpy. Textbook
cross-checks pin the rest: numpy's IEEE float16 conversion for the half
writer away from ties, geometric identities for the camera matrices,
finite differences for the normal-consistency gradient.
"""
import base64
import json
import os
import struct
import subprocess
import zlib

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "_bin", "assets_cli")
F32 = np.float32


@pytest.fixture(scope="module")
def cli():
    if not os.path.exists(EXE):
        from opendressi_amd.build import LIB, build_graph_test
        if not os.path.exists(LIB):
            pytest.fail("opendressi_amd/libdressi_hip.so is not built (run __graft_entry__.build())")
        build_graph_test()

    def run(*args, ok=True):
        res = subprocess.run([EXE, *map(str, args)], capture_output=True, text=True, timeout=60)
        if ok and res.returncode != 0:
            raise AssertionError(f"assets_cli {args[0]} failed: {res.stderr}")
        return res

    return run


def write_img(path, a):
    a = np.asarray(a, F32)
    if a.ndim == 1:
        a = a[None, :, None]
    elif a.ndim == 2:
        a = a[None, :, :]
    h, w, c = a.shape
    with open(path, "wb") as f:
        f.write(struct.pack("<3I", w, h, c))
        f.write(np.ascontiguousarray(a).tobytes())


def read_img(path):
    with open(path, "rb") as f:
        w, h, c = struct.unpack("<3I", f.read(12))
        return np.frombuffer(f.read(), F32).reshape(h, w, c).copy()


def read_mesh(prefix):
    pos = read_img(prefix + ".pos")[0]
    uv = read_img(prefix + ".uv")[0]
    faces = read_img(prefix + ".faces")[0].astype(np.int64)
    return pos, uv, faces


def normalise_mul(p):
    """(p - centre) * (1 / extent) in float32 (OBJ)."""
    lo, hi = p.min(0), p.max(0)
    ext = (hi - lo).max()
    return ((p - F32(0.5) * (lo + hi)) * (F32(1) / ext)).astype(F32)


def normalise_div(p):
    """(p - centre) / max(extent, 1e-12) in float32 (glTF)."""
    lo, hi = p.min(0), p.max(0)
    ext = max(F32(1e-12), (hi - lo).max())
    return ((p - F32(0.5) * (lo + hi)) / ext).astype(F32)


# ---------------------------------------------------------------------- OBJ


def unweld(v, vt, corners):
    """One vertex per (v, vt) pair in first-use order over the triangle
    corners; uv = (u, 1 - v), (0, 0) without texcoords."""
    key_of, pos, uv, idx = {}, [], [], []
    for k in corners:
        if k not in key_of:
            key_of[k] = len(pos)
            pos.append(v[k[0]])
            uv.append([vt[k[1]][0], F32(1) - vt[k[1]][1]] if k[1] >= 0 else [0, 0])
        idx.append(key_of[k])
    return (np.asarray(pos, F32), np.asarray(uv, F32), np.asarray(idx, np.int64).reshape(-1, 3))


def test_obj_unwelds_flips_and_normalises(cli, tmp_path):
    rng = np.random.default_rng(3)
    v = (rng.standard_normal((6, 3)) * 3 + 1).astype(F32)
    vt = rng.random((5, 2)).astype(F32)
    text = ["# test", "o first"]
    text += [f"v {x!r} {y!r} {z!r}" for x, y, z in v.tolist()]
    text += [f"vt {a!r} {b!r}" for a, b in vt.tolist()]
    # (v, vt) corners, 1-based in the file; one face with relative indices,
    # one without texcoords, one v//vn, CRLF on a line
    faces = [[(0, 0), (1, 1), (2, 2)], [(2, 2), (1, 1), (3, 3)], [(3, -1), (4, -1), (5, -1)],
             [(0, 4), (2, 2), (5, 4)]]
    text.append("f 1/1 2/2 3/3")
    text.append("f -4/-3 -5/-4 -3/-2\r")
    text.append("f 4//1 5//1 6//1")
    text.append("g second")
    text.append("vn 0 0 1")
    text.append("f 1/5/1 3/3/1 6/5/1")
    p = tmp_path / "m.obj"
    p.write_text("\n".join(text) + "\n")
    cli("obj", p, tmp_path / "out")
    pos, uv, idx = read_mesh(str(tmp_path / "out"))
    v32 = np.asarray([np.float32(float(x)) for x in np.asarray(v, np.float64).ravel()],
                     F32).reshape(-1, 3)
    vt32 = vt.astype(F32)
    e_pos, e_uv, e_idx = unweld(v32, vt32, [c for f in faces for c in f])
    assert np.array_equal(idx, e_idx)
    assert np.array_equal(uv, e_uv)
    assert np.array_equal(pos, normalise_mul(e_pos))
    # normalised: centred, maximum extent 1
    ext = pos.max(0) - pos.min(0)
    assert abs(ext.max() - 1) < 1e-6
    assert np.allclose(pos.max(0) + pos.min(0), 0, atol=1e-6)


def _quad_obj(tmp_path, v, name):
    text = [f"v {x!r} {y!r} {z!r}" for x, y, z in np.asarray(v, np.float64).tolist()]
    text.append("f 1 2 3 4")
    text.append("f 1 2 3 4 5")
    p = tmp_path / name
    p.write_text("\n".join(text) + "\n")
    return p


def test_obj_quads_split_along_the_shorter_diagonal(cli, tmp_path):
    # diagonal 0-2 shorter: (0,1,2),(0,2,3); else (0,1,3),(1,2,3); the
    # pentagon is a fan
    short02 = np.array([[0, 0, 0], [2, -0.2, 0], [1, 1, 0], [-1, 1, 0], [0, 3, 0]], F32)
    short13 = np.array([[0, 0, 0], [1, 0, 0], [3, 2, 0], [0, 1, 0], [0, 3, 0]], F32)
    for v, tris in ((short02, [0, 1, 2, 0, 2, 3]), (short13, [0, 1, 3, 1, 2, 3])):
        p = _quad_obj(tmp_path, v, "q.obj")
        cli("obj", p, tmp_path / "q")
        pos, uv, idx = read_mesh(str(tmp_path / "q"))
        corners = [(i, -1) for i in tris + [0, 1, 2, 0, 2, 3, 0, 3, 4]]
        e_pos, e_uv, e_idx = unweld(v, None, corners)
        assert np.array_equal(idx, e_idx)
        assert np.array_equal(pos, normalise_mul(e_pos))
        assert not uv.any()


def test_obj_errors(cli, tmp_path):
    r = cli("obj", tmp_path / "missing.obj", tmp_path / "x", ok=False)
    assert r.returncode == 2 and "Failed to load OBJ" in r.stderr
    p = tmp_path / "bad.obj"
    p.write_text("v 0 0 0\nv 1 0 0\nf 1 2 7\n")
    r = cli("obj", p, tmp_path / "x", ok=False)
    assert r.returncode == 2 and "bad index" in r.stderr
    p.write_text("v 0 0 0\nv 1 0 0\n")
    r = cli("obj", p, tmp_path / "x", ok=False)
    assert r.returncode == 2 and "no triangles" in r.stderr


# --------------------------------------------------------------------- glTF


def gltf_doc(pos, uv, idx, idx_type, interleave):
    """Buffer bytes and the JSON document of a one-primitive mesh."""
    n = len(pos)
    views, accessors = [], []
    if interleave:  # pos + uv in one view, 20-byte stride, offset accessors
        inter = np.zeros((n, 5), F32)
        inter[:, :3] = pos
        inter[:, 3:] = uv
        blob = b"\0" * 8 + inter.tobytes()
        views.append({"buffer": 0, "byteOffset": 8, "byteLength": n * 20, "byteStride": 20})
        accessors.append({"bufferView": 0, "componentType": 5126, "count": n, "type": "VEC3"})
        accessors.append({"bufferView": 0, "byteOffset": 12, "componentType": 5126, "count": n,
                          "type": "VEC2"})
    else:
        blob = pos.astype(F32).tobytes()
        views.append({"buffer": 0, "byteLength": len(blob)})
        accessors.append({"bufferView": 0, "componentType": 5126, "count": n, "type": "VEC3"})
        accessors.append(None)
    dt = {5121: np.uint8, 5123: np.uint16, 5125: np.uint32}[idx_type]
    while len(blob) % 4:
        blob += b"\0"
    ib = np.asarray(idx, dt).tobytes()
    views.append({"buffer": 0, "byteOffset": len(blob), "byteLength": len(ib)})
    blob += ib
    accessors.append({"bufferView": len(views) - 1, "componentType": idx_type,
                      "count": int(np.size(idx)), "type": "SCALAR"})
    attrs = {"POSITION": 0}
    if accessors[1] is not None:
        attrs["TEXCOORD_0"] = 1
        acc = accessors
        idx_acc = 2
    else:
        acc = [accessors[0], accessors[2]]
        idx_acc = 1
    doc = {"asset": {"version": "2.0"}, "bufferViews": views, "accessors": acc,
           "buffers": [{"byteLength": len(blob)}],
           "meshes": [{"primitives": [{"attributes": attrs, "indices": idx_acc}]},
                      {"primitives": []}]}
    return blob, doc


def _check_gltf(cli, tmp_path, path, pos, uv, idx):
    cli("gltf", path, tmp_path / "g")
    gp, guv, gi = read_mesh(str(tmp_path / "g"))
    assert np.array_equal(gi, np.asarray(idx).reshape(-1, 3))
    assert np.array_equal(gp, normalise_div(pos))
    e_uv = np.zeros((len(pos), 2), F32) if uv is None else np.stack([uv[:, 0], F32(1) - uv[:, 1]], 1)
    assert np.array_equal(guv, e_uv)


def test_gltf_embedded_external_and_binary(cli, tmp_path):
    rng = np.random.default_rng(5)
    pos = (rng.standard_normal((7, 3)) * 2).astype(F32)
    uv = rng.random((7, 2)).astype(F32)
    idx = rng.integers(0, 7, 12)
    # .gltf, base64 data URI, interleaved, u16 indices
    blob, doc = gltf_doc(pos, uv, idx, 5123, True)
    doc["buffers"][0]["uri"] = "data:application/octet-stream;base64," + base64.b64encode(blob).decode()
    (tmp_path / "a.gltf").write_text(json.dumps(doc, indent=1))
    _check_gltf(cli, tmp_path, tmp_path / "a.gltf", pos, uv, idx)
    # .gltf with an external, percent-encoded .bin, u8 indices, no uv
    blob, doc = gltf_doc(pos, None, idx, 5121, False)
    doc["buffers"][0]["uri"] = "mesh%20data.bin"
    (tmp_path / "mesh data.bin").write_bytes(blob)
    (tmp_path / "b.gltf").write_text(json.dumps(doc))
    _check_gltf(cli, tmp_path, tmp_path / "b.gltf", pos, None, idx)
    # .glb, u32 indices
    blob, doc = gltf_doc(pos, uv, idx, 5125, True)
    js = json.dumps(doc).encode()
    js += b" " * (-len(js) % 4)
    body = struct.pack("<II", len(js), 0x4E4F534A) + js + struct.pack("<II", len(blob), 0x004E4942) + blob
    (tmp_path / "c.glb").write_bytes(struct.pack("<III", 0x46546C67, 2, 12 + len(body)) + body)
    _check_gltf(cli, tmp_path, tmp_path / "c.glb", pos, uv, idx)


def test_gltf_errors(cli, tmp_path):
    pos = np.eye(3, dtype=F32)
    blob, doc = gltf_doc(pos, None, [0, 1, 2], 5125, False)
    doc["buffers"][0]["uri"] = "data:application/octet-stream;base64," + base64.b64encode(blob).decode()
    del doc["meshes"][0]["primitives"][0]["indices"]
    (tmp_path / "n.gltf").write_text(json.dumps(doc))
    r = cli("gltf", tmp_path / "n.gltf", tmp_path / "x", ok=False)
    assert r.returncode == 2 and "POSITION + indices" in r.stderr
    doc["meshes"] = []
    (tmp_path / "n.gltf").write_text(json.dumps(doc))
    r = cli("gltf", tmp_path / "n.gltf", tmp_path / "x", ok=False)
    assert r.returncode == 2 and "no mesh primitives" in r.stderr
    (tmp_path / "j.gltf").write_text("{\"asset\": ")
    r = cli("gltf", tmp_path / "j.gltf", tmp_path / "x", ok=False)
    assert r.returncode == 2 and "Failed to load glTF" in r.stderr


# ---------------------------------------------------------------------- EXR


def exr_predict(raw):
    """OpenEXR's zip/rle pre-pass: even bytes then odd bytes, then the
    difference predictor (+128)."""
    b = np.frombuffer(raw, np.uint8)
    t = np.concatenate([b[0::2], b[1::2]]).astype(np.int16)
    d = t.copy()
    d[1:] = (t[1:] - t[:-1] + 128) & 0xFF
    return d.astype(np.uint8).tobytes()


def exr_unpredict(data):
    t = np.frombuffer(data, np.uint8).astype(np.int64)
    t = np.cumsum(np.concatenate([t[:1], t[1:] - 128])) & 0xFF
    half = (len(t) + 1) // 2
    out = np.empty(len(t), np.uint8)
    out[0::2] = t[:half]
    out[1::2] = t[half:]
    return out.tobytes()


def rle_encode(data):
    out, i, n = bytearray(), 0, len(data)
    while i < n:
        j = i
        while j < n and j - i < 127 and data[j] == data[i]:
            j += 1
        if j - i >= 3:
            out += bytes([j - i - 1, data[i]])
            i = j
            continue
        j = i
        while j < n and j - i < 127 and not (j + 2 < n and data[j] == data[j + 1] == data[j + 2]):
            j += 1
        out += bytes([(256 - (j - i)) & 0xFF]) + data[i:j]
        i = j
    return bytes(out)


def attr(name, typ, value):
    return name.encode() + b"\0" + typ.encode() + b"\0" + struct.pack("<i", len(value)) + value


def write_exr(path, chans, compression):
    """chans: list of (name, 'half'|'float', array HxW) in the order given
    (the file's channel list order)."""
    h, w = chans[0][2].shape
    ch = b""
    for name, typ, _ in chans:
        ch += name.encode() + b"\0" + struct.pack("<iB3xii", 1 if typ == "half" else 2, 0, 1, 1)
    ch += b"\0"
    box = struct.pack("<4i", 0, 0, w - 1, h - 1)
    hdr = struct.pack("<II", 20000630, 2)
    hdr += attr("channels", "chlist", ch) + attr("compression", "compression", bytes([compression]))
    hdr += attr("dataWindow", "box2i", box) + attr("displayWindow", "box2i", box)
    hdr += attr("lineOrder", "lineOrder", b"\0") + attr("pixelAspectRatio", "float", struct.pack("<f", 1))
    hdr += attr("screenWindowCenter", "v2f", struct.pack("<2f", 0, 0))
    hdr += attr("screenWindowWidth", "float", struct.pack("<f", 1)) + b"\0"
    per = 16 if compression == 3 else 1
    blocks = []
    for y0 in range(0, h, per):
        raw = b""
        for y in range(y0, min(h, y0 + per)):
            for _, typ, a in chans:
                raw += a[y].astype(np.float16 if typ == "half" else F32).tobytes()
        if compression in (2, 3):
            data = zlib.compress(exr_predict(raw))
        elif compression == 1:
            data = rle_encode(exr_predict(raw))
        else:
            data = raw
        if len(data) >= len(raw):
            data = raw
        blocks.append(struct.pack("<ii", y0, len(data)) + data)
    table_end = len(hdr) + 8 * len(blocks)
    offs, pos = [], table_end
    for b in blocks:
        offs.append(pos)
        pos += len(b)
    with open(path, "wb") as f:
        f.write(hdr + struct.pack(f"<{len(offs)}Q", *offs) + b"".join(blocks))


def read_exr(path):
    """A small OpenEXR reader (scanline, NONE / ZIPS / ZIP, HALF / FLOAT):
    {name: array}, plus the compression."""
    d = open(path, "rb").read()
    assert struct.unpack("<I", d[:4])[0] == 20000630
    o, chans, comp, box = 8, [], None, None
    while d[o] != 0:
        e = d.index(b"\0", o)
        name = d[o:e].decode()
        e2 = d.index(b"\0", e + 1)
        size = struct.unpack("<i", d[e2 + 1:e2 + 5])[0]
        val = d[e2 + 5:e2 + 5 + size]
        if name == "channels":
            q = 0
            while val[q] != 0:
                z = val.index(b"\0", q)
                chans.append((val[q:z].decode(), struct.unpack("<i", val[z + 1:z + 5])[0]))
                q = z + 17
        elif name == "compression":
            comp = val[0]
        elif name == "dataWindow":
            box = struct.unpack("<4i", val)
        o = e2 + 5 + size
    o += 1
    w, h = box[2] - box[0] + 1, box[3] - box[1] + 1
    per = 16 if comp == 3 else 1
    nb = (h + per - 1) // per
    offs = struct.unpack(f"<{nb}Q", d[o:o + 8 * nb])
    out = {n: np.zeros((h, w), F32) for n, _ in chans}
    for off in offs:
        y0, size = struct.unpack("<ii", d[off:off + 8])
        data = d[off + 8:off + 8 + size]
        lines = min(per, h - y0)
        expect = sum(w * (2 if t == 1 else 4) for _, t in chans) * lines
        if size < expect:
            data = exr_unpredict(zlib.decompress(data))
        q = 0
        for y in range(y0, y0 + lines):
            for n, t in chans:
                dt = np.float16 if t == 1 else F32
                nbytes = w * np.dtype(dt).itemsize
                out[n][y] = np.frombuffer(data[q:q + nbytes], dt).astype(F32)
                q += nbytes
    return out, comp, [n for n, _ in chans]


@pytest.mark.parametrize("compression", [0, 1, 2, 3])
def test_exr_load_compressions_and_types(cli, tmp_path, compression):
    rng = np.random.default_rng(compression)
    h, w = 37, 21
    r, g, b, a = (rng.standard_normal((4, h, w)) * 4).astype(F32)
    g[5:9] = 0.5  # runs for RLE
    # channel list in name order: A, B, G, R; B float, the rest half
    chans = [("A", "half", a), ("B", "float", b), ("G", "half", g), ("R", "half", r)]
    p = tmp_path / "t.exr"
    write_exr(p, chans, compression)
    cli("exr_load", p, tmp_path / "t.img")
    img = read_img(str(tmp_path / "t.img"))
    assert img.shape == (h, w, 3)
    h16 = lambda x: x.astype(np.float16).astype(F32)
    assert np.array_equal(img[..., 0], h16(r))
    assert np.array_equal(img[..., 1], h16(g))
    assert np.array_equal(img[..., 2], b)


def test_exr_single_channel_layers_and_missing(cli, tmp_path):
    y = np.linspace(-2, 5, 6 * 4, dtype=F32).reshape(6, 4)
    write_exr(tmp_path / "y.exr", [("Y", "float", y)], 3)
    cli("exr_load", tmp_path / "y.exr", tmp_path / "y.img")
    img = read_img(str(tmp_path / "y.img"))
    assert all(np.array_equal(img[..., c], y) for c in range(3))
    # layer prefixes are dropped (name after the last '.')
    write_exr(tmp_path / "l.exr", [("d.B", "float", y * 3), ("d.G", "float", y * 2),
                                   ("d.R", "float", y)], 2)
    cli("exr_load", tmp_path / "l.exr", tmp_path / "l.img")
    img = read_img(str(tmp_path / "l.img"))
    assert np.array_equal(img[..., 0], y) and np.array_equal(img[..., 2], y * 3)
    write_exr(tmp_path / "m.exr", [("G", "float", y), ("R", "float", y)], 0)
    r = cli("exr_load", tmp_path / "m.exr", tmp_path / "m.img", ok=False)
    assert r.returncode == 2 and "B channel not found" in r.stderr


def test_exr_save_round_trip_and_half_rounding(cli, tmp_path):
    rng = np.random.default_rng(11)
    h, w = 33, 20
    img = (rng.standard_normal((h, w, 3)) * 100).astype(F32)
    # ties between two halfs round away from zero; others to nearest
    ties = np.array([1 + 2.0 ** -11, -(1 + 3 * 2.0 ** -11), 2.0 ** -25, 3 * 2.0 ** -25,
                     65519.0, 65520.0, 1e-30, 1e6, 0.0, -0.0], F32)
    img.reshape(-1)[:len(ties)] = ties
    write_img(tmp_path / "s.img", img)
    cli("exr_save", tmp_path / "s.img", tmp_path / "s.exr")
    chans, comp, names = read_exr(tmp_path / "s.exr")
    assert comp == 3 and names == ["B", "G", "R"]
    got = np.stack([chans["R"], chans["G"], chans["B"]], -1)
    with np.errstate(over="ignore"):
        rne = img.astype(np.float16).astype(F32)
    flat, gflat = img.reshape(-1), got.reshape(-1)
    tie_vals = {float(x) for x in ties[:6]}
    for i, x in enumerate(flat):
        if float(x) in tie_vals and float(x) not in (65519.0,):
            continue
        assert gflat[i] == rne.reshape(-1)[i] or (np.isnan(gflat[i]) and np.isnan(rne.reshape(-1)[i])), (i, x)
    # exact ties: the neighbour further from zero
    assert gflat[0] == F32(1 + 2.0 ** -10)
    assert gflat[1] == F32(-(1 + 2 * 2.0 ** -10))
    assert gflat[2] == F32(2.0 ** -24)
    assert gflat[3] == F32(2 * 2.0 ** -24)
    assert gflat[4] == F32(65504.0) and np.isinf(gflat[5])
    # float subnormals / tiny values become zero, overflow infinity
    assert gflat[6] == 0 and np.isinf(gflat[7])
    # small images are stored uncompressed; the loader reads both back
    write_img(tmp_path / "small.img", img[:5, :7])
    cli("exr_save", tmp_path / "small.img", tmp_path / "small.exr")
    chans, comp, _ = read_exr(tmp_path / "small.exr")
    assert comp == 0
    for name in ("s", "small"):
        cli("exr_load", tmp_path / f"{name}.exr", tmp_path / f"{name}.back")
    back = read_img(str(tmp_path / "s.back"))
    assert np.array_equal(back, got)
    r = cli("exr_save", tmp_path / "missing.img", tmp_path / "x.exr", ok=False)
    assert r.returncode == 2


# ---------------------------------------------------------------------- PNG


def png_chunk(typ, data):
    return struct.pack(">I", len(data)) + typ + data + struct.pack(">I", zlib.crc32(typ + data))


def png_filter(rows, bpp, kinds):
    out = b""
    prev = bytes(len(rows[0]))
    for row, k in zip(rows, kinds):
        f = bytearray(len(row))
        for i in range(len(row)):
            a = row[i - bpp] if i >= bpp else 0
            b = prev[i]
            c = prev[i - bpp] if i >= bpp else 0
            if k == 0:
                pred = 0
            elif k == 1:
                pred = a
            elif k == 2:
                pred = b
            elif k == 3:
                pred = (a + b) // 2
            else:
                p = a + b - c
                pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
                pred = a if pa <= pb and pa <= pc else (b if pb <= pc else c)
            f[i] = (row[i] - pred) & 0xFF
        out += bytes([k]) + bytes(f)
        prev = row
    return out


def pack_rows(samples, depth):
    """samples: H x (W*channels) ints -> packed row bytes."""
    rows = []
    for s in samples:
        if depth == 16:
            rows.append(np.asarray(s, ">u2").tobytes())
        elif depth == 8:
            rows.append(bytes(np.asarray(s, np.uint8)))
        else:
            bits = "".join(format(int(v), f"0{depth}b") for v in s)
            bits += "0" * (-len(bits) % 8)
            rows.append(bytes(int(bits[i:i + 8], 2) for i in range(0, len(bits), 8)))
    return rows


ADAM7 = [(0, 0, 8, 8), (4, 0, 8, 8), (0, 4, 4, 8), (2, 0, 4, 4), (0, 2, 2, 4), (1, 0, 2, 2), (0, 1, 1, 2)]


def write_png(path, samples, color, depth, palette=None, interlace=False, seed=0):
    """samples: H x W x channels integers."""
    h, w, ch = samples.shape
    bits = ch * depth
    bpp = max(1, bits // 8)
    rng = np.random.default_rng(seed)
    raw = b""
    passes = ADAM7 if interlace else [(0, 0, 1, 1)]
    for x0, y0, dx, dy in passes:
        sub = samples[y0::dy, x0::dx]
        if sub.size == 0:
            continue
        rows = pack_rows(sub.reshape(sub.shape[0], -1), depth)
        raw += png_filter(rows, bpp, rng.integers(0, 5, len(rows)))
    data = b"\x89PNG\r\n\x1a\n"
    data += png_chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, depth, color, 0, 0, int(interlace)))
    if palette is not None:
        data += png_chunk(b"PLTE", bytes(np.asarray(palette, np.uint8).ravel()))
    z = zlib.compress(raw)
    data += png_chunk(b"IDAT", z[:len(z) // 2]) + png_chunk(b"IDAT", z[len(z) // 2:])
    data += png_chunk(b"IEND", b"")
    open(path, "wb").write(data)


def read_png_rgb8(path):
    d = open(path, "rb").read()
    assert d[:8] == b"\x89PNG\r\n\x1a\n"
    o, idat = 8, b""
    while o < len(d):
        n = struct.unpack(">I", d[o:o + 4])[0]
        typ, body = d[o + 4:o + 8], d[o + 8:o + 8 + n]
        assert struct.unpack(">I", d[o + 8 + n:o + 12 + n])[0] == zlib.crc32(typ + body)
        if typ == b"IHDR":
            w, h, depth, color, _, _, il = struct.unpack(">IIBBBBB", body)
            assert (depth, color, il) == (8, 2, 0)
        elif typ == b"IDAT":
            idat += body
        o += 12 + n
    raw = zlib.decompress(idat)
    row = w * 3
    out = np.zeros((h, row), np.uint8)
    prev = np.zeros(row, np.int64)
    for y in range(h):
        f = raw[y * (row + 1)]
        line = np.frombuffer(raw[y * (row + 1) + 1:(y + 1) * (row + 1)], np.uint8).astype(np.int64)
        cur = np.zeros(row, np.int64)
        for i in range(row):
            a = cur[i - 3] if i >= 3 else 0
            b = prev[i]
            c = prev[i - 3] if i >= 3 else 0
            pred = [0, a, b, (a + b) // 2, 0][f]
            if f == 4:
                p = a + b - c
                pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
                pred = a if pa <= pb and pa <= pc else (b if pb <= pc else c)
            cur[i] = (line[i] + pred) & 0xFF
        out[y] = cur
        prev = cur
    return out.reshape(h, w, 3)


PNG_CASES = [  # color, depth, channels, interlace
    (2, 8, 3, False), (6, 8, 4, False), (0, 8, 1, False), (4, 8, 2, True), (2, 16, 3, False),
    (6, 16, 4, True), (0, 16, 1, False), (0, 1, 1, False), (0, 2, 1, True), (0, 4, 1, False),
    (3, 8, 1, False), (3, 4, 1, True), (3, 1, 1, False),
]


@pytest.mark.parametrize("color,depth,ch,interlace", PNG_CASES)
def test_png_load_layouts(cli, tmp_path, color, depth, ch, interlace):
    rng = np.random.default_rng(depth * 10 + color)
    h, w = 13, 11
    top = (1 << depth) - 1
    palette = None
    if color == 3:
        n = 1 << depth
        palette = rng.integers(0, 256, (n, 3))
    samples = rng.integers(0, top + 1, (h, w, ch))
    p = tmp_path / "t.png"
    write_png(p, samples, color, depth, palette, interlace, seed=color + depth)
    cli("png_load", p, tmp_path / "t.img")
    img = read_img(str(tmp_path / "t.img"))
    # stb's 8-bit RGB view: 16-bit keeps the high byte, gray below 8 bits
    # scales to 0..255, gray is replicated, alpha dropped, palette expanded
    if color == 3:
        rgb = palette[samples[..., 0]]
    else:
        s = samples >> 8 if depth == 16 else samples
        if depth < 8:
            s = s * {1: 0xFF, 2: 0x55, 4: 0x11}[depth]
        rgb = np.repeat(s[..., :1], 3, -1) if ch <= 2 else s[..., :3]
    assert np.array_equal(img, rgb.astype(F32) / F32(255))


def test_png_save_round_trip(cli, tmp_path):
    rng = np.random.default_rng(2)
    img = (rng.random((9, 14, 3)) * 1.4 - 0.2).astype(F32)
    write_img(tmp_path / "c.img", img)
    cli("png_save", tmp_path / "c.img", tmp_path / "c.png")
    expect = (np.clip(img, 0, 1) * F32(255) + F32(0.5)).astype(np.uint8)
    assert np.array_equal(read_png_rgb8(tmp_path / "c.png"), expect)
    cli("png_load", tmp_path / "c.png", tmp_path / "c.back")
    assert np.array_equal(read_img(str(tmp_path / "c.back")), expect.astype(F32) / F32(255))
    gray = rng.random((5, 6, 1)).astype(F32)
    write_img(tmp_path / "g.img", gray)
    cli("png_save", tmp_path / "g.img", tmp_path / "g.png")
    g8 = (np.clip(gray, 0, 1) * F32(255) + F32(0.5)).astype(np.uint8)
    assert np.array_equal(read_png_rgb8(tmp_path / "g.png"), np.repeat(g8, 3, -1))
    write_img(tmp_path / "two.img", np.zeros((2, 2, 2), F32))
    r = cli("png_save", tmp_path / "two.img", tmp_path / "two.png", ok=False)
    assert r.returncode == 2 and "Failed to save image" in r.stderr
    (tmp_path / "not.png").write_bytes(b"GIF89a....")
    r = cli("png_load", tmp_path / "not.png", tmp_path / "x", ok=False)
    assert r.returncode == 2 and "Failed to load image" in r.stderr


# ------------------------------------------------------------ image helpers


def test_srgb_downsample_tile(cli, tmp_path):
    rng = np.random.default_rng(4)
    img = (rng.random((7, 9, 3)) * 1.2 - 0.1).astype(F32)
    write_img(tmp_path / "i.img", img)
    cli("srgb", tmp_path / "i.img", tmp_path / "s.img")
    s = read_img(str(tmp_path / "s.img"))
    ref = np.power(np.maximum(img.astype(np.float64), 0), float(F32(2.2)))
    assert np.allclose(s, ref, rtol=3e-7, atol=1e-30) and (s[img <= 0] == 0).all()
    # constant images stay constant; a ramp in x halves to pair means; odd
    # extents repeat the last row / column
    const = np.full((5, 7, 2), 0.375, F32)
    write_img(tmp_path / "c.img", const)
    cli("down", tmp_path / "c.img", tmp_path / "cd.img")
    cd = read_img(str(tmp_path / "cd.img"))
    assert cd.shape == (3, 4, 2) and (cd == F32(0.375)).all()
    ramp = np.broadcast_to(np.arange(7, dtype=F32)[None, :, None], (5, 7, 1)).copy()
    write_img(tmp_path / "r.img", ramp)
    cli("down", tmp_path / "r.img", tmp_path / "rd.img")
    rd = read_img(str(tmp_path / "rd.img"))[..., 0]
    assert np.array_equal(rd, np.broadcast_to(np.array([0.5, 2.5, 4.5, 6], F32), (3, 4)))
    one = np.ones((1, 1, 1), F32)
    write_img(tmp_path / "o.img", one)
    cli("down", tmp_path / "o.img", tmp_path / "od.img")
    assert read_img(str(tmp_path / "od.img")).shape == (1, 1, 1)
    # tiles: gray replicated, grid row-major, empty cells zero
    a = rng.random((4, 3, 3)).astype(F32)
    b = rng.random((4, 3, 1)).astype(F32)
    write_img(tmp_path / "a.img", a)
    write_img(tmp_path / "b.img", b)
    cli("tile", 2, tmp_path / "t.img", tmp_path / "a.img", tmp_path / "b.img", tmp_path / "a.img")
    t = read_img(str(tmp_path / "t.img"))
    assert t.shape == (8, 6, 3)
    assert np.array_equal(t[:4, :3], a) and np.array_equal(t[:4, 3:], np.repeat(b, 3, -1))
    assert np.array_equal(t[4:, :3], a) and not t[4:, 3:].any()


# ----------------------------------------------------------------- matrices


def mat(cli, tmp_path, *args):
    cli(*args, tmp_path / "m.img")
    return read_img(str(tmp_path / "m.img")).reshape(4, 4).T  # row-major view


def test_camera_matrices(cli, tmp_path):
    eye, center, up = np.array([1.5, 2.0, 3.0]), np.array([0.2, -0.1, 0.3]), np.array([0, 1.0, 0])
    v = mat(cli, tmp_path, "lookat", *eye, *center, *up).astype(np.float64)
    # orthonormal rotation, eye -> origin, center on the -z axis
    assert np.allclose(v[:3, :3] @ v[:3, :3].T, np.eye(3), atol=1e-6)
    assert np.allclose(v @ np.append(eye, 1), [0, 0, 0, 1], atol=1e-5)
    d = np.linalg.norm(center - eye)
    assert np.allclose(v @ np.append(center, 1), [0, 0, -d, 1], atol=1e-5)
    assert (v @ np.array([0, 1.0, 0, 0]))[1] > 0.5  # up stays up
    fovy, aspect, n, f = 0.8, 1.5, 0.1, 10.0
    p = mat(cli, tmp_path, "persp", fovy, aspect, n, f).astype(np.float64)
    for z, depth in ((-n, 0.0), (-f, 1.0)):
        c = p @ np.array([0, 0, z, 1.0])
        assert abs(c[2] / c[3] - depth) < 1e-6
    t = 1 / np.tan(fovy / 2)
    c = p @ np.array([0, 1.0, -1.0, 1])
    assert abs(c[1] / c[3] + t) < 1e-5  # y down
    c = p @ np.array([1.0, 0, -1.0, 1])
    assert abs(c[0] / c[3] - t / aspect) < 1e-5
    # Mul, TransformToClip and ChainRuleClipToPos against float64 products
    rng = np.random.default_rng(9)
    a, b = rng.standard_normal((2, 4, 4)).astype(F32)
    write_img(tmp_path / "a.img", a.T.reshape(-1))  # column-major files
    write_img(tmp_path / "b.img", b.T.reshape(-1))
    ab = mat(cli, tmp_path, "mul", tmp_path / "a.img", tmp_path / "b.img")
    assert np.allclose(ab, a.astype(np.float64) @ b, atol=1e-5)
    pos = rng.standard_normal((10, 3)).astype(F32)
    write_img(tmp_path / "p.img", pos[None])
    cli("clip", tmp_path / "p.img", tmp_path / "a.img", tmp_path / "c.img")
    clip = read_img(str(tmp_path / "c.img"))[0]
    ph = np.concatenate([pos, np.ones((10, 1), F32)], 1).astype(np.float64)
    assert np.allclose(clip, ph @ a.T.astype(np.float64), atol=1e-5)
    g = rng.standard_normal((10, 4)).astype(F32)
    write_img(tmp_path / "g.img", g[None])
    cli("chain", tmp_path / "g.img", tmp_path / "a.img", tmp_path / "gp.img")
    gp = read_img(str(tmp_path / "gp.img"))[0]
    assert np.allclose(gp, g.astype(np.float64) @ a[:, :3].astype(np.float64), atol=1e-5)


# ------------------------------------------------------------------ geometry


def test_sphere_generators(cli, tmp_path):
    cli("ico", 2, tmp_path / "ico")
    pos, uv, faces = read_mesh(str(tmp_path / "ico"))
    assert pos.shape == (162, 3) and faces.shape == (320, 3) and not uv.any()
    assert np.allclose(np.linalg.norm(pos, axis=1), 1, atol=1e-6)
    import opendressi_amd as od
    ref_pos, ref_faces = od.icosphere(2)
    assert np.array_equal(pos, np.asarray(ref_pos, F32).reshape(-1, 3))
    assert np.array_equal(faces, np.asarray(ref_faces).reshape(-1, 3))
    cli("uvsphere", 4, 6, tmp_path / "uvs")
    pos, uv, faces = read_mesh(str(tmp_path / "uvs"))
    assert pos.shape == (35, 3) and faces.shape == (2 * 4 * 6 - 12, 3)
    assert np.array_equal(uv[7], [F32(0), F32(1) / F32(4)])
    cli("uvsphere", 1, 1, tmp_path / "uvc")  # clamped to 2 x 3
    assert read_mesh(str(tmp_path / "uvc"))[0].shape == (12, 3)


def test_transfer_deformation_by_direction(cli, tmp_path):
    cli("ico", 1, tmp_path / "ctrl")
    rest, _, faces = read_mesh(str(tmp_path / "ctrl"))
    rng = np.random.default_rng(6)
    dst = rng.standard_normal((50, 3)).astype(F32)
    write_img(tmp_path / "rest.img", rest[None])
    write_img(tmp_path / "faces.img", faces.astype(F32)[None])
    write_img(tmp_path / "dst.img", dst[None])
    # rest -> rest: each direction lands on the control surface, on its ray
    cli("transfer", tmp_path / "rest.img", tmp_path / "faces.img", tmp_path / "rest.img",
        tmp_path / "dst.img", tmp_path / "o.img")
    o = read_img(str(tmp_path / "o.img"))[0].astype(np.float64)
    dirs = dst / np.linalg.norm(dst, axis=1, keepdims=True)
    assert np.allclose(np.cross(o, dirs), 0, atol=1e-5)
    assert ((o * dirs).sum(1) > 0.79).all() and (np.linalg.norm(o, axis=1) <= 1 + 1e-6).all()
    # a scaled deformation scales the transfer
    write_img(tmp_path / "def.img", (rest * F32(2))[None])
    cli("transfer", tmp_path / "rest.img", tmp_path / "faces.img", tmp_path / "def.img",
        tmp_path / "dst.img", tmp_path / "o2.img")
    o2 = read_img(str(tmp_path / "o2.img"))[0]
    assert np.allclose(o2, 2 * o, atol=1e-5)


def test_regulariser_gradients(cli, tmp_path):
    # tetrahedron: every vertex neighbours the other three
    pos = np.array([[0, 0, 0], [1, 0, 0], [0, 1, 0], [0, 0, 1]], F32)
    faces = np.array([[0, 2, 1], [0, 1, 3], [0, 3, 2], [1, 2, 3]], F32)
    write_img(tmp_path / "p.img", pos[None])
    write_img(tmp_path / "f.img", faces[None])
    cli("lap", tmp_path / "p.img", tmp_path / "f.img", 0.5, tmp_path / "l.img")
    lap = read_img(str(tmp_path / "l.img"))[0]
    mean_others = (pos.sum(0) - pos) / 3
    assert np.allclose(lap, 0.5 * (pos - mean_others), atol=1e-7)
    # normal consistency: gradient against central differences of the energy
    cli("ico", 1, tmp_path / "ico")
    ipos, _, ifaces = read_mesh(str(tmp_path / "ico"))
    rng = np.random.default_rng(8)
    ipos = (ipos + rng.standard_normal(ipos.shape) * 0.05).astype(F32)
    write_img(tmp_path / "ip.img", ipos[None])
    write_img(tmp_path / "if.img", ifaces.astype(F32)[None])
    r = cli("ncons", tmp_path / "ip.img", tmp_path / "if.img", 0.7, tmp_path / "n.img")
    g = read_img(str(tmp_path / "n.img"))[0]
    assert r.stdout.split()[1] == "0" and int(r.stdout.split()[3]) == 120

    def energy(p):
        e = np.zeros(len(ifaces), np.float64)
        a, b, c = p[ifaces[:, 0]], p[ifaces[:, 1]], p[ifaces[:, 2]]
        n = np.cross(b - a, c - a)
        n /= np.linalg.norm(n, axis=1, keepdims=True)
        edges = {}
        for fi, f in enumerate(ifaces):
            for k in range(3):
                edges.setdefault(tuple(sorted((f[k], f[(k + 1) % 3]))), []).append(fi)
        return 0.7 * sum(1 - n[x] @ n[y] for x, y in edges.values())

    p64 = ipos.astype(np.float64)
    fd = np.zeros_like(p64)
    for i in range(len(p64)):
        for c in range(3):
            d = np.zeros_like(p64)
            d[i, c] = 1e-6
            fd[i, c] = (energy(p64 + d) - energy(p64 - d)) / 2e-6
    assert np.abs(g - fd).max() < 2e-3 * max(1.0, np.abs(fd).max())
    # one face turned over flips its three adjacent pairs
    bad = ifaces.copy()
    bad[0] = bad[0, ::-1]
    write_img(tmp_path / "bf.img", bad.astype(F32)[None])
    r = cli("ncons", tmp_path / "ip.img", tmp_path / "bf.img", 0.7, tmp_path / "n2.img")
    assert r.stdout.split()[1] == "3"


def test_adam_step(cli, tmp_path):
    # a constant gradient: bias correction makes m_hat = g and v_hat = g^2,
    # so every step moves each parameter by lr * g / (|g| + eps)
    params = np.array([1.0, -2.0, 0.5, 3.0], F32)
    g = np.array([0.3, -1e-3, 4.0, 0.0], F32)
    write_img(tmp_path / "p.img", params)
    write_img(tmp_path / "g.img", np.tile(g, 5))
    cli("adam", tmp_path / "p.img", tmp_path / "g.img", 0.01, 5, tmp_path / "o.img")
    out = read_img(str(tmp_path / "o.img")).reshape(-1)
    step = 0.01 * g / (np.abs(g) + 1e-8)
    assert np.allclose(out, params - 5 * step, atol=2e-6)
    assert out[3] == params[3]


def test_save_obj_and_textured_obj(cli, tmp_path):
    pos = np.array([[0.5, -1, 0.25], [1e-7, 2, 3], [123456.7, 0, -0.125]], F32)
    uv = np.array([[0, 0.25], [1, 1], [0.5, 0.75]], F32)
    faces = np.array([[0, 1, 2]], F32)
    for name, arr in (("p", pos), ("u", uv), ("f", faces)):
        write_img(tmp_path / f"{name}.img", arr[None])
    cli("save_obj", tmp_path / "p.img", tmp_path / "u.img", tmp_path / "f.img", tmp_path / "a.obj")
    assert (tmp_path / "a.obj").read_text() == (
        "v 0.5 -1 0.25\nv 1e-07 2 3\nv 123457 0 -0.125\nf 1 2 3\n")
    cli("save_obj", tmp_path / "p.img", tmp_path / "u.img", tmp_path / "f.img",
        tmp_path / "t.obj", "tex.png")
    assert (tmp_path / "t.mtl").read_text() == (
        "newmtl material0\nKa 0 0 0\nKd 1 1 1\nd 1\nillum 1\nmap_Kd tex.png\n")
    text = (tmp_path / "t.obj").read_text().splitlines()
    assert text[:2] == ["mtllib t.mtl", "usemtl material0"]
    assert text[5:] == ["vt 0 0.75", "vt 1 0", "vt 0.5 0.25", "f 1/1 2/2 3/3"]
    # reloading gives the uv back (v flipped twice)
    cli("obj", tmp_path / "t.obj", tmp_path / "back")
    _, back_uv, back_f = read_mesh(str(tmp_path / "back"))
    assert np.array_equal(back_uv, uv) and np.array_equal(back_f, [[0, 1, 2]])


# --------------------------------------------------------------------- JPEG
#
# The reference decodes JPEG with stb_image (absent here), so decoder parity
# with it is unpinned. What ITU-T T.81 fixes is pinned instead: the test
# writes baseline files itself from quantised DCT blocks (its own Huffman
# tables, byte stuffing, restart markers) and checks the decoded samples
# against closed forms of the inverse DCT (DC-only blocks: F q / 8 + 128;
# one AC term: a product of two cosines) and against the definition
# evaluated with numpy, the JFIF colour transform, and the triangle
# upsampling filter on a two-level chroma edge.


def zigzag_natural():
    """Natural index of the k-th zig-zag coefficient: diagonals r + c = s,
    odd ones walked with the row rising, even ones with it falling."""
    out = []
    for s in range(15):
        rows = range(max(0, s - 7), min(s, 7) + 1)
        rows = rows if s % 2 else reversed(rows)
        out += [r * 8 + (s - r) for r in rows]
    return out


ZZ = zigzag_natural()


class _Bits:
    def __init__(self):
        self.acc, self.n, self.out = 0, 0, bytearray()

    def put(self, v, n):
        for i in range(n - 1, -1, -1):
            self.acc = (self.acc << 1) | ((v >> i) & 1)
            self.n += 1
            if self.n == 8:
                self._byte(self.acc)
                self.acc, self.n = 0, 0

    def _byte(self, b):
        self.out.append(b)
        if b == 0xFF:
            self.out.append(0x00)

    def flush(self):
        if self.n:
            self.put((1 << (8 - self.n)) - 1, 8 - self.n)  # pad with ones


def _cat(v):
    return int(abs(int(v))).bit_length()


def _flat_huffman(symbols):
    """Every symbol the same code length L with 2^L > count (the all-ones
    code unused): (BITS, HUFFVAL, {symbol: (code, L)})."""
    syms = sorted(set(symbols)) or [0]
    L = max(1, int(np.ceil(np.log2(len(syms) + 1))))
    counts = [0] * 16
    counts[L - 1] = len(syms)
    return counts, syms, {s: (i, L) for i, s in enumerate(syms)}


def _block_symbols(coef, pred):
    """(dc category, dc bits) and the AC (run/size, bits) list of one block
    (natural-order ints)."""
    zz = [int(coef[ZZ[k]]) for k in range(64)]
    diff = zz[0] - pred
    s = _cat(diff)
    dc = (s, diff if diff >= 0 else diff + (1 << s) - 1)
    ac, run = [], 0
    for k in range(1, 64):
        v = zz[k]
        if v == 0:
            run += 1
            continue
        while run > 15:
            ac.append((0xF0, 0, 0))
            run -= 16
        s = _cat(v)
        ac.append(((run << 4) | s, v if v >= 0 else v + (1 << s) - 1, s))
        run = 0
    if run:
        ac.append((0x00, 0, 0))
    return dc, ac, zz[0]


def write_jpeg(path, comps, width, height, q, restart=0, sof=0xC0, app14=None, ids=None):
    """comps: [(h, v, blocks)] with blocks {rows, cols, 64} natural-order
    quantised coefficients (interleaved scan for several components, each
    covering its MCUs; one component: its own blocks); q: {64} zig-zag
    quantisation table shared by all."""
    ids = ids or list(range(1, len(comps) + 1))
    hmax = max(c[0] for c in comps)
    vmax = max(c[1] for c in comps)
    units = []  # per restart unit: [(comp index, block)]
    if len(comps) == 1:
        b = comps[0][2]
        units = [[(0, b[r, c])] for r in range(b.shape[0]) for c in range(b.shape[1])]
    else:
        mx = -(-width // (8 * hmax))
        my = -(-height // (8 * vmax))
        for y in range(my):
            for x in range(mx):
                u = []
                for ci, (h, v, b) in enumerate(comps):
                    u += [(ci, b[y * v + j, x * h + i]) for j in range(v) for i in range(h)]
                units.append(u)
    # symbols, with the DC predictions (reset at restarts)
    coded, dcs, acs = [], [], []
    pred = [0] * len(comps)
    for n, u in enumerate(units):
        if restart and n and n % restart == 0:
            pred = [0] * len(comps)
            coded.append(None)
        for ci, blk in u:
            dc, ac, pred[ci] = _block_symbols(blk, pred[ci])
            coded.append((dc, ac))
            dcs.append(dc[0])
            acs += [a[0] for a in ac]
    dbits, dvals, dcode = _flat_huffman(dcs)
    abits, avals, acode = _flat_huffman(acs)
    bw, seg, rst = _Bits(), bytearray(), 0
    for c in coded:
        if c is None:
            bw.flush()
            seg += bw.out + bytes([0xFF, 0xD0 + rst % 8])
            bw, rst = _Bits(), rst + 1
            continue
        (s, bits), ac = c
        bw.put(*dcode[s])
        bw.put(bits, s)
        for rs, b, s2 in ac:
            bw.put(*acode[rs])
            bw.put(b, s2)
    bw.flush()
    seg += bw.out

    def marker(m, body):
        return bytes([0xFF, m]) + struct.pack(">H", len(body) + 2) + body

    out = b"\xff\xd8" + marker(0xE0, b"JFIF\x00\x01\x01\x00\x00\x01\x00\x01\x00\x00")
    if app14 is not None:
        out += marker(0xEE, b"Adobe" + bytes([0, 100, 0, 0, 0, 0, app14]))
    out += marker(0xDB, bytes([0]) + bytes(int(x) for x in q))
    sofb = struct.pack(">BHHB", 8, height, width, len(comps))
    for ci, (h, v, _) in enumerate(comps):
        sofb += bytes([ids[ci], (h << 4) | v, 0])
    out += marker(sof, sofb)
    out += marker(0xC4, bytes([0x00]) + bytes(dbits) + bytes(dvals))
    out += marker(0xC4, bytes([0x10]) + bytes(abits) + bytes(avals))
    if restart:
        out += marker(0xDD, struct.pack(">H", restart))
    sos = bytes([len(comps)]) + b"".join(bytes([ids[ci], 0x00]) for ci in range(len(comps)))
    out += marker(0xDA, sos + bytes([0, 63, 0])) + bytes(seg) + b"\xff\xd9"
    open(path, "wb").write(out)


def idct_ref(blk, qn):
    """T.81 A.3.3 in float64 for one block (natural-order coefficients,
    natural-order quantisation), + 128, rounded half up, clamped."""
    F = blk.astype(np.float64).reshape(8, 8) * qn.reshape(8, 8)
    x = np.arange(8)
    C = np.where(np.arange(8) == 0, 1 / np.sqrt(2), 1.0)
    T = 0.5 * C[None, :] * np.cos((2 * x[:, None] + 1) * np.arange(8)[None, :] * np.pi / 16)
    s = T @ F @ T.T  # s[y, x] = sum_v sum_u T[y, v] F[v, u] T[x, u]
    return np.clip(np.floor(s + 128.5), 0, 255)


def plane_of(blocks, qn):
    r, c = blocks.shape[:2]
    out = np.zeros((r * 8, c * 8))
    for i in range(r):
        for j in range(c):
            out[i * 8:i * 8 + 8, j * 8:j * 8 + 8] = idct_ref(blocks[i, j], qn)
    return out


def jfif_rgb(y, cb, cr):
    cb, cr = cb - 128.0, cr - 128.0
    r = y + 1.402 * cr
    g = y - 0.344136 * cb - 0.714136 * cr
    b = y + 1.772 * cb
    return np.clip(np.floor(np.stack([r, g, b], -1) + 0.5), 0, 255)


def _load_rgb8(cli, tmp_path, path):
    cli("png_load", path, tmp_path / "o.img")
    return np.rint(read_img(tmp_path / "o.img") * 255).astype(np.int64)


def test_jpeg_closed_forms_gray(cli, tmp_path):
    q = np.full(64, 1, np.int64)
    q[ZZ.index(1)] = 3  # (v, u) = (0, 1) dequantised by 3
    blocks = np.zeros((2, 3, 64), np.int64)
    blocks[0, 0, 0] = 8 * 40        # DC only: 40 + 128 everywhere
    blocks[0, 1, 0] = -8 * 100      # 28
    blocks[0, 2, 0] = 8 * 200       # clamps at 255
    blocks[1, 0, 1] = 50            # one AC term along x
    blocks[1, 1, 0] = -8 * 300      # clamps at 0
    blocks[1, 2, 8] = -20           # (v, u) = (1, 0): along y
    write_jpeg(tmp_path / "g.jpg", [(1, 1, blocks)], 20, 13, np.asarray(
        [q[ZZ[k]] for k in range(64)]))
    got = _load_rgb8(cli, tmp_path, tmp_path / "g.jpg")
    assert got.shape == (13, 20, 3)
    assert (got[..., 0] == got[..., 1]).all() and (got[..., 0] == got[..., 2]).all()
    g = got[..., 0]
    assert (g[0:8, 0:8] == 168).all() and (g[0:8, 8:16] == 28).all()
    assert (g[0:8, 16:20] == 255).all() and (g[8:13, 8:16] == 0).all()
    x = np.arange(8)
    ax = 128 + 0.25 * (1 / np.sqrt(2)) * 150 * np.cos((2 * x + 1) * np.pi / 16)
    assert (g[8:13, 0:8] == np.floor(ax + 0.5)[None, :]).all()
    ay = 128 + 0.25 * (1 / np.sqrt(2)) * -20 * np.cos((2 * np.arange(5) + 1) * np.pi / 16)
    assert (g[8:13, 16:20] == np.floor(ay + 0.5)[:, None]).all()


def _rand_blocks(rng, r, c, dc_scale=30, ac=6):
    b = np.zeros((r, c, 64), np.int64)
    b[..., 0] = rng.integers(-dc_scale, dc_scale + 1, (r, c))
    for k in rng.integers(1, 64, 6):
        b[..., ZZ[k]] = rng.integers(-ac, ac + 1, (r, c))
    return b


def test_jpeg_444_random_blocks_restarts_and_stuffing(cli, tmp_path):
    rng = np.random.default_rng(3)
    qz = rng.integers(1, 9, 64)
    qn = np.zeros(64)
    qn[ZZ] = qz
    Y, Cb, Cr = (_rand_blocks(rng, 2, 3) for _ in range(3))
    comps = [(1, 1, Y), (1, 1, Cb), (1, 1, Cr)]
    want = jfif_rgb(plane_of(Y, qn), plane_of(Cb, qn), plane_of(Cr, qn))[:16, :24]
    outs = []
    for restart in (0, 1, 4):
        write_jpeg(tmp_path / f"c{restart}.jpg", comps, 24, 16, qz, restart=restart)
        outs.append(_load_rgb8(cli, tmp_path, tmp_path / f"c{restart}.jpg"))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    d = np.abs(outs[0] - want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99


def test_jpeg_byte_stuffing(cli, tmp_path):
    # DC differences of +-255 (eight one bits, or eight zero bits) at every
    # bit alignment: the coded data holds 0xFF bytes, written as 0xFF 0x00
    # (+255, -255) pairs with a 1..7-bit difference between them to walk
    # through the alignments
    diffs = [0]
    for k in range(1, 8):
        diffs += [255, -255, (1 << k) - 1]
    dc = np.cumsum(diffs)
    blocks = np.zeros((1, len(dc), 64), np.int64)
    blocks[0, :, 0] = dc
    q = np.ones(64, np.int64)
    write_jpeg(tmp_path / "f.jpg", [(1, 1, blocks)], 8 * len(dc), 8, q)
    data = open(tmp_path / "f.jpg", "rb").read()
    assert b"\xff\x00" in data[data.index(b"\xff\xda"):data.index(b"\xff\xd9")]
    g = _load_rgb8(cli, tmp_path, tmp_path / "f.jpg")[..., 0]
    want = np.clip(np.floor(dc / 8.0 + 128.5), 0, 255)
    assert (g == np.repeat(want, 8)[None, :]).all()


def test_jpeg_420_constant_chroma_and_triangle_filter(cli, tmp_path):
    rng = np.random.default_rng(4)
    qz = np.ones(64, np.int64)
    qn = np.ones(64)
    Y = _rand_blocks(rng, 2, 4)
    cb = np.zeros((1, 2, 64), np.int64)
    cr = np.zeros((1, 2, 64), np.int64)
    cb[0, :, 0] = 8 * 20      # Cb 148 everywhere
    cr[0, 0, 0] = -8 * 16     # Cr 112 on the left chroma block,
    cr[0, 1, 0] = 8 * 48      # 176 on the right one
    write_jpeg(tmp_path / "s.jpg", [(2, 2, Y), (1, 1, cb), (1, 1, cr)], 32, 16, qz)
    got = _load_rgb8(cli, tmp_path, tmp_path / "s.jpg")
    y = plane_of(Y, qn)[:16, :32]
    # columns 0..14 see Cr 112 only, 17..31 Cr 176 only; the filter mixes
    # 3:1 at the edge: col(i) = 4 c, out(15) = (12 a + 4 b + 7) >> 4,
    # out(16) = (12 b + 4 a + 8) >> 4
    a, b = 112, 176
    crs = np.where(np.arange(32) < 16, a, b).astype(np.float64)
    crs[15] = (12 * a + 4 * b + 7) >> 4
    crs[16] = (12 * b + 4 * a + 8) >> 4
    want = jfif_rgb(y, np.full_like(y, 148.0), np.broadcast_to(crs, y.shape))
    d = np.abs(got - want)
    assert d.max() <= 1 and (d == 0).mean() > 0.99
    assert (np.abs(got[:, :15] - jfif_rgb(y[:, :15], 148.0 + 0 * y[:, :15], 112.0 + 0 * y[:, :15])) <= 1).all()


def test_jpeg_rgb_components_progressive_and_truncated(cli, tmp_path):
    b = np.zeros((1, 1, 64), np.int64)
    comps = [(1, 1, b + np.eye(1, 64, 0, dtype=np.int64) * 8 * k) for k in (10, -20, 30)]
    qz = np.ones(64, np.int64)
    write_jpeg(tmp_path / "a.jpg", comps, 8, 8, qz, app14=0)
    assert (_load_rgb8(cli, tmp_path, tmp_path / "a.jpg") == [138, 108, 158]).all()
    write_jpeg(tmp_path / "n.jpg", comps, 8, 8, qz, ids=[ord("R"), ord("G"), ord("B")])
    assert (_load_rgb8(cli, tmp_path, tmp_path / "n.jpg") == [138, 108, 158]).all()
    write_jpeg(tmp_path / "p.jpg", comps, 8, 8, qz, sof=0xC2)
    r = cli("png_load", tmp_path / "p.jpg", tmp_path / "x", ok=False)
    assert r.returncode != 0 and "baseline" in r.stderr
    data = open(tmp_path / "a.jpg", "rb").read()
    (tmp_path / "t.jpg").write_bytes(data[:data.index(b"\xff\xc4")])
    r = cli("png_load", tmp_path / "t.jpg", tmp_path / "x", ok=False)
    assert r.returncode != 0 and "JPEG" in r.stderr


# ---------------------------------------------------------- glTF scenes
#
# LoadGltfScene on hand-built files: the node transform is chosen so that
# float32 evaluates it exactly (a 180-degree turn about z, scales 2, 3, 4),
# so positions, normals (area-weighted, through the normal matrix) and
# generated tangents have closed forms; textures come from a data URI PNG,
# a bufferView JPEG (one gray component, replicated), a gray + alpha PNG
# (channel c reads component min(c, 1)) and absent slots.


def _b64(data):
    return "data:application/octet-stream;base64," + base64.b64encode(data).decode()


def _scene_doc(pos, uv, idx, extra_attrs=None, node=None, images=None, material=None,
               extra_views=b""):
    blob = np.asarray(pos, F32).tobytes()
    views = [{"buffer": 0, "byteOffset": 0, "byteLength": len(blob)}]
    acc = [{"bufferView": 0, "componentType": 5126, "count": len(pos), "type": "VEC3"}]
    attrs = {"POSITION": 0}
    for name, arr, typ in ([("TEXCOORD_0", uv, "VEC2")] + (extra_attrs or [])):
        data = np.asarray(arr, F32).tobytes()
        views.append({"buffer": 0, "byteOffset": len(blob), "byteLength": len(data)})
        blob += data
        acc.append({"bufferView": len(views) - 1, "componentType": 5126, "count": len(arr),
                    "type": typ})
        attrs[name] = len(acc) - 1
    ib = np.asarray(idx, np.uint16).tobytes()
    views.append({"buffer": 0, "byteOffset": len(blob), "byteLength": len(ib)})
    blob += ib
    acc.append({"bufferView": len(views) - 1, "componentType": 5123, "count": len(idx),
                "type": "SCALAR"})
    prim = {"attributes": attrs, "indices": len(acc) - 1}
    doc = {"asset": {"version": "2.0"}, "accessors": acc, "bufferViews": views,
           "meshes": [{"primitives": [prim]}], "nodes": [{"name": "empty"}, node or {"mesh": 0}]}
    if images is not None:
        doc["images"], doc["textures"] = [], []
        for kind, data in images:
            if kind == "uri":
                doc["images"].append({"uri": _b64(data)})
            else:
                doc["bufferViews"].append({"buffer": 0, "byteOffset": len(blob),
                                           "byteLength": len(data)})
                blob += data + b"\0" * (-len(data) % 4)
                doc["images"].append({"bufferView": len(doc["bufferViews"]) - 1,
                                      "mimeType": kind})
            doc["textures"].append({"source": len(doc["images"]) - 1})
        doc["textures"].append({"sampler": 0})  # a texture without a source
    if material is not None:
        doc["materials"] = [material]
        prim["material"] = 0
    doc["buffers"] = [{"byteLength": len(blob)}]
    return blob, doc


def test_gltf_scene_transform_generated_frames_and_textures(cli, tmp_path):
    pos = np.array([[0, 0, 0], [1, 0, 0], [1, 1, 0], [0, 1, 0]], F32)
    uv = np.array([[0, 1.25], [1, 1.25], [1, 2], [0, 2]], F32)  # V offset by a whole period
    idx = [0, 1, 2, 0, 2, 3]
    node = {"mesh": 0, "translation": [1, 2, 3], "rotation": [0, 0, 1, 0], "scale": [2, 3, 4]}
    base = np.array([[[255, 0, 10], [1, 2, 3]], [[9, 99, 200], [0, 128, 255]]])
    write_png(tmp_path / "b.png", base, 2, 8)
    occ = np.array([[[10, 200], [20, 100]], [[30, 0], [40, 255]]])
    write_png(tmp_path / "o.png", occ, 4, 8)
    blocks = np.zeros((1, 1, 64), np.int64)
    blocks[0, 0, 0] = 8 * 50
    write_jpeg(tmp_path / "m.jpg", [(1, 1, blocks)], 8, 8, np.ones(64, np.int64))
    images = [("uri", open(tmp_path / "b.png", "rb").read()),
              ("image/jpeg", open(tmp_path / "m.jpg", "rb").read()),
              ("image/png", open(tmp_path / "o.png", "rb").read())]
    material = {"pbrMetallicRoughness": {"baseColorTexture": {"index": 0},
                                         "metallicRoughnessTexture": {"index": 1}},
                "occlusionTexture": {"index": 2}, "emissiveTexture": {"index": 3}}
    blob, doc = _scene_doc(pos, uv, idx, node=node, images=images, material=material)
    doc["buffers"][0]["uri"] = _b64(blob)
    (tmp_path / "s.gltf").write_text(json.dumps(doc))
    cli("gltf_scene", tmp_path / "s.gltf", tmp_path / "r", "raw")
    p, u, f = read_mesh(str(tmp_path / "r"))
    want = np.stack([-2 * pos[:, 0] + 1, -3 * pos[:, 1] + 2, 4 * pos[:, 2] + 3], 1)
    assert np.array_equal(p, want) and np.array_equal(f, np.reshape(idx, (-1, 3)))
    assert np.array_equal(u, uv - np.array([0, 1], F32))
    n = read_img(str(tmp_path / "r.normal"))[0]
    t = read_img(str(tmp_path / "r.tangent"))[0]
    assert np.array_equal(n, np.tile([0, 0, 1], (4, 1)).astype(F32))
    # uv u runs along +x: tangent +x (w = +1 for this winding), turned to -x
    assert np.array_equal(t, np.tile([-1, 0, 0, 1], (4, 1)).astype(F32))
    assert np.array_equal(np.rint(read_img(str(tmp_path / "r.base")) * 255), base)
    assert np.array_equal(np.rint(read_img(str(tmp_path / "r.mr")) * 255), np.full((8, 8, 3), 178))
    o = np.rint(read_img(str(tmp_path / "r.occ")) * 255)
    assert np.array_equal(o, np.stack([occ[..., 0], occ[..., 1], occ[..., 1]], -1))
    for slot in ("nmap", "emis"):
        assert read_img(str(tmp_path / f"r.{slot}")).size == 0
    # normalised: centred, maximum extent 1 (as LoadGltfMesh)
    cli("gltf_scene", tmp_path / "s.gltf", tmp_path / "q")
    assert np.array_equal(read_mesh(str(tmp_path / "q"))[0], normalise_div(want))


def test_gltf_scene_given_frames_matrix_glb_and_errors(cli, tmp_path):
    pos = np.array([[0, 0, 0], [2, 0, 0], [0, 2, 0]], F32)
    nrm = np.array([[0, 0, 1], [0, 0, 1], [0, 0, 1]], F32)
    tan = np.array([[1, 0, 0, -1], [1, 0, 0, -1], [0, 1, 0, 1]], F32)
    # matrix: x -> y, y -> -x, z -> 2 z, translated by (5, 0, 0) (column-major)
    m = [0, 1, 0, 0, -1, 0, 0, 0, 0, 0, 2, 0, 5, 0, 0, 1]
    blob, doc = _scene_doc(pos, np.zeros((3, 2), F32), [0, 1, 2],
                           extra_attrs=[("NORMAL", nrm, "VEC3"), ("TANGENT", tan, "VEC4")],
                           node={"mesh": 0, "matrix": m})
    js = json.dumps(doc).encode()
    js += b" " * (-len(js) % 4)
    blob += b"\0" * (-len(blob) % 4)
    body = struct.pack("<II", len(js), 0x4E4F534A) + js + struct.pack("<II", len(blob), 0x004E4942) + blob
    (tmp_path / "g.glb").write_bytes(struct.pack("<III", 0x46546C67, 2, 12 + len(body)) + body)
    cli("gltf_scene", tmp_path / "g.glb", tmp_path / "r", "raw")
    p = read_mesh(str(tmp_path / "r"))[0]
    assert np.array_equal(p, np.stack([5 - pos[:, 1], pos[:, 0], 2 * pos[:, 2]], 1))
    assert np.array_equal(read_img(str(tmp_path / "r.normal"))[0], nrm)
    t = read_img(str(tmp_path / "r.tangent"))[0]
    assert np.array_equal(t[:, :3], np.array([[0, 1, 0], [0, 1, 0], [-1, 0, 0]], F32))
    assert np.array_equal(t[:, 3], tan[:, 3])
    for slot in ("base", "mr", "nmap", "occ", "emis"):
        assert read_img(str(tmp_path / f"r.{slot}")).size == 0  # no material
    # a 16-bit texture is refused
    write_png(tmp_path / "w.png", np.full((2, 2, 3), 1000), 2, 16)
    blob, doc = _scene_doc(pos, np.zeros((3, 2), F32), [0, 1, 2],
                           images=[("uri", open(tmp_path / "w.png", "rb").read())],
                           material={"pbrMetallicRoughness": {"baseColorTexture": {"index": 0}}})
    doc["buffers"][0]["uri"] = _b64(blob)
    (tmp_path / "w.gltf").write_text(json.dumps(doc))
    r = cli("gltf_scene", tmp_path / "w.gltf", tmp_path / "x", ok=False)
    assert r.returncode != 0 and "8-bit" in r.stderr
    doc["meshes"] = []
    (tmp_path / "e.gltf").write_text(json.dumps(doc))
    r = cli("gltf_scene", tmp_path / "e.gltf", tmp_path / "x", ok=False)
    assert r.returncode != 0 and "no mesh primitives" in r.stderr
