"""CPU checks of the format restatement (oracle/formats.py) and of the
library's host-only readers (point clouds, PLY headers). No GPU is used."""
import struct

import numpy as np
import pytest

from oracle import formats as FM

F = np.float32


def _params(n, seed):
    g = np.random.default_rng(seed)
    return {"means": g.normal(0, 1, (n, 3)).astype(F), "scales": g.normal(-4, 1, (n, 3)).astype(F),
            "rotations": g.normal(0, 1, (n, 4)).astype(F), "opacities": g.normal(0, 2, n).astype(F),
            "sh0": g.normal(0, 1.5, (n, 3)).astype(F), "sh_rest": g.normal(0, 0.2, (n, 45)).astype(F)}


def test_ply_header_is_happly_text():
    # hapPLY's writeHeader: magic, format line with version 1.0, its own
    # comment, then "element <name> <count>" and "property <type> <name>"
    want = ("ply\nformat binary_little_endian 1.0\n"
            "comment Written with hapPLY (https://github.com/nmwsharp/happly)\n"
            "element vertex 2\nproperty float x\nproperty float y\nproperty float z\n"
            "property uchar red\nproperty uchar green\nproperty uchar blue\nend_header\n").encode()
    assert FM.ply_header(2, False) == want
    full = FM.ply_header(7, True).decode().split("\n")
    assert full[3] == "element vertex 7"
    props = [ln.split()[2] for ln in full if ln.startswith("property")]
    assert len(props) == 3 + 3 + 3 + 45 + 1 + 3 + 4
    assert props[9:12] == ["f_rest_r_0", "f_rest_g_0", "f_rest_b_0"] and props[53] == "f_rest_b_14"
    assert props[-4:] == ["rot_w", "rot_x", "rot_y", "rot_z"]


def _brute_rows(p, full):
    """save_ply's property vectors, then hapPLY's writeDataBinary loop: for
    each vertex, each property in order, its little-endian bytes."""
    n = p["means"].shape[0]
    cols = []
    for k in range(3):
        cols.append(("f", [float(p["means"][i, k]) for i in range(n)]))
    for k in range(3):
        vals = []
        for i in range(n):
            t = F(F(p["sh0"][i, k]) * F(0.28209479177387814)) + F(0.5)
            t = F(0.0) if t < 0 else (F(1.0) if t > 1 else F(t))
            vals.append(int(F(t * F(255.0))))
        cols.append(("B", vals))
    if full:
        for k in range(3):
            cols.append(("f", [float(p["sh0"][i, k]) for i in range(n)]))
        for coeff in range(15):
            for c in range(3):
                cols.append(("f", [float(p["sh_rest"][i, coeff * 3 + c]) for i in range(n)]))
        cols.append(("f", [float(v) for v in p["opacities"]]))
        for k in range(3):
            cols.append(("f", [float(p["scales"][i, k]) for i in range(n)]))
        for k in range(4):
            cols.append(("f", [float(p["rotations"][i, k]) for i in range(n)]))
    out = bytearray()
    for i in range(n):
        for fmt, vals in cols:
            out += struct.pack("<" + fmt, vals[i])
    return bytes(out)


@pytest.mark.parametrize("full", [False, True])
def test_oracle_ply_rows_brute_force(full):
    p = _params(37, 1)
    p["sh0"][0] = [-10.0, 0.0, 10.0]   # clamped low, the 0.5 midpoint (127), clamped high
    data = FM.ply_bytes(p, full)
    head = FM.ply_header(37, full)
    assert data[:len(head)] == head
    rows = data[len(head):]
    assert len(rows) == 37 * (239 if full else 15)
    assert rows == _brute_rows(p, full)
    assert list(rows[12:15]) == [0, 127, 255]


def test_colour_byte_closed_form():
    # colour = sh0 C0 + 0.5 in [0, 1], times 255, truncated
    v = np.array([-1e9, -0.5 / 0.28209479177387814, 0.0, 0.5 / 0.28209479177387814, 1e9], F)
    assert list(FM.colour_bytes(v)) == [0, 0, 127, 255, 255]
    x = np.linspace(-2, 2, 4001).astype(F)
    c = FM.colour_bytes(x)
    ref = np.floor(np.clip(x.astype(np.float64) * 0.28209479177387814 + 0.5, 0, 1) * 255)
    assert np.max(np.abs(c.astype(np.float64) - ref)) <= 1   # float rounding at exact integers only
    assert np.mean(c == ref) > 0.99


def _tiled_loop(src, w, h, bgr):
    """from_cv2 as the reference's three loops (image_format.cu:68-90)."""
    c = src.shape[2]
    tw = (w + 7) // 8
    total = ((w + 7) // 8 * 8) * ((h + 7) // 8 * 8)
    out = np.zeros(c * total, np.uint8)
    for ch in range(c):
        for y in range(h):
            for x in range(w):
                lin = ((y >> 3) * tw + (x >> 3)) * 64 + (y & 7) * 8 + (x & 7)
                out[ch * total + lin] = src[y, x, (2 - ch) if bgr else ch]
    return out


@pytest.mark.parametrize("wh", [(1, 1), (13, 9), (40, 17)])
def test_oracle_image_converters_vs_loops(wh):
    w, h = wh
    src = np.random.default_rng(w).integers(0, 256, (h, w, 3)).astype(np.uint8)
    for bgr in (True, False):
        t = FM.from_cv2(src, w, h, bgr)
        assert np.array_equal(t, _tiled_loop(src, w, h, bgr))
        assert np.array_equal(FM.to_cv2(t, w, h, 3, bgr), src)
    f = FM.from_cv2(src, w, h, True, "float32")
    assert f.dtype == F and np.array_equal(f, (F(1.0) / F(255.0)) * _tiled_loop(src, w, h, True).astype(F))
    # narrowing truncates clamp(255 v): 1/255 widening then narrowing loses up to one step
    back = FM.to_cv2(f, w, h, 3, True).astype(int)
    assert np.all((back == src) | (back == src.astype(int) - 1))
    assert list(FM.narrow(np.array([-1.0, 0.5, 2.0, np.nan], F))) == [0, 127, 255, 0]


def test_colmap_points_restatement():
    text = "# header\n\n1 0.5 1.5 -2 255 0 51 0.1 3 4\n2 1 2\n3 1 2 3 10 20 30 0.5\n#x 1 2 3 4 5 6 7\n"
    p, c = FM.colmap_points(text)
    assert np.array_equal(p, np.array([[0.5, 1.5, -2], [1, 2, 3]], F))
    assert np.allclose(c, np.array([[1, 0, 0.2], [10 / 255, 20 / 255, 30 / 255]], F))


# ---------------------------------------------------------------- library host readers


def test_point_cloud_load_colmap(tmp_path):
    from tinygs_amd import io
    text = "# POINT3D_ID, X, Y, Z, R, G, B, ERROR, TRACK[]\n\n7 0.25 -1 3.5 12 34 56 0.7 1 2 3 4\n" \
           "8 1 2\n9 -0.125 8 9 200 100 0 1.5\n"
    f = tmp_path / "points3D.txt"
    f.write_text(text)
    pc = io.load_point_cloud(str(f))
    p, c = FM.colmap_points(text)
    assert np.array_equal(pc.points, p) and np.array_equal(pc.colors, c)


@pytest.mark.parametrize("fmt", ["ascii", "binary_little_endian", "binary_big_endian"])
def test_point_cloud_load_ply(tmp_path, fmt):
    from tinygs_amd import io
    g = np.random.default_rng(4)
    n = 50
    xyz = g.normal(0, 3, (n, 3))
    rgb = g.integers(0, 256, (n, 3)).astype(np.uint8)
    cols = [("nx", "float", g.normal(0, 1, n).astype(F)), ("x", "double", xyz[:, 0]), ("y", "double", xyz[:, 1]),
            ("z", "float", xyz[:, 2].astype(F)), ("blue", "uchar", rgb[:, 2]), ("red", "uchar", rgb[:, 0]),
            ("green", "uchar", rgb[:, 1]), ("quality", "int", g.integers(-5, 5, n))]
    f = tmp_path / "cloud.ply"
    FM.write_ply(str(f), cols, fmt, extra_elements=(("camera", 2, [("k", "float"), ("id", "int")]),))
    info = io.ply_info(str(f))
    assert info == {"n_vertices": n, "format": fmt, "has_gaussians": False, "has_colors": True}
    pc = io.load_ply(str(f))
    want = np.stack([xyz[:, 0].astype(F), xyz[:, 1].astype(F), xyz[:, 2].astype(F)], 1)
    # positions are read as double and rounded to float (ascii: repr() round-trips the doubles)
    assert np.array_equal(pc.points, want)
    assert np.array_equal(pc.colors, rgb.astype(F) / F(255.0))


def test_point_cloud_load_errors(tmp_path):
    from tinygs_amd import io
    with pytest.raises(RuntimeError, match="Unsupported point cloud file format"):
        io.load_point_cloud(str(tmp_path / "a.xyz"))
    with pytest.raises(RuntimeError, match="could not open"):
        io.load_point_cloud(str(tmp_path / "missing.ply"))
    f = tmp_path / "nocolor.ply"
    FM.write_ply(str(f), [("x", "float", np.zeros(3, F)), ("y", "float", np.zeros(3, F)),
                          ("z", "float", np.zeros(3, F))])
    with pytest.raises(RuntimeError, match="colors"):
        io.load_point_cloud(str(f))
    t = tmp_path / "trunc.ply"
    FM.write_ply(str(t), [(c, "float", np.zeros(4, F)) for c in "xyz"] + [(c, "uchar", np.zeros(4, np.uint8))
                                                                           for c in ("red", "green", "blue")])
    t.write_bytes(t.read_bytes()[:-5])
    with pytest.raises(RuntimeError, match="truncated"):
        io.load_point_cloud(str(t))
    bad = tmp_path / "bad.ply"
    bad.write_bytes(b"ply\nformat binary_little_endian 1.0\nelement vertex 1\nproperty list uchar int idx\n"
                    b"end_header\n\x00")
    with pytest.raises(RuntimeError, match="list property"):
        io.ply_info(str(bad))
    assert io.ply_info(str(f))["has_colors"] is False


@pytest.mark.parametrize("fmt", ["ascii", "binary_little_endian"])
def test_point_cloud_hostile_counts(tmp_path, fmt):
    # element counts come from the header: a count far beyond what the file
    # holds must fail at once (no allocation of it, no loop over it)
    from tinygs_amd import io
    vert = "property float x\nproperty float y\nproperty float z\nproperty uchar red\nproperty uchar green\n" \
           "property uchar blue\n"
    body = b"0.5 1 2 10 20 30\n" if fmt == "ascii" else struct.pack("<fffBBB", 0.5, 1, 2, 10, 20, 30)
    huge = 10 ** 15
    cases = {"vertex": f"element vertex {huge}\n{vert}",
             "skipped": f"element face {huge}\nproperty int a\nelement vertex 1\n{vert}"}
    for name, elems in cases.items():
        f = tmp_path / f"{name}.ply"
        f.write_bytes(f"ply\nformat {fmt} 1.0\n{elems}end_header\n".encode() + body)
        with pytest.raises(RuntimeError, match="truncated"):
            io.load_point_cloud(str(f))
    # an element without properties holds no bytes, whatever its count
    f = tmp_path / "empty_elem.ply"
    f.write_bytes(f"ply\nformat {fmt} 1.0\nelement camera {huge}\nelement vertex 1\n{vert}end_header\n".encode()
                  + body)
    pc = io.load_point_cloud(str(f))
    assert np.array_equal(pc.points, np.array([[0.5, 1, 2]], F))
    assert np.array_equal(pc.colors, np.array([[10, 20, 30]], F) / F(255.0))
