"""TEST INFRASTRUCTURE -- CPU restatement of the on-disk formats and image
layout converters.

Only tests/ may import this module; the product (tinygs_amd) never does.

  ply_header / ply_bytes   save_ply (tinygs/src/core/pointcloud.cpp:111-240)
                           through hapPLY (tinygs/src/core/happly.h: header
                           :1973-2010, element header :1084-1091, binary rows
                           :1120-1126): one little-endian row per vertex, the
                           properties in the order they were added
  write_ply                a general PLY writer (any property order / types,
                           ascii or either byte order) to build reader inputs
  colmap_points            load_from_colmap (pointcloud.cpp:19-73)
  from_cv2 / to_cv2        image_format.cu:68-114 with the loader's widening
                           (tinygs/src/dataloader/dataloader.cu:18-95) and the
                           export's narrowing (tinygs/src/orchestrator.cu:
                           922-935)
"""
from __future__ import annotations

import numpy as np

F = np.float32
HAPPLY_COMMENT = "Written with hapPLY (https://github.com/nmwsharp/happly)"
C0 = F(0.28209479177387814)


def ply_properties(full: bool) -> list[tuple[str, str]]:
    """(name, PLY type) of save_ply's vertex properties, in order."""
    props = [("x", "float"), ("y", "float"), ("z", "float"), ("red", "uchar"), ("green", "uchar"), ("blue", "uchar")]
    if full:
        props += [("f_dc_r", "float"), ("f_dc_g", "float"), ("f_dc_b", "float")]
        for k in range(15):
            props += [(f"f_rest_{c}_{k}", "float") for c in "rgb"]
        props += [("opacity", "float"), ("scale_0", "float"), ("scale_1", "float"), ("scale_2", "float")]
        props += [("rot_w", "float"), ("rot_x", "float"), ("rot_y", "float"), ("rot_z", "float")]
    return props


def ply_header(n: int, full: bool) -> bytes:
    lines = ["ply", "format binary_little_endian 1.0", "comment " + HAPPLY_COMMENT, f"element vertex {n}"]
    lines += [f"property {t} {name}" for name, t in ply_properties(full)]
    lines.append("end_header")
    return ("\n".join(lines) + "\n").encode()


def colour_bytes(sh0: np.ndarray) -> np.ndarray:
    """(unsigned char)(clamp(sh0 * C0 + 0.5, 0, 1) * 255), float arithmetic
    with one rounding per operation, truncation to integer."""
    t = np.asarray(sh0, F) * C0
    t = (t + F(0.5)).astype(F)
    t = np.where(t < F(0.0), F(0.0), np.where(F(1.0) < t, F(1.0), t))
    return (t * F(255.0)).astype(F).astype(np.uint8)


_NP = {"char": "i1", "uchar": "u1", "short": "<i2", "ushort": "<u2", "int": "<i4", "uint": "<u4",
       "float": "<f4", "double": "<f8"}


def ply_bytes(p: dict, full: bool) -> bytes:
    """The whole file save_ply writes for parameters p (means (n,3), scales
    (n,3), rotations (n,4) r x y z, opacities (n,), sh0 (n,3), sh_rest
    (n,45) or (n,15,3); SH given as the float values stored)."""
    n = int(np.asarray(p["means"]).shape[0])
    props = ply_properties(full)
    dt = np.dtype([(name, _NP[t]) for name, t in props])   # packed: no alignment padding
    rows = np.zeros(n, dt)
    m = np.asarray(p["means"], F).reshape(n, 3)
    sh0 = np.asarray(p["sh0"], F).reshape(n, 3)
    col = colour_bytes(sh0)
    for k, name in enumerate("xyz"):
        rows[name] = m[:, k]
    for k, name in enumerate(("red", "green", "blue")):
        rows[name] = col[:, k]
    if full:
        shr = np.asarray(p["sh_rest"], F).reshape(n, 45)
        for k, c in enumerate("rgb"):
            rows[f"f_dc_{c}"] = sh0[:, k]
        for j in range(45):
            rows[f"f_rest_{'rgb'[j % 3]}_{j // 3}"] = shr[:, j]
        rows["opacity"] = np.asarray(p["opacities"], F).reshape(n)
        s = np.asarray(p["scales"], F).reshape(n, 3)
        for k in range(3):
            rows[f"scale_{k}"] = s[:, k]
        q = np.asarray(p["rotations"], F).reshape(n, 4)
        for k, c in enumerate("wxyz"):
            rows[f"rot_{c}"] = q[:, k]
    return ply_header(n, full) + rows.tobytes()


def write_ply(path, columns: list[tuple[str, str, np.ndarray]], fmt: str = "binary_little_endian",
              extra_elements: tuple = ()):
    """A PLY with one vertex element of the given (name, type, values)
    columns in order; fmt ascii / binary_little_endian / binary_big_endian.
    extra_elements: (name, count, [(prop, type)]) elements written before the
    vertex element, filled with zeros (scalar properties only)."""
    n = len(columns[0][2]) if columns else 0
    lines = ["ply", f"format {fmt} 1.0", "comment oracle test file"]
    for name, count, props in extra_elements:
        lines.append(f"element {name} {count}")
        lines += [f"property {t} {pn}" for pn, t in props]
    lines.append(f"element vertex {n}")
    lines += [f"property {t} {name}" for name, t, _ in columns]
    lines.append("end_header")
    head = ("\n".join(lines) + "\n").encode()
    if fmt == "ascii":
        body = []
        for name, count, props in extra_elements:
            body += [" ".join("0" for _ in props)] * count
        for i in range(n):
            vals = []
            for _, t, v in columns:
                x = v[i]
                vals.append(repr(float(x)) if t in ("float", "double") else str(int(x)))
            body.append(" ".join(vals))
        data = ("\n".join(body) + "\n").encode()
    else:
        end = "<" if fmt == "binary_little_endian" else ">"
        parts = []
        for name, count, props in extra_elements:
            edt = np.dtype([(pn, end + _NP[t][-2:]) for pn, t in props])
            parts.append(np.zeros(count, edt).tobytes())
        dt = np.dtype([(name, end + _NP[t][-2:]) for name, t, _ in columns])
        rows = np.zeros(n, dt)
        for name, _, v in columns:
            rows[name] = v
        parts.append(rows.tobytes())
        data = b"".join(parts)
    with open(path, "wb") as f:
        f.write(head + data)


def colmap_points(text: str) -> tuple[np.ndarray, np.ndarray]:
    """load_from_colmap: lines that are empty or start with '#' are skipped;
    numbers are read from the start of the line until one fails to parse; a
    line with >= 7 gives XYZ from columns 1-3 and RGB / 255 from 4-6."""
    pts, cols = [], []
    for line in text.split("\n"):
        if not line or line[0] == "#":
            continue
        vals = []
        for tok in line.split():
            try:
                vals.append(F(float(tok)))
            except ValueError:
                break
        if len(vals) >= 7:
            pts.append(vals[1:4])
            cols.append([F(v) / F(255.0) for v in vals[4:7]])
    return np.array(pts, F).reshape(-1, 3), np.array(cols, F).reshape(-1, 3)


# ---------------------------------------------------------------- images

CHAR_TO_FLOAT = F(1.0) / F(255.0)


def tiled_index(width: int, height: int) -> np.ndarray:
    """(H, W) per-channel index of pixel (y, x) in the 8x8-tiled plane
    (get_linear_index_tiled, tinygs/include/tinygs/common.hpp:404-408)."""
    tw = (width + 7) // 8
    y = np.arange(height)[:, None]
    x = np.arange(width)[None, :]
    return ((y // 8) * tw + x // 8) * 64 + (y % 8) * 8 + (x % 8)


def widen(v: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "uint8":
        return np.asarray(v, np.uint8)
    f = (CHAR_TO_FLOAT * np.asarray(v, F)).astype(F)
    return f.astype(np.float16) if dtype == "float16" else f


def narrow(v: np.ndarray) -> np.ndarray:
    """uint8 of min(max(255 v, 0), 255) truncated; NaN -> 0."""
    a = np.asarray(v)
    if a.dtype == np.uint8:
        return a
    t = np.asarray(a, F) * F(255.0)
    return np.fmin(np.fmax(t, F(0.0)), F(255.0)).astype(np.uint8)


def from_cv2(src: np.ndarray, width: int, height: int, bgr: bool = True, dtype: str = "uint8") -> np.ndarray:
    """(H, W, C) u8 -> padded tiled planar buffer; padding zero."""
    c = src.shape[2]
    tw, th = (width + 7) // 8, (height + 7) // 8
    cs = tw * th * 64
    out = np.zeros(c * cs, np.uint8)
    idx = tiled_index(width, height)
    for ch in range(c):
        sc = c - 1 - ch if bgr else ch
        out[ch * cs + idx] = src[:, :, sc]
    return widen(out, dtype)


def to_cv2(src: np.ndarray, width: int, height: int, channels: int, bgr: bool = True) -> np.ndarray:
    """padded tiled planar buffer -> (H, W, C) u8."""
    tw, th = (width + 7) // 8, (height + 7) // 8
    cs = tw * th * 64
    b = narrow(src)
    out = np.zeros((height, width, channels), np.uint8)
    idx = tiled_index(width, height)
    for ch in range(channels):
        dc = channels - 1 - ch if bgr else ch
        out[:, :, dc] = b[ch * cs + idx]
    return out
