"""On-disk formats and image layout converters, over the C ABI.

Mirrors tinygs/include/tinygs/core/pointcloud.hpp:11-26 (PointCloud,
load_from_colmap, load_ply, load_point_cloud, save_ply) and
tinygs/include/tinygs/utils/image_format.hpp (from_cv2, to_cv2,
half_to_float_gpu, float_to_half_gpu, hwc_to_chw, chw_to_hwc):

  save_ply(filename, gaussians, full_features)   pointcloud.cpp:111-240, from
                                                 device arrays (no host copy of
                                                 the Gaussians)
  load_gaussians_ply(filename)                   the inverse of a full-feature
                                                 save_ply (restart from an
                                                 export)
  load_point_cloud / load_ply / load_from_colmap pointcloud.cpp:19-109
  from_cv2 / to_cv2                              image_format.cu:68-114 on the
                                                 device; with a float / half
                                                 Image the u8 widening of the
                                                 data loader (dataloader.cu:
                                                 18-95) or the export's
                                                 narrowing (orchestrator.cu:
                                                 896-937) is folded in
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import os

import numpy as np

from . import _lib
from .core import DataType, GPUGaussian3d, stream_ptr
from .image import ImageShape


@dataclasses.dataclass
class PointCloud:
    points: np.ndarray   # (n, 3) float32
    colors: np.ndarray   # (n, 3) float32 in [0, 1]


def _fn(filename) -> bytes:
    return os.fsencode(filename)


def save_ply(filename, gs: GPUGaussian3d, full_features: bool = False, stream=None):
    """save_ply (pointcloud.cpp:111-240): binary PLY of the Gaussians, byte
    for byte what the reference's hapPLY writer produces."""
    g = gs.to_c()
    _lib.check(_lib.load().tgs_ply_save(_fn(filename), C.byref(g), int(bool(full_features)), stream_ptr(stream)),
               "save_ply")


def ply_info(filename) -> dict:
    info = _lib.tgs_ply_info()
    _lib.check(_lib.load().tgs_ply_read_info(_fn(filename), C.byref(info)), "ply_info")
    return {"n_vertices": int(info.n_vertices), "format": ("ascii", "binary_little_endian",
                                                           "binary_big_endian")[info.format],
            "has_gaussians": bool(info.has_gaussians), "has_colors": bool(info.has_colors)}


def load_gaussians_ply(filename, sh_dtype: str = DataType.Float32, sh_degree: int = 3, device: str = "cuda",
                       stream=None) -> GPUGaussian3d:
    """Gaussians of a full-feature PLY (the reference's property names or the
    common 3DGS ones) into new device arrays."""
    n = ply_info(filename)["n_vertices"]
    g = GPUGaussian3d(n, sh_dtype, device=device)
    g.set_sh_degree(sh_degree)
    c = g.to_c()
    _lib.check(_lib.load().tgs_ply_load_gaussians(_fn(filename), C.byref(c), stream_ptr(stream)),
               "load_gaussians_ply")
    return g


def load_point_cloud(filename) -> PointCloud:
    """load_point_cloud (pointcloud.cpp:94-109): .ply or COLMAP points3D .txt."""
    L = _lib.load()
    n = C.c_int64(0)
    _lib.check(L.tgs_point_cloud_load(_fn(filename), C.byref(n), None, None), "load_point_cloud")
    pts = np.zeros((n.value, 3), np.float32)
    cols = np.zeros((n.value, 3), np.float32)
    if n.value:
        _lib.check(L.tgs_point_cloud_load(_fn(filename), C.byref(n), pts.ctypes.data, cols.ctypes.data),
                   "load_point_cloud")
    return PointCloud(pts[:n.value], cols[:n.value])


def load_ply(filename) -> PointCloud:
    if not str(filename).lower().endswith(".ply"):
        raise RuntimeError("load_ply expects a .ply file")
    return load_point_cloud(filename)


def load_from_colmap(filename) -> PointCloud:
    if not str(filename).lower().endswith(".txt"):
        raise RuntimeError("load_from_colmap expects a .txt file")
    return load_point_cloud(filename)


# ---------------------------------------------------------------- images

_DTYPE = {"float32": _lib.TGS_DTYPE_FLOAT32, "float16": _lib.TGS_DTYPE_FLOAT16, "uint8": _lib.TGS_DTYPE_UINT8}


def _dtype_code(t) -> int:
    name = str(t).replace("torch.", "")
    if name not in _DTYPE:
        raise RuntimeError(f"unsupported image dtype {t}")
    return _DTYPE[name]


def from_cv2(dst, src, shape: ImageShape, bgr: bool = True, stream=None):
    """from_cv2(dst, src, shape) (image_format.cu:68-90): src an (H, W, C) u8
    device tensor (BGR when bgr), dst the padded tiled device tensor (uint8,
    float32 or float16: the widening (1 / 255) v of the data loader folded
    in); padding written as zero."""
    if tuple(src.shape) != (shape.height, shape.width, shape.channel) or str(src.dtype) != "torch.uint8":
        raise RuntimeError("from_cv2: src must be a uint8 (H, W, C) tensor of the shape")
    if dst.numel() != shape.padded_size:
        raise RuntimeError("from_cv2: dst must hold the padded size")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise RuntimeError("from_cv2: tensors must be contiguous")
    _lib.check(_lib.load().tgs_image_from_hwc_u8(src.data_ptr(), shape.width, shape.height, shape.channel, int(bgr),
                                                 dst.data_ptr(), _dtype_code(dst.dtype), stream_ptr(stream)),
               "from_cv2")


def to_cv2(dst, src, shape: ImageShape, bgr: bool = True, stream=None):
    """to_cv2 (image_format.cu:93-114) for a uint8 src; for float32 / float16
    the export's truncation of clamp(255 v, 0, 255) (orchestrator.cu:922-935).
    dst is an (H, W, C) uint8 device tensor."""
    if tuple(dst.shape) != (shape.height, shape.width, shape.channel) or str(dst.dtype) != "torch.uint8":
        raise RuntimeError("to_cv2: dst must be a uint8 (H, W, C) tensor of the shape")
    if src.numel() != shape.padded_size:
        raise RuntimeError("to_cv2: src must hold the padded size")
    if not (src.is_contiguous() and dst.is_contiguous()):
        raise RuntimeError("to_cv2: tensors must be contiguous")
    _lib.check(_lib.load().tgs_image_to_hwc_u8(src.data_ptr(), _dtype_code(src.dtype), shape.width, shape.height,
                                               shape.channel, int(bgr), dst.data_ptr(), stream_ptr(stream)),
               "to_cv2")


def convert(dst, src, stream=None):
    """Elementwise dtype conversion between uint8 / float16 / float32 device
    tensors of the same size."""
    if dst.numel() != src.numel():
        raise RuntimeError("convert: sizes differ")
    _lib.check(_lib.load().tgs_convert(src.data_ptr(), _dtype_code(src.dtype), dst.data_ptr(), _dtype_code(dst.dtype),
                                       src.numel(), stream_ptr(stream)), "convert")


def half_to_float_gpu(dst, src, n: int | None = None, stream=None):
    """image_format.cu:133-135."""
    convert(dst if n is None else dst[:n], src if n is None else src[:n], stream)


def float_to_half_gpu(dst, src, n: int | None = None, stream=None):
    """image_format.cu:137-139."""
    convert(dst if n is None else dst[:n], src if n is None else src[:n], stream)


def hwc_to_chw(src: np.ndarray, shape: ImageShape) -> np.ndarray:
    """hwc_to_chw (image_format.cu:11-23, :39-51), host arrays."""
    return np.ascontiguousarray(np.asarray(src).reshape(shape.height, shape.width, shape.channel).transpose(2, 0, 1))


def chw_to_hwc(src: np.ndarray, shape: ImageShape) -> np.ndarray:
    """chw_to_hwc (image_format.cu:25-37, :53-65), host arrays."""
    return np.ascontiguousarray(np.asarray(src).reshape(shape.channel, shape.height, shape.width).transpose(1, 2, 0))
