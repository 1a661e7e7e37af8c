"""Host-side mirror of the reference's data types for the FastGS path.

Names and meanings follow tinygs:
  GPUGaussian3d        tinygs/include/tinygs/core/gpu_gaussian.hpp:9-73
  ImageShape / Image   tinygs/include/tinygs/core/image.hpp:35-85
  GPUBatchInput/Output tinygs/include/tinygs/dataloader/dataloader.hpp:8-19
  RasterizeContext     tinygs/include/tinygs/rasterizer/rasterizer.hpp:9-29
  LossContext          tinygs/include/tinygs/loss/loss.hpp:6-12
Device memory is held in torch tensors (plumbing only); all compute goes
through the C ABI of libtinygs_amd.so.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
from typing import Optional

import numpy as np

from . import _lib
from .image import ImageShape


class DataType:
    Float32 = "float32"
    Float16 = "float16"


def _torch():
    import torch
    return torch


class GPUGaussian3d:
    """SoA Gaussian parameters on the device (or their gradients)."""

    FIELDS = ("means", "scales", "rotations", "opacities", "sh_coefficient_0", "sh_coefficients_rest")

    def __init__(self, n: int = 0, sh_dtype: str = DataType.Float32, device: str = "cuda"):
        torch = _torch()
        f32 = torch.float32
        shd = torch.float16 if sh_dtype == DataType.Float16 else torch.float32
        self.m_means = torch.zeros((n, 3), dtype=f32, device=device)
        self.m_scales = torch.zeros((n, 3), dtype=f32, device=device)
        self.m_rotations = torch.zeros((n, 4), dtype=f32, device=device)
        self.m_opacities = torch.zeros((n,), dtype=f32, device=device)
        self.m_sh_coefficient_0 = torch.zeros((n, 3), dtype=shd, device=device)
        self.m_sh_coefficients_rest = torch.zeros((n, 15, 3), dtype=shd, device=device)
        self.sh_dtype = sh_dtype
        self.m_current_sh_degree = 0
        self.m_scene_scale = 1.0

    # accessors named as in gpu_gaussian.hpp
    def size(self) -> int:
        return int(self.m_means.shape[0])

    def means(self):
        return self.m_means

    def scales(self):
        return self.m_scales

    def rotations(self):
        return self.m_rotations

    def opacities(self):
        return self.m_opacities

    def sh_coefficient_0(self):
        return self.m_sh_coefficient_0

    def sh_coefficients_rest(self):
        return self.m_sh_coefficients_rest

    def scene_scale(self) -> float:
        return self.m_scene_scale

    def set_scene_scale(self, s: float):
        self.m_scene_scale = float(s)

    def set_sh_degree(self, d: int):
        self.m_current_sh_degree = min(3, int(d))

    def get_sh_degree(self) -> int:
        return self.m_current_sh_degree

    def tensors(self):
        return [self.m_means, self.m_scales, self.m_rotations, self.m_opacities, self.m_sh_coefficient_0,
                self.m_sh_coefficients_rest]

    def memset(self, value: int = 0):
        for t in self.tensors():
            if value == 0:
                t.zero_()
            else:
                t.view(_torch().uint8).fill_(value)

    memset_async = memset

    def zero_(self, stream=None):
        """memset_async(0) ordered on `stream` (the caller's gradient zeroing
        at the start of an accumulation cycle, orchestrator.cu:351-353)."""
        torch = _torch()
        if stream is None:
            self.memset(0)
            return
        with torch.cuda.stream(stream):
            self.memset(0)

    def clone(self) -> "GPUGaussian3d":
        g = GPUGaussian3d.__new__(GPUGaussian3d)
        for name in ("m_means", "m_scales", "m_rotations", "m_opacities", "m_sh_coefficient_0",
                     "m_sh_coefficients_rest"):
            setattr(g, name, getattr(self, name).clone())
        g.sh_dtype = self.sh_dtype
        g.m_current_sh_degree = self.m_current_sh_degree
        g.m_scene_scale = self.m_scene_scale
        return g

    def append(self, num_dup: int):
        """GPUGaussian3d::append (gpu_gaussian.cu:161-170): num_dup zero rows
        appended to every array."""
        if num_dup <= 0:
            raise RuntimeError("append: num_dup must be positive")
        torch = _torch()
        for name in ("m_means", "m_scales", "m_rotations", "m_opacities", "m_sh_coefficient_0",
                     "m_sh_coefficients_rest"):
            t = getattr(self, name)
            z = torch.zeros((num_dup,) + tuple(t.shape[1:]), dtype=t.dtype, device=t.device)
            setattr(self, name, torch.cat([t, z]))

    def reorder(self, indices, stream=None):
        """GPUGaussian3d::reorder(uint* indices, stream) (gpu_gaussian.cu:
        273-310): in place, row i becomes old row indices[i] (device int32 /
        uint32 tensor of size() indices)."""
        c = self.to_c()
        _lib.check(_lib.load().tgs_gaussians_reorder(C.byref(c), ptr(indices), stream_ptr(stream)),
                   "GPUGaussian3d::reorder")

    def remove(self, kept_rows, num_kept: int, stream=None):
        """GPUGaussian3d::remove (gpu_gaussian.cu:117-158): keep the rows
        listed (in order) in the device int32 tensor kept_rows[:num_kept]."""
        dst = GPUGaussian3d(num_kept, self.sh_dtype, device=self.m_means.device)
        src_c, dst_c = self.to_c(), dst.to_c()
        _lib.check(_lib.load().tgs_gaussians_gather(C.byref(src_c), C.byref(dst_c), ptr(kept_rows),
                                                    stream_ptr(stream)), "GPUGaussian3d::remove")
        for name in ("m_means", "m_scales", "m_rotations", "m_opacities", "m_sh_coefficient_0",
                     "m_sh_coefficients_rest"):
            setattr(self, name, getattr(dst, name))

    def gradient_like(self) -> "GPUGaussian3d":
        """Zeroed fp32 gradient buffers of the same size."""
        return GPUGaussian3d(self.size(), DataType.Float32, device=self.m_means.device)

    @classmethod
    def from_scene(cls, scene, device: str = "cuda") -> "GPUGaussian3d":
        torch = _torch()
        sh_dtype = DataType.Float16 if getattr(scene, "sh_dtype", "float32") == "float16" else DataType.Float32
        g = cls(0, sh_dtype, device)
        shd = torch.float16 if sh_dtype == DataType.Float16 else torch.float32
        g.m_means = torch.from_numpy(np.ascontiguousarray(scene.means, np.float32)).to(device)
        g.m_scales = torch.from_numpy(np.ascontiguousarray(scene.scales, np.float32)).to(device)
        g.m_rotations = torch.from_numpy(np.ascontiguousarray(scene.rotations, np.float32)).to(device)
        g.m_opacities = torch.from_numpy(np.ascontiguousarray(scene.opacities, np.float32)).to(device)
        g.m_sh_coefficient_0 = torch.from_numpy(np.ascontiguousarray(scene.sh0, np.float32)).to(device).to(shd)
        g.m_sh_coefficients_rest = torch.from_numpy(np.ascontiguousarray(scene.sh_rest, np.float32)).to(device).to(shd)
        g.m_current_sh_degree = scene.sh_degree
        return g

    def to_c(self) -> _lib.tgs_gaussians:
        for t in self.tensors():
            if not t.is_contiguous():
                raise ValueError("GPUGaussian3d tensors must be contiguous")
        return _lib.tgs_gaussians(
            self.m_means.data_ptr(), self.m_scales.data_ptr(), self.m_rotations.data_ptr(),
            self.m_opacities.data_ptr(), self.m_sh_coefficient_0.data_ptr(),
            self.m_sh_coefficients_rest.data_ptr(), self.size(), self.m_current_sh_degree,
            _lib.TGS_DTYPE_FLOAT16 if self.sh_dtype == DataType.Float16 else _lib.TGS_DTYPE_FLOAT32,
            self.m_scene_scale)


@dataclasses.dataclass
class Image:
    shape: ImageShape
    data_type: str = DataType.Float32
    data: object = None  # torch tensor on the device, padded 8x8-tiled

    @classmethod
    def empty(cls, shape: ImageShape, device: str = "cuda", data_type: str = DataType.Float32) -> "Image":
        torch = _torch()
        dt = torch.float16 if data_type == DataType.Float16 else torch.float32
        return cls(shape, data_type, torch.zeros(shape.padded_size, dtype=dt, device=device))

    def __bool__(self):
        return self.data is not None

    def size(self) -> int:
        return self.shape.size()


@dataclasses.dataclass
class GPUBatchInput:
    """Camera of one view. K and w2c are row-major numpy matrices here; the C
    ABI receives them in glm column-major order as the reference stores them."""
    width: int = 0
    height: int = 0
    near: float = 0.01
    far: float = 100.0
    K: np.ndarray = dataclasses.field(default_factory=lambda: np.eye(3))
    w2c: np.ndarray = dataclasses.field(default_factory=lambda: np.eye(4))
    timestamp: int = 0

    @classmethod
    def from_camera(cls, cam) -> "GPUBatchInput":
        K = np.array([[cam.fx, 0.0, cam.cx], [0.0, cam.fy, cam.cy], [0.0, 0.0, 1.0]])
        return cls(cam.width, cam.height, cam.near, cam.far, K, np.asarray(cam.w2c, np.float64))

    def to_c(self) -> _lib.tgs_camera:
        c = _lib.tgs_camera()
        c.width, c.height = int(self.width), int(self.height)
        c.near_plane, c.far_plane = float(self.near), float(self.far)
        k = np.asarray(self.K, np.float32).T.reshape(-1)
        w = np.asarray(self.w2c, np.float32).T.reshape(-1)
        for i in range(9):
            c.K[i] = float(k[i])
        for i in range(16):
            c.w2c[i] = float(w[i])
        return c


@dataclasses.dataclass
class GPUBatchOutput:
    image: Image = dataclasses.field(default_factory=lambda: Image(ImageShape(0, 0)))


@dataclasses.dataclass
class RasterizeContext:
    prepare_input_gradients: bool = False
    inference: bool = False
    stream: object = None          # torch.cuda.Stream or None (current stream)
    grad_scaler: float = 1.0
    fwd_input: GPUBatchInput = dataclasses.field(default_factory=GPUBatchInput)
    fwd_output: GPUBatchOutput = dataclasses.field(default_factory=GPUBatchOutput)
    grad_input: GPUBatchInput = dataclasses.field(default_factory=GPUBatchInput)
    grad_output: GPUBatchOutput = dataclasses.field(default_factory=GPUBatchOutput)
    gaussians_grad: Optional[GPUGaussian3d] = None
    densification_info: object = None   # torch float32 tensor (n, 4) or None


@dataclasses.dataclass
class LossContext:
    pred: Image = None
    target: Image = None
    loss: Image = None
    grad: Image = None
    stream: object = None


def stream_ptr(stream) -> C.c_void_p:
    torch = _torch()
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()
