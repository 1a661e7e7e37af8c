"""Synthetic multi-view dataset and SimpleDataLoader for the training loop.

SimpleDataLoader mirrors tinygs's SimpleDataLoader
(tinygs/src/dataloader/simple.cpp:9-103): views in a Fisher-Yates
permutation drawn from pcg32 (seeded 0, reseeded by set_params' "seed"),
a fresh permutation per epoch, near 0.1 / far 100. The dataset renders its
targets once on the GPU from a ground-truth Gaussian set (the synthetic
stand-in for image files) and keeps them resident in HBM, so next() moves
no pixels.
"""
from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np

from . import _lib
from .core import DataType, GPUBatchInput, GPUGaussian3d, Image, RasterizeContext
from .rasterizer import create_rasterizer


def gaussians_from_arrays(p: dict, sh_degree: int = 3, device: str = "cuda") -> GPUGaussian3d:
    import torch
    g = GPUGaussian3d(0)
    g.m_means = torch.from_numpy(np.ascontiguousarray(p["means"], np.float32)).to(device)
    g.m_scales = torch.from_numpy(np.ascontiguousarray(p["scales"], np.float32)).to(device)
    g.m_rotations = torch.from_numpy(np.ascontiguousarray(p["rotations"], np.float32)).to(device)
    g.m_opacities = torch.from_numpy(np.ascontiguousarray(p["opacities"], np.float32)).to(device)
    g.m_sh_coefficient_0 = torch.from_numpy(np.ascontiguousarray(p["sh0"], np.float32)).to(device)
    g.m_sh_coefficients_rest = torch.from_numpy(
        np.ascontiguousarray(p["sh_rest"], np.float32).reshape(-1, 15, 3)).to(device)
    g.m_current_sh_degree = sh_degree
    return g


@dataclasses.dataclass
class View:
    camera: object      # scenes.Camera
    target: Image       # device image, 8x8-tiled, of the dataset's data type


class SyntheticViewDataset:
    """DatasetBase over synthetic views: camera i and its target, the render
    of the ground-truth Gaussians (SH degree 3) from camera i. data_type is
    the dataset's image type (the reference's "data_type", e.g.
    configs/default.json:4): float16 targets are the float32 renders
    rounded to nearest half on the device (float_to_half_gpu,
    image_format.cu:117-139)."""

    def __init__(self, scene, device: str = "cuda", data_type: str = DataType.Float32):
        import torch
        gt = gaussians_from_arrays(scene.gt, 3, device)
        r = create_rasterizer("fastgs")
        r.set_gaussians(gt)
        self.views = []
        self.data_type = data_type
        for cam in scene.cameras:
            ctx = RasterizeContext()
            ctx.fwd_input = GPUBatchInput.from_camera(cam)
            ctx.fwd_output.image = Image.empty(cam.shape, device)
            r.forward(ctx)
            target = ctx.fwd_output.image
            if data_type == DataType.Float16:
                half = Image.empty(cam.shape, device, DataType.Float16)
                _lib.check(_lib.load().tgs_convert(target.data.data_ptr(), _lib.TGS_DTYPE_FLOAT32,
                                                   half.data.data_ptr(), _lib.TGS_DTYPE_FLOAT16,
                                                   target.data.numel(), None), "float_to_half")
                target = half
            self.views.append(View(cam, target))
        torch.cuda.synchronize()
        self.width, self.height = scene.width, scene.height

    def size(self) -> int:
        return len(self.views)

    def __getitem__(self, i: int) -> View:
        return self.views[i]

    def camera_positions(self) -> np.ndarray:
        return np.stack([v.camera.cam_pos for v in self.views])


class SimpleDataLoader:
    def __init__(self, dataset):
        self.m_dataset = dataset
        self.m_rng = _lib.tgs_pcg32()
        _lib.load().tgs_pcg32_seed(C.byref(self.m_rng), 0, 1)
        self.m_permutation = []
        self.m_current_index = 0
        self.generate_permutation()

    def generate_permutation(self):
        n = self.m_dataset.size()
        perm = list(range(n))
        L = _lib.load()
        for i in range(n - 1, 0, -1):
            j = int(L.tgs_pcg32_next_uint(C.byref(self.m_rng), i + 1))
            perm[i], perm[j] = perm[j], perm[i]
        self.m_permutation = perm
        self.m_current_index = 0

    def set_params(self, params: dict):
        if "seed" in params:
            _lib.load().tgs_pcg32_seed(C.byref(self.m_rng), int(params["seed"]), 1)

    def reset(self):
        self.generate_permutation()

    def next(self):
        """(GPUBatchInput, target Image) of the next view."""
        if self.m_current_index >= len(self.m_permutation):
            self.generate_permutation()
        v = self.m_dataset[self.m_permutation[self.m_current_index]]
        self.m_current_index += 1
        return GPUBatchInput.from_camera(v.camera), v.target

    def get_dataset(self):
        return self.m_dataset
