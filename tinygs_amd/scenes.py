"""Seeded synthetic scenes for the FastGS training path (configs 1-5).

Parameters follow the SoA layout of tinygs's GPUGaussian3d
(tinygs/include/tinygs/core/gpu_gaussian.hpp:67-72): means (N,3), scales (N,3)
log-space, rotations (N,4) stored (r, x, y, z), opacities (N,) logits,
sh0 (N,3), sh_rest (N,15,3) -- always 15 bases per Gaussian
(tinygs/src/core/gpu_gaussian.cu:25).

Random numbers come from numpy's PCG64 (O'Neill's PCG family); every field
draws from its own child stream of ``SeedSequence(seed)`` so that changing N
for one field does not shift the others.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np

from .image import ImageShape


@dataclasses.dataclass
class Camera:
    """Pinhole camera in the reference's conventions.

    ``w2c`` is the row-major 4x4 world-to-camera matrix (the reference keeps a
    glm column-major matrix and transposes it on upload, fastgs.cu:95-100);
    the camera looks along +z and depth = row 2 . [mu, 1].
    ``K`` entries: fx = K[0][0], fy = K[1][1], cx = K[2][0], cy = K[2][1] in glm
    indexing (camera.hpp:29-35); here they are kept as scalars.
    """

    width: int
    height: int
    fx: float
    fy: float
    cx: float
    cy: float
    w2c: np.ndarray  # (4,4) float64, row-major
    near: float = 0.01
    far: float = 100.0

    @property
    def cam_pos(self) -> np.ndarray:
        """Camera centre = column 3 of inverse(w2c) (fastgs.cu:96,100), from the
        float32 matrix the rasterizer receives, inverted in double."""
        return np.linalg.inv(self.w2c.astype(np.float32).astype(np.float64))[:3, 3]

    @property
    def shape(self) -> ImageShape:
        return ImageShape(self.width, self.height, 3)

    @property
    def grid(self) -> tuple[int, int]:
        return ((self.width + 15) // 16, (self.height + 15) // 16)

    def as_array(self) -> np.ndarray:
        """Flat float32[23]: fx fy cx cy near far, w2c rows 0-2, cam_pos, W, H."""
        out = np.zeros(23, dtype=np.float32)
        out[0:6] = [self.fx, self.fy, self.cx, self.cy, self.near, self.far]
        out[6:18] = self.w2c[:3, :].astype(np.float32).reshape(-1)
        out[18:21] = self.cam_pos.astype(np.float32)
        out[21] = float(self.width)
        out[22] = float(self.height)
        return out


@dataclasses.dataclass
class Scene:
    means: np.ndarray
    scales: np.ndarray
    rotations: np.ndarray
    opacities: np.ndarray
    sh0: np.ndarray
    sh_rest: np.ndarray
    sh_degree: int
    camera: Camera
    target: np.ndarray  # padded 8x8-tiled image, float32[3 * channel_stride]
    name: str = ""
    sh_dtype: str = "float32"

    @property
    def n(self) -> int:
        return int(self.means.shape[0])


def look_at(position, target=(0.0, 0.0, 0.0), up=(0.0, 1.0, 0.0)) -> np.ndarray:
    """Row-major w2c of a camera at ``position`` looking at ``target`` (+z forward)."""
    p = np.asarray(position, dtype=np.float64)
    z = np.asarray(target, dtype=np.float64) - p
    z /= np.linalg.norm(z)
    x = np.cross(z, -np.asarray(up, dtype=np.float64))
    if np.linalg.norm(x) < 1e-9:
        x = np.cross(z, np.array([1.0, 0.0, 0.0]))
    x /= np.linalg.norm(x)
    y = np.cross(z, x)
    R = np.stack([x, y, z])
    w2c = np.eye(4)
    w2c[:3, :3] = R
    w2c[:3, 3] = -R @ p
    return w2c


def _streams(seed: int, n: int):
    return [np.random.Generator(np.random.PCG64(s)) for s in np.random.SeedSequence(seed).spawn(n)]


def _unit_quats(rng, n):
    q = rng.standard_normal((n, 4))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return q.astype(np.float32)


def _random_unit(rng):
    v = rng.standard_normal(3)
    return v / np.linalg.norm(v)


def _target(rng, cam: Camera) -> np.ndarray:
    shape = cam.shape
    return rng.random(shape.padded_size, dtype=np.float64).astype(np.float32)


def config1(seed: int = 1, n: int = 1024) -> Scene:
    """Tiny scene: BASELINE config 1 (64x64, SH degree 0, camera at (0,0,-3))."""
    r = _streams(seed, 8)
    means = r[0].uniform(-1.0, 1.0, (n, 3)).astype(np.float32)
    scales = r[1].normal(-3.0, 0.3, (n, 3)).astype(np.float32)
    rots = _unit_quats(r[2], n)
    opac = r[3].normal(0.0, 1.0, n).astype(np.float32)
    sh0 = r[4].uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    sh_rest = np.zeros((n, 15, 3), dtype=np.float32)
    w2c = np.eye(4)
    w2c[2, 3] = 3.0
    cam = Camera(64, 64, 64.0, 64.0, 32.0, 32.0, w2c)
    return Scene(means, scales, rots, opac, sh0, sh_rest, 0, cam, _target(r[5], cam), "config1")


def config2(seed: int = 2, n: int = 100_000, width: int = 800, height: int = 800) -> Scene:
    """100k Gaussians, 800x800, SH degree 3."""
    r = _streams(seed, 10)
    means = r[0].standard_normal((n, 3))
    norm = np.linalg.norm(means, axis=1, keepdims=True)
    means = np.where(norm > 2.0, means * (2.0 / np.maximum(norm, 1e-12)), means).astype(np.float32)
    scales = r[1].normal(-4.0, 0.5, (n, 3)).astype(np.float32)
    rots = _unit_quats(r[2], n)
    opac = r[3].normal(0.0, 1.5, n).astype(np.float32)
    sh0 = r[4].uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    sh_rest = r[5].normal(0.0, 0.05, (n, 15, 3)).astype(np.float32)
    pos = 4.0 * _random_unit(r[6])
    cam = Camera(width, height, 1100.0 * width / 800.0, 1100.0 * height / 800.0, width / 2.0, height / 2.0, look_at(pos))
    return Scene(means, scales, rots, opac, sh0, sh_rest, 3, cam, _target(r[7], cam), "config2")


def config3(seed: int = 3, n: int = 1_000_000, width: int = 1920, height: int = 1080,
            sh_dtype: str = "float16") -> Scene:
    """BASELINE config 3 (the headline): 1M Gaussians, 1920x1080, SH degree 3
    stored as fp16, 32 isotropic clusters in a 6x6x6 box, 2% scale outliers."""
    r = _streams(seed, 12)
    centres = r[0].uniform(-3.0, 3.0, (32, 3))
    which = r[1].integers(0, 32, n)
    means = (centres[which] + r[2].normal(0.0, 0.3, (n, 3))).astype(np.float32)
    scales = r[3].normal(-4.5, 0.8, (n, 3))
    outlier = r[4].random(n) < 0.02
    scales[outlier] = -1.5
    scales = scales.astype(np.float32)
    rots = _unit_quats(r[5], n)
    opac = r[6].normal(0.5, 1.5, n).astype(np.float32)
    sh0 = r[7].uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    sh_rest = r[8].normal(0.0, 0.05, (n, 15, 3)).astype(np.float32)
    if sh_dtype == "float16":
        sh0 = sh0.astype(np.float16).astype(np.float32)
        sh_rest = sh_rest.astype(np.float16).astype(np.float32)
    pos = 10.0 * _random_unit(r[9])
    sx, sy = width / 1920.0, height / 1080.0
    cam = Camera(width, height, 1200.0 * sx, 1200.0 * sy, width / 2.0, height / 2.0, look_at(pos))
    return Scene(means, scales, rots, opac, sh0, sh_rest, 3, cam, _target(r[10], cam), "config3", sh_dtype)


def config4(seed: int = 4, n: int = 3_000_000, width: int = 3840, height: int = 2160,
            depth: float = 2.0, focal: float = 2000.0) -> Scene:
    """high-overlap stress. Means uniform in a unit cube on
    the optical axis (centre at ``depth``), camera at the origin looking +z.

    A projected Gaussian's radius is a fixed fraction of the cube's projected
    width (3 sigma ~ 0.09 of it at log-scale -3.5), so the focal length trades
    covered tiles against instances per Gaussian. At 480x270 with focal 800
    and 60k Gaussians the cube fills the frame and the median tile holds about
    3,100 Gaussians (the reduced parity case). At 3840x2160 the same geometry
    with 3M Gaussians would make ~5e9 instances (hundreds of GB of sort and
    checkpoint buffers), so the full-size default keeps focal 2000: the cube
    covers the central ~1000x1000 pixels, whose tiles hold a median of tens
    of thousands of Gaussians (5.5e8 instances)."""
    r = _streams(seed, 10)
    means = r[0].uniform(-0.5, 0.5, (n, 3))
    means[:, 2] += depth
    means = means.astype(np.float32)
    scales = r[1].normal(-3.5, 0.6, (n, 3)).astype(np.float32)
    rots = _unit_quats(r[2], n)
    opac = r[3].normal(-1.0, 1.0, n).astype(np.float32)
    sh0 = r[4].uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    sh_rest = r[5].normal(0.0, 0.05, (n, 15, 3)).astype(np.float32)
    cam = Camera(width, height, focal, focal, width / 2.0, height / 2.0, np.eye(4))
    return Scene(means, scales, rots, opac, sh0, sh_rest, 3, cam, _target(r[6], cam), "config4")


def config2_gaussians(seed: int, n: int) -> dict:
    """Gaussian parameters drawn as in config 2 (means ~N(0,1)^3 clipped to a
    radius-2 ball, log-scales ~N(-4,0.5), opacity logits ~N(0,1.5), SH degree
    3: DC ~U(0,1), higher bands ~N(0,0.05))."""
    r = _streams(seed, 6)
    means = r[0].standard_normal((n, 3))
    norm = np.linalg.norm(means, axis=1, keepdims=True)
    means = np.where(norm > 2.0, means * (2.0 / np.maximum(norm, 1e-12)), means).astype(np.float32)
    return {"means": means, "scales": r[1].normal(-4.0, 0.5, (n, 3)).astype(np.float32),
            "rotations": _unit_quats(r[2], n), "opacities": r[3].normal(0.0, 1.5, n).astype(np.float32),
            "sh0": r[4].uniform(0.0, 1.0, (n, 3)).astype(np.float32),
            "sh_rest": r[5].normal(0.0, 0.05, (n, 15, 3)).astype(np.float32)}


@dataclasses.dataclass
class TrainingScene:
    """a ground-truth Gaussian set rendered from many
    cameras (the targets) and an initial Gaussian set to train."""
    gt: dict
    init: dict
    cameras: list
    width: int
    height: int
    name: str = "config5"


def config5(seed: int = 5, n_init: int = 500_000, n_gt: int = 400_000, width: int = 1600, height: int = 1060,
            n_cameras: int = 200, radius: float = 4.0) -> TrainingScene:
    """500k initial Gaussians seeded as in config 2,
    width x height views from n_cameras random cameras on a sphere of the
    given radius looking at the origin, targets rendered from a fixed seeded
    ground-truth set of 400k Gaussians (drawn as in config 2, other seed).
    The focal length keeps config 2's 1100 px per 800 px of width."""
    r = _streams(seed, 3)
    f = 1100.0 * width / 800.0
    # near / far of SimpleDataLoader::next (simple.cpp:60-61)
    cams = [Camera(width, height, f, f, width / 2.0, height / 2.0, look_at(radius * _random_unit(r[0])), 0.1, 100.0)
            for _ in range(n_cameras)]
    return TrainingScene(config2_gaussians(seed + 1000, n_gt), config2_gaussians(seed + 2000, n_init), cams, width,
                         height)


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4}


def make(config: int, **kw) -> Scene:
    return CONFIGS[config](**kw)


def grad_image(seed: int, shape: ImageShape, scale: float | None = None) -> np.ndarray:
    """Seeded dL/dimage ~ U(0,1)/P (the hand check of examples/single_gs.cpp:171-174)."""
    rng = _streams(seed, 1)[0]
    p = shape.width * shape.height
    s = (1.0 / p) if scale is None else scale
    return (rng.random(shape.padded_size) * s).astype(np.float32)


def perturb_sh_degree(scene: Scene, degree: int) -> Scene:
    return dataclasses.replace(scene, sh_degree=degree)


def active_sh_bases(degree: int) -> int:
    return (degree + 1) * (degree + 1)


__all__ = ["Camera", "Scene", "look_at", "config1", "config2", "config3", "config4", "make",
           "grad_image", "active_sh_bases", "CONFIGS", "math"]
