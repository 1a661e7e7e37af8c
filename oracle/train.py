"""TEST INFRASTRUCTURE — CPU restatement of the training loop.

Only tests/ (and the fixture script under tests/golden/) may import this
module; the product (tinygs_amd) never does.

Chains the float oracle stages the way tinygs's Orchestrator::train_step
(tinygs/src/orchestrator.cu:335-439) does, with the pieces around it:
  SimpleDataLoader permutation (pcg32 seeded 0, Fisher-Yates with
  next_uint(bound))                         tinygs/src/dataloader/simple.cpp:17-57
  scene scale (max camera distance to the
  mean of the means)                        orchestrator.cu:215-231, :298
  forward (max screen radii into the densification info), L1 + SSIM, blend
  backward, preprocess backward (counters and gradient norms into the
  densification info), SimpleAdam (lr of means times the scene scale)
  DefaultStrategy                           oracle/strategy.py
  SH degree schedule                        orchestrator.cu:750-761
  PsnrMetric                                tinygs/src/loss/psnr.cu:72-128
"""
from __future__ import annotations

import numpy as np

from . import oracle as O
from . import strategy as S

F = np.float32
GROUPS = ("means", "opacities", "rotations", "scales", "sh0", "sh_rest")
WIDTH = {"means": 3, "opacities": 1, "rotations": 4, "scales": 3, "sh0": 3, "sh_rest": 45}


def next_bounded(rng: S.Pcg32, bound: int) -> int:
    """pcg32::next_uint(bound) (pcg32.hpp:68-94)."""
    threshold = ((~bound + 1) & 0xFFFFFFFF) % bound
    while True:
        r = rng.next_uint()
        if r >= threshold:
            return r % bound


class Loader:
    def __init__(self, n: int):
        self.n = n
        self.rng = S.Pcg32()
        self.rng.seed(0, 1)
        self.perm = []
        self.cur = 0
        self.permute()

    def permute(self):
        perm = list(range(self.n))
        for i in range(self.n - 1, 0, -1):
            j = next_bounded(self.rng, i + 1)
            perm[i], perm[j] = perm[j], perm[i]
        self.perm = perm
        self.cur = 0

    def next(self) -> int:
        if self.cur >= len(self.perm):
            self.permute()
        v = self.perm[self.cur]
        self.cur += 1
        return v


def scene_scale(means: np.ndarray, cam_positions: np.ndarray) -> float:
    pc = np.asarray(means, F).reshape(-1, 3)
    inv = F(1.0) / F(pc.shape[0])
    mean = (pc * inv).sum(axis=0, dtype=F)
    d = np.linalg.norm(np.asarray(cam_positions, F) - mean, axis=1)
    return float(F(d.max()))


def psnr(pred: np.ndarray, target: np.ndarray, shape) -> float:
    d = np.clip(np.asarray(pred, F), F(0.0), F(1.0)) - np.asarray(target, F)
    sq = (d * d).astype(np.float64).sum()
    mse = F(sq) / F(shape.size())
    return 100.0 if mse == 0 else float(F(-10.0) * F(np.log10(mse)))


class _View:
    """Scene-like object the oracle stages take."""

    def __init__(self, p, sh_degree, camera, target):
        self.means, self.scales, self.rotations = p["means"], p["scales"], p["rotations"]
        self.opacities, self.sh0 = p["opacities"], p["sh0"]
        self.sh_rest = p["sh_rest"].reshape(-1, 15, 3)
        self.sh_degree, self.camera, self.target = sh_degree, camera, target
        self.sh_dtype = "float32"

    @property
    def n(self):
        return int(self.means.shape[0])


def render_targets(gt: dict, cameras) -> list:
    out = []
    for cam in cameras:
        v = _View({k: np.asarray(a, F).reshape(a.shape[0], -1) if k != "opacities" else np.asarray(a, F)
                   for k, a in gt.items()}, 3, cam, None)
        out.append(O.render(v, "f")[2]["image"])
    return out


class Trainer:
    def __init__(self, scene, strategy_params: dict, lr: dict | None = None, eps: float = 1e-8,
                 sh_degree_interval: int = 1000, max_sh_degree: int = 3, l1_w: float = 0.8, ssim_w: float = 0.2,
                 targets: list | None = None):
        self.cameras = scene.cameras
        # targets[i] may be None for views the run never reads
        self.targets = targets if targets is not None else render_targets(scene.gt, scene.cameras)
        self.p = {k: np.asarray(v, F).reshape(v.shape[0], -1).copy() if k != "opacities" else np.asarray(v, F).copy()
                  for k, v in scene.init.items()}
        self.p["sh_rest"] = self.p["sh_rest"].reshape(-1, 45)
        n = self.p["means"].shape[0]
        self.m1 = {k: np.zeros((n, WIDTH[k]) if WIDTH[k] > 1 else n, F) for k in GROUPS}
        self.m2 = {k: np.zeros((n, WIDTH[k]) if WIDTH[k] > 1 else n, F) for k in GROUPS}
        self.loader = Loader(len(self.cameras))
        self.strategy = S.DefaultStrategy(strategy_params)
        self.lr = dict(lr or {"means": 1.6e-4, "opacities": 5e-2, "rotations": 1e-3, "scales": 5e-3, "shs": 2.5e-3})
        self.eps = eps
        self.sh_interval, self.max_sh = sh_degree_interval, max_sh_degree
        self.sh_degree = 0
        self.l1_w, self.ssim_w = l1_w, ssim_w
        self.info = None
        self.adam_steps = 0
        self.step_count = 0
        self.scale = scene_scale(self.p["means"], np.stack([c.cam_pos for c in self.cameras]))

    def train_step(self):
        i = self.loader.next()
        cam, target = self.cameras[i], self.targets[i]
        v = _View(self.p, self.sh_degree, cam, target)
        shape = cam.shape
        radii = None if self.info is None else np.ascontiguousarray(self.info[:, 3])
        pre = O.preprocess(v, "f", max_radii=radii)
        if radii is not None:
            self.info[:, 3] = radii
        bins = O.bin(v, pre, "f")
        fwd = O.blend_forward(v, pre, bins, "f", True)
        loss = np.zeros(shape.padded_size, F)
        gimg = np.zeros(shape.padded_size, F)
        O.l1(fwd["image"], target, shape, F(self.l1_w), loss, gimg)
        O.ssim(fwd["image"], target, shape, F(self.ssim_w), loss, gimg)
        g2d = O.blend_backward(v, pre, bins, fwd, gimg, "f")
        dens = None if self.info is None else np.ascontiguousarray(self.info.reshape(-1))
        grads = O.preprocess_backward(v, pre, g2d, "f", densif=dens)
        if dens is not None:
            self.info = dens.reshape(-1, 4)
        self.adam_steps += 1
        theta = {k: self.p[k].reshape(-1) for k in GROUPS}
        m1 = {k: self.m1[k].reshape(-1) for k in GROUPS}
        m2 = {k: self.m2[k].reshape(-1) for k in GROUPS}
        lr = dict(self.lr, scene_scale=self.scale)
        O.adam_step(theta, grads, m1, m2, lr, self.adam_steps, grad_scale=1.0, eps=self.eps, max_grad=1.0)
        W, H = cam.width, cam.height
        self.info = self.strategy.step(self.p, self.m1, self.m2, self.info, 1.0, self.scale, W, H)
        if self.step_count % self.sh_interval == 0:
            self.sh_degree = min(self.step_count // self.sh_interval, self.max_sh)
        self.step_count += 1

    def eval_psnr(self, views) -> float:
        vals = []
        for i in views:
            cam = self.cameras[i]
            img = O.render(_View(self.p, self.sh_degree, cam, None), "f")[2]["image"]
            vals.append(psnr(img, self.targets[i], cam.shape))
        return float(np.mean(vals))
