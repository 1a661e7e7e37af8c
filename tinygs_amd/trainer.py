"""The training loop around the FastGS path.

Mirrors tinygs's Orchestrator (tinygs/include/tinygs/orchestrator.hpp:24-120,
tinygs/src/orchestrator.cu): OrchestratorConfig's names and defaults; train()
recomputes the scene scale first (:295-298); train_step (:335-439) takes the
next view, runs forward, the weighted losses (weight * grad_scaler), backward,
the LR scheduler and SimpleAdam step (gradients scaled by
1 / (grad_scaler * accumulate_grad_steps)), the densification strategy, the
scene-scale recompute and the SH-degree schedule (:750-761); PsnrMetric
(tinygs/src/loss/psnr.cu:72-128); the LR schedulers of
tinygs/src/optim/lr_scheduler.cpp.

Gradients of the parameters are handed to Adam sparsely (rows that received
a gradient; the others are zero) and L1 + SSIM run as one fused evaluation
that assigns the loss / gradient images, which together replace the
reference's per-step zeroing (orchestrator.cu:351-355) with the same
results. Morton reordering (reorder_gaussians_interval) runs at initialize()
and every interval steps, as in the reference (orchestrator.cu:718-720,
429-432).
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import logging
import math
import time

import numpy as np

from . import _lib
from .core import DataType, Image, LossContext, RasterizeContext, stream_ptr
from .loss import create_loss, evaluate_l1_ssim

log = logging.getLogger("tinygs_amd.trainer")


# ---------------------------------------------------------------- LR schedulers (lr_scheduler.cpp)

class LrSchedulerBase:
    def __init__(self, optimizer, initial_lr: float):
        self.m_optimizer = optimizer
        self.m_current_lr = float(initial_lr)
        if optimizer is not None:
            optimizer.set_lr(self.m_current_lr)

    def update_lr(self, lr: float):
        self.m_current_lr = float(np.float32(lr))
        if self.m_optimizer is not None:
            self.m_optimizer.set_lr(self.m_current_lr)

    def get_lr(self) -> float:
        return self.m_current_lr


class ConstantLR(LrSchedulerBase):
    def step(self) -> float:
        self.update_lr(self.m_current_lr)
        return self.m_current_lr

    def reset(self):
        pass

    def get_params(self) -> dict:
        return {"type": "constant", "lr": self.m_current_lr}

    def set_params(self, params: dict):
        if "lr" in params:
            self.update_lr(params["lr"])


class ExponentialLR(LrSchedulerBase):
    """lr_scheduler.cpp:58-100: lr = initial_lr * decay_rate ** step_count
    (std::pow in double, rounded to float), step_count incremented after."""

    def __init__(self, optimizer, initial_lr: float, decay_rate: float):
        super().__init__(optimizer, initial_lr)
        self.m_initial_lr = float(np.float32(initial_lr))
        self.m_decay_rate = float(np.float32(decay_rate))
        self.m_step_count = 0

    def _lr(self) -> float:
        return float(np.float32(self.m_initial_lr * math.pow(self.m_decay_rate, self.m_step_count)))

    def step(self) -> float:
        lr = self._lr()
        self.m_step_count += 1
        self.update_lr(lr)
        return lr

    def reset(self):
        self.m_step_count = 0
        self.update_lr(self.m_initial_lr)

    def get_params(self) -> dict:
        return {"type": "exponential", "initial_lr": self.m_initial_lr, "decay_rate": self.m_decay_rate,
                "step_count": self.m_step_count}

    def set_params(self, params: dict):
        if "initial_lr" in params:
            self.m_initial_lr = float(np.float32(params["initial_lr"]))
        if "decay_rate" in params:
            self.m_decay_rate = float(np.float32(params["decay_rate"]))
        if "step_count" in params:
            self.m_step_count = int(params["step_count"])
        self.update_lr(self._lr())


def create_lr_scheduler(kind: str, optimizer, params: dict | None = None):
    params = params or {}
    k = kind.lower()
    if k == "constant":
        return ConstantLR(optimizer, params.get("lr", 1.0))
    if k == "exponential":
        return ExponentialLR(optimizer, params.get("initial_lr", 1.0), params.get("decay_rate", 1.0))
    raise RuntimeError(f"Unknown lr scheduler type: {kind}")


# ---------------------------------------------------------------- PSNR

class PsnrMetric:
    """psnr.cu:72-128 through tgs_psnr (the device reduction)."""

    def evaluate(self, pred: Image, target: Image, stream=None) -> float:
        if pred.shape != target.shape:
            raise RuntimeError("Prediction and target shapes must match")
        if pred.data_type != target.data_type:
            raise RuntimeError("PSNR: prediction and target data type must be the same")
        dt = _lib.TGS_DTYPE_FLOAT16 if pred.data_type == DataType.Float16 else _lib.TGS_DTYPE_FLOAT32
        ctx = _lib.tgs_loss_context(pred.data.data_ptr(), target.data.data_ptr(), None, None, pred.shape.width,
                                    pred.shape.height, pred.shape.channel, dt)
        out = C.c_float()
        _lib.check(_lib.load().tgs_psnr(C.byref(ctx), C.byref(out), stream_ptr(stream)), "PsnrMetric::evaluate")
        return float(out.value)


# ---------------------------------------------------------------- orchestrator

@dataclasses.dataclass
class OrchestratorConfig:
    """orchestrator.hpp:24-70 (the fields the training path reads).
    train_data_type / eval_data_type: "float32" or "float16" images; float16
    renders with the fp16-image rasterizer and runs the fp16 losses, as the
    reference's default configs do (configs/default.json:99-100)."""
    max_steps: int = 30000
    accumulate_grad_steps: int = 1
    sh_degree_interval: int = 1000
    max_sh_degree: int = 3
    grad_scaler: float = 1.0
    scene_scale_recompute_interval: int = 1000
    reorder_gaussians_interval: int = 1000
    train_data_type: str = DataType.Float32
    eval_data_type: str = DataType.Float32


@dataclasses.dataclass
class TrainingState:
    current_step: int = 0
    current_loss: float = 0.0


class Orchestrator:
    def __init__(self, config: OrchestratorConfig, gaussians, gradients, rasterizer, optimizer, dataloader,
                 losses=(("l1", 0.8), ("fused_ssim", 0.2)), strategy=None, lr_scheduler=None, stream=None):
        import torch
        self.m_config = config
        self.m_gaussians = gaussians
        self.m_gradients = gradients
        self.m_rasterizer = rasterizer
        self.m_optimizer = optimizer
        self.m_dataloader = dataloader
        self.m_strategy = strategy
        self.m_lr_scheduler = lr_scheduler
        self.m_losses = [(create_loss(k), float(w)) for k, w in losses]
        self.m_state = TrainingState()
        self.stream = stream
        ds = dataloader.get_dataset()
        from .image import ImageShape
        shape = ImageShape(ds.width, ds.height, 3)
        for dt in (config.train_data_type, config.eval_data_type):
            if dt not in (DataType.Float32, DataType.Float16):
                raise RuntimeError(f"unsupported image data type {dt}")
        if int(config.accumulate_grad_steps) < 1:
            raise RuntimeError("accumulate_grad_steps must be at least 1")
        # orchestrator.cu:682-707: render, loss and gradient images of the training data type
        self.m_pred = Image.empty(shape, data_type=config.train_data_type)
        self.m_loss = Image.empty(shape, data_type=config.train_data_type)
        self.m_grad = Image.empty(shape, data_type=config.train_data_type)
        self.m_eval_pred = (self.m_pred if config.eval_data_type == config.train_data_type
                            else Image.empty(shape, data_type=config.eval_data_type))
        self.m_ctx = RasterizeContext(stream=stream, grad_scaler=config.grad_scaler)
        self.m_ctx.fwd_output.image = self.m_pred
        self.m_ctx.grad_output.image = self.m_grad
        self.m_ctx.gaussians_grad = gradients
        rasterizer.set_gaussians(gaussians)
        self._torch = torch

    # orchestrator.cu:215-231
    def recompute_scene_scale(self):
        pc = self.m_gaussians.means().detach().cpu().numpy().astype(np.float32)
        inv = np.float32(1.0) / np.float32(pc.shape[0])
        mean = (pc * inv).sum(axis=0, dtype=np.float32)
        d = np.linalg.norm(self.m_dataloader.get_dataset().camera_positions().astype(np.float32) - mean, axis=1)
        scale = float(np.float32(d.max())) if d.size else 0.0
        self.m_gaussians.set_scene_scale(scale)
        log.info("Recompute scene scale: %g", scale)

    # orchestrator.cu:750-761
    def update_sh_degree(self):
        c = self.m_config
        if self.m_state.current_step % c.sh_degree_interval == 0:
            d = min(self.m_state.current_step // c.sh_degree_interval, c.max_sh_degree)
            self.m_gaussians.set_sh_degree(int(d))

    def train_step(self):
        """orchestrator.cu:335-439.

        With accumulate_grad_steps == 1 the gradients go to Adam sparsely
        (the backward writes only rows that received a gradient, Adam reads
        only those), which equals zeroing, accumulating and a dense step.
        With more steps per cycle the gradients are zeroed at the cycle start
        (:351-353), every backward accumulates into them, and the cycle's last
        step runs a dense Adam step scaled by 1 / (grad_scaler * steps)
        (:390-404)."""
        c = self.m_config
        st = self.m_state
        accum = int(c.accumulate_grad_steps)
        if st.current_step % accum == 0 and accum > 1:
            self.m_gradients.zero_(self.stream)
        cam, target = self.m_dataloader.next()
        if target.data_type != c.train_data_type:
            raise RuntimeError("Prediction and target data type must be the same (dataset images are "
                               f"{target.data_type}, train_data_type is {c.train_data_type})")
        ctx = self.m_ctx
        ctx.fwd_input = cam
        ctx.gaussians_grad = self.m_gradients
        self.m_rasterizer.forward(ctx)
        lctx = LossContext(self.m_pred, target, self.m_loss, self.m_grad, self.stream)
        (l1, w1), (_, w2) = self.m_losses
        evaluate_l1_ssim(l1, lctx, w1 * c.grad_scaler, w2 * c.grad_scaler, assign=True)
        self.m_rasterizer.backward(ctx, sparse=accum == 1)
        if (st.current_step + 1) % accum == 0:
            if self.m_lr_scheduler is not None:
                self.m_lr_scheduler.step()
            # float arithmetic as in :401-403
            scale = float(np.float32(np.float32(1.0) / np.float32(c.grad_scaler)) / np.float32(accum))
            mask = self.m_rasterizer.grad_row_mask() if accum == 1 else None
            self.m_optimizer.step(scale, self.stream, row_mask=mask)
        if self.m_strategy is not None:
            self.m_strategy.step(ctx)
        if st.current_step > 0:
            if c.scene_scale_recompute_interval > 0 and st.current_step % c.scene_scale_recompute_interval == 0:
                self.recompute_scene_scale()
            if c.reorder_gaussians_interval > 0 and st.current_step % c.reorder_gaussians_interval == 0:
                self.reorder_gaussians()
        self.update_sh_degree()
        st.current_step += 1

    def initialize(self):
        """The part of orchestrator.cu:639-730 that touches the path: Morton
        reordering of the Gaussians before the first step whenever
        reorder_gaussians_interval > 0 (:718-720)."""
        if self.m_config.reorder_gaussians_interval > 0:
            self.reorder_gaussians()
        self.m_initialized = True

    def reorder_gaussians(self):
        """orchestrator.cu:26-90, 1038-1061: permute the Gaussians, their
        gradients, the optimiser's moments and the densification info by the
        Morton code of the means (stable, so equal codes keep their order)."""
        from . import morton
        idx = morton.morton_order(self.m_gaussians.means(), self.stream)
        self.m_gaussians.reorder(idx, self.stream)
        self.m_gradients.reorder(idx, self.stream)
        self.m_optimizer.reorder(idx, self.stream)
        di = self.m_ctx.densification_info
        if di is not None:
            self.m_ctx.densification_info = morton.gather_rows(di, idx, self.stream)
        if self.m_strategy is not None and hasattr(self.m_strategy, "on_reorder"):
            self.m_strategy.on_reorder(self.m_ctx)

    def train(self, n_steps: int):
        """orchestrator.cu:295-330 for n_steps steps: initialize (once), the
        scene scale, then the steps."""
        if len(self.m_losses) != 2:
            raise RuntimeError("the loop runs the fused L1 + SSIM loss pair")
        if not getattr(self, "m_initialized", False):
            self.initialize()
        self.recompute_scene_scale()
        for _ in range(n_steps):
            self.train_step()

    def eval_psnr(self, views=None) -> float:
        """Mean PSNR over the dataset's views (or the given indices)."""
        ds = self.m_dataloader.get_dataset()
        idx = range(ds.size()) if views is None else views
        m = PsnrMetric()
        vals = []
        ctx = RasterizeContext(stream=self.stream)
        ctx.fwd_output.image = self.m_eval_pred   # orchestrator.cu:446-456: eval_data_type
        for i in idx:
            v = ds[i]
            from .core import GPUBatchInput
            ctx.fwd_input = GPUBatchInput.from_camera(v.camera)
            self.m_rasterizer.forward(ctx)
            vals.append(m.evaluate(self.m_eval_pred, v.target, self.stream))
        return float(np.mean(vals)) if vals else 0.0
