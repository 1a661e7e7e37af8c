"""Densification strategy over the C ABI.

Mirrors tinygs's StrategyParams / StrategyBase / DefaultStrategy /
create_strategy (tinygs/include/tinygs/strategy/strategy.hpp:7-121,
tinygs/src/strategy/strategy.cpp:10-177, tinygs/src/strategy/default.cu):
same parameter names and defaults, same step schedule (refine every
``refine_every`` steps inside [start_refine, end_refine]: duplicate / split,
then prune, then fresh densification info; opacity reset every
``reset_every`` steps), same RNG (pcg32 seeded with ``seed``, stream 1) and
the same order of the Gaussian / gradient / optimiser updates. The device
work (selection, compaction, split, row gathers, random numbers) runs in the
HIP kernels behind the tgs_densify_* / tgs_prune_select / tgs_*_gather entry
points; tensor sizing is torch's (plumbing).

Only "default" is built; "mcmc" and "improved" raise.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import logging

import numpy as np

from . import _lib
from .core import GPUGaussian3d, RasterizeContext, ptr, stream_ptr

log = logging.getLogger("tinygs_amd.strategy")


def _f32mul(a, b) -> float:
    """float * float as the reference evaluates its thresholds."""
    return float(np.float32(a) * np.float32(b))

PCG32_DEFAULT_STATE = 0x853C49E6748FEA9B
PCG32_DEFAULT_STREAM = 0xDA3E39CB94B95BDB


@dataclasses.dataclass
class StrategyParams:
    pruning_opacity_threshold: float = 0.005
    pruning_scale_threshold: float = 0.1
    max_screen_size: float = 10.0
    duplicate_grad_threshold: float = 0.0002
    duplicate_scale_threshold: float = 0.01
    reset_reset_optimizer: bool = False
    absgrad: bool = False
    refine_every: int = 100
    start_refine: int = 500
    end_refine: int = 15_000
    max_num_gaussians: int = 10_000_000
    reset_every: int = 3_000
    seed: int = 42

    def to_json(self) -> dict:
        return dataclasses.asdict(self)

    def from_json(self, config: dict):
        for f in dataclasses.fields(self):
            if f.name in config:
                cur = getattr(self, f.name)
                setattr(self, f.name, bool(config[f.name]) if isinstance(cur, bool) else type(cur)(config[f.name]))


class StrategyBase:
    def __init__(self, gaussians: GPUGaussian3d, gaussians_grad: GPUGaussian3d, optimizer):
        self.m_gaussians = gaussians
        self.m_gaussians_grad = gaussians_grad
        self.m_optimizer = optimizer
        self.m_params = StrategyParams()
        self.m_step_count = 0

    def step(self, ctx: RasterizeContext):
        self.step_impl(ctx)
        self.m_step_count += 1

    def this_step(self) -> int:
        return self.m_step_count

    def step_impl(self, ctx: RasterizeContext):
        raise NotImplementedError

    def reset(self):
        raise NotImplementedError

    def on_remove(self, kept_flag, kept_rows, num_kept: int, stream=None):
        """strategy.cpp:19-31: Gaussians, gradients, then the optimiser."""
        if num_kept <= 0:
            return
        if self.m_gaussians is not None:
            self.m_gaussians.remove(kept_rows, num_kept, stream)
        if self.m_gaussians_grad is not None:
            self.m_gaussians_grad.remove(kept_rows, num_kept, stream)
        if self.m_optimizer is not None:
            self.m_optimizer.remove(kept_flag, num_kept, stream)

    def on_duplicate(self, num_duplications: int, stream=None):
        """strategy.cpp:33-45: rows appended to the Gaussians, gradients and
        optimiser state (the new rows are filled afterwards)."""
        if num_duplications <= 0:
            return
        if self.m_gaussians is not None:
            self.m_gaussians.append(num_duplications)
        if self.m_gaussians_grad is not None:
            self.m_gaussians_grad.append(num_duplications)
        if self.m_optimizer is not None:
            self.m_optimizer.duplicate(num_duplications, stream)

    def on_reset_opacity(self, stream=None):
        """strategy.cpp:55-63."""
        if self.m_optimizer is not None:
            self.m_optimizer.reset_opacity(stream)
            if self.m_params.reset_reset_optimizer:
                log.info("Reset optimizer after reset opacity!")
                self.m_optimizer.reset(stream)

    def set_params(self, config: dict):
        self.m_params.from_json(config)

    def get_params(self) -> dict:
        return self.m_params.to_json()


class DefaultStrategy(StrategyBase):
    """default.cu:17-359."""

    def __init__(self, gaussians, gaussians_grad, optimizer):
        super().__init__(gaussians, gaussians_grad, optimizer)
        # pcg32's default constructor; set_params reseeds (default.cu:349-352)
        self.m_rng = _lib.tgs_pcg32(PCG32_DEFAULT_STATE, PCG32_DEFAULT_STREAM)

    def set_params(self, config: dict):
        super().set_params(config)
        _lib.load().tgs_pcg32_seed(C.byref(self.m_rng), int(self.m_params.seed) & (2**64 - 1), 1)

    def get_params(self) -> dict:
        p = super().get_params()
        p["type"] = "default"
        return p

    def reset(self):
        pass

    @staticmethod
    def _fresh_info(n: int, like):
        import torch
        return torch.zeros((n, 4), dtype=torch.float32, device=like.device)

    def step_impl(self, ctx: RasterizeContext):
        """default.cu:40-69."""
        import torch
        s = ctx.stream
        torch.cuda.synchronize()
        g = self.m_gaussians
        if ctx.densification_info is None:
            ctx.densification_info = self._fresh_info(g.size(), g.means())
        p = self.m_params
        step = self.this_step()
        if step % p.refine_every == 0 and p.start_refine <= step <= p.end_refine:
            if g.size() < p.max_num_gaussians:
                self.duplicate(ctx)
            self.prune(ctx)
            ctx.densification_info = self._fresh_info(g.size(), g.means())
        if p.reset_every > 0 and step % p.reset_every == 0 and p.start_refine <= step < p.end_refine:
            gc = g.to_c()
            _lib.check(_lib.load().tgs_reset_opacity(C.byref(gc), _f32mul(2.0, p.pruning_opacity_threshold),
                                                     stream_ptr(s)),
                       "reset_opacity")
            self.on_reset_opacity(s)

    def duplicate(self, ctx: RasterizeContext):
        """default.cu:71-297."""
        import torch
        s = ctx.stream
        g = self.m_gaussians
        n = g.size()
        info = ctx.densification_info
        if info is None or int(info.shape[0]) != n:
            log.warning("Densification info is not provided or has wrong size, skip duplication.")
            return
        p = self.m_params
        dev = g.means().device
        flags = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
        src = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        n_dup, n_split = C.c_int64(), C.c_int64()
        L = _lib.load()
        gc = g.to_c()
        _lib.check(L.tgs_densify_select(C.byref(gc), ptr(info), _f32mul(p.duplicate_grad_threshold, ctx.grad_scaler),
                                        _f32mul(p.duplicate_scale_threshold, g.scene_scale()), int(p.absgrad),
                                        ptr(flags), ptr(src), C.byref(n_dup), C.byref(n_split), stream_ptr(s)),
                   "DefaultStrategy::duplicate")
        grows = n_dup.value + n_split.value
        log.info("Add %d gaussians (%d total, %d split, %d duplicate)", grows, grows + n, n_split.value, n_dup.value)
        self.last_counts = {"duplicate": n_dup.value, "split": n_split.value}
        if grows == 0:
            return
        self.on_duplicate(grows, s)
        rnd = torch.empty(grows * 6, dtype=torch.float32, device=dev)
        _lib.check(L.tgs_random_logistic(C.byref(self.m_rng), grows * 6, ptr(rnd), 0.0, 1.0, stream_ptr(s)),
                   "generate_random_logistic")
        gc = g.to_c()
        _lib.check(L.tgs_densify_apply(C.byref(gc), n, ptr(src), grows, ptr(flags), ptr(rnd), stream_ptr(s)),
                   "DefaultStrategy::duplicate")

    def prune(self, ctx: RasterizeContext):
        """default.cu:300-341."""
        import torch
        s = ctx.stream
        g = self.m_gaussians
        p = self.m_params
        n = g.size()
        info = ctx.densification_info
        n_info = int(info.shape[0])
        cam = ctx.fwd_input
        limit_ss = _f32mul(max(cam.width, cam.height), p.max_screen_size)
        dev = g.means().device
        alive = torch.empty(max(n, 1), dtype=torch.uint8, device=dev)
        kept = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        n_kept = C.c_int64()
        gc = g.to_c()
        _lib.check(_lib.load().tgs_prune_select(
            C.byref(gc), ptr(info), n_info, float(p.pruning_opacity_threshold),
            _f32mul(p.pruning_scale_threshold, g.scene_scale()), limit_ss,
            int(self.this_step() > p.reset_every), ptr(alive), ptr(kept), C.byref(n_kept), stream_ptr(s)),
            "DefaultStrategy::prune")
        log.info("Remove %d dead gaussians (kept %d)", n - n_kept.value, n_kept.value)
        self.last_counts = dict(getattr(self, "last_counts", {}), kept=n_kept.value)
        self.on_remove(alive, kept, n_kept.value, s)


def create_strategy(strategy_type: str, gaussians, gaussians_grad, optimizer) -> StrategyBase:
    t = strategy_type.lower()
    if t == "default":
        return DefaultStrategy(gaussians, gaussians_grad, optimizer)
    if t in ("mcmc", "improved"):
        raise RuntimeError(f"Strategy '{strategy_type}' is not built (only 'default')")
    raise RuntimeError(f"Unknown strategy type: {strategy_type}")
