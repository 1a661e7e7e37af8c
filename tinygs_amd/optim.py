"""SimpleAdam over the C ABI.

Mirrors tinygs's OptimizerBase / SimpleAdam / create_optimizer
(tinygs/include/tinygs/optim/optim.hpp:39-106,
tinygs/include/tinygs/optim/simple_adam.hpp:30-87, tinygs/src/optim/optim.cu:86-105).
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .core import GPUGaussian3d, stream_ptr

GROUPS = ("means", "opacities", "rotations", "scales", "sh0", "sh_rest")


class OptimizerBase:
    def __init__(self, gaussians: GPUGaussian3d, gaussians_grad: GPUGaussian3d):
        self.m_gaussians = gaussians
        self.m_gaussians_grad = gaussians_grad

    def get_gaussians(self):
        return self.m_gaussians

    def get_gaussians_grad(self):
        return self.m_gaussians_grad


class SimpleAdam(OptimizerBase):
    def __init__(self, gaussians: GPUGaussian3d, gaussians_grad: GPUGaussian3d):
        super().__init__(gaussians, gaussians_grad)
        if gaussians.size() != gaussians_grad.size():
            raise RuntimeError("SimpleAdam::step: gaussians and gaussians_grad must have same size")
        self._cp = gaussians.to_c()
        self._cg = gaussians_grad.to_c()
        h = C.c_void_p()
        _lib.check(_lib.load().tgs_adam_create(C.byref(self._cp), C.byref(self._cg), C.byref(h)), "create_optimizer")
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib.load().tgs_adam_destroy(h)
            except Exception:
                pass
            self._h = None

    def _rebind(self):
        self._cp = self.m_gaussians.to_c()
        self._cg = self.m_gaussians_grad.to_c()
        _lib.check(_lib.load().tgs_adam_set_gaussians(self._h, C.byref(self._cp), C.byref(self._cg)), "set_gaussians")

    def step(self, scale: float, stream=None, row_mask: int | None = None, device_step: bool = False,
             rows: str | None = None, same_step: bool = False):
        """OptimizerBase::step. row_mask: device address of a per-Gaussian
        byte mask (a sparse backward's); unmarked gradient rows are taken as
        zero without being read. device_step=True keeps the step count and
        bias corrections on the device (TGS_ADAM_DEVICE_STEP), so the step
        can be captured into a graph and replayed. rows="unmarked" / "marked"
        updates only the rows whose mask byte is 0 / nonzero
        (TGS_ADAM_ROWS_UNMARKED / _MARKED), same_step=True repeats the last
        call's step count (TGS_ADAM_SAME_STEP): one step in two parts."""
        self._rebind()
        L = _lib.load()
        flags = _lib.TGS_ADAM_DEVICE_STEP if device_step else 0
        if rows is not None:
            flags |= {"unmarked": _lib.TGS_ADAM_ROWS_UNMARKED, "marked": _lib.TGS_ADAM_ROWS_MARKED}[rows]
        if same_step:
            flags |= _lib.TGS_ADAM_SAME_STEP
        if flags:
            _lib.check(L.tgs_adam_step_ex(self._h, float(scale), C.c_void_p(row_mask) if row_mask else None,
                                          flags, stream_ptr(stream)), "SimpleAdam::step")
        elif row_mask is None:
            _lib.check(L.tgs_adam_step(self._h, float(scale), stream_ptr(stream)), "SimpleAdam::step")
        else:
            _lib.check(L.tgs_adam_step_masked(self._h, float(scale), C.c_void_p(row_mask), stream_ptr(stream)),
                       "SimpleAdam::step")

    def device_steps(self, stream=None) -> int:
        """The step count of the device-step mode (waits for the stream)."""
        v = C.c_int64()
        _lib.check(_lib.load().tgs_adam_device_steps(self._h, C.byref(v), stream_ptr(stream)), "device_steps")
        return v.value

    def reset(self, stream=None):
        _lib.check(_lib.load().tgs_adam_reset(self._h, stream_ptr(stream)), "SimpleAdam::reset")

    def remove(self, kept_flag, num_kept: int, stream=None):
        """SimpleAdam::remove (simple_adam.cu:841-906). The reference builds
        its row mapping from the optimiser's Gaussians, which StrategyBase has
        already shrunk to num_kept rows: the kept rows among the first
        num_kept flags, in order, then row 0 for the remaining moment rows.
        That mapping is reproduced here."""
        torch = __import__("torch")
        rows = torch.zeros(max(num_kept, 1), dtype=torch.int32, device=kept_flag.device)
        cnt = C.c_int64()
        L = _lib.load()
        _lib.check(L.tgs_flags_compact(C.c_void_p(kept_flag.data_ptr()), int(num_kept), C.c_void_p(rows.data_ptr()),
                                       C.byref(cnt), stream_ptr(stream)), "SimpleAdam::remove")
        _lib.check(L.tgs_adam_gather(self._h, C.c_void_p(rows.data_ptr()), int(num_kept), stream_ptr(stream)),
                   "SimpleAdam::remove")

    def duplicate(self, num_duplicate: int, stream=None):
        """SimpleAdam::duplicate (simple_adam.cu:908-924): zero moment rows
        for the appended Gaussians."""
        if num_duplicate <= 0:
            return
        _lib.check(_lib.load().tgs_adam_append(self._h, int(num_duplicate), stream_ptr(stream)),
                   "SimpleAdam::duplicate")

    def reset_indices(self, indices, num_reset: int | None = None, stream=None):
        """SimpleAdam::reset(int* indices, int num_reset) (simple_adam.cu:
        944-979): zero both moments of the given rows (device int32 tensor)."""
        n = int(indices.numel() if num_reset is None else num_reset)
        _lib.check(_lib.load().tgs_adam_reset_rows(self._h, C.c_void_p(indices.data_ptr()), n, stream_ptr(stream)),
                   "SimpleAdam::reset")

    def reorder(self, indices, stream=None):
        """SimpleAdam::reorder(uint* indices) (simple_adam.cu:1037-1097):
        new row i = old row indices[i] (device int32/uint32 tensor, one per row)."""
        _lib.check(_lib.load().tgs_adam_reorder(self._h, C.c_void_p(indices.data_ptr()), stream_ptr(stream)),
                   "SimpleAdam::reorder")

    def reset_opacity(self, stream=None):
        """SimpleAdam::reset_opacity (simple_adam.cu:981-985)."""
        _lib.check(_lib.load().tgs_adam_reset_opacity(self._h, stream_ptr(stream)), "SimpleAdam::reset_opacity")

    def set_lr(self, lr: float):
        _lib.check(_lib.load().tgs_adam_set_lr(self._h, float(lr)), "set_lr")

    def get_lr(self) -> float:
        return float(_lib.load().tgs_adam_get_lr(self._h))

    def global_steps(self) -> int:
        return int(_lib.load().tgs_adam_global_steps(self._h))

    def get_params(self) -> dict:
        p = _lib.tgs_adam_params()
        _lib.check(_lib.load().tgs_adam_get_params(self._h, C.byref(p)), "get_params")
        return {f: getattr(p, f) for f, _ in p._fields_}

    def set_params(self, config: dict):
        p = _lib.tgs_adam_params()
        _lib.check(_lib.load().tgs_adam_get_params(self._h, C.byref(p)), "get_params")
        alias = {"eps": "epsilon"}
        for k, v in config.items():
            k = alias.get(k, k)
            if k == "decay_reduction":
                p.decay_mean = 1 if v == "mean" else 0
            elif hasattr(p, k):
                setattr(p, k, v)
            else:
                raise RuntimeError(f"SimpleAdam: unknown parameter {k}")
        _lib.check(_lib.load().tgs_adam_set_params(self._h, C.byref(p)), "set_params")

    def moments(self, group: str):
        import torch
        k = GROUPS.index(group)
        a, b = C.c_void_p(), C.c_void_p()
        _lib.check(_lib.load().tgs_adam_moments(self._h, k, C.byref(a), C.byref(b)), "moments")
        mult = (3, 1, 4, 3, 3, 45)[k]
        n = mult * self.m_gaussians.size()
        dev = self.m_gaussians.means().device
        m1 = torch.empty(n, dtype=torch.float32, device=dev)
        m2 = torch.empty(n, dtype=torch.float32, device=dev)
        _lib.copy_device(a.value, 4 * n, m1)
        _lib.copy_device(b.value, 4 * n, m2)
        return m1, m2


def create_optimizer(optimizer_type: str, gaussians: GPUGaussian3d, gaussians_grad: GPUGaussian3d):
    t = optimizer_type.lower()
    if t == "simple_adam":
        return SimpleAdam(gaussians, gaussians_grad)
    raise RuntimeError(f"Unknown optimizer type: {optimizer_type}")
