"""L1Loss / FusedSSIMLoss over the C ABI.

Mirrors tinygs's LossBase / create_loss (tinygs/include/tinygs/loss/loss.hpp:15-47,
tinygs/src/loss/loss.cu:13-27): evaluate(ctx, scale) accumulates the loss
and gradient images.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from .core import DataType, LossContext, ptr, stream_ptr


class LossBase:
    def evaluate(self, ctx: LossContext, scale: float):
        raise NotImplementedError

    def name(self) -> str:
        raise NotImplementedError


class _CLoss(LossBase):
    _type = b""

    def __init__(self):
        h = C.c_void_p()
        _lib.check(_lib.load().tgs_loss_create(self._type, C.byref(h)), "create_loss")
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib.load().tgs_loss_destroy(h)
            except Exception:
                pass
            self._h = None

    def _context(self, ctx: LossContext):
        if ctx.pred.data_type != ctx.target.data_type:
            raise RuntimeError(f"{self.name()}: prediction and target data type must be the same")
        # l1.cu:130-146, fused_ssim.cu:863-906: float32 and float16 images
        dts = {DataType.Float32: _lib.TGS_DTYPE_FLOAT32, DataType.Float16: _lib.TGS_DTYPE_FLOAT16}
        if ctx.pred.data_type not in dts:
            raise RuntimeError(f"{self.name()}: only float32 and float16 are supported")
        shape = ctx.pred.shape
        return _lib.tgs_loss_context(ptr(ctx.pred.data), ptr(ctx.target.data),
                                     ptr(ctx.loss.data) if ctx.loss else None,
                                     ptr(ctx.grad.data) if ctx.grad else None,
                                     shape.width, shape.height, shape.channel, dts[ctx.pred.data_type])

    def evaluate(self, ctx: LossContext, scale: float):
        c = self._context(ctx)
        _lib.check(_lib.load().tgs_loss_evaluate(self._h, C.byref(c), float(scale), stream_ptr(ctx.stream)),
                   self.name())


def evaluate_l1_ssim(loss: LossBase, ctx: LossContext, l1_scale: float, ssim_scale: float, assign: bool = False):
    """L1 (scale l1_scale) then fused SSIM (scale ssim_scale) of one prediction
    in two launches: the same result as evaluating an L1Loss and then a
    FusedSSIMLoss with those scales. assign=True writes the loss / gradient
    images instead of accumulating (as if they had been zeroed first).
    `loss` is any loss object of this module (it holds the SSIM scratch)."""
    c = loss._context(ctx)
    flags = _lib.TGS_LOSS_ASSIGN if assign else 0
    _lib.check(_lib.load().tgs_loss_l1_ssim(loss._h, C.byref(c), float(l1_scale), float(ssim_scale), flags,
                                            stream_ptr(ctx.stream)), "l1_ssim")


class L1Loss(_CLoss):
    _type = b"l1"

    def name(self) -> str:
        return "l1"


class FusedSSIMLoss(_CLoss):
    _type = b"fused_ssim"

    def name(self) -> str:
        return "fused_ssim"


def create_loss(loss_type: str) -> LossBase:
    t = loss_type.lower()
    if t == "l1":
        return L1Loss()
    if t == "fused_ssim":
        return FusedSSIMLoss()
    raise RuntimeError(f"Unknown loss type: {loss_type}")
