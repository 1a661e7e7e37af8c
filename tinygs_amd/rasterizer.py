"""FastGSRasterizer over the C ABI.

Mirrors tinygs's RasterizerBase / FastGSRasterizer / create_rasterizer
(tinygs/include/tinygs/rasterizer/rasterizer.hpp:38-61,
tinygs/include/tinygs/rasterizer/fastgs.hpp:14-37,
tinygs/src/rasterizer/rasterizer.cpp:44-53): same method names, same
accumulation and error behaviour (RuntimeError where the reference throws
std::runtime_error).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .core import DataType, GPUGaussian3d, RasterizeContext, ptr, stream_ptr


class RasterizerBase:
    def forward(self, ctx: RasterizeContext):
        raise NotImplementedError

    def backward(self, ctx: RasterizeContext):
        raise NotImplementedError

    def set_gaussians(self, gaussians: GPUGaussian3d):
        self.m_gaussians = gaussians

    def get_params(self) -> dict:
        raise NotImplementedError

    def set_params(self, params: dict):
        raise NotImplementedError


class FastGSRasterizer(RasterizerBase):
    def __init__(self):
        L = _lib.load()
        h = C.c_void_p()
        _lib.check(L.tgs_rasterizer_create(b"fastgs", C.byref(h)), "create_rasterizer")
        self._h = h
        self.m_gaussians = None
        self.m_params = {"f16_grad_scaler": 1.0, "enable_pose_opt": False}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib.load().tgs_rasterizer_destroy(h)
            except Exception:
                pass
            self._h = None

    def set_gaussians(self, gaussians: GPUGaussian3d):
        self.m_gaussians = gaussians
        self._cg = gaussians.to_c()
        _lib.check(_lib.load().tgs_rasterizer_set_gaussians(self._h, C.byref(self._cg)), "set_gaussians")

    def forward(self, ctx: RasterizeContext, no_sync: bool = False):
        """no_sync=True: the forward does not wait for the instance count and
        uses the capacity of reserve() instead (TGS_FORWARD_NO_SYNC), so it can
        be queued ahead or captured into a HIP graph; check status() later."""
        if self.m_gaussians is None:
            raise RuntimeError("Gaussians not set")
        # the pointers may have changed (e.g. tensors replaced); rebind
        self._cg = self.m_gaussians.to_c()
        L = _lib.load()
        _lib.check(L.tgs_rasterizer_set_gaussians(self._h, C.byref(self._cg)), "set_gaussians")
        img = ctx.fwd_output.image
        # fastgs.cu:143-188: a float16 image selects the fp16-image rasterizer (FGS16)
        if img.data_type == DataType.Float32:
            dt = _lib.TGS_DTYPE_FLOAT32
        elif img.data_type == DataType.Float16:
            dt = _lib.TGS_DTYPE_FLOAT16
        else:
            raise RuntimeError("FastGSRasterizer: float32 or float16 images only")
        cam = ctx.fwd_input.to_c()
        _lib.check(L.tgs_rasterizer_forward_ex(self._h, C.byref(cam), ptr(img.data), dt,
                                               ptr(ctx.densification_info),
                                               _lib.TGS_FORWARD_NO_SYNC if no_sync else 0,
                                               stream_ptr(ctx.stream)), "forward")

    def reserve(self, max_instances: int, grid_tiles: int, stream=None):
        """Instance capacity of no-sync forwards (tgs_rasterizer_reserve)."""
        _lib.check(_lib.load().tgs_rasterizer_reserve(self._h, int(max_instances), int(grid_tiles),
                                                      stream_ptr(stream)), "reserve")

    def status(self, clear_capacity_flag: bool = False, stream=None) -> int:
        """Waits for the queued work and returns the device state of the
        forwards so far: 0, or _lib.TGS_ERR_CAPACITY when a no-sync forward
        needed more instances than reserved. Other failures raise."""
        rc = _lib.load().tgs_rasterizer_status(self._h, 1 if clear_capacity_flag else 0, stream_ptr(stream))
        if rc == _lib.TGS_ERR_CAPACITY:
            return rc
        _lib.check(rc, "status")
        return 0

    def backward(self, ctx: RasterizeContext, assign: bool = False, sparse: bool = False, keep_2d: bool = False):
        """Accumulates into ctx.gaussians_grad (reference contract). assign=True
        writes the gradients instead (zero for culled Gaussians): the caller's
        zeroing fused into the backward. sparse=True writes only the rows that
        received a gradient (see grad_row_mask); the others keep their old
        contents and stand for zero."""
        if self.m_gaussians is None or ctx.gaussians_grad is None:
            raise RuntimeError("Gaussians or gradient gaussians not set")
        if assign and sparse:
            raise RuntimeError("assign and sparse are exclusive")
        g = ctx.gaussians_grad.to_c()
        L = _lib.load()
        pose = bool(self.m_params["enable_pose_opt"])
        flags = (_lib.TGS_BACKWARD_ASSIGN if assign else 0) | (_lib.TGS_BACKWARD_SPARSE if sparse else 0) | \
            (_lib.TGS_BACKWARD_POSE if pose else 0) | (_lib.TGS_BACKWARD_KEEP_2D if keep_2d else 0)
        _lib.check(L.tgs_rasterizer_backward_ex(self._h, ptr(ctx.grad_output.image.data),
                                                ptr(ctx.fwd_output.image.data), C.byref(g),
                                                ptr(ctx.densification_info), flags,
                                                stream_ptr(ctx.stream)), "backward")
        # fastgs.cu:373-383: grad_input.w2c is the pose gradient (zero without
        # pose optimisation); row-major here, like GPUBatchInput.w2c
        if pose:
            out = (C.c_float * 16)()
            _lib.check(L.tgs_rasterizer_grad_w2c(self._h, out, stream_ptr(ctx.stream)), "backward")
            ctx.grad_input.w2c = np.array(out, dtype=np.float64).reshape(4, 4).T.copy()
        else:
            ctx.grad_input.w2c = np.zeros((4, 4))

    def grad_row_mask(self) -> int:
        """Device address of the byte mask [n] of the last sparse backward
        (1: the row was written, 0: its gradient is zero and was not written)."""
        m = C.c_void_p()
        _lib.check(_lib.load().tgs_rasterizer_grad_row_mask(self._h, C.byref(m)), "grad_row_mask")
        return m.value

    def backward_rows(self, stream=None) -> int:
        """Device address of the byte mask [n] of the rows a sparse backward
        after the last forward will write, queued on `stream` before that
        backward runs (equal to grad_row_mask after it)."""
        m = C.c_void_p()
        _lib.check(_lib.load().tgs_rasterizer_backward_rows(self._h, C.byref(m), stream_ptr(stream)),
                   "backward_rows")
        return m.value

    def counts(self):
        v, i, t = C.c_int64(), C.c_int64(), C.c_int64()
        _lib.check(_lib.load().tgs_rasterizer_counts(self._h, C.byref(v), C.byref(i), C.byref(t)), "counts")
        return v.value, i.value, t.value

    def debug_view(self) -> dict:
        """Copies of the internal buffers of the last forward (tests only)."""
        import torch
        dv = _lib.tgs_debug_view()
        _lib.check(_lib.load().tgs_rasterizer_debug_view(self._h, C.byref(dv)), "debug_view")
        n = self.m_gaussians.size()
        V, I, T = dv.n_visible, dv.n_instances, dv.n_tiles
        dev = self.m_gaussians.means().device
        cs = None

        def grab(p, count, dtype):
            t = torch.empty(max(int(count), 0), dtype=dtype, device=dev)
            if p and count:
                _lib.copy_device(p, t.numel() * t.element_size(), t)
            return t

        out = {
            "n_touched": grab(dv.n_touched, n, torch.int32),
            "bounds": grab(dv.bounds, 4 * n, torch.int32).view(-1, 4)[:, :2].reshape(-1),
            "mean2d": grab(dv.mean2d, 2 * n, torch.float32),
            "conic_opacity": grab(dv.conic_opacity, 4 * n, torch.float32),
            "color": grab(dv.color, 4 * n, torch.float32),
            # the library sorts depth bits minus the near plane's bits; add them back
            "depth_sorted_keys": ((grab(dv.depth_sorted_keys, V, torch.int32).long() + int(dv.depth_key_base))
                                  & 0xFFFFFFFF).to(torch.int32),
            "depth_sorted_prims": grab(dv.depth_sorted_prims, V, torch.int32),
            "instance_tiles": grab(dv.instance_tiles, I, torch.int32),
            "instance_prims": grab(dv.instance_prims, I, torch.int32),
            "tile_ranges": grab(dv.tile_ranges, 2 * T, torch.int32),
            "tile_max": grab(dv.tile_max, T, torch.int32),
            "n_visible": V, "n_instances": I, "n_tiles": T,
            "image_dtype": int(dv.image_dtype),
        }
        del cs
        return out

    def debug_grad2d(self) -> dict:
        """The summed 2D gradients of the last backward run with keep_2d=True,
        in the oracle's layout (tests only)."""
        import torch
        dv = _lib.tgs_debug_view()
        _lib.check(_lib.load().tgs_rasterizer_debug_view(self._h, C.byref(dv)), "debug_view")
        if not dv.grad2d:
            raise RuntimeError("no backward with keep_2d since the last forward")
        n = self.m_gaussians.size()
        t = torch.empty(12 * n, dtype=torch.float32, device=self.m_gaussians.means().device)
        _lib.copy_device(dv.grad2d, t.numel() * 4, t)
        g = t.cpu().numpy().reshape(n, 12)
        return {"grad_mean2d": np.ascontiguousarray(g[:, 0:2]).reshape(-1),
                "absgrad": np.ascontiguousarray(g[:, 2:4]).reshape(-1),
                "grad_conic": np.ascontiguousarray(g[:, 4:7]).reshape(-1),
                "grad_color": np.ascontiguousarray(g[:, 7:10]).reshape(-1),
                "alpha_sum": np.ascontiguousarray(g[:, 10]),
                # fp32 images: each primitive's marks of written records of ranks 0..31
                "record_masks": np.ascontiguousarray(g[:, 11]).view(np.uint32)}

    def debug_records(self) -> dict:
        """First record slot per primitive and the 2D-gradient records of the
        last backward (12 floats per instance slot); with fp32 images also
        each sorted instance's rank among its primitive's instances and the
        bits of the written record slots (tests only)."""
        import torch
        dv = _lib.tgs_debug_view()
        _lib.check(_lib.load().tgs_rasterizer_debug_view(self._h, C.byref(dv)), "debug_view")
        n = self.m_gaussians.size()
        I = int(dv.n_instances)
        dev = self.m_gaussians.means().device
        fs = torch.empty(max(n, 1), dtype=torch.int32, device=dev)
        rec = torch.empty(12 * max(I, 1), dtype=torch.float32, device=dev)
        _lib.copy_device(dv.first_slot, fs.numel() * 4, fs)
        _lib.copy_device(dv.records, rec.numel() * 4, rec)
        out = {"first_slot": fs.cpu().numpy().view(np.uint32)[:n],
               "records": rec.cpu().numpy()[: 12 * I].reshape(-1, 12)}
        if dv.instance_ranks:
            rk = torch.empty(max(I, 1), dtype=torch.int16, device=dev)
            bits = torch.empty(max((I + 31) // 32, 1), dtype=torch.int32, device=dev)
            _lib.copy_device(dv.instance_ranks, rk.numel() * 2, rk)
            _lib.copy_device(dv.record_bits, bits.numel() * 4, bits)
            out["ranks"] = rk.cpu().numpy().view(np.uint16)[:I]
            out["bits"] = bits.cpu().numpy().view(np.uint32)[: (I + 31) // 32]
        return out

    def debug_n_contrib(self, shape) -> "object":
        import torch
        dv = _lib.tgs_debug_view()
        _lib.check(_lib.load().tgs_rasterizer_debug_view(self._h, C.byref(dv)), "debug_view")
        if dv.image_dtype == _lib.TGS_DTYPE_FLOAT16:   # FGS16: 16-bit counts
            t = torch.empty(shape.channel_stride, dtype=torch.int16, device=self.m_gaussians.means().device)
            return _lib.copy_device(dv.n_contrib, t.numel() * 2, t)
        t = torch.empty(shape.channel_stride, dtype=torch.int32, device=self.m_gaussians.means().device)
        return _lib.copy_device(dv.n_contrib, t.numel() * 4, t)

    def get_params(self) -> dict:
        return {"type": "fastgs", **self.m_params}

    def set_params(self, params: dict):
        """enable_pose_opt turns on the pose gradient (FastGSRasterizerParams,
        fastgs.hpp:6-12). The reference's set_params ignores its argument
        (fastgs.cu:398), so there the flag keeps its default (off)."""
        if "enable_pose_opt" in params:
            self.m_params["enable_pose_opt"] = bool(params["enable_pose_opt"])
        if "f16_grad_scaler" in params:
            self.m_params["f16_grad_scaler"] = float(params["f16_grad_scaler"])


def create_rasterizer(rasterizer_type: str) -> RasterizerBase:
    t = rasterizer_type.lower()
    if t == "fastgs":
        return FastGSRasterizer()
    raise RuntimeError(f"Unknown rasterizer type: {rasterizer_type}")
