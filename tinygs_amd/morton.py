"""Morton reordering of the Gaussians (Orchestrator::reorder_gaussians,
tinygs/src/orchestrator.cu:26-90, 1038-1061) over the C ABI: the order by
the 30-bit Morton code of the means (tgs_morton_order) and the gather of
the densification info rows (tgs_densification_reorder)."""
from __future__ import annotations

import ctypes as C

from . import _lib
from .core import stream_ptr


def morton_order(means, stream=None):
    """Device int32 tensor [n]: the Gaussians in stable order of the Morton
    code of their means (row i of the reordered arrays is old row idx[i])."""
    import torch
    n = int(means.shape[0])
    if means.dtype != torch.float32 or not means.is_contiguous():
        raise ValueError("means must be a contiguous float32 tensor (n, 3)")
    idx = torch.empty(max(n, 1), dtype=torch.int32, device=means.device)
    _lib.check(_lib.load().tgs_morton_order(C.c_void_p(means.data_ptr()), n, C.c_void_p(idx.data_ptr()),
                                            stream_ptr(stream)), "reorder")
    return idx[:n]


def gather_rows(info, idx, stream=None):
    """densification_update (orchestrator.cu:1023-1032): a new (n, 4) float32
    tensor whose row i is info's row idx[i]."""
    import torch
    out = torch.empty_like(info)
    _lib.check(_lib.load().tgs_densification_reorder(C.c_void_p(info.data_ptr()), C.c_void_p(out.data_ptr()),
                                                     C.c_void_p(idx.data_ptr()), int(info.shape[0]),
                                                     stream_ptr(stream)), "reorder densification info")
    return out
