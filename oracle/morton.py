"""TEST INFRASTRUCTURE — CPU restatement of the Morton order of
Orchestrator::reorder_gaussians (tinygs/src/orchestrator.cu:26-90) and of
its densification-info gather (:1023-1032, 1052-1059).

Only tests/ may import this module; the product (tinygs_amd) never does.

reorder() (orchestrator.cu:26-90):
  min / max of the means per axis (thrust::reduce with fminf / fmaxf, :39-49)
  inv_d = 1 / max(max - min, 1e-8) in float on the host (:52-54)
  t = min(max((p - min) * inv_d, 0), 1); q = (uint)(t * 1023) (:61-68)
  code = morton3D(qx, qy, qz): bit k of qx at bit 3k, of qy at 3k + 1, of qz
  at 3k + 2 (common_device.cuh:170-182)
  stable radix sort of (code, index) over bits 0..29 (:71-89); the sorted
  indices are the new row order.
"""
from __future__ import annotations

import numpy as np

F = np.float32


def interleave_bits(qx: int, qy: int, qz: int) -> int:
    """morton3D by its definition, one bit at a time (10 bits per axis)."""
    code = 0
    for k in range(10):
        code |= ((qx >> k) & 1) << (3 * k)
        code |= ((qy >> k) & 1) << (3 * k + 1)
        code |= ((qz >> k) & 1) << (3 * k + 2)
    return code


def _spread(v: np.ndarray) -> np.ndarray:
    """Vectorised interleave: bit k of v (k < 10) to bit 3k."""
    v = v.astype(np.uint64) & 0x3FF
    out = np.zeros_like(v)
    for k in range(10):
        out |= ((v >> np.uint64(k)) & np.uint64(1)) << np.uint64(3 * k)
    return out


def quantise(means: np.ndarray) -> np.ndarray:
    """(n, 3) uint32 10-bit grid coordinates of the means in their box."""
    m = np.asarray(means, F).reshape(-1, 3)
    lo = np.fmin.reduce(m, axis=0) if len(m) else np.full(3, np.finfo(F).max, F)
    hi = np.fmax.reduce(m, axis=0) if len(m) else np.full(3, -np.finfo(F).max, F)
    ext = (hi - lo).astype(F)
    ext = np.where(ext < F(1e-8), F(1e-8), ext).astype(F)   # std::max(ext, 1e-8f)
    inv = (F(1.0) / ext).astype(F)
    t = np.minimum(np.maximum(((m - lo).astype(F) * inv).astype(F), F(0.0)), F(1.0)).astype(F)
    return (t * F(1023.0)).astype(F).astype(np.uint32)


def codes(means: np.ndarray) -> np.ndarray:
    q = quantise(means)
    c = _spread(q[:, 0]) | (_spread(q[:, 1]) << np.uint64(1)) | (_spread(q[:, 2]) << np.uint64(2))
    return c.astype(np.uint32)


def morton_order(means: np.ndarray) -> np.ndarray:
    """int64 [n]: row i of the reordered arrays is old row order[i]."""
    return np.argsort(codes(means), kind="stable")


def densification_reorder(info: np.ndarray, order: np.ndarray) -> np.ndarray:
    return np.asarray(info)[np.asarray(order)]
