"""The reference's image layout: channel-planar, padded to multiples of 8,
8x8-tiled (tinygs/include/tinygs/common.hpp:366-414,
tinygs/include/tinygs/core/image.hpp:35-85).

Pixel (row y, column x) of channel c lives at
``c * channel_stride + ((y>>3) * tiled_width + (x>>3)) * 64 + (y&7) * 8 + (x&7)``
with ``tiled_width = ceil(W/8)`` and ``channel_stride = ceil(W/8)*ceil(H/8)*64``.
"""
from __future__ import annotations

import dataclasses

import numpy as np


@dataclasses.dataclass(frozen=True)
class ImageShape:
    width: int
    height: int
    channel: int = 3

    @property
    def tiled_width(self) -> int:
        return (self.width + 7) >> 3

    @property
    def tiled_height(self) -> int:
        return (self.height + 7) >> 3

    @property
    def padded_width(self) -> int:
        return self.tiled_width << 3

    @property
    def padded_height(self) -> int:
        return self.tiled_height << 3

    @property
    def channel_stride(self) -> int:
        return self.tiled_width * self.tiled_height * 64

    @property
    def padded_size(self) -> int:
        return self.padded_width * self.padded_height * self.channel

    def size(self) -> int:
        return self.width * self.height * self.channel


def tiled_index(shape: ImageShape) -> np.ndarray:
    """(H, W) array of physical per-channel indices."""
    y = np.arange(shape.height)[:, None]
    x = np.arange(shape.width)[None, :]
    return (((y >> 3) * shape.tiled_width + (x >> 3)) << 6) + ((y & 7) << 3) + (x & 7)


def to_hwc(buf: np.ndarray, shape: ImageShape) -> np.ndarray:
    """Tiled planar buffer -> (H, W, C) array."""
    idx = tiled_index(shape)
    return np.stack([buf[c * shape.channel_stride + idx] for c in range(shape.channel)], axis=-1)


def from_hwc(img: np.ndarray, shape: ImageShape, fill: float = 0.0) -> np.ndarray:
    """(H, W, C) array -> tiled planar buffer (padding set to ``fill``)."""
    out = np.full(shape.padded_size, fill, dtype=img.dtype)
    idx = tiled_index(shape)
    for c in range(shape.channel):
        out[c * shape.channel_stride + idx] = img[..., c]
    return out


def valid_mask(shape: ImageShape) -> np.ndarray:
    """Boolean mask over one tiled plane: True where the pixel is inside W x H."""
    m = np.zeros(shape.channel_stride, dtype=bool)
    m[tiled_index(shape)] = True
    return m
