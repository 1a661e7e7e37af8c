"""tinygs_amd — MI355X-native (gfx950) FastGS training path for tinygs.

The hot path (preprocess, binning, blend forward/backward, preprocess
backward, L1 / fused SSIM, SimpleAdam) runs as hand-written HIP kernels in
libtinygs_amd.so behind the C ABI of include/tinygs_amd.h. This package
mirrors tinygs's plugin interfaces on top of it:

  create_rasterizer("fastgs") -> FastGSRasterizer   (rasterizer.cpp:44-53)
  create_loss("l1" | "fused_ssim")                  (loss.cu:13-27)
  create_optimizer("simple_adam", params, grads)    (optim.cu:86-105)

Importing the package does not load the library; the first rasterizer /
loss / optimizer call does, and raises if it has not been built.
"""
from . import image, scenes  # noqa: F401
from .image import ImageShape  # noqa: F401


def load_library():
    from . import _lib
    return _lib.load()


def __getattr__(name):
    # lazy imports keep `import tinygs_amd` free of torch for CPU-only tooling
    if name in ("FastGSRasterizer", "RasterizerBase", "create_rasterizer"):
        from . import rasterizer
        return getattr(rasterizer, name)
    if name in ("L1Loss", "FusedSSIMLoss", "LossBase", "create_loss"):
        from . import loss
        return getattr(loss, name)
    if name in ("SimpleAdam", "OptimizerBase", "create_optimizer"):
        from . import optim
        return getattr(optim, name)
    if name in ("GPUGaussian3d", "Image", "GPUBatchInput", "GPUBatchOutput", "RasterizeContext", "LossContext",
                "DataType"):
        from . import core
        return getattr(core, name)
    if name in ("TrainStep",):
        from . import train
        return getattr(train, name)
    raise AttributeError(name)
