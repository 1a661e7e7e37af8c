"""Shared helpers for the parity tests: run a scene through the HIP path (via
the C ABI) and through the CPU oracle, and compare with stated tolerances."""
from __future__ import annotations

import numpy as np

# Tolerances (north star: binning bit-exact, fp32 pixels within 1e-5 relative,
# gradients within 1e-4 relative).
PIXEL_RTOL = 1e-5
PIXEL_ATOL = 1e-7
GRAD_NORMWISE_RTOL = 1e-4      # max |gpu - cpu| <= 1e-4 * max |cpu| per parameter group


def gpu_render(scene, with_debug=True, densif=False):
    import torch
    from tinygs_amd.core import GPUGaussian3d, GPUBatchInput, Image, RasterizeContext
    from tinygs_amd.rasterizer import create_rasterizer
    g = GPUGaussian3d.from_scene(scene)
    r = create_rasterizer("fastgs")
    r.set_gaussians(g)
    ctx = RasterizeContext()
    ctx.fwd_input = GPUBatchInput.from_camera(scene.camera)
    ctx.fwd_output.image = Image.empty(scene.camera.shape)
    ctx.fwd_output.image.data.fill_(np.nan)   # padding must be written by the forward
    if densif:
        ctx.densification_info = torch.zeros((scene.n, 4), dtype=torch.float32, device="cuda")
    r.forward(ctx)
    torch.cuda.synchronize()
    out = {"r": r, "g": g, "ctx": ctx, "image": ctx.fwd_output.image.data.cpu().numpy()}
    if with_debug:
        dv = r.debug_view()
        out["dv"] = {k: (v.cpu().numpy() if hasattr(v, "cpu") else v) for k, v in dv.items()}
        out["n_contrib"] = r.debug_n_contrib(scene.camera.shape).cpu().numpy().view(np.uint32)
    return out


def gpu_backward(run, grad_image_np):
    import torch
    from tinygs_amd.core import Image
    ctx = run["ctx"]
    grads = run["g"].gradient_like()
    ctx.gaussians_grad = grads
    ctx.grad_output.image = Image(ctx.fwd_output.image.shape, "float32",
                                  torch.from_numpy(np.ascontiguousarray(grad_image_np, np.float32)).cuda())
    run["r"].backward(ctx)
    torch.cuda.synchronize()
    return {
        "means": grads.means().cpu().numpy().reshape(-1),
        "scales": grads.scales().cpu().numpy().reshape(-1),
        "rotations": grads.rotations().cpu().numpy().reshape(-1),
        "opacities": grads.opacities().cpu().numpy().reshape(-1),
        "sh0": grads.sh_coefficient_0().cpu().numpy().reshape(-1),
        "sh_rest": grads.sh_coefficients_rest().cpu().numpy().reshape(-1),
    }


def normwise_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.abs(b).max() if b.size else 0.0
    if scale == 0.0:
        return float(np.abs(a).max()) if a.size else 0.0
    return float(np.abs(a - b).max() / scale)


def assert_grads_close(gpu, ref, rtol=GRAD_NORMWISE_RTOL, groups=None):
    worst = {}
    for k in groups or ref:
        e = normwise_err(gpu[k], ref[k])
        worst[k] = e
        assert e <= rtol, (k, e, worst)
    return worst
