"""Parity at the benchmarked sizes: config 3 (1M Gaussians, 1920x1080, SH 3
stored as fp16; the headline iteration, run exactly as bench.py runs it:
TrainStep with the fused L1 + SSIM in assign mode, the sparse backward and the
masked SimpleAdam) and config 2 (100k Gaussians, 800x800, fp32 SH) against the
CPU oracle on the same seeded scene.

Bars (config-3 column of the baseline plan):
* binning bit-exact: n_touched, tile bounds, depth order, instance lists,
  tile ranges;
* pixels bit-exact with the oracle on the same fp16-rounded SH (the stated
  per-channel tolerance 2^-10 absolute and 1e-5 relative are asserted too);
* the loss gradient image: L1 exact, SSIM within 1e-5 normwise;
* the rasterizer backward, fed the GPU's loss gradient image, in two parts:
  (a) the blend backward's summed 2D gradients (records summed in the fixed
  order the oracle restates) at the gradient bar of tests/helpers.py, and
  (b) the 3D gradient chain of the preprocess backward given the GPU's own
  2D gradients, exact; then (c) end to end, where the chain amplifies (a)'s
  per-record rounding by a Gaussian's anisotropy (rotations of needle-shaped
  Gaussians: bar 1e-3);
* the gradients of a second backward after the same forward, and of a whole
  second iteration of a twin, are bit-identical to the first's;
* SimpleAdam bit-exact given the GPU's gradients.
The oracle runs on all host cores (its results do not depend on the count).
"""
import os

import numpy as np
import pytest

from tinygs_amd import scenes
from tinygs_amd.image import tiled_index

from helpers import PIXEL_ATOL, PIXEL_RTOL, assert_grads_close, normwise_err

pytestmark = pytest.mark.gpu

# (c) end to end, per group: the common bars (normwise 1e-4, elementwise floor
# 6e-5 max|cpu|), except rotations. The 2D-gradient records are summed in a
# fixed order that the oracle restates (rank order, and above 16 records the
# 16-lane split by 8-slot bytes with an xor butterfly), so what is left
# between GPU and oracle is each record's own rounding: the hardware exp2
# (v_exp_f32) and the order of the pixel sums inside a bucket. The 3D chain
# amplifies that by a Gaussian's anisotropy: for the needle-shaped Gaussians
# of config 3 (log-scales about -5.5, -1.4, -5.2) the rotation gradient
# differs from the oracle's by 4.4e-4 normwise (measured; worst element
# 4.4e-4 max|cpu| on one of 0.13 max|cpu|) while the 2D sums differ by 4e-6
# and the chain itself is bit-exact; config 2's rotations measure 2.2e-5.
# Log-scales measured 3.7e-5 (config 3), within the common bars.
END_TO_END_RTOL = {"means": 1e-4, "scales": 1e-4, "rotations": 1e-3, "opacities": 1e-4, "sh0": 1e-4,
                   "sh_rest": 1e-4}
END_TO_END_ATOL_FRAC = {"rotations": 1e-3}

LR = {"means": 1.6e-4, "scene_scale": 1.0, "opacities": 5e-2, "rotations": 1e-3, "scales": 5e-3, "shs": 5e-3}


def _host_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))


def _run(scene, orc, sparse):
    import torch
    from tinygs_amd.train import TrainStep
    print(f"[fullsize] {scene.name}: N={scene.n} {scene.camera.width}x{scene.camera.height} "
          f"sh_storage={scene.sh_dtype} sparse={sparse}", flush=True)
    ts = TrainStep(scene, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=sparse)
    ts.zero()
    ts.forward()
    torch.cuda.synchronize()
    dv = ts.rasterizer.debug_view()
    dv = {k: (v.cpu().numpy() if hasattr(v, "cpu") else v) for k, v in dv.items()}
    ncontrib = ts.rasterizer.debug_n_contrib(scene.camera.shape).cpu().numpy().view(np.uint32)
    img = ts.image()
    ts.losses_and_grad()
    ts.backward(keep_2d=True)
    torch.cuda.synchronize()
    gimg = ts.grad_image()
    g2d_gpu = ts.rasterizer.debug_grad2d()
    g = ts.grads
    grads = {"means": g.means(), "scales": g.scales(), "rotations": g.rotations(), "opacities": g.opacities(),
             "sh0": g.sh_coefficient_0(), "sh_rest": g.sh_coefficients_rest()}
    grads = {k: v.cpu().numpy().reshape(-1) for k, v in grads.items()}
    # the same backward again, and a whole second iteration (forward, loss,
    # backward) of a twin: bit-identical gradients (a fixed summation order)
    ts.backward()
    torch.cuda.synchronize()
    for k, t in zip(grads, g.tensors()):
        assert np.array_equal(t.detach().cpu().numpy().reshape(-1).view(np.uint32), grads[k].view(np.uint32)), k
    twin = TrainStep(scene, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=sparse)
    twin.zero()
    twin.forward()
    twin.losses_and_grad()
    twin.backward()
    torch.cuda.synchronize()
    # (both start from zeroed gradient arrays, so the rows a sparse backward
    # leaves unwritten agree too)
    for k, t in zip(grads, twin.grads.tensors()):
        got = t.detach().cpu().numpy().reshape(-1)
        assert np.array_equal(got.view(np.uint32), grads[k].view(np.uint32)), ("twin", k)
    del twin
    ts.optimize()
    torch.cuda.synchronize()
    theta = ts.params()
    print("[fullsize] GPU iteration done; CPU oracle on "
          f"{_host_threads()} threads", flush=True)

    orc.set_threads(_host_threads())
    pre, bins, fwd = orc.render(scene, "f")
    n = scene.n
    vis = pre["n_touched"] > 0
    # binning: bit-exact
    assert np.array_equal(dv["n_touched"].view(np.uint32), pre["n_touched"])
    b = dv["bounds"].view(np.uint32).reshape(n, 2)
    ob = pre["bounds"].reshape(n, 4).astype(np.uint32)
    assert np.array_equal(b[vis, 0] & 0xffff, ob[vis, 0]) and np.array_equal(b[vis, 0] >> 16, ob[vis, 1])
    assert np.array_equal(b[vis, 1] & 0xffff, ob[vis, 2]) and np.array_equal(b[vis, 1] >> 16, ob[vis, 3])
    assert dv["n_visible"] == bins["n_visible"] and dv["n_instances"] == bins["n_instances"]
    assert np.array_equal(dv["depth_sorted_prims"].view(np.uint32), bins["sorted_prims"])
    assert np.array_equal(dv["instance_tiles"].view(np.uint32), bins["inst_tile"])
    assert np.array_equal(dv["instance_prims"].view(np.uint32), bins["inst_prim"])
    assert np.array_equal(dv["tile_ranges"].view(np.uint32), bins["ranges"])
    print(f"[fullsize] binning bit-exact: V={bins['n_visible']} I={bins['n_instances']}", flush=True)
    # pixels
    ref_img = fwd["image"].astype(np.float32)
    err = np.abs(img - ref_img)
    assert err.max() <= 2.0 ** -10
    assert np.all(err <= PIXEL_RTOL * np.abs(ref_img) + PIXEL_ATOL), err.max()
    assert np.array_equal(img.view(np.uint32), ref_img.view(np.uint32))
    assert np.array_equal(ncontrib, fwd["n_contrib"])
    assert np.array_equal(dv["tile_max"].view(np.uint32), fwd["tile_max"])
    # loss gradient image (L1 + SSIM) over the valid pixels
    shape = scene.camera.shape
    loss = np.zeros(shape.padded_size, np.float32)
    ref_gimg = np.zeros(shape.padded_size, np.float32)
    orc.l1(fwd["image"], scene.target, shape, np.float32(0.8), loss, ref_gimg)
    orc.ssim(fwd["image"], scene.target, shape, np.float32(0.2), loss, ref_gimg)
    idx = np.concatenate([c * shape.channel_stride + tiled_index(shape).reshape(-1) for c in range(3)])
    e_gimg = normwise_err(gimg[idx], ref_gimg[idx])
    print(f"[fullsize] loss gradient image normwise {e_gimg:.2e}", flush=True)
    assert e_gimg < 1e-5
    # (a) the blend backward on the GPU's loss gradient image: the summed 2D
    # gradients (the quantities that summation order touches)
    g2d = orc.blend_backward(scene, pre, bins, fwd, gimg, "f")
    one_minus_o = np.float32(1) - pre["conic_opacity"].reshape(n, 4)[:, 3].astype(np.float32)
    g2d_gpu["grad_opacity"] = (g2d_gpu["alpha_sum"] * one_minus_o).astype(np.float32)
    print("[fullsize] 2D gradients (blend backward):", flush=True)
    assert_grads_close({k: g2d_gpu[k] for k in ("grad_mean2d", "grad_conic", "grad_color", "grad_opacity")}, g2d)
    # (b) the gradient chain (preprocess backward) on the GPU's own 2D gradients
    g2d_gpu["absgrad"] = np.zeros_like(g2d_gpu["absgrad"])
    chain = orc.preprocess_backward(scene, pre, g2d_gpu, "f")
    # the kernel and the oracle evaluate the same chain in the same operation
    # order: equal values (a row that no bucket reached keeps the sparse
    # backward's +0 where the oracle's chain of zeros may give -0)
    for k in grads:
        c = chain[k].astype(np.float32)
        bad = grads[k] != c
        assert not bad.any(), (k, int(bad.sum()), grads[k][bad][:5], c[bad][:5])
    print("[fullsize] gradient chain on the GPU's 2D gradients: equal values", flush=True)
    # (c) end to end
    ref = orc.preprocess_backward(scene, pre, g2d, "f")
    print("[fullsize] end to end:", flush=True)
    assert_grads_close(grads, ref, rtol=END_TO_END_RTOL, atol_frac=END_TO_END_ATOL_FRAC)
    # SimpleAdam on the GPU's gradients: bit-exact
    th0 = orc.params(scene, "f")
    m1 = {k: np.zeros_like(v) for k, v in th0.items()}
    m2 = {k: np.zeros_like(v) for k, v in th0.items()}
    orc.adam_step(th0, grads, m1, m2, LR, 1, grad_scale=1.0, eps=1e-15, sh_half=scene.sh_dtype == "float16")
    for k in th0:
        assert np.array_equal(theta[k].view(np.uint32), th0[k].view(np.uint32)), k


def test_config3_full_size_iteration(hip, orc):
    _run(scenes.config3(), orc, sparse=True)


def test_config2_full_size_iteration(hip, orc):
    _run(scenes.config2(), orc, sparse=True)
