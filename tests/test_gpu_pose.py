"""Pose-optimisation gradient dL/dw2c (kernels_backward.cuh:256-269 summed as
backward.cu:332-348, handed over as fastgs.cu:373-383) on the GPU against the
CPU restatement (oracle preprocess_backward's grad_w2c, itself pinned by
finite differences in tests/test_oracle.py)."""
import ctypes as C

import numpy as np
import pytest

from tinygs_amd import scenes
from helpers import gpu_render

pytestmark = pytest.mark.gpu


def _oracle_pose(orc, scene, gimg, prec):
    pre, bins, fwd = orc.render(scene, prec)
    g2d = orc.blend_backward(scene, pre, bins, fwd, gimg, prec)
    gw = np.zeros(16, np.float32 if prec == "f" else np.float64)
    orc.preprocess_backward(scene, pre, g2d, prec, grad_w2c=gw)
    return gw.reshape(4, 4).T.astype(np.float64)   # row-major dL/dw2c


def _gpu_pose(scene, gimg, assign=False, sparse=False):
    import torch
    from tinygs_amd.core import Image
    run = gpu_render(scene, with_debug=False)
    r, ctx = run["r"], run["ctx"]
    r.set_params({"enable_pose_opt": True})
    assert r.get_params()["enable_pose_opt"] is True
    ctx.gaussians_grad = run["g"].gradient_like()
    ctx.grad_output.image = Image(ctx.fwd_output.image.shape, "float32",
                                  torch.from_numpy(np.ascontiguousarray(gimg, np.float32)).cuda())
    r.backward(ctx, assign=assign, sparse=sparse)
    return np.array(ctx.grad_input.w2c, np.float64), run


@pytest.mark.parametrize("case", ["config1", "config2_reduced", "sh0"])
def test_pose_gradient_matches_oracle(hip, orc, case):
    if case == "config1":
        s = scenes.config1()
    elif case == "config2_reduced":
        s = scenes.config2(seed=17, n=20000, width=320, height=240)
    else:
        s = scenes.perturb_sh_degree(scenes.config2(seed=18, n=5000, width=160, height=128), 0)
    print(f"[pose] {case} n={s.n}", flush=True)
    gimg = scenes.grad_image(21, s.camera.shape)
    got, _ = _gpu_pose(s, gimg)
    ref_f = _oracle_pose(orc, s, gimg, "f")
    ref_d = _oracle_pose(orc, s, gimg, "d")
    assert np.all(got[3] == 0.0) and np.abs(got).max() > 0
    # the sum cancels over many primitives: the bar is 1e-4 of the largest
    # entry or three times the float oracle's own distance to the double one
    tol = max(1e-4 * np.abs(ref_d).max(), 3 * np.abs(ref_f - ref_d).max())
    assert np.abs(got - ref_f).max() <= tol, (got, ref_f, tol)


def test_pose_gradient_same_in_every_mode_and_zero_when_off(hip):
    s = scenes.config2(seed=19, n=8000, width=192, height=128)
    gimg = scenes.grad_image(22, s.camera.shape)
    a, _ = _gpu_pose(s, gimg)
    b, _ = _gpu_pose(s, gimg, assign=True)
    c, run = _gpu_pose(s, gimg, sparse=True)
    # the pose sum and the per-primitive 2D gradients run in fixed orders: the
    # same bits in every mode
    assert np.array_equal(a, b) and np.array_equal(a, c)
    # off: grad_input.w2c is zero (the reference's memset) and the C getter refuses
    from tinygs_amd import _lib
    r, ctx = run["r"], run["ctx"]
    r.set_params({"enable_pose_opt": False})
    r.forward(ctx)
    r.backward(ctx)
    assert np.array_equal(ctx.grad_input.w2c, np.zeros((4, 4)))
    out = (C.c_float * 16)()
    assert _lib.load().tgs_rasterizer_grad_w2c(r._h, out, None) == 3   # TGS_ERR_STATE


def test_pose_gradient_nothing_visible(hip):
    s = scenes.config1()
    w2c = s.camera.w2c.copy()
    w2c[2, 3] = -50.0   # everything behind the camera
    cam = scenes.Camera(s.camera.width, s.camera.height, s.camera.fx, s.camera.fy, s.camera.cx, s.camera.cy, w2c)
    s2 = scenes.Scene(s.means, s.scales, s.rotations, s.opacities, s.sh0, s.sh_rest, s.sh_degree, cam,
                      np.zeros(cam.shape.padded_size, np.float32))
    got, _ = _gpu_pose(s2, np.ones(cam.shape.padded_size, np.float32))
    assert np.array_equal(got, np.zeros((4, 4)))
