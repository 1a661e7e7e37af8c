"""The C++ class surface (include/tinygs_amd/tinygs.hpp) end to end: a C++
program runs one Orchestrator::train_step-ordered iteration through
create_rasterizer / create_loss / create_optimizer, and its outputs are checked
against the CPU oracle with the same tolerances as the Python-side tests.

The float16 case is the training data type of four of the reference's six
shipped configs (configs/default.json:99): the image's data type selects the
fp16-image rasterizer (fastgs.cu:143-188, 273-274) and the fp16 losses
(l1.cu:123-146, fused_ssim.cu:863-906). Its pixels are bit-exact against the
oracle's half restatement (orc.h_render), the loss gradient image within one
half ulp of the oracle's fp16 L1 then SSIM, the 2D sums (rebuilt from the
program's gradient image by orc.h_blend_backward) feed the oracle's chain,
which equals the program's 3D gradients (the opacity-logit sums, kept in
double in completion order, within 2 float ulps), and Adam is bit-exact on
the program's own gradients."""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from tinygs_amd import scenes
from tinygs_amd.image import tiled_index

from helpers import PIXEL_ATOL, PIXEL_RTOL, assert_grads_close, normwise_err

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "_build", "train_step")
GROUPS = [("means", 3), ("scales", 3), ("rotations", 4), ("opacities", 1), ("sh0", 3), ("sh_rest", 45)]


def _binary():
    if not os.path.exists(BIN):
        from tinygs_amd import build as hb
        hb.build_cpp_test()
    return BIN


def _write_input(path, s, l1_w, ssim_w, eps, shs_lr, image_half=False):
    cam = s.camera
    K = np.array([[cam.fx, 0.0, cam.cx], [0.0, cam.fy, cam.cy], [0.0, 0.0, 1.0]], np.float32)
    with open(path, "wb") as f:
        f.write(np.int64(s.n).tobytes())
        f.write(np.array([s.sh_degree, 1 if s.sh_dtype == "float16" else 0, 1 if image_half else 0],
                         np.int32).tobytes())
        f.write(np.array([cam.width, cam.height], np.uint32).tobytes())
        f.write(np.array([cam.near, cam.far], np.float32).tobytes())
        f.write(K.T.reshape(-1).tobytes())                                   # glm column-major
        f.write(np.asarray(cam.w2c, np.float32).T.reshape(-1).tobytes())
        f.write(np.array([l1_w, ssim_w, 1.0, eps, shs_lr], np.float32).tobytes())
        for name, _ in GROUPS:
            f.write(np.ascontiguousarray(getattr(s, name), np.float32).reshape(-1).tobytes())
        f.write(np.ascontiguousarray(s.target, np.float16 if image_half else np.float32).tobytes())


def _read_output(path, s, image_half=False):
    n = s.n
    npad = s.camera.shape.padded_size
    buf = open(path, "rb").read()
    off = 0

    def take(count, dtype):
        nonlocal off
        a = np.frombuffer(buf, dtype=dtype, count=count, offset=off)
        off += a.nbytes
        return a

    idt = np.uint16 if image_half else np.float32
    out = {"image": take(npad, idt), "grad_image": take(npad, idt)}
    out["grads"] = {k: take(m * n, np.float32) for k, m in GROUPS}
    out["params"] = {k: take(m * n, np.float32) for k, m in GROUPS}
    out["counts"] = take(3, np.int64)
    assert off == len(buf)
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["config1_l1", "config3_fp16_sh"])
def test_cpp_train_step(hip, orc, tmp_path, case):
    if case == "config1_l1":
        s, l1_w, ssim_w, shs_lr = scenes.config1(), 1.0, 0.0, 2.5e-3
    else:
        s, l1_w, ssim_w, shs_lr = scenes.config3(seed=21, n=20000, width=320, height=180), 0.8, 0.2, 5e-3
    eps = 1e-15
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    _write_input(src, s, l1_w, ssim_w, eps, shs_lr)
    print(f"cpp train_step case={case} n={s.n}", flush=True)
    r = subprocess.run([_binary(), str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    got = _read_output(dst, s)

    lr = {"means": 1.6e-4, "scene_scale": 1.0, "opacities": 5e-2, "rotations": 1e-3, "scales": 5e-3, "shs": shs_lr}
    ref = orc.run_iteration(s, l1_w, ssim_w, lr=lr, eps=eps)
    assert np.allclose(got["image"], ref["fwd"]["image"], rtol=PIXEL_RTOL, atol=PIXEL_ATOL)
    shape = s.camera.shape
    idx = np.concatenate([c * shape.channel_stride + tiled_index(shape).reshape(-1) for c in range(3)])
    assert normwise_err(got["grad_image"][idx], ref["grad_image"][idx]) < 1e-5
    assert got["counts"][1] == len(ref["bins"]["inst_prim"])
    assert_grads_close(got["grads"], ref["grads"])
    # Adam applied to the program's own gradients: bit-exact
    theta = orc.params(s, "f")
    m1 = {k: np.zeros_like(v) for k, v in theta.items()}
    m2 = {k: np.zeros_like(v) for k, v in theta.items()}
    orc.adam_step(theta, got["grads"], m1, m2, lr, 1, grad_scale=1.0, eps=eps, sh_half=s.sh_dtype == "float16")
    for k in theta:
        assert np.array_equal(got["params"][k].view(np.uint32), theta[k].view(np.uint32)), k


def _run(tmp_path, s, l1_w, ssim_w, eps, shs_lr, image_half):
    src, dst = tmp_path / "in.bin", tmp_path / "out.bin"
    _write_input(src, s, l1_w, ssim_w, eps, shs_lr, image_half)
    r = subprocess.run([_binary(), str(src), str(dst)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    return _read_output(dst, s, image_half)


@pytest.mark.gpu
@pytest.mark.parametrize("case", ["config1_l1", "config2_l1_ssim"])
def test_cpp_train_step_float16_images(hip, orc, tmp_path, case):
    if case == "config1_l1":
        s, l1_w, ssim_w = scenes.config1(), 1.0, 0.0
    else:
        s, l1_w, ssim_w = scenes.config2(seed=11, n=6000, width=246, height=182), 0.8, 0.2
    eps, shs_lr = 1e-15, 5e-3
    print(f"cpp train_step float16 images case={case} n={s.n}", flush=True)
    got = _run(tmp_path, s, l1_w, ssim_w, eps, shs_lr, True)
    shape = s.camera.shape
    pre, bins, fwd = orc.h_render(s)
    assert np.array_equal(got["image"], fwd["image"])
    assert got["counts"][1] == bins["n_instances"]
    # loss gradient: L1 then SSIM on the half image and target, each
    # accumulation rounded to half (l1.cu:67-107, fused_ssim.cu:445-693)
    f = lambda a: a.view(np.float16).astype(np.float32)
    tgt = np.ascontiguousarray(s.target, np.float16)
    loss = np.zeros(shape.padded_size, np.float32)
    g = np.zeros(shape.padded_size, np.float32)
    if l1_w:
        loss, g = orc.l1(f(got["image"]), tgt.astype(np.float32), shape, np.float32(l1_w), loss, g)
        loss, g = (loss.astype(np.float16).astype(np.float32), g.astype(np.float16).astype(np.float32))
    if ssim_w:
        loss, g = orc.ssim(f(got["image"]), tgt.astype(np.float32), shape, np.float32(ssim_w), loss.copy(),
                           g.copy())
    idx = np.concatenate([c * shape.channel_stride + tiled_index(shape).reshape(-1) for c in range(3)])
    r16 = g[idx].astype(np.float16)
    gg = f(got["grad_image"])[idx].astype(np.float64)
    ulp = np.abs(np.spacing(r16).astype(np.float64))
    assert np.all(np.abs(gg - r16.astype(np.float64)) <= ulp), np.abs(gg - r16.astype(np.float64)).max()
    # the oracle's 2D sums of the program's gradient image through the oracle's chain
    ob = orc.h_blend_backward(s, pre, bins, fwd, got["grad_image"])
    g_in = dict(ob["g2d"])
    g_in["absgrad"] = np.zeros_like(g_in["absgrad"])
    chain = orc.h_preprocess_backward(s, pre, g_in)
    for key, _ in GROUPS:
        c = chain[key].astype(np.float32)
        if key == "opacities":
            assert np.all(np.abs(got["grads"][key] - c) <= 2.4e-7 * np.abs(c)), key
        else:
            bad = got["grads"][key] != c
            assert not bad.any(), (key, int(bad.sum()), got["grads"][key][bad][:5], c[bad][:5])
    lr = {"means": 1.6e-4, "scene_scale": 1.0, "opacities": 5e-2, "rotations": 1e-3, "scales": 5e-3, "shs": shs_lr}
    theta = orc.params(s, "f")
    m1 = {k: np.zeros_like(v) for k, v in theta.items()}
    m2 = {k: np.zeros_like(v) for k, v in theta.items()}
    orc.adam_step(theta, got["grads"], m1, m2, lr, 1, grad_scale=1.0, eps=eps, sh_half=s.sh_dtype == "float16")
    for k in theta:
        assert np.array_equal(got["params"][k].view(np.uint32), theta[k].view(np.uint32)), k
