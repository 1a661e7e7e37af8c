"""Forward entry checks and the forward that does not wait for its counts.

* fp32 images: a tile grid beyond the 65,536 tiles of the reference's 16-bit
  tile keys (kernels_forward.cuh:477,521; forward.cu:214) is refused before
  anything is launched; the largest allowed grid renders like the oracle.
  (fp16 images sort 32-bit tile keys: tests/test_gpu_fgs16.py renders a
  78,250-tile grid.)
* TGS_FORWARD_NO_SYNC: same binning, pixels and gradients as the forward that
  waits, and a forward that outgrows its reserved instance capacity is
  reported by tgs_rasterizer_status without touching memory out of bounds.
"""
import numpy as np
import pytest

from tinygs_amd import scenes

from helpers import assert_grads_close, gpu_backward, gpu_render
from test_gpu_parity import _check_forward, _grad_image

pytestmark = pytest.mark.gpu


def _with_camera(s, width, height, f):
    cam = scenes.Camera(width, height, f, f, width / 2.0, height / 2.0, s.camera.w2c)
    return scenes.Scene(s.means, s.scales, s.rotations, s.opacities, s.sh0, s.sh_rest, s.sh_degree, cam,
                        np.zeros(cam.shape.padded_size, np.float32))


def test_fp32_tile_grid_beyond_16_bit_keys_refused_before_launch(hip):
    import torch
    from tinygs_amd.core import GPUBatchInput, GPUGaussian3d, Image, RasterizeContext
    from tinygs_amd.rasterizer import create_rasterizer
    s = _with_camera(scenes.config1(seed=3, n=64), 5000, 4000, 4000.0)   # 313 x 250 = 78,250 tiles
    print("[tiles] 5000x4000 camera", flush=True)
    r = create_rasterizer("fastgs")
    r.set_gaussians(GPUGaussian3d.from_scene(s))
    ctx = RasterizeContext()
    ctx.fwd_input = GPUBatchInput.from_camera(s.camera)
    ctx.fwd_output.image = Image.empty(s.camera.shape)
    ctx.fwd_output.image.data.fill_(np.nan)
    torch.cuda.synchronize()
    with pytest.raises(RuntimeError, match="65,536 tiles"):
        r.forward(ctx)
    with pytest.raises(RuntimeError, match="65,536 tiles"):
        r.forward(ctx, no_sync=True)
    torch.cuda.synchronize()
    assert bool(torch.isnan(ctx.fwd_output.image.data).all())   # nothing was written
    with pytest.raises(RuntimeError, match="no forward yet"):
        r.counts()


def test_largest_tile_grid_matches_oracle(hip, orc):
    # 4096 x 4096: exactly 65,536 tiles, the tile keys need all 16 bits (two passes)
    s = _with_camera(scenes.config1(seed=5, n=2000), 4096, 4096, 2048.0)
    print("[tiles] 4096x4096 camera", flush=True)
    run, (pre, bins, fwd) = _check_forward(s, orc)
    assert run["dv"]["n_tiles"] == 65536 and bins["n_instances"] > 100_000
    assert run["dv"]["instance_tiles"].view(np.uint32).max() >= 32768   # the top key bit is sorted


def _no_sync_render(s, capacity):
    import torch
    from tinygs_amd.core import GPUBatchInput, GPUGaussian3d, Image, RasterizeContext
    from tinygs_amd.rasterizer import create_rasterizer
    g = GPUGaussian3d.from_scene(s)
    r = create_rasterizer("fastgs")
    r.set_gaussians(g)
    ctx = RasterizeContext()
    ctx.fwd_input = GPUBatchInput.from_camera(s.camera)
    ctx.fwd_output.image = Image.empty(s.camera.shape)
    ctx.fwd_output.image.data.fill_(np.nan)
    gx, gy = s.camera.grid
    r.reserve(capacity, gx * gy)
    r.forward(ctx, no_sync=True)
    return {"r": r, "g": g, "ctx": ctx}


def test_no_sync_forward_matches_waiting_forward(hip, orc):
    import torch
    s = scenes.config2(seed=11, n=20000, width=320, height=240)
    print("[no-sync] config2 20k 320x240", flush=True)
    ref_run, (pre, bins, fwd) = _check_forward(s, orc)
    I = bins["n_instances"]
    run = _no_sync_render(s, I + 777)
    assert run["r"].status() == 0
    torch.cuda.synchronize()
    dv = run["r"].debug_view()
    assert dv["n_instances"] == I and dv["n_visible"] == bins["n_visible"]
    for k in ("instance_tiles", "instance_prims", "tile_ranges", "depth_sorted_prims", "tile_max"):
        assert np.array_equal(dv[k].cpu().numpy(), ref_run["dv"][k]), k
    img = run["ctx"].fwd_output.image.data.cpu().numpy()
    assert np.array_equal(img.view(np.uint32), fwd["image"].astype(np.float32).view(np.uint32))
    # the backward after a no-sync forward
    gimg = _grad_image(s)
    g2d = orc.blend_backward(s, pre, bins, fwd, gimg, "f")
    ref = orc.preprocess_backward(s, pre, g2d, "f")
    run["image"] = img
    got = gpu_backward(run, gimg)
    assert_grads_close(got, ref)


def test_no_sync_capacity_overflow_reported(hip, orc):
    import torch
    from tinygs_amd import _lib
    s = scenes.config2(seed=12, n=20000, width=320, height=240)
    pre, bins, fwd = orc.render(s, "f")
    I = bins["n_instances"]
    print(f"[no-sync] capacity {I // 2} of {I}", flush=True)
    run = _no_sync_render(s, I // 2)
    r = run["r"]
    assert r.status(clear_capacity_flag=True) == _lib.TGS_ERR_CAPACITY
    assert r.counts()[1] == I          # the true count is still reported
    assert r.status() == 0             # the flag was cleared
    # the debug view covers only the instances the buffers hold
    dv = r.debug_view()
    assert dv["n_instances"] == I // 2 and dv["instance_prims"].numel() == I // 2
    assert r.debug_records()["records"].shape[0] <= I // 2
    # enough capacity: a no-sync forward on the same handle renders exactly
    r.reserve(I, s.camera.grid[0] * s.camera.grid[1])
    r.forward(run["ctx"], no_sync=True)
    assert r.status() == 0
    torch.cuda.synchronize()
    img = run["ctx"].fwd_output.image.data.cpu().numpy()
    assert np.array_equal(img.view(np.uint32), fwd["image"].astype(np.float32).view(np.uint32))


def test_no_sync_train_step_matches_waiting(hip):
    """Repeated TrainSteps whose forwards do not wait for the host against
    ones that do: images, gradients and parameters bit-identical after every
    step (the gradient sums run in a fixed order, so the two runs cannot
    drift apart)."""
    import torch
    from tinygs_amd.train import TrainStep
    s = scenes.config3(seed=24, n=30000, width=320, height=192)
    a = TrainStep(s, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=False)
    b = TrainStep(s, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=False, no_sync=True)
    for step in range(4):
        for ts in (a, b):
            ts.step()
        torch.cuda.synchronize()
        assert np.array_equal(a.image().view(np.uint32), b.image().view(np.uint32)), step
        for ga, gb in zip(a.grads.tensors(), b.grads.tensors()):
            assert np.array_equal(ga.cpu().numpy().view(np.uint32), gb.cpu().numpy().view(np.uint32)), step
        pa, pb = a.params(), b.params()
        for k in pa:
            assert np.array_equal(pa[k].view(np.uint32), pb[k].view(np.uint32)), (step, k)
    b.check_status()
    assert b.rasterizer.counts()[1] == a.rasterizer.counts()[1]


def test_reserve_that_grows_drops_forward_state(hip):
    """Growing the instance buffers loses the last forward's lists and
    checkpoints, so a backward after such a reserve is refused."""
    import torch
    from tinygs_amd.core import Image
    s = scenes.config1(seed=7)
    run = gpu_render(s, with_debug=False)
    I = run["r"].counts()[1]
    run["r"].reserve(8 * I + 100000, 16)
    run["ctx"].gaussians_grad = run["g"].gradient_like()
    run["ctx"].grad_output.image = Image(s.camera.shape, "float32",
                                         torch.from_numpy(_grad_image(s)).cuda())
    with pytest.raises(RuntimeError, match="without a preceding forward"):
        run["r"].backward(run["ctx"])


def test_no_sync_train_step_capacity_check_raises_and_regrows(hip):
    """A TrainStep whose scene grows past the reserved instance capacity
    (larger Gaussians, as after densification) raises at its next capacity
    check, and the step after that runs with room for the new count."""
    import torch
    from tinygs_amd.train import TrainStep
    s = scenes.config2(seed=13, n=8000, width=256, height=192)
    ts = TrainStep(s, l1_weight=0.8, ssim_weight=0.2, eps=1e-15, no_sync=True, check_interval=1)
    print("[no-sync] capacity check: two steps", flush=True)
    ts.step()          # waits once: sizes and reserves the capacity
    ts.step()          # no-sync from here on
    ts.check_status()
    before = ts._capacity[0]
    with torch.no_grad():
        ts.gaussians.scales().add_(1.5)   # every Gaussian 4.5x larger: several times the instances
    ts.step()          # checks the earlier steps (fine), then overflows
    with pytest.raises(RuntimeError, match="outgrew its instance capacity"):
        ts.step()
    assert ts._capacity[0] > before
    ts.step()          # reserves the new capacity first
    ts.check_status()


def test_binning_scan_give_up_reported_by_its_forward(hip, orc):
    """A look-back wait of the binning that gives up is reported by the call
    that queued it. The give-up is forced from the host (spin bound 0: each
    look-back with a predecessor stops at once and sets the flag, so every
    kernel still runs to its end; the emission and the blend then skip their
    work). The waiting forward fails and the backward after it is refused; a
    no-sync forward's failure is reported once by status(); with the bound
    restored the same handle renders like the oracle."""
    import torch
    from tinygs_amd import _lib
    from tinygs_amd.core import GPUBatchInput, GPUGaussian3d, Image, RasterizeContext
    from tinygs_amd.rasterizer import create_rasterizer
    s = scenes.config2(seed=14, n=50000, width=320, height=240)   # several scan workgroups per pass
    pre, bins, fwd = orc.render(s, "f")
    g = GPUGaussian3d.from_scene(s)
    r = create_rasterizer("fastgs")
    r.set_gaussians(g)
    ctx = RasterizeContext()
    ctx.fwd_input = GPUBatchInput.from_camera(s.camera)
    ctx.fwd_output.image = Image.empty(s.camera.shape)
    ctx.gaussians_grad = g.gradient_like()
    ctx.grad_output.image = Image(s.camera.shape, "float32", torch.from_numpy(_grad_image(s)).cuda())
    L = _lib.load()
    torch.cuda.synchronize()
    print("[give-up] waiting forward with the look-back bound at 0", flush=True)
    _lib.check(L.tgs_selftest_lookback_spins(0), "spins")
    try:
        with pytest.raises(RuntimeError, match="binning failed on the device"):
            r.forward(ctx)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="without a preceding forward"):
            r.backward(ctx)
        print("[give-up] no-sync forward with the look-back bound at 0", flush=True)
        r.reserve(bins["n_instances"] + 1000, s.camera.grid[0] * s.camera.grid[1])
        r.forward(ctx, no_sync=True)
        with pytest.raises(RuntimeError, match="binning failed on the device"):
            r.status()
        assert r.status() == 0   # reported once
    finally:
        torch.cuda.synchronize()
        _lib.check(L.tgs_selftest_lookback_spins(0xFFFFFFFF), "spins")
    print("[give-up] bound restored", flush=True)
    r.forward(ctx)
    torch.cuda.synchronize()
    img = ctx.fwd_output.image.data.cpu().numpy()
    assert np.array_equal(img.view(np.uint32), fwd["image"].astype(np.float32).view(np.uint32))
    r.backward(ctx)
