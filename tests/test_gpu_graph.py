"""A whole training step captured into a HIP graph and replayed: no-sync
forward (reserved instance capacity, look-back epochs advanced on the
device), fused L1 + SSIM in assign mode, sparse backward and masked Adam
with the step count on the device. Each replay is checked against an eager
twin fed the same scene, with eager work and synchronisation between the
replays: parameters, image and loss gradient bit-exact after every step.

The scene keeps every Gaussian inside one tile (small Gaussians near tile
centres), so each has one 2D-gradient record per step and the step is
deterministic: the per-primitive sums of several records follow the order
in which buckets finish, which would make twins drift apart by rounding
whether or not a graph is used."""
import numpy as np
import pytest

from tinygs_amd import scenes

pytestmark = pytest.mark.gpu


def _state(ts):
    import torch
    torch.cuda.synchronize()
    out = {k: v.copy() for k, v in ts.params().items()}
    out["image"] = ts.pred.data.cpu().numpy().copy()
    out["grad_image"] = ts.grad_img.data.cpu().numpy().copy()
    return out


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint16 if a.dtype == np.float16 else np.uint32)


def _tile_centred_scene(k=12, seed=4):
    """k Gaussians per 16x16 tile of a 128x96 view, each projecting within
    3 px of its tile's centre with a footprint of a few pixels."""
    rng = np.random.default_rng(seed)
    W, H, f = 128, 96, 100.0
    w2c = np.eye(4)
    w2c[2, 3] = 3.0
    cam = scenes.Camera(W, H, f, f, W / 2.0, H / 2.0, w2c)
    gw, gh = W // 16, H // 16
    n = gw * gh * k
    tile = np.repeat(np.arange(gw * gh), k)
    px = (tile % gw) * 16 + 8 + rng.uniform(-3, 3, n)
    py = (tile // gw) * 16 + 8 + rng.uniform(-3, 3, n)
    z = rng.uniform(-0.5, 0.5, n)
    depth = z + 3.0
    means = np.stack([(px - W / 2.0) * depth / f, (py - H / 2.0) * depth / f, z], 1).astype(np.float32)
    scales = rng.normal(-4.6, 0.1, (n, 3)).astype(np.float32)
    rots = rng.standard_normal((n, 4)).astype(np.float32)
    opac = rng.normal(0.0, 1.0, n).astype(np.float32)
    sh0 = rng.uniform(0.0, 1.0, (n, 3)).astype(np.float32)
    shr = rng.normal(0.0, 0.05, (n, 15, 3)).astype(np.float32)
    target = rng.random(cam.shape.padded_size).astype(np.float32)
    return scenes.Scene(means, scales, rots, opac, sh0, shr, 3, cam, target, "tile_centred")


@pytest.mark.parametrize("image_dtype", ["float32", "float16"])
def test_captured_step_replays_match_eager_steps(hip, image_dtype):
    import torch
    from tinygs_amd.train import TrainStep
    scene = _tile_centred_scene()
    s = torch.cuda.Stream()
    kw = dict(l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=True, no_sync=True, stream=s,
              image_dtype=image_dtype)
    eager = TrainStep(scene, **kw)
    graphed = TrainStep(scene, **kw)
    print(f"[graph] {image_dtype}: two eager warm-up steps each", flush=True)
    with torch.cuda.stream(s):
        for ts in (eager, graphed):
            ts.step()
            ts.step()
    s.synchronize()
    # the premise: one tile, so one record, per Gaussian
    v, inst, _ = eager.rasterizer.counts()
    assert inst == v, (inst, v)
    a, b = _state(eager), _state(graphed)
    for k in a:
        assert np.array_equal(_bits(a[k]), _bits(b[k])), k
    g = graphed.capture_step()
    s.synchronize()
    for rep in range(4):
        with torch.cuda.stream(s):
            eager.step()
        s.synchronize()
        print(f"[graph] replay {rep}", flush=True)
        g.replay()
        s.synchronize()
        a, b = _state(eager), _state(graphed)
        for k in a:
            bad = _bits(a[k]) != _bits(b[k])
            assert not bad.any(), (rep, k, int(bad.sum()))
    eager.check_status()
    graphed.check_status()
    assert graphed.optimizer.device_steps(s) == 6
    assert eager.optimizer.device_steps(s) == 6
