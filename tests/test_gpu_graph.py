"""A whole training step captured into a HIP graph and replayed: no-sync
forward (reserved instance capacity, look-back epochs advanced on the
device), fused L1 + SSIM in assign mode, sparse backward and masked Adam
with the step count on the device. Each replay is checked against an eager
twin fed the same scene, with eager work and synchronisation between the
replays: parameters, image and loss gradient bit-exact after every step.

fp32 images run a general scene: each primitive's 2D-gradient records are
summed in a fixed order, so a step repeats bit for bit. The fp16-image
rasterizer sums its half records exactly but adds the opacity-logit parts in
double in the order the buckets finish, so its case keeps every Gaussian
inside one tile (one record each), which makes its step deterministic too."""
import numpy as np
import pytest

from helpers import tile_centred_scene

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


@pytest.mark.parametrize("image_dtype,overlap", [("float32", False), ("float16", False), ("float32", True)])
def test_captured_step_replays_match_eager_steps(hip, image_dtype, overlap):
    """overlap: Adam's rows without gradient on a second stream (a fork and a
    join inside the captured step)."""
    import torch
    from tinygs_amd import scenes
    from tinygs_amd.train import TrainStep
    one_tile = image_dtype == "float16"
    scene = tile_centred_scene() if one_tile else scenes.config3(seed=41, n=20000, width=256, height=160)
    s = torch.cuda.Stream()
    kw = dict(l1_weight=0.8, ssim_weight=0.2, eps=1e-15, shs_lr=5e-3, sparse_grads=True, no_sync=True, stream=s,
              image_dtype=image_dtype, overlap_adam=overlap)
    eager = TrainStep(scene, **kw)
    graphed = TrainStep(scene, **kw)
    print(f"[graph] {image_dtype} overlap={overlap}: two eager warm-up steps each", flush=True)
    with torch.cuda.stream(s):
        for ts in (eager, graphed):
            ts.step()
            ts.step()
    s.synchronize()
    v, inst, _ = eager.rasterizer.counts()
    if one_tile:   # the premise: one tile, so one record, per Gaussian
        assert inst == v, (inst, v)
    else:
        assert inst > v, (inst, v)   # primitives over several tiles: several records each
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
    # the replays advanced only the device count: the host count follows it,
    # and a host-counted step after them continues at step 7 in both twins
    assert graphed.optimizer.global_steps() == 6 and eager.optimizer.global_steps() == 6
    with torch.cuda.stream(s):
        for ts in (eager, graphed):
            ts.zero()
            ts.forward()
            ts.losses_and_grad()
            ts.backward()
            ts.optimizer.step(1.0 / ts.grad_scaler, s, row_mask=ts.rasterizer.grad_row_mask(), device_step=False)
    s.synchronize()
    a, b = _state(eager), _state(graphed)
    for k in a:
        assert np.array_equal(_bits(a[k]), _bits(b[k])), ("host step", k)
    assert graphed.optimizer.global_steps() == 7 and eager.optimizer.global_steps() == 7


def test_device_step_adam_matches_host_step(hip):
    """Device-counted Adam steps (each launch reads the corrections of its step,
    computed one step ahead on the device, and its last workgroup to finish
    advances the count) equal host-counted steps bit for bit: over a grid of
    more than 64 workgroups, across a change of the betas, and for a step in
    two parts (rows without a gradient, then the others at the same count)."""
    import torch
    from tinygs_amd.core import GPUGaussian3d
    from tinygs_amd.optim import SimpleAdam
    n = 40_000
    rng = np.random.default_rng(11)
    fields = ("means", "scales", "rotations", "opacities", "sh_coefficient_0", "sh_coefficients_rest")

    def twin():
        g, gr = GPUGaussian3d(n, device="cuda"), GPUGaussian3d(n, device="cuda")
        return g, gr

    (ga, gra), (gb, grb) = twin(), twin()
    for f in fields:
        v = torch.from_numpy(rng.standard_normal(getattr(ga, f)().numel()).astype(np.float32)).cuda()
        getattr(ga, f)().copy_(v.view_as(getattr(ga, f)()))
        getattr(gb, f)().copy_(v.view_as(getattr(gb, f)()))
    A, B = SimpleAdam(ga, gra), SimpleAdam(gb, grb)
    s = torch.cuda.current_stream()

    def new_grads():
        for f in fields:
            v = torch.from_numpy((1e-2 * rng.standard_normal(getattr(gra, f)().numel())).astype(np.float32)).cuda()
            getattr(gra, f)().copy_(v.view_as(getattr(gra, f)()))
            getattr(grb, f)().copy_(v.view_as(getattr(grb, f)()))

    def same(tag):
        torch.cuda.synchronize()
        for f in fields:
            a, b = getattr(ga, f)().cpu().numpy(), getattr(gb, f)().cpu().numpy()
            assert np.array_equal(_bits(a), _bits(b)), (tag, f)

    for step in range(6):
        new_grads()
        if step == 3:
            for o in (A, B):
                o.set_params({"beta1": 0.8, "beta2": 0.99})
        A.step(1.0, s)
        B.step(1.0, s, device_step=True)
        same(step)
    new_grads()
    mask = torch.from_numpy((rng.random(n) < 0.1).astype(np.uint8)).cuda()
    A.step(1.0, s, row_mask=mask.data_ptr())
    B.step(1.0, s, row_mask=mask.data_ptr(), device_step=True, rows="unmarked")
    B.step(1.0, s, row_mask=mask.data_ptr(), device_step=True, rows="marked", same_step=True)
    same("two parts")
    assert B.device_steps(s) == 7 and A.global_steps() == 7
