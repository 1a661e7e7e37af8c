"""The training loop (Orchestrator + SimpleAdam + DefaultStrategy + data
loader) on a reduced config-5 scene against the CPU oracle's trajectory
(tests/golden/config5_reduced.json, written by make_config5_reduced.py from
oracle/train.py)."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config5_reduced.json")


def _orchestrator(fx):
    from tinygs_amd import scenes
    from tinygs_amd.data import SimpleDataLoader, SyntheticViewDataset, gaussians_from_arrays
    from tinygs_amd.optim import create_optimizer
    from tinygs_amd.rasterizer import create_rasterizer
    from tinygs_amd.strategy import create_strategy
    from tinygs_amd.trainer import Orchestrator, OrchestratorConfig
    sc = scenes.config5(**fx["scene"])
    ds = SyntheticViewDataset(sc)
    g = gaussians_from_arrays(sc.init, 0)
    grads = g.gradient_like()
    opt = create_optimizer("simple_adam", g, grads)
    st = create_strategy("default", g, grads, opt)
    st.set_params(fx["strategy"])
    return Orchestrator(OrchestratorConfig(), g, grads, create_rasterizer("fastgs"), opt, SimpleDataLoader(ds),
                        strategy=st), g, st


def test_config5_reduced_trajectory_matches_oracle(hip):
    """Forty iterations with densification every 10 (duplicate / split /
    prune) and an opacity reset at 30: the Gaussian count and the
    duplicate / split / kept counts of every refine are the oracle's, and the
    mean PSNR over four views at iterations 10, 20, 30 and 40 is within
    0.02 dB of it (the loop differs from the oracle only by float rounding of
    sums)."""
    with open(GOLDEN) as f:
        fx = json.load(f)
    orch, g, st = _orchestrator(fx)
    orch.recompute_scene_scale()
    assert abs(g.scene_scale() - fx["scene_scale"]) <= 1e-6 * fx["scene_scale"]
    traj = fx["trajectory"]
    for it in range(1, fx["iters"] + 1):
        orch.train_step()
        key = str(it)
        if key in traj["counts"]:
            assert st.last_counts == traj["counts"][key], it
        if key in traj["psnr"] and traj["psnr"][key] is not None:
            assert g.size() == traj["gaussians"][key], it
            p = orch.eval_psnr(fx["eval_views"])
            assert abs(p - traj["psnr"][key]) < 0.02, (it, p, traj["psnr"][key])


GOLDEN_FULL = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config5_iter{}.json")


@pytest.mark.parametrize("iters", [100, 250])
def test_config5_full_size_matches_oracle(hip, iters):
    """The full config-5 loop (500k initial Gaussians, 200 views of
    1600x1060, refine every 100 from 100) against the CPU oracle's run of the
    same loop (tests/golden/config5_iter<N>.json, written by
    make_config5_fixture.py): at iteration 100, where the benchmark quotes
    its PSNR, and at 250, after the refines at steps 101 and 201 (densify,
    then prune). The mean PSNR over views 0-19 within 0.02 dB, the Gaussian
    count within 0.1% (a refine's thresholds meet float sums whose rounding
    differs between the two) and the parameter means."""
    with open(GOLDEN_FULL.format(iters)) as f:
        fx = json.load(f)
    orch, g, st = _orchestrator({"scene": {}, "strategy": fx["strategy"]})
    orch.recompute_scene_scale()
    assert abs(g.scene_scale() - fx["scene_scale"]) <= 1e-6 * fx["scene_scale"]
    for it in range(fx["iters"]):
        orch.train_step()
    print(f"[config5 full] iteration {iters}: {g.size()} Gaussians (oracle {fx['gaussians']})", flush=True)
    assert abs(g.size() - fx["gaussians"]) <= 1e-3 * fx["gaussians"]
    p = orch.eval_psnr(fx["eval_views"])
    print(f"[config5 full] PSNR {p:.4f} (oracle {fx['psnr']:.4f})", flush=True)
    assert abs(p - fx["psnr"]) < 0.02, (p, fx["psnr"])
    got = {"means": g.means(), "scales": g.scales(), "rotations": g.rotations(), "opacities": g.opacities(),
           "sh0": g.sh_coefficient_0().float(), "sh_rest": g.sh_coefficients_rest().float()}
    for k, v in got.items():
        m = float(v.double().abs().mean())
        assert abs(m - fx["param_abs_means"][k]) <= 1e-3 * fx["param_abs_means"][k] + 1e-7, (k, m)


@pytest.mark.parametrize("wh", [(37, 21), (64, 48), (1, 1)])
def test_psnr_closed_form(hip, wh):
    """tgs_psnr against -10 log10(MSE) in double precision: MSE over every
    padded element of (saturate(pred) - target)^2 divided by W H C
    (psnr.cu:72-128), with prediction values outside [0, 1] and nonzero
    padding; 100 for identical images."""
    import torch
    from tinygs_amd.core import Image
    from tinygs_amd.image import ImageShape
    from tinygs_amd.trainer import PsnrMetric
    shape = ImageShape(*wh)
    g = np.random.default_rng(wh[0])
    pred = g.uniform(-0.3, 1.3, shape.padded_size).astype(np.float32)
    target = g.uniform(0.0, 1.0, shape.padded_size).astype(np.float32)
    a = Image(shape, data=torch.from_numpy(pred).cuda())
    b = Image(shape, data=torch.from_numpy(target).cuda())
    got = PsnrMetric().evaluate(a, b)
    d = np.clip(pred.astype(np.float64), 0.0, 1.0) - target
    want = -10.0 * np.log10((d * d).sum() / shape.size())
    assert abs(got - want) < 1e-4 * max(1.0, abs(want)), (got, want)
    assert PsnrMetric().evaluate(b, b) == 100.0


@pytest.mark.parametrize("wh", [(64, 48), (101, 67)])
def test_psnr_float16_closed_form(hip, wh):
    """tgs_psnr on half images (psnr.cu:38-70, 72-128): each half widened to
    float, saturate(pred) - target squared in float, summed over the padded
    elements and divided by W H C; against the same in double precision."""
    import torch
    from tinygs_amd.core import DataType, Image
    from tinygs_amd.image import ImageShape
    from tinygs_amd.trainer import PsnrMetric
    shape = ImageShape(*wh)
    g = np.random.default_rng(wh[1])
    pred = g.uniform(-0.3, 1.3, shape.padded_size).astype(np.float16)
    target = g.uniform(0.0, 1.0, shape.padded_size).astype(np.float16)
    a = Image(shape, DataType.Float16, torch.from_numpy(pred).cuda())
    b = Image(shape, DataType.Float16, torch.from_numpy(target).cuda())
    got = PsnrMetric().evaluate(a, b)
    d = np.clip(pred.astype(np.float64), 0.0, 1.0) - target.astype(np.float64)
    want = -10.0 * np.log10((d * d).sum() / shape.size())
    assert abs(got - want) < 1e-4 * max(1.0, abs(want)), (got, want)
    assert PsnrMetric().evaluate(b, b) == 100.0
    with pytest.raises(RuntimeError):
        PsnrMetric().evaluate(a, Image(shape, DataType.Float32, torch.zeros(shape.padded_size).cuda()))


def _small_loop(data_type="float32", accum=1, views=4):
    from tinygs_amd import scenes
    from tinygs_amd.data import SimpleDataLoader, SyntheticViewDataset, gaussians_from_arrays
    from tinygs_amd.optim import create_optimizer
    from tinygs_amd.rasterizer import create_rasterizer
    from tinygs_amd.trainer import Orchestrator, OrchestratorConfig
    sc = scenes.config5(n_init=3000, n_gt=2000, n_cameras=views, width=96, height=64)
    ds = SyntheticViewDataset(sc, data_type=data_type)
    g = gaussians_from_arrays(sc.init, 0)
    grads = g.gradient_like()
    opt = create_optimizer("simple_adam", g, grads)
    cfg = OrchestratorConfig(train_data_type=data_type, eval_data_type=data_type, accumulate_grad_steps=accum,
                             reorder_gaussians_interval=0, grad_scaler=4.0)
    return sc, ds, Orchestrator(cfg, g, grads, create_rasterizer("fastgs"), opt, SimpleDataLoader(ds)), g, opt


def _twin(sc, ds, data_type):
    """The same Gaussians and Adam state driven by the bare entry points."""
    from tinygs_amd.core import Image, LossContext, RasterizeContext
    from tinygs_amd.data import SimpleDataLoader, gaussians_from_arrays
    from tinygs_amd.loss import create_loss
    from tinygs_amd.optim import create_optimizer
    from tinygs_amd.rasterizer import create_rasterizer
    from tinygs_amd.image import ImageShape
    g = gaussians_from_arrays(sc.init, 0)
    grads = g.gradient_like()
    opt = create_optimizer("simple_adam", g, grads)
    r = create_rasterizer("fastgs")
    r.set_gaussians(g)
    shape = ImageShape(ds.width, ds.height, 3)
    ctx = RasterizeContext(grad_scaler=4.0)
    ctx.fwd_output.image = Image.empty(shape, data_type=data_type)
    ctx.grad_output.image = Image.empty(shape, data_type=data_type)
    ctx.gaussians_grad = grads
    return {"g": g, "grads": grads, "opt": opt, "r": r, "ctx": ctx, "loader": SimpleDataLoader(ds),
            "loss": Image.empty(shape, data_type=data_type), "l1": create_loss("l1")}


def _state(g):
    return [t.detach().cpu().numpy().copy() for t in g.tensors()]


@pytest.mark.parametrize("data_type", ["float32", "float16"])
def test_orchestrator_step_equals_bare_entry_points(hip, data_type):
    """One Orchestrator step at train_data_type float32 / float16 (dataset
    images of the same type; grad_scaler 4) is the bare sequence forward ->
    fused L1 + SSIM (weights x grad_scaler) -> sparse backward -> masked Adam
    with scale 1 / grad_scaler, bit for bit; training then raises the PSNR
    (fp16 PsnrMetric on fp16 images)."""
    import numpy as np
    import torch
    from tinygs_amd.core import LossContext
    from tinygs_amd.loss import evaluate_l1_ssim
    sc, ds, orch, g, opt = _small_loop(data_type)
    t = _twin(sc, ds, data_type)
    print(f"[loop] one step, {data_type} images", flush=True)
    orch.recompute_scene_scale()
    t["g"].set_scene_scale(g.scene_scale())
    orch.train_step()
    cam, target = t["loader"].next()
    ctx = t["ctx"]
    ctx.fwd_input = cam
    t["r"].forward(ctx)
    lctx = LossContext(ctx.fwd_output.image, target, t["loss"], ctx.grad_output.image, None)
    evaluate_l1_ssim(t["l1"], lctx, 0.8 * 4.0, 0.2 * 4.0, assign=True)
    t["r"].backward(ctx, sparse=True)
    t["opt"].step(float(np.float32(1.0) / np.float32(4.0)), None, row_mask=t["r"].grad_row_mask())
    torch.cuda.synchronize()
    assert orch.m_pred.data.dtype == (torch.float16 if data_type == "float16" else torch.float32)
    for a, b in zip(_state(g), _state(t["g"])):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    p0 = orch.eval_psnr()
    orch.train(40)
    p1 = orch.eval_psnr()
    print(f"[loop] {data_type}: PSNR {p0:.3f} -> {p1:.3f} dB after 40 steps", flush=True)
    assert p1 > p0 + 0.5


def test_gradient_accumulation_over_two_steps(hip, orc):
    """accumulate_grad_steps = 2 (orchestrator.cu:343-353, 390-404): the
    gradients are zeroed at the cycle start, both backwards accumulate, and
    only the second step runs Adam, scaled by 1 / (grad_scaler * 2). The
    accumulated gradients equal the sum of the two views' oracle gradients
    (within the gradient bars), and the step is Adam bit-exact on them."""
    import numpy as np
    import torch
    from helpers import assert_grads_close
    sc, ds, orch, g, opt = _small_loop("float32", accum=2)
    orch.recompute_scene_scale()
    theta0 = _state(g)
    orch.train_step()
    torch.cuda.synchronize()
    assert all(np.array_equal(a, b) for a, b in zip(theta0, _state(g)))   # no step after the first view
    orch.train_step()
    torch.cuda.synchronize()
    got_grads = _state(orch.m_gradients)
    # the oracle: both views' gradients at the initial parameters, summed
    from oracle import train as T
    from tinygs_amd.data import SimpleDataLoader
    ld = SimpleDataLoader(ds)
    names = ("means", "scales", "rotations", "opacities", "sh0", "sh_rest")
    init = {k: np.asarray(v, np.float32).reshape(v.shape[0], -1) if k != "opacities" else np.asarray(v, np.float32)
            for k, v in sc.init.items()}
    init["sh_rest"] = init["sh_rest"].reshape(-1, 45)
    ref = {k: 0.0 for k in names}
    for _ in range(2):
        view = ds[ld.m_permutation[ld.m_current_index]]
        ld.next()
        v = T._View(init, 0, view.camera, view.target.data.cpu().numpy())
        out = orc.run_iteration(v, 0.8 * 4.0, 0.2 * 4.0, lr=None, eps=1e-8)
        for k in names:
            ref[k] = ref[k] + out["grads"][k].astype(np.float64)
    assert_grads_close({k: a.reshape(-1) for k, a in zip(names, got_grads)},
                       {k: ref[k].astype(np.float32) for k in names})
    # Adam on the accumulated gradients, scale 1 / (4 * 2)
    th = orc.params(v, "f")
    m1 = {k: np.zeros_like(a) for k, a in th.items()}
    m2 = {k: np.zeros_like(a) for k, a in th.items()}
    lr = {"means": 1.6e-4, "scene_scale": g.scene_scale(), "opacities": 5e-2, "rotations": 1e-3,
          "scales": 5e-3, "shs": 2.5e-3}
    scale = float(np.float32(np.float32(1.0) / np.float32(4.0)) / np.float32(2.0))
    orc.adam_step(th, {k: a.reshape(-1) for k, a in zip(names, got_grads)}, m1, m2, lr, 1, grad_scale=scale,
                  eps=1e-8)
    for k, a in zip(names, _state(g)):
        assert np.array_equal(a.reshape(-1).view(np.uint32), th[k].view(np.uint32)), k
