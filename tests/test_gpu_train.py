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
