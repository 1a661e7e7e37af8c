"""Morton reordering (Orchestrator::reorder_gaussians, orchestrator.cu:
26-90, 1038-1061) on the GPU: tgs_morton_order bit-exact against the
oracle's order (oracle/morton.py), and the reorder of the Gaussians, their
gradients, the Adam moments and the densification info consistent with it."""
import numpy as np
import pytest

from oracle import morton as M

pytestmark = pytest.mark.gpu

GROUPS = ("means", "opacities", "rotations", "scales", "sh0", "sh_rest")


def _means(n, seed):
    rng = np.random.default_rng(seed)
    centres = rng.uniform(-3, 3, (16, 3))
    m = centres[rng.integers(0, 16, n)] + rng.normal(0, 0.3, (n, 3))
    m = m.astype(np.float32)
    if n > 64:
        m[10:60] = m[3]                    # equal codes: stable order
    return m


@pytest.mark.parametrize("n,seed", [(1, 0), (4097, 1), (200_000, 2)])
def test_morton_order_matches_oracle(hip, n, seed):
    import torch
    from tinygs_amd.morton import morton_order
    m = _means(n, seed)
    print(f"[morton] n={n}", flush=True)
    got = morton_order(torch.from_numpy(m).cuda()).cpu().numpy().astype(np.int64)
    assert np.array_equal(got, M.morton_order(m))


def test_morton_order_degenerate_axis(hip):
    import torch
    from tinygs_amd.morton import morton_order
    m = _means(5000, 3)
    m[:, 1] = 0.25                          # zero extent: clamped to 1e-8
    got = morton_order(torch.from_numpy(m).cuda()).cpu().numpy().astype(np.int64)
    assert np.array_equal(got, M.morton_order(m))


def test_orchestrator_reorder_permutes_every_row_array(hip):
    """After two training steps (nonzero moments and densification info),
    reorder_gaussians permutes parameters, gradients, both Adam moments and
    the densification info by the same Morton order."""
    import torch
    from tinygs_amd import scenes
    from tinygs_amd.data import SimpleDataLoader, SyntheticViewDataset, gaussians_from_arrays
    from tinygs_amd.optim import create_optimizer
    from tinygs_amd.rasterizer import create_rasterizer
    from tinygs_amd.trainer import Orchestrator, OrchestratorConfig
    sc = scenes.config5(n_init=3000, n_gt=2000, n_cameras=4, width=96, height=64)
    g = gaussians_from_arrays(sc.init, 0)
    grads = g.gradient_like()
    opt = create_optimizer("simple_adam", g, grads)
    orch = Orchestrator(OrchestratorConfig(reorder_gaussians_interval=0), g, grads, create_rasterizer("fastgs"),
                        opt, SimpleDataLoader(SyntheticViewDataset(sc)))
    orch.m_ctx.densification_info = torch.rand((g.size(), 4), device="cuda")
    orch.train(2)
    torch.cuda.synchronize()
    before = {"p": [t.cpu().numpy().copy() for t in g.tensors()],
              "g": [t.cpu().numpy().copy() for t in grads.tensors()],
              "m": {k: tuple(a.cpu().numpy().copy() for a in opt.moments(k)) for k in GROUPS},
              "d": orch.m_ctx.densification_info.cpu().numpy().copy()}
    order = M.morton_order(before["p"][0])
    orch.reorder_gaussians()
    torch.cuda.synchronize()
    for a, t in zip(before["p"], g.tensors()):
        assert np.array_equal(t.cpu().numpy(), a[order])
    for a, t in zip(before["g"], grads.tensors()):
        assert np.array_equal(t.cpu().numpy(), a[order])
    for k in GROUPS:
        (a1, a2), (m1, m2) = before["m"][k], opt.moments(k)
        w = a1.size // g.size()
        assert np.array_equal(m1.cpu().numpy().reshape(-1, w), a1.reshape(-1, w)[order])
        assert np.array_equal(m2.cpu().numpy().reshape(-1, w), a2.reshape(-1, w)[order])
    assert np.array_equal(orch.m_ctx.densification_info.cpu().numpy(), before["d"][order])
