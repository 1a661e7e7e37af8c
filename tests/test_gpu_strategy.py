"""Densification kernels and DefaultStrategy on the GPU against the CPU
restatement (oracle/strategy.py): bit-exact (deterministic exp / log, IEEE
division and square root on both sides)."""
import ctypes as C

import numpy as np
import pytest

from oracle import strategy as S

pytestmark = pytest.mark.gpu

F = np.float32
GROUPS = ("means", "opacities", "rotations", "scales", "sh0", "sh_rest")
WIDTH = {"means": 3, "opacities": 1, "rotations": 4, "scales": 3, "sh0": 3, "sh_rest": 45}


def _bits(a):
    return np.ascontiguousarray(a, F).view(np.uint32)


def _rand_params(n, seed):
    g = np.random.default_rng(seed)
    return {"means": g.normal(0, 1, (n, 3)).astype(F), "scales": g.normal(-4.3, 1.0, (n, 3)).astype(F),
            "rotations": (g.standard_normal((n, 4)) * 1.2).astype(F), "opacities": g.normal(0, 2.5, n).astype(F),
            "sh0": g.random((n, 3)).astype(F), "sh_rest": g.normal(0, 0.1, (n, 45)).astype(F)}


def _rand_info(n, seed):
    g = np.random.default_rng(seed)
    info = np.zeros((n, 4), F)
    info[:, 0] = g.integers(0, 5, n)
    info[:, 1] = (g.random(n) * 8e-4).astype(F)
    info[:, 2] = (g.random(n) * 1.6e-3).astype(F)
    info[:, 3] = (g.random(n) * 900.0).astype(F)
    return info


def _gaussians(p, sh_dtype="float32"):
    import torch
    from tinygs_amd.core import GPUGaussian3d
    g = GPUGaussian3d(0, sh_dtype)
    shd = torch.float16 if sh_dtype == "float16" else torch.float32
    g.m_means = torch.from_numpy(p["means"]).cuda()
    g.m_scales = torch.from_numpy(p["scales"]).cuda()
    g.m_rotations = torch.from_numpy(p["rotations"]).cuda()
    g.m_opacities = torch.from_numpy(p["opacities"]).cuda()
    g.m_sh_coefficient_0 = torch.from_numpy(p["sh0"]).cuda().to(shd)
    g.m_sh_coefficients_rest = torch.from_numpy(p["sh_rest"].reshape(-1, 15, 3)).cuda().to(shd)
    g.m_current_sh_degree = 3
    return g


def _host(g):
    return {"means": g.means().cpu().numpy(), "scales": g.scales().cpu().numpy(),
            "rotations": g.rotations().cpu().numpy(), "opacities": g.opacities().cpu().numpy(),
            "sh0": g.sh_coefficient_0().float().cpu().numpy(),
            "sh_rest": g.sh_coefficients_rest().float().cpu().numpy().reshape(-1, 45)}


def _round_half(p):
    q = dict(p)
    q["sh0"] = p["sh0"].astype(np.float16).astype(F)
    q["sh_rest"] = p["sh_rest"].astype(np.float16).astype(F)
    return q


@pytest.mark.parametrize("n", [1, 5, 12, 4663])
def test_random_logistic_bit_exact(hip, n):
    import torch
    from tinygs_amd import _lib
    L = _lib.load()
    rng = _lib.tgs_pcg32()
    L.tgs_pcg32_seed(C.byref(rng), 42, 1)
    ref = S.Pcg32()
    ref.seed(42, 1)
    assert (rng.state, rng.inc) == (ref.state, ref.inc)
    for _ in range(2):   # two calls: the stream continues where the first left it
        out = torch.empty(n, dtype=torch.float32, device="cuda")
        _lib.check(L.tgs_random_logistic(C.byref(rng), n, out.data_ptr(), 0.0, 1.0, None))
        torch.cuda.synchronize()
        want = S.random_logistic(ref, n)
        assert np.array_equal(_bits(out.cpu().numpy()), _bits(want))
        assert (rng.state, rng.inc) == (ref.state, ref.inc)


@pytest.mark.parametrize("sh_dtype", ["float32", "float16"])
def test_densify_select_and_apply_bit_exact(hip, sh_dtype):
    import torch
    from tinygs_amd import _lib
    L = _lib.load()
    n = 20000
    p = _rand_params(n, 1)
    if sh_dtype == "float16":
        p = _round_half(p)
    info = _rand_info(n, 2)
    g = _gaussians(p, sh_dtype)
    dinfo = torch.from_numpy(info).cuda()
    flags = torch.empty(n, dtype=torch.uint8, device="cuda")
    src = torch.empty(n, dtype=torch.int32, device="cuda")
    nd, ns = C.c_int64(), C.c_int64()
    gc = g.to_c()
    _lib.check(L.tgs_densify_select(C.byref(gc), dinfo.data_ptr(), 2e-4, 0.012, 0, flags.data_ptr(),
                                    src.data_ptr(), C.byref(nd), C.byref(ns), None))
    want = S.densify_select(info, p["scales"], F(2e-4), F(0.012), False)
    assert np.array_equal(flags.cpu().numpy(), want)
    wsrc = np.nonzero(want)[0]
    assert nd.value == int((want == 1).sum()) and ns.value == int((want == 2).sum())
    assert nd.value > 100 and ns.value > 100
    grows = wsrc.size
    assert np.array_equal(src[:grows].cpu().numpy(), wsrc)
    g.append(grows)
    rng = _lib.tgs_pcg32()
    L.tgs_pcg32_seed(C.byref(rng), 9, 1)
    rnd = torch.empty(6 * grows, dtype=torch.float32, device="cuda")
    _lib.check(L.tgs_random_logistic(C.byref(rng), 6 * grows, rnd.data_ptr(), 0.0, 1.0, None))
    gc = g.to_c()
    _lib.check(L.tgs_densify_apply(C.byref(gc), n, src.data_ptr(), grows, flags.data_ptr(), rnd.data_ptr(), None))
    torch.cuda.synchronize()
    q = {k: np.concatenate([v, np.zeros((grows,) + v.shape[1:], F)]) for k, v in p.items()}
    S.densify_apply(q, n, wsrc, want, rnd.cpu().numpy())
    got = _host(g)
    for k in q:
        assert np.array_equal(_bits(got[k]), _bits(q[k])), k


def test_prune_gather_reset_bit_exact(hip):
    import torch
    from tinygs_amd import _lib
    L = _lib.load()
    n = 30000
    p = _rand_params(n, 3)
    p["rotations"][::211] = 0.0
    info = _rand_info(25000, 4)
    g = _gaussians(p)
    dinfo = torch.from_numpy(info).cuda()
    for prune_large in (0, 1):
        alive = torch.empty(n, dtype=torch.uint8, device="cuda")
        kept = torch.empty(n, dtype=torch.int32, device="cuda")
        nk = C.c_int64()
        gc = g.to_c()
        _lib.check(L.tgs_prune_select(C.byref(gc), dinfo.data_ptr(), 25000, 0.005, 0.05, 640.0, prune_large,
                                      alive.data_ptr(), kept.data_ptr(), C.byref(nk), None))
        want = S.prune_alive(p, info, 25000, F(0.005), F(0.05), F(640.0), bool(prune_large))
        assert np.array_equal(alive.cpu().numpy(), want)
        wk = np.nonzero(want)[0]
        assert nk.value == wk.size and np.array_equal(kept[:wk.size].cpu().numpy(), wk)
    h = g.clone()
    h.remove(kept, nk.value)
    got = _host(h)
    for k in p:
        assert np.array_equal(_bits(got[k]), _bits(p[k][wk])), k
    gc = h.to_c()
    _lib.check(L.tgs_reset_opacity(C.byref(gc), 0.01, None))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(h.opacities().cpu().numpy()), _bits(S.reset_opacity(p["opacities"][wk], F(0.01))))


def _set_moments(opt, m1, m2):
    from tinygs_amd import _lib
    import torch
    for k, name in enumerate(GROUPS):
        a, b = C.c_void_p(), C.c_void_p()
        _lib.check(_lib.load().tgs_adam_moments(opt._h, k, C.byref(a), C.byref(b)))
        for ptr, arr in ((a, m1[name]), (b, m2[name])):
            t = torch.from_numpy(np.ascontiguousarray(arr, F).reshape(-1)).cuda()
            torch.cuda.synchronize()
            rc = _lib.hip().hipMemcpy(ptr, C.c_void_p(t.data_ptr()), C.c_size_t(4 * t.numel()), 3)
            assert rc == 0


@pytest.mark.parametrize("sh_dtype", ["float32", "float16"])
def test_default_strategy_steps_match_oracle(hip, sh_dtype):
    """DefaultStrategy.step over six steps (refine at 2 and 4, opacity reset at
    4, large Gaussians pruned after step 3) against the CPU restatement:
    parameters, optimiser moments (including SimpleAdam::remove's mapping
    over the already-shrunk Gaussian count), counts and RNG state."""
    import torch
    from tinygs_amd import _lib
    from tinygs_amd.core import GPUBatchInput, RasterizeContext
    from tinygs_amd.optim import create_optimizer
    from tinygs_amd.strategy import create_strategy
    n = 6000
    p = _rand_params(n, 5)
    if sh_dtype == "float16":
        p = _round_half(p)
    g = _gaussians(p, sh_dtype)
    grads = g.gradient_like()
    opt = create_optimizer("simple_adam", g, grads)
    rg = np.random.default_rng(6)
    m1 = {k: rg.normal(0, 1, (n, WIDTH[k]) if WIDTH[k] > 1 else n).astype(F) for k in GROUPS}
    m2 = {k: rg.random((n, WIDTH[k]) if WIDTH[k] > 1 else n).astype(F) for k in GROUPS}
    _set_moments(opt, m1, m2)
    cfg = {"refine_every": 2, "start_refine": 2, "end_refine": 5, "reset_every": 4, "seed": 77,
           "duplicate_grad_threshold": 3e-4, "duplicate_scale_threshold": 0.012, "pruning_scale_threshold": 0.3,
           "max_screen_size": 0.5}
    st = create_strategy("default", g, grads, opt)
    st.set_params(cfg)
    ref = S.DefaultStrategy(cfg)
    q = {k: v.copy() for k, v in p.items()}
    rm1 = {k: v.copy() for k, v in m1.items()}
    rm2 = {k: v.copy() for k, v in m2.items()}
    ctx = RasterizeContext()
    ctx.fwd_input = GPUBatchInput(width=320, height=240)
    ctx.grad_scaler = 1.0
    g.set_scene_scale(1.5)
    for step in range(6):
        info = _rand_info(g.size(), 100 + step)
        ctx.densification_info = torch.from_numpy(info).cuda()
        st.step(ctx)
        ref.step(q, rm1, rm2, info, 1.0, 1.5, 320, 240)
        torch.cuda.synchronize()
        assert g.size() == q["means"].shape[0] == grads.size(), step
        got = _host(g)
        for k in q:
            assert np.array_equal(_bits(got[k]), _bits(q[k])), (step, k)
        for name in GROUPS:
            a, b = opt.moments(name)
            assert np.array_equal(_bits(a.cpu().numpy()), _bits(rm1[name].reshape(-1))), (step, name)
            assert np.array_equal(_bits(b.cpu().numpy()), _bits(rm2[name].reshape(-1))), (step, name)
        assert (st.m_rng.state, st.m_rng.inc) == (ref.rng.state, ref.rng.inc)
        assert int(ctx.densification_info.shape[0]) == g.size()
    assert getattr(st, "last_counts", {}) == ref.counts
    assert g.size() != n


@pytest.mark.parametrize("sh_dtype", ["float32", "float16"])
def test_gaussians_reorder_is_a_gather(hip, sh_dtype):
    """GPUGaussian3d::reorder (gpu_gaussian.cu:273-310): new row i = old row
    indices[i], in place, for every array; out-of-range indices are refused
    before anything changes."""
    import torch
    n = 3001
    p = _rand_params(n, 31)
    g = _gaussians(p, sh_dtype)
    before = _host(g)
    perm = np.random.default_rng(5).permutation(n).astype(np.int32)
    g.reorder(torch.from_numpy(perm).cuda())
    torch.cuda.synchronize()
    after = _host(g)
    for k in GROUPS:
        assert np.array_equal(_bits(after[k]), _bits(before[k][perm])), k
    bad = perm.copy()
    bad[17] = n
    with pytest.raises(RuntimeError, match="outside"):
        g.reorder(torch.from_numpy(bad).cuda())
    torch.cuda.synchronize()
    for k, v in _host(g).items():
        assert np.array_equal(_bits(v), _bits(after[k])), k   # untouched


def test_adam_reorder_and_reset_rows(hip):
    """SimpleAdam::reorder (simple_adam.cu:1037-1097) gathers every moment row;
    SimpleAdam::reset(indices, n) (:944-979) zeroes both moments of the listed
    rows and nothing else."""
    import torch
    from tinygs_amd.optim import create_optimizer
    n = 2049
    p = _rand_params(n, 32)
    g = _gaussians(p)
    gg = g.gradient_like()
    for t in gg.tensors():
        t.copy_(torch.randn(t.shape, device="cuda"))
    opt = create_optimizer("simple_adam", g, gg)
    opt.step(1.0)   # nonzero moments
    torch.cuda.synchronize()
    mom = {k: [m.cpu().numpy().reshape(n, -1).copy() for m in opt.moments(k)] for k in GROUPS}
    perm = np.random.default_rng(6).permutation(n).astype(np.int32)
    opt.reorder(torch.from_numpy(perm).cuda())
    torch.cuda.synchronize()
    for k in GROUPS:
        for a, b in zip(opt.moments(k), mom[k]):
            assert np.array_equal(_bits(a.cpu().numpy().reshape(n, -1)), _bits(b[perm])), k
    rows = np.array([0, 5, 5, 2048, 1000], np.int32)
    opt.reset_indices(torch.from_numpy(rows).cuda())
    torch.cuda.synchronize()
    keep = np.setdiff1d(np.arange(n), rows)
    for k in GROUPS:
        for a, b in zip(opt.moments(k), mom[k]):
            a = a.cpu().numpy().reshape(n, -1)
            assert np.all(a[rows] == 0) and np.array_equal(_bits(a[keep]), _bits(b[perm][keep])), k
    with pytest.raises(RuntimeError, match="outside"):
        opt.reset_indices(torch.tensor([n], dtype=torch.int32, device="cuda"))
