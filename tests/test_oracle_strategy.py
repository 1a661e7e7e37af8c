"""CPU checks of the densification restatement (oracle/strategy.py) against
known answers, closed forms and brute force -- no GPU needed."""
import math

import numpy as np
import pytest

from oracle import strategy as S

F = np.float32


def test_pcg32_known_answer():
    # pcg32_srandom_r(&rng, 42, 54) then pcg32_random_r: the published
    # output of the PCG reference demo (pcg32-demo.c, pcg-c-basic)
    r = S.Pcg32()
    r.seed(42, 54)
    got = [r.next_uint() for _ in range(6)]
    assert got == [0xA15C02B7, 0x7B47F409, 0xBA1D3330, 0x83D2F293, 0xBFA4784B, 0xCBED606E]


def test_pcg32_advance_and_floats():
    r = S.Pcg32()
    r.seed(7)
    a = S.Pcg32(r.state, r.inc)
    seq = [a.next_uint() for _ in range(1000)]
    for k in (0, 1, 5, 999):
        b = S.Pcg32(r.state, r.inc)
        b.advance(k)
        assert b.next_uint() == seq[k]
    # a full-period step back: advancing by -k returns to the earlier state
    b = S.Pcg32(r.state, r.inc)
    b.advance(37)
    b.advance(-37)
    assert (b.state, b.inc) == (r.state, r.inc)
    c = S.Pcg32(r.state, r.inc)
    fl = np.array([c.next_float() for _ in range(20000)], F)
    assert fl.min() >= 0.0 and fl.max() < 1.0
    # 23 random mantissa bits: every value is a multiple of 2^-23
    assert np.all(fl * F(2.0 ** 23) == np.floor(fl * F(2.0 ** 23)))


def test_logit_logistic():
    assert S.logit(np.array([0.5], F))[0] == 0.0
    p = np.linspace(1e-4, 1 - 1e-4, 999).astype(F)
    back = S.logistic(S.logit(p))
    assert np.max(np.abs(back - p)) < 2e-6
    # logit clamps at 1e-9: logit(0) = -log(1e9 - 1)
    assert abs(float(S.logit(np.array([0.0], F))[0]) + math.log(1e9 - 1)) < 1e-4
    x = np.linspace(-8, 8, 101).astype(F)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(S.logistic(x) - ref)) < 1e-6


def test_random_logistic_layout_and_moments():
    # element i + T j reads stream position 4 i + j (T = ceil(n / 4))
    r = S.Pcg32()
    r.seed(3)
    n = 10
    t = (n + 3) // 4
    u = []
    c = S.Pcg32(r.state, r.inc)
    for _ in range(4 * t):
        u.append(c.next_float())
    out = S.random_logistic(r, n)
    for idx in range(n):
        i, j = idx % t, idx // t
        assert out[idx] == S.logit(np.array([u[4 * i + j]], F))[0] * F(0.551328895)
    # stream advanced by exactly n
    d = S.Pcg32(c.state, c.inc)
    e = S.Pcg32()
    e.seed(3)
    e.advance(n)
    assert r.state == e.state
    # logistic with scale sqrt(3) / pi: zero mean, unit variance
    big = S.random_logistic(r, 200_000)
    assert abs(float(big.mean())) < 0.01
    assert abs(float(big.std()) - 1.0) < 0.01


def _rand_params(n, seed):
    g = np.random.default_rng(seed)
    q = g.standard_normal((n, 4)).astype(F) * F(1.3)
    return {"means": g.normal(0, 1, (n, 3)).astype(F), "scales": g.normal(-4, 1.2, (n, 3)).astype(F),
            "rotations": q, "opacities": g.normal(0, 2, n).astype(F), "sh0": g.random((n, 3)).astype(F),
            "sh_rest": g.normal(0, 0.1, (n, 45)).astype(F)}


def test_densify_select_brute_force():
    g = np.random.default_rng(5)
    n = 3000
    info = np.zeros((n, 4), F)
    info[:, 0] = g.integers(0, 4, n)
    info[:, 1] = g.random(n) * 1e-3
    info[:, 2] = g.random(n) * 2e-3
    scales = g.normal(-4.6, 0.7, (n, 3)).astype(F)
    for absgrad in (False, True):
        flags = S.densify_select(info, scales, 2e-4, 0.01, absgrad)
        for i in range(n):
            acc = info[i, 2] if absgrad else info[i, 1]
            grad = acc / max(info[i, 0], 1.0)
            if abs(grad - 2e-4) < 1e-9:
                continue
            s = max(math.exp(v) for v in scales[i])
            if abs(s - 0.01) < 1e-9:
                continue
            want = 0 if not (grad > 2e-4 and info[i, 0] > 0) else (2 if s > 0.01 else 1)
            assert flags[i] == want, i


def test_split_closed_forms():
    n = 64
    p = _rand_params(n, 6)
    flags = np.full(n, 2, np.uint8)
    flags[::3] = 1
    src = np.nonzero(flags)[0]
    g = src.size
    orig = {k: v.copy() for k, v in p.items()}
    for k in p:
        p[k] = np.concatenate([p[k], np.zeros((g,) + p[k].shape[1:], F)])
    rnd = np.random.default_rng(7).normal(0, 1, 6 * g).astype(F)
    S.densify_apply(p, n, src, flags, rnd)
    for i, s in enumerate(src):
        t = n + i
        assert np.array_equal(p["rotations"][t], orig["rotations"][s])
        assert np.array_equal(p["sh_rest"][t], orig["sh_rest"][s])
        if flags[s] == 1:
            for k in ("means", "scales", "opacities"):
                assert np.array_equal(p[k][t], orig[k][s])
            continue
        # scale / 1.6 in activated space, both children
        want = orig["scales"][s].astype(np.float64) - math.log(1.6)
        assert np.max(np.abs(p["scales"][t] - want)) < 1e-5 and np.array_equal(p["scales"][t], p["scales"][s])
        # two children of opacity 1 - sqrt(1 - o) composite to o
        o = 1.0 / (1.0 + math.exp(-float(orig["opacities"][s])))
        oc = 1.0 / (1.0 + math.exp(-float(p["opacities"][t])))
        if o < 0.999:
            assert abs((1.0 - (1.0 - oc) ** 2) - o) < 5e-6
        # offsets: R^T (r * (exp(s) + 1e-5)) with R the rotation matrix of the raw quaternion
        r, x, y, z = orig["rotations"][s].astype(np.float64)
        R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - r * z), 2 * (x * z + r * y)],
                      [2 * (x * y + r * z), 1 - 2 * (x * x + z * z), 2 * (y * z - r * x)],
                      [2 * (x * z - r * y), 2 * (y * z + r * x), 1 - 2 * (x * x + y * y)]])
        a = np.exp(orig["scales"][s].astype(np.float64)) + 1e-5
        off1 = R.T @ (rnd[6 * i:6 * i + 3].astype(np.float64) * a)
        off2 = R.T @ (rnd[6 * i + 3:6 * i + 6].astype(np.float64) * a)
        scale = np.abs(R).sum() * a.max() * 4 + 1e-3
        assert np.max(np.abs(p["means"][t] - (orig["means"][s] + off1))) < 1e-5 * scale
        assert np.max(np.abs(p["means"][s] - (orig["means"][s] + off2))) < 1e-5 * scale


def test_prune_brute_force():
    n = 2000
    p = _rand_params(n, 8)
    p["rotations"][::97] = 0.0
    info = np.zeros((1500, 4), F)
    info[:, 3] = np.random.default_rng(9).random(1500) * 40
    for prune_large in (False, True):
        alive = S.prune_alive(p, info, 1500, 0.005, 0.05, 30.0, prune_large)
        for i in range(n):
            s = max(math.exp(v) for v in p["scales"][i])
            o = 1.0 / (1.0 + math.exp(-float(p["opacities"][i])))
            if min(abs(s - 0.05), abs(o - 0.005)) < 1e-7:
                continue
            ws = s < 0.05
            ss = i >= 1500 or info[i, 3] < 30.0
            deg = np.abs(p["rotations"][i]).sum() > 1.1920929e-07
            want = (o > 0.005) and ((ws and ss) or not prune_large) and deg
            assert alive[i] == int(want), i


def test_reset_opacity_caps_at_threshold():
    x = np.linspace(-10, 10, 201).astype(F)
    y = S.reset_opacity(x, F(0.01))
    o = S.logistic(y)
    assert np.all(o <= 0.01 + 1e-7)
    low = S.logistic(x) < 0.0099
    assert np.max(np.abs(y[low] - x[low])) < 1e-5


def test_adam_remove_mapping_of_the_reference():
    # SimpleAdam::remove maps over the first num_kept flags only (the
    # Gaussians are already shrunk); the zero-initialised tail reads row 0
    alive = np.array([1, 0, 1, 1, 0, 1], np.uint8)
    assert list(S.adam_remove_rows(alive, 4)) == [0, 2, 3, 0]
    assert list(S.adam_remove_rows(np.ones(5, np.uint8), 5)) == [0, 1, 2, 3, 4]


def test_strategy_schedule():
    st = S.DefaultStrategy({"refine_every": 2, "start_refine": 2, "end_refine": 6, "reset_every": 4, "seed": 1})
    n = 50
    p = _rand_params(n, 11)
    m1 = {"means": np.zeros((n, 3), F), "opacities": np.ones(n, F), "rotations": np.zeros((n, 4), F),
          "scales": np.zeros((n, 3), F), "sh0": np.zeros((n, 3), F), "sh_rest": np.zeros((n, 45), F)}
    m2 = {k: v.copy() for k, v in m1.items()}
    info = np.zeros((n, 4), F)
    resets = []
    for step in range(8):
        before = p["opacities"].copy()
        info = st.step(p, m1, m2, info, 1.0, 1.0, 64, 64)
        if not np.array_equal(before, p["opacities"]) and step in (4,):
            resets.append(step)
        m1["opacities"][:] = 1.0
    assert resets == [4]
    assert st.step_count == 8
