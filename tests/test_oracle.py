"""Pins the CPU oracle against mathematics, independently of the GPU build.

The reference holds no golden vectors or tests for this path (its tests/
directory has only a gtest main), so each oracle function is checked against
closed forms, brute force on tiny inputs and double-precision finite
differences, chosen so that a dropped term, a wrong sign or a transposed
operand fails at least one check.
"""
import math

import numpy as np
import pytest

from tinygs_amd import scenes
from tinygs_amd.image import ImageShape, to_hwc, from_hwc, tiled_index


# ---------------------------------------------------------------- exp / log / half

def test_expf_accuracy(orc):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-103.0, 88.7, 200000), rng.uniform(-20, 0, 200000),
                        np.linspace(-1e-3, 1e-3, 2001)]).astype(np.float32)
    y = orc.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    normal = ref > 1.2e-38
    ulp = np.abs(y[normal] - ref[normal]) / np.spacing(ref[normal].astype(np.float32)).astype(np.float64)
    assert ulp.max() <= 2.0, ulp.max()
    # subnormal range: absolute error within one subnormal ulp
    sub = (ref <= 1.2e-38) & (ref > 0)
    assert np.all(np.abs(y[sub] - ref[sub]) <= 2 * 1.4e-45)


def test_exp2_core_accuracy(orc):
    """The blend forward's 2^x (degree-5 minimax, -150 <= x <= 0): within
    2.2e-7 relative (about 4 ulps) of libm's double exp2 over the normal range,
    2^k times the polynomial's value at 0 at the integers k, and the same
    relative error plus half a subnormal ulp below 2^-126."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-150, 0, 400000), rng.uniform(-9, 0, 400000), -np.arange(0, 151.0),
                        np.linspace(-0.5, 0.0, 4001)]).astype(np.float32)
    y = orc.exp2_core(x).astype(np.float64)
    ref = np.exp2(x.astype(np.float64))
    normal = ref > 1.2e-38
    rel = np.abs(y[normal] - ref[normal]) / ref[normal]
    assert rel.max() <= 2.2e-7, rel.max()
    ints = x == np.round(x)
    assert np.array_equal(y[ints & normal], ref[ints & normal] * float.fromhex("0x1.000002p+0"))
    sub = ~normal   # the polynomial's error plus half a subnormal ulp from ldexp
    assert np.all(np.abs(y[sub] - ref[sub]) <= 2.2e-7 * ref[sub] + 0.5 * 2.0 ** -149)


def test_expf_special(orc):
    x = np.array([0.0, -0.0, 1.0, -1.0, 89.0, -104.0, np.inf, -np.inf, np.nan], np.float32)
    y = orc.expf(x)
    assert y[0] == 1.0 and y[1] == 1.0
    assert abs(y[2] - math.e) <= 2.4e-7 * math.e and abs(y[3] - 1 / math.e) <= 1.2e-7
    assert np.isinf(y[4]) and y[5] == 0.0 and np.isinf(y[6]) and y[7] == 0.0 and np.isnan(y[8])


def test_logf_accuracy(orc):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(1.0, 255.0, 200000), np.exp(rng.uniform(-80, 80, 200000)),
                        1.0 + np.linspace(-1e-3, 1e-3, 2001)]).astype(np.float32)
    x = x[x > 0]
    y = orc.logf(x).astype(np.float64)
    ref = np.log(x.astype(np.float64))
    tol = np.maximum(np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64), 1e-45)
    err = np.abs(y - ref) / tol
    assert err.max() <= 2.0, err.max()
    assert orc.logf(np.array([1.0], np.float32))[0] == 0.0
    assert np.isneginf(orc.logf(np.array([0.0], np.float32))[0])


def test_half_rounding_matches_numpy(orc):
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(100000) * 10, rng.uniform(-70000, 70000, 10000),
                        rng.uniform(-1e-4, 1e-4, 10000), np.array([65504, 65519.99, 65520, 2.0 ** -25, 2.0 ** -24])]
                       ).astype(np.float32)
    bits = orc.half_bits(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(bits, ref)


# ---------------------------------------------------------------- preprocess

def _one_gaussian_scene(mean, scale, quat, opac, sh0=(0.3, 0.5, 0.7), cam=None, sh_rest=None, deg=0):
    c = cam or scenes.Camera(64, 64, 64.0, 64.0, 32.0, 32.0, np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 3.0], [0, 0, 0, 1]]))
    return scenes.Scene(np.array([mean], np.float32), np.array([scale], np.float32), np.array([quat], np.float32),
                        np.array([opac], np.float32), np.array([sh0], np.float32),
                        np.zeros((1, 15, 3), np.float32) if sh_rest is None else np.array([sh_rest], np.float32),
                        deg, c, np.zeros(c.shape.padded_size, np.float32))


def _ewa_double(scene, i):
    """Closed-form EWA projection (Zwicker et al. 2001) in double precision."""
    cam = scene.camera
    W = cam.w2c.astype(np.float64)
    mu = scene.means[i].astype(np.float64)
    t = W[:3, :3] @ mu + W[:3, 3]
    q = scene.rotations[i].astype(np.float64)
    q = q / np.linalg.norm(q)
    r, x, y, z = q
    R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - r * z), 2 * (x * z + r * y)],
                  [2 * (x * y + r * z), 1 - 2 * (x * x + z * z), 2 * (y * z - r * x)],
                  [2 * (x * z - r * y), 2 * (y * z + r * x), 1 - 2 * (x * x + y * y)]])
    S = np.diag(np.exp(scene.scales[i].astype(np.float64)))
    Sig = R @ S @ S @ R.T
    J = np.array([[cam.fx / t[2], 0, -cam.fx * t[0] / t[2] ** 2], [0, cam.fy / t[2], -cam.fy * t[1] / t[2] ** 2]])
    cov2 = J @ W[:3, :3] @ Sig @ W[:3, :3].T @ J.T + 0.3 * np.eye(2)
    mean2 = np.array([cam.fx * t[0] / t[2] + cam.cx, cam.fy * t[1] / t[2] + cam.cy])
    return mean2, cov2


def test_preprocess_matches_closed_form_ewa(orc):
    s = scenes.config1(seed=11, n=256)
    pre = orc.preprocess(s, "f")
    vis = np.nonzero(pre["n_touched"])[0]
    assert len(vis) > 150
    for i in vis[:100]:
        mean2, cov2 = _ewa_double(s, i)
        m = pre["mean2d"][2 * i:2 * i + 2]
        assert np.allclose(m, mean2, rtol=1e-5, atol=1e-4)
        a, b, c, o = pre["conic_opacity"][4 * i:4 * i + 4]
        conic = np.array([[a, b], [b, c]], np.float64)
        prod = conic @ cov2
        assert np.allclose(prod, np.eye(2), atol=2e-4), prod
        assert abs(o - 1 / (1 + math.exp(-float(s.opacities[i])))) < 1e-6
        assert abs(pre["power_thr"][i] - math.log(255 * float(o))) < 1e-5


def test_preprocess_rotation_invariance(orc):
    """Rotating a Gaussian about its own axis by a quaternion that commutes with
    an isotropic scale leaves the 2D footprint unchanged."""
    base = _one_gaussian_scene((0.1, -0.2, 0.3), (-2.0, -2.0, -2.0), (1, 0, 0, 0), 0.5)
    rot = _one_gaussian_scene((0.1, -0.2, 0.3), (-2.0, -2.0, -2.0), (0.3, 0.5, -0.7, 0.2), 0.5)
    a = orc.preprocess(base, "d")
    b = orc.preprocess(rot, "d")
    assert np.allclose(a["conic_opacity"], b["conic_opacity"], rtol=1e-9)


def _real_sh(deg_bases, d):
    """Real spherical harmonics from their closed forms with the 3DGS sign
    convention (degree 0..3), at unit direction d."""
    x, y, z = d
    pi = math.pi
    c1 = math.sqrt(3 / (4 * pi))
    c2a = 0.5 * math.sqrt(15 / pi)
    c2b = 0.25 * math.sqrt(5 / pi)
    c2c = 0.25 * math.sqrt(15 / pi)
    c3a = 0.25 * math.sqrt(35 / (2 * pi))
    c3b = 0.5 * math.sqrt(105 / pi)
    c3c = 0.25 * math.sqrt(21 / (2 * pi))
    c3d = 0.25 * math.sqrt(7 / pi)
    c3e = 0.25 * math.sqrt(105 / pi)
    vals = [-c1 * y, c1 * z, -c1 * x,
            c2a * x * y, -c2a * y * z, c2b * (3 * z * z - 1), -c2a * x * z, c2c * (x * x - y * y),
            -c3a * y * (3 * x * x - y * y), c3b * x * y * z, -c3c * y * (5 * z * z - 1), c3d * z * (5 * z * z - 3),
            -c3c * x * (5 * z * z - 1), c3e * z * (x * x - y * y), -c3a * x * (x * x - 3 * y * y)]
    return np.array(vals[:deg_bases - 1])


def test_sh_constants_against_closed_form(orc):
    rng = np.random.default_rng(3)
    for trial in range(5):
        mean = rng.uniform(-0.3, 0.3, 3)
        for b in range(15):
            rest = np.zeros((15, 3), np.float32)
            rest[b, 1] = 1.0
            s = _one_gaussian_scene(mean, (-2.5, -2.5, -2.5), (1, 0, 0, 0), 2.0, sh0=(0, 0, 0), sh_rest=rest, deg=3)
            pre = orc.preprocess(s, "d")
            assert pre["n_touched"][0] > 0
            v = s.means[0].astype(np.float64) - s.camera.cam_pos
            d = v / np.linalg.norm(v)
            expect = _real_sh(16, d)[b]
            col = pre["color"][0:3]
            assert abs(col[0] - 0.5) < 1e-12 and abs(col[2] - 0.5) < 1e-12
            assert abs((col[1] - 0.5) - expect) < 1e-9, (b, col[1] - 0.5, expect)
    # degree 0: c = 0.5 + C0 * dc with C0 = 1 / (2 sqrt(pi))
    s = _one_gaussian_scene((0, 0, 0), (-2.5, -2.5, -2.5), (1, 0, 0, 0), 2.0, sh0=(1.0, -1.0, 0.25))
    col = orc.preprocess(s, "d")["color"][:3]
    c0 = 1 / (2 * math.sqrt(math.pi))
    assert np.allclose(col, 0.5 + c0 * np.array([1.0, -1.0, 0.25]), atol=1e-12)


def test_tile_culling_is_conservative(orc):
    """Brute force: every tile dropped inside the bounds rectangle holds no
    pixel centre where the Gaussian's alpha reaches 1/255."""
    s = scenes.config1(seed=5, n=400)
    pre = orc.preprocess(s, "f")
    bins = orc.bin(s, pre, "f")
    gw, gh = s.camera.grid
    kept = set(zip(bins["inst_tile"].tolist(), bins["inst_prim"].tolist()))
    dropped_checked = 0
    for i in np.nonzero(pre["n_touched"])[0]:
        x0, x1, y0, y1 = pre["bounds"][4 * i:4 * i + 4]
        a, b, c, o = pre["conic_opacity"][4 * i:4 * i + 4].astype(np.float64)
        mx, my = pre["mean2d"][2 * i:2 * i + 2].astype(np.float64)
        for ty in range(y0, y1):
            for tx in range(x0, x1):
                t = ty * gw + tx
                if (t, i) in kept:
                    continue
                px = np.arange(tx * 16, tx * 16 + 16) + 0.5
                py = np.arange(ty * 16, ty * 16 + 16) + 0.5
                dx = mx - px[None, :]
                dy = my - py[:, None]
                sig = 0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy
                alpha = o * np.exp(-sig)
                assert alpha.max() < 1 / 255 * (1 + 1e-4), (i, t, alpha.max())
                dropped_checked += 1
    assert dropped_checked > 10


def test_bin_matches_stable_sort_of_64bit_keys(orc):
    s = scenes.config1(seed=6, n=1024)
    pre = orc.preprocess(s, "f")
    bins = orc.bin(s, pre, "f")
    gw, gh = s.camera.grid
    # independent emission: every (tile, prim) passing the culling, index order
    tiles, prims = [], []
    for i in range(s.n):
        if pre["n_touched"][i] == 0:
            continue
        x0, x1, y0, y1 = pre["bounds"][4 * i:4 * i + 4]
        cand = [(ty * gw + tx) for ty in range(y0, y1) for tx in range(x0, x1)]
        got = set(bins["inst_tile"][bins["inst_prim"] == i].tolist())
        assert len(got) == pre["n_touched"][i]
        assert got.issubset(set(cand))
        tiles += sorted(got)
        prims += [i] * len(got)
    depth_bits = pre["depth"].astype(np.float32).view(np.uint32).astype(np.uint64)
    keys = (np.array(tiles, np.uint64) << np.uint64(32)) | depth_bits[np.array(prims)]
    order = np.argsort(keys, kind="stable")
    assert np.array_equal(np.array(tiles)[order], bins["inst_tile"])
    assert np.array_equal(np.array(prims)[order], bins["inst_prim"])
    # ranges: linear scan
    r = bins["ranges"].reshape(-1, 2)
    for t in range(gw * gh):
        idx = np.nonzero(bins["inst_tile"] == t)[0]
        if len(idx) == 0:
            assert r[t, 0] == 0 and r[t, 1] == 0
        else:
            assert r[t, 0] == idx[0] and r[t, 1] == idx[-1] + 1 and len(idx) == idx[-1] + 1 - idx[0]


# ---------------------------------------------------------------- blend forward

def _blend_numpy(s, pre, bins):
    """Independent per-pixel front-to-back loop (double evaluation of the
    reference thresholds, kernels_forward.cuh:643-674)."""
    cam = s.camera
    gw, gh = cam.grid
    H, W = cam.height, cam.width
    img = np.zeros((H, W, 3))
    nc = np.zeros((H, W), np.int64)
    r = bins["ranges"].reshape(-1, 2)
    for y in range(H):
        for x in range(W):
            t = (y // 16) * gw + (x // 16)
            T, C = 1.0, np.zeros(3)
            for j in range(r[t, 1] - r[t, 0]):
                p = bins["inst_prim"][r[t, 0] + j]
                a, b, c, o = pre["conic_opacity"][4 * p:4 * p + 4].astype(np.float64)
                dx = pre["mean2d"][2 * p] - (x + 0.5)
                dy = pre["mean2d"][2 * p + 1] - (y + 0.5)
                sig = 0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy
                if sig < 0:
                    continue
                al = min(o * math.exp(-sig), 0.999)
                if al < 1 / 255:
                    continue
                if T * (1 - al) < 1e-4:
                    break
                C += T * al * np.maximum(pre["color"][3 * p:3 * p + 3], 0)
                T *= 1 - al
                nc[y, x] = j + 1
            img[y, x] = C
    return img, nc


def test_blend_forward_matches_bruteforce(orc):
    s = scenes.config1(seed=7, n=600)
    pre, bins, fwd = orc.render(s, "f")
    img, nc = _blend_numpy(s, pre, bins)
    got = to_hwc(fwd["image"], s.camera.shape)
    assert np.allclose(got, img, rtol=1e-5, atol=2e-6)
    idx = tiled_index(s.camera.shape)
    assert np.array_equal(fwd["n_contrib"][idx], nc)
    gw, gh = s.camera.grid
    for t in range(gw * gh):
        ty, tx = divmod(t, gw)
        assert fwd["tile_max"][t] == nc[ty * 16:ty * 16 + 16, tx * 16:tx * 16 + 16].max()


def test_blend_forward_padding_zeroed_and_odd_size(orc):
    s = scenes.config1(seed=8, n=300)
    cam = scenes.Camera(61, 45, 60.0, 60.0, 30.0, 22.0, s.camera.w2c)
    s = scenes.Scene(s.means, s.scales, s.rotations, s.opacities, s.sh0, s.sh_rest, 0, cam,
                     np.zeros(cam.shape.padded_size, np.float32))
    pre, bins, fwd = orc.render(s, "f")
    img, nc = _blend_numpy(s, pre, bins)
    assert np.allclose(to_hwc(fwd["image"], cam.shape), img, rtol=1e-5, atol=2e-6)
    mask = np.zeros(cam.shape.padded_size, bool)
    for c in range(3):
        mask[c * cam.shape.channel_stride + tiled_index(cam.shape)] = True
    assert np.all(fwd["image"][~mask] == 0)


# ---------------------------------------------------------------- gradients (finite differences)

def _fd_scene(seed=21, n=24, deg=3, size=32):
    rng = np.random.default_rng(seed)
    means = np.concatenate([rng.uniform(-0.6, 0.6, (n, 2)), rng.uniform(-0.4, 0.4, (n, 1))], 1).astype(np.float32)
    scales = rng.normal(-2.0, 0.25, (n, 3)).astype(np.float32)
    rots = rng.standard_normal((n, 4)).astype(np.float32)
    opac = rng.normal(-0.5, 0.8, n).astype(np.float32)
    sh0 = rng.uniform(0.2, 1.0, (n, 3)).astype(np.float32)
    shr = rng.normal(0, 0.2, (n, 15, 3)).astype(np.float32)
    w2c = scenes.look_at((0.4, -0.3, -3.0))
    cam = scenes.Camera(size, size, 40.0, 42.0, size / 2 + 0.3, size / 2 - 0.2, w2c)
    return scenes.Scene(means, scales, rots, opac, sh0, shr, deg, cam, np.zeros(cam.shape.padded_size, np.float32))


def _loss_d(orc, s, prm, weights):
    pre = orc.preprocess(s, "d", prm=prm)
    bins = orc.bin(s, pre, "d")
    fwd = orc.blend_forward(s, pre, bins, "d")
    return float(np.dot(fwd["image"], weights)), pre, bins, fwd


@pytest.mark.parametrize("seed", [21, 22])
def test_backward_matches_finite_differences(orc, seed):
    s = _fd_scene(seed)
    shape = s.camera.shape
    weights = np.random.default_rng(seed + 100).uniform(-1, 1, shape.padded_size)
    prm = orc.params(s, "d")
    L0, pre, bins, fwd = _loss_d(orc, s, prm, weights)
    g2d = orc.blend_backward(s, pre, bins, fwd, weights, "d", exact_grad=True)
    grads = orc.preprocess_backward(s, pre, g2d, "d", prm=prm, exact_grad=True)
    h = 1e-6
    checked = 0
    worst = 0.0
    for name in ("means", "scales", "rotations", "opacities", "sh0", "sh_rest"):
        arr = prm[name]
        idx = np.arange(arr.size)
        if name == "sh_rest":
            idx = idx[::7]
        for k in idx:
            p_ = dict(prm)
            a = arr.copy(); a[k] += h; p_[name] = a
            Lp = _loss_d(orc, s, p_, weights)[0]
            a = arr.copy(); a[k] -= h; p_[name] = a
            Lm = _loss_d(orc, s, p_, weights)[0]
            fd = (Lp - Lm) / (2 * h)
            # skip points where a threshold (tile cull, alpha cut, termination)
            # lies inside [-h, h]: one-sided differences disagree there
            if abs((Lp - L0) - (L0 - Lm)) > 1e-3 * (abs(Lp - L0) + abs(L0 - Lm)) + 1e-12:
                continue
            an = grads[name][k]
            # relative error, with a floor at 1e-3 of the group's largest
            # gradient where central differences carry roundoff ~1e-9
            err = abs(an - fd) / (abs(fd) + 1e-3 * np.abs(grads[name]).max() + 1e-9)
            worst = max(worst, err)
            assert err < 1e-4, (name, k, an, fd)
            checked += 1
    assert checked > 200


def test_quirk_alpha_below_threshold_enters_backward(orc):
    """Reference backward has no alpha >= 1/255 test (kernels_backward.cuh:864-871):
    a faint Gaussian in front of the last contributor receives a gradient and
    scales the transmittance seen by later Gaussians of the same bucket."""
    cam = scenes.Camera(16, 16, 16.0, 16.0, 8.0, 8.0, np.array([[1, 0, 0, 0], [0, 1, 0, 0], [0, 0, 1, 4.0], [0, 0, 0, 1]], float))
    # prim 0: faint (o ~ 1/300 -> culled entirely); make it just visible with
    # a steep fall-off so some pixels see alpha < 1/255 while the centre does not
    means = np.array([[0.0, 0.0, 0.0], [0.05, 0.0, 1.0]], np.float32)
    scales = np.array([[-1.6, -1.6, -1.6], [-0.3, -0.3, -0.3]], np.float32)
    rots = np.array([[1, 0, 0, 0], [1, 0, 0, 0]], np.float32)
    opac = np.array([-4.0, 0.5], np.float32)
    sh0 = np.array([[0.5, 0.5, 0.5], [1.0, 0.0, 0.0]], np.float32)
    s = scenes.Scene(means, scales, rots, opac, sh0, np.zeros((2, 15, 3), np.float32), 0, cam,
                     np.zeros(cam.shape.padded_size, np.float32))
    pre, bins, fwd = orc.render(s, "f")
    assert bins["n_instances"] == 2 and list(bins["inst_prim"]) == [0, 1]
    gimg = np.ones(cam.shape.padded_size, np.float32)
    ref = orc.blend_backward(s, pre, bins, fwd, gimg, "f", exact_grad=False)
    ex = orc.blend_backward(s, pre, bins, fwd, gimg, "f", exact_grad=True)
    # prim 1 sees T reduced by prim 0's sub-threshold alpha in the reference mode
    assert ref["grad_color"][3] < ex["grad_color"][3]
    # and prim 0 receives colour gradient from pixels where it was skipped
    assert ref["grad_color"][0] > ex["grad_color"][0]


def test_quirk_quaternion_gradient_scaled_by_inverse_norm(orc):
    """Reference quaternion gradient divides by |q|^3 (kernels_backward.cuh:332);
    the exact derivative has |q|^2. Equal for unit quaternions, ratio |q| otherwise."""
    s = _fd_scene(23)
    prm = orc.params(s, "d")
    w = np.random.default_rng(1).uniform(-1, 1, s.camera.shape.padded_size)
    pre, bins, fwd = orc.render(s, "d")
    g2d = orc.blend_backward(s, pre, bins, fwd, w, "d", exact_grad=False)
    ref = orc.preprocess_backward(s, pre, g2d, "d", prm=prm, exact_grad=False)
    ex = orc.preprocess_backward(s, pre, g2d, "d", prm=prm, exact_grad=True)
    qn = np.linalg.norm(s.rotations.astype(np.float64), axis=1)
    vis = pre["n_touched"] > 0
    r = ref["rotations"].reshape(-1, 4)[vis] * qn[vis, None]
    e = ex["rotations"].reshape(-1, 4)[vis]
    # det epsilon differs between the modes too; it is 1e-8 against det ~ 1e2
    assert np.allclose(r, e, rtol=1e-6, atol=1e-12)
    # unit quaternions: identical up to the determinant epsilon
    s1 = _fd_scene(23)
    s1.rotations[:] = s1.rotations / np.linalg.norm(s1.rotations, axis=1, keepdims=True)
    prm1 = orc.params(s1, "d")
    pre, bins, fwd = orc.render(s1, "d")
    g2d = orc.blend_backward(s1, pre, bins, fwd, w, "d")
    a = orc.preprocess_backward(s1, pre, g2d, "d", prm=prm1)["rotations"]
    b = orc.preprocess_backward(s1, pre, g2d, "d", prm=prm1, exact_grad=True)["rotations"]
    assert np.allclose(a, b, rtol=1e-6, atol=1e-12)


# ---------------------------------------------------------------- losses

def test_l1_closed_form(orc):
    shape = ImageShape(19, 13)
    rng = np.random.default_rng(4)
    pred = rng.uniform(-0.5, 1.5, shape.padded_size).astype(np.float32)
    targ = rng.uniform(0, 1, shape.padded_size).astype(np.float32)
    pred[5] = targ[5]
    loss, grad = orc.l1(pred, targ, shape, np.float32(0.8))
    s = np.float32(0.8) / np.float32(shape.size())
    d = np.clip(pred, 0, 1) - targ
    assert np.allclose(loss, np.abs(d) * s, rtol=1e-6)
    assert np.allclose(grad, np.where(d >= 0, 1, -1) * s)
    assert grad[5] == s  # sign(+0) = +1


def _ssim_double(pred_hwc, targ_hwc):
    """Brute-force SSIM map (Wang et al. 2004) with the 11x11 Gaussian window,
    sigma 1.5, zero padding, C1 = 1e-4, C2 = 9e-4."""
    g = np.exp(-(np.arange(11) - 5) ** 2 / (2 * 1.5 ** 2))
    g /= g.sum()
    w2 = np.outer(g, g)
    H, W = pred_hwc.shape
    P = np.pad(pred_hwc, 5)
    Tg = np.pad(targ_hwc, 5)
    out = np.zeros((H, W))
    for y in range(H):
        for x in range(W):
            a = P[y:y + 11, x:x + 11]
            b = Tg[y:y + 11, x:x + 11]
            m1, m2 = (w2 * a).sum(), (w2 * b).sum()
            s1 = (w2 * a * a).sum() - m1 * m1
            s2 = (w2 * b * b).sum() - m2 * m2
            s12 = (w2 * a * b).sum() - m1 * m2
            C1, C2 = 1e-4, 9e-4
            out[y, x] = ((2 * m1 * m2 + C1) * (2 * s12 + C2)) / ((m1 * m1 + m2 * m2 + C1) * (s1 + s2 + C2))
    return out


def test_ssim_window_weights_are_gaussian_sigma_1p5(orc):
    from oracle import oracle as O  # noqa: F401  (weights live in the C source)
    g = np.exp(-(np.arange(11) - 5) ** 2 / (2 * 1.5 ** 2))
    g /= g.sum()
    ref = np.array([0.001028380123898387, 0.0075987582094967365, 0.036000773310661316, 0.10936068743467331,
                    0.21300552785396576, 0.26601171493530273, 0.21300552785396576, 0.10936068743467331,
                    0.036000773310661316, 0.0075987582094967365, 0.001028380123898387])
    assert np.allclose(g, ref, rtol=1e-6)


def test_ssim_matches_bruteforce_and_fd(orc):
    shape = ImageShape(21, 17)
    rng = np.random.default_rng(5)
    targ = rng.uniform(0, 1, shape.padded_size)
    pred = np.clip(targ + rng.normal(0, 0.2, shape.padded_size), 0, 1)
    loss, grad = orc.ssim(pred, targ, shape, 1.0, prec="d")
    ref_map = np.stack([_ssim_double(to_hwc(pred, shape)[..., c], to_hwc(targ, shape)[..., c]) for c in range(3)], -1)
    got = to_hwc(loss, shape) * (shape.width * shape.height)
    assert np.allclose(got, 1 - ref_map, atol=1e-10)
    # gradient of total loss sum vs central differences
    def total(p):
        l, _ = orc.ssim(p, targ, shape, 1.0, prec="d")
        return l.sum()
    idx = tiled_index(shape)
    for (y, x, c) in [(0, 0, 0), (5, 7, 1), (16, 20, 2), (8, 10, 0), (3, 19, 1)]:
        k = c * shape.channel_stride + idx[y, x]
        h = 1e-6
        pp = pred.copy(); pp[k] += h
        pm = pred.copy(); pm[k] -= h
        fd = (total(pp) - total(pm)) / (2 * h)
        assert abs(grad[k] - fd) < 1e-6 * max(1.0, abs(fd)), (y, x, c, grad[k], fd)
    # float oracle stages its inputs in fp16 for the statistics only
    lf, gf = orc.ssim(pred.astype(np.float32), targ.astype(np.float32), shape, np.float32(1.0), prec="f")
    assert np.allclose(lf, loss, atol=5e-5)
    assert np.allclose(gf, grad, atol=5e-5)


# ---------------------------------------------------------------- adam

def test_adam_closed_form(orc):
    rng = np.random.default_rng(6)
    n = 1000
    theta = rng.standard_normal(n).astype(np.float32)
    grad = rng.standard_normal(n).astype(np.float32) * 3
    m1 = np.zeros(n, np.float32)
    m2 = np.zeros(n, np.float32)
    th0 = theta.copy()
    lr, b1, b2, eps, clip = np.float32(1e-2), 0.9, 0.999, 1e-15, 1.0
    for step in (1, 2, 3):
        bc1, bc2 = orc.bias_corrections(step, b1, b2)
        orc.lib().orc_f_adam(n, theta, grad, m1, m2, lr, b1, b2, eps, 1.0, bc1, bc2, clip, 0, 0, 0.0, 0)
    # double-precision Kingma & Ba with clipped gradient, same gradient each step
    g = np.clip(grad.astype(np.float64), -clip, clip)
    m = np.zeros(n)
    v = np.zeros(n)
    th = th0.astype(np.float64)
    b1f, b2f = float(np.float32(b1)), float(np.float32(b2))
    for step in (1, 2, 3):
        m = b1f * m + (1 - b1f) * g
        v = b2f * v + (1 - b2f) * g * g
        mh = m / (1 - b1f ** step)
        vh = np.sqrt(v) / np.sqrt(1 - b2f ** step)
        th = th - 1e-2 * mh / (vh + eps)
    assert np.allclose(theta, th, rtol=1e-5, atol=1e-6)
    assert np.allclose(m1, m, rtol=1e-5, atol=1e-7)


def test_adam_learning_rate_rules(orc):
    lrs = orc.adam_lrs({"means": 1.6e-4, "scene_scale": 2.0, "opacities": 5e-2, "rotations": 1e-3,
                        "scales": 5e-3, "shs": 5e-3})
    assert np.isclose(lrs["means"], 3.2e-4) and np.isclose(lrs["sh_rest"], 2.5e-4)
    assert np.isclose(lrs["sh0"], 5e-3)


# ---------------------------------------------------------------- pose-optimisation gradient

def test_pose_gradient_translation_matches_fd(orc):
    """dL/dw2c translation column (kernels_backward.cuh:256-269 summed as
    backward.cu:332-345) against central differences of the loss in the
    translation entries of w2c. With SH degree 0 the camera centre does not
    enter the image, so the mean path the reference differentiates is the
    whole derivative in t."""
    s = _fd_scene(31, deg=0)
    shape = s.camera.shape
    weights = np.random.default_rng(131).uniform(-1, 1, shape.padded_size)
    prm = orc.params(s, "d")
    cam = orc.cam_array(s.camera, "d")
    pre = orc.preprocess(s, "d", prm=prm, cam=cam)
    bins = orc.bin(s, pre, "d")
    fwd = orc.blend_forward(s, pre, bins, "d")
    g2d = orc.blend_backward(s, pre, bins, fwd, weights, "d", exact_grad=True)
    gw = np.zeros(16)
    orc.preprocess_backward(s, pre, g2d, "d", prm=prm, cam=cam, exact_grad=True, grad_w2c=gw)
    assert np.all(gw[3::4] == 0.0)   # row 3 of the gradient is zero

    def loss(c):
        p = orc.preprocess(s, "d", prm=prm, cam=c)
        b = orc.bin(s, p, "d")
        return float(np.dot(orc.blend_forward(s, p, b, "d")["image"], weights))

    h = 1e-6
    for k in range(3):
        cp, cm = cam.copy(), cam.copy()
        cp[6 + 4 * k + 3] += h
        cm[6 + 4 * k + 3] -= h
        fd = (loss(cp) - loss(cm)) / (2 * h)
        assert abs(gw[12 + k] - fd) <= 1e-5 * (abs(fd) + np.abs(gw).max()), (k, gw[12 + k], fd)


def test_pose_gradient_is_outer_product_of_mean_gradients(orc):
    """With SH degree 0 the mean gradient is R^T dL/dmean_cam, so the pose
    gradient's rotation block is sum_i (R dL/dmean_i) mean_i^T and its
    translation column sum_i R dL/dmean_i (a transposed or dropped factor
    fails this)."""
    s = _fd_scene(32, n=40, deg=0)
    weights = np.random.default_rng(132).uniform(-1, 1, s.camera.shape.padded_size)
    prm = orc.params(s, "d")
    pre = orc.preprocess(s, "d", prm=prm)
    bins = orc.bin(s, pre, "d")
    fwd = orc.blend_forward(s, pre, bins, "d")
    g2d = orc.blend_backward(s, pre, bins, fwd, weights, "d")
    gw = np.zeros(16)
    grads = orc.preprocess_backward(s, pre, g2d, "d", prm=prm, grad_w2c=gw)
    # R is the float32 rounding of a rotation (R R^T = I to ~5e-8), so the
    # identity holds to that relative accuracy
    R = s.camera.w2c[:3, :3].astype(np.float32).astype(np.float64)
    dc = grads["means"].reshape(-1, 3) @ R.T           # rows: R g_i
    m = prm["means"].reshape(-1, 3)
    G = gw.reshape(4, 4).T                               # row-major dL/dw2c
    tol = 1e-6 * np.abs(G).max()
    assert np.max(np.abs(G[:3, :3] - dc.T @ m)) < tol
    assert np.max(np.abs(G[:3, 3] - dc.sum(0))) < tol
    assert np.abs(G).max() > 0


def test_screen_radius_updated_per_32_primitive_group(orc):
    """kernels_forward.cuh:261-263,342-348: the screen radius is folded into the
    densification info by every thread of a 32-lane warp that has a thread
    still active after the depth / opacity / quaternion culls, culled or not;
    warps with none leave before it."""
    from helpers import culled_group_scene, screen_radius_double
    s = culled_group_scene()
    mr = np.zeros(s.n, np.float32)
    pre = orc.preprocess(s, "f", max_radii=mr)
    vis = pre["n_touched"] > 0
    assert not vis[32:64].any() and vis[80] and vis[:32].sum() > 10
    # a group with no active primitive is left untouched
    assert np.all(mr[32:64] == 0)
    checked = 0
    for i in list(range(0, 32)) + list(range(64, 160)):
        want = screen_radius_double(s, i)
        if want is None:      # q = 0 (NaN radius) or depth 0: fmaxf keeps the old 0 or takes inf
            assert mr[i] == 0 or np.isinf(mr[i]), (i, mr[i])
            continue
        assert abs(float(mr[i]) - want) <= 1.0, (i, mr[i], want)
        checked += 1
    assert checked > 90
    # culled primitives of live groups do get a radius
    for i in (3, 7, 11, 15, 19, 64, 65):
        assert not vis[i] and mr[i] > 0, i
    # folding is a running max: a second pass with a larger stored value keeps it
    mr2 = np.full(s.n, 1e6, np.float32)
    orc.preprocess(s, "f", max_radii=mr2)
    assert np.all(mr2 == 1e6)
