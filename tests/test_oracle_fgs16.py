"""Pins of the oracle's FGS16 restatement (oracle/fgs16_impl.inc) by checks
that do not retype it:

* preprocess against the fp32 oracle (itself pinned by closed-form EWA): the
  same mean2d, the conic rounded to nearest half by numpy, the 8-bit colour
  as saturate(c) * 255 truncated, the opacity sigmoid of the half logit;
* the half tile test against brute force over the tile's pixel centres in
  float64 (kept where the exact minimum power is clearly below the
  threshold, dropped where clearly above);
* binning: instances sorted by (tile, depth), n_touched per primitive;
* the blend forward against a float64 model of the FGS16 semantics (8-bit
  colour, alpha <= 0.99 and no 1/255 cut, transmittance stop, count of
  processed Gaussians);
* the blend backward's 2D gradients against central finite differences of
  that float64 model (the record scalings -1/255, -128/255, 1 and
  (1 - o) / 255, the half conic-b convention of the fp32 path);
* the per-primitive reduction: correctly rounded sums of the records'
  halves (numpy's float64 -> float16 conversion of exact sums).
"""
import numpy as np
import pytest

from tinygs_amd import scenes
from tinygs_amd.image import tiled_index, to_hwc


def _h(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def _small(seed=11, n=3000, w=118, h=86):
    return scenes.config2(seed=seed, n=n, width=w, height=h)


def test_fgs16_preprocess_against_fp32(orc):
    s = _small()
    p16 = orc.h_preprocess(s)
    p32 = orc.preprocess(s, "f")
    n = s.n
    both = (p16["n_touched"] > 0) & (p32["n_touched"] > 0)
    assert both.sum() > 500
    m16 = p16["mean2d"].reshape(n, 2)[both]
    m32 = p32["mean2d"].reshape(n, 2)[both]
    assert np.array_equal(m16.view(np.uint32), m32.view(np.uint32))
    conic32 = p32["conic_opacity"].reshape(n, 4)[both, :3].astype(np.float32)
    assert np.array_equal(p16["conic"].reshape(n, 3)[both], conic32.astype(np.float16).view(np.uint16))
    col32 = p32["color"].reshape(n, 3)[both].astype(np.float32)
    rgb = (np.clip(col32, 0, 1) * np.float32(255)).astype(np.uint8)
    assert np.array_equal(p16["rgb"].reshape(n, 3)[both], rgb)
    # opacity: sigmoid of the half-rounded logit, rounded to half (one half ulp
    # for the sigmoid's own rounding)
    lg = s.opacities.astype(np.float16).astype(np.float64)[both]
    want = 1.0 / (1.0 + np.exp(-lg))
    got = _h(p16["opacity"][both])
    assert np.all(np.abs(got - want) <= 2.0 ** -11 * want + 1e-7)
    assert np.allclose(p16["power_thr"][both], np.log(255.0 * got), rtol=1e-6, atol=1e-6)
    # visibility differs only through the half tile test / opacity: a few primitives
    diff = (p16["n_touched"] > 0) != (p32["n_touched"] > 0)
    assert diff.sum() <= 0.01 * both.sum()


def test_fgs16_logit_rounded_before_sigmoid(orc):
    """A logit whose float sigmoid passes the 1/255 cut but whose half-rounded
    value does not: culled by FGS16 (kernels_forward.cuh:314-322), kept by fp32."""
    base = scenes.config1(seed=3, n=1)
    cut = np.log(1 / 255 / (1 - 1 / 255))
    lo = None
    for k in range(1, 200):
        x = np.float32(cut + 2e-5 * k)
        hx = np.float16(x).astype(np.float64)
        if 1 / (1 + np.exp(-np.float64(x))) > (1 / 255) * (1 + 1e-5) and 1 / (1 + np.exp(-hx)) < (1 / 255) * (1 - 1e-5):
            lo = x
            break
    assert lo is not None
    s = scenes.Scene(np.array([[0.05, 0.03, 0.0]], np.float32), np.full((1, 3), -1.0, np.float32),
                     np.array([[1, 0, 0, 0]], np.float32), np.array([lo], np.float32),
                     np.full((1, 3), 0.5, np.float32), np.zeros((1, 15, 3), np.float32), 0, base.camera,
                     base.target)
    assert orc.preprocess(s, "f")["n_touched"][0] > 0
    assert orc.h_preprocess(s)["n_touched"][0] == 0


def test_fgs16_tile_test_against_bruteforce(orc):
    s = _small(seed=12, n=1500)
    pre = orc.h_preprocess(s)
    bins = orc.h_bin(s, pre)
    gw, gh = s.camera.grid
    kept = set(zip(bins["inst_tile"].tolist(), bins["inst_prim"].tolist()))
    clear_in = clear_out = 0
    conic = _h(pre["conic"]).reshape(-1, 3)
    for i in np.nonzero(pre["n_touched"])[0]:
        x0, x1, y0, y1 = pre["bounds"][4 * i:4 * i + 4]
        a, b, c = conic[i]
        pt = float(pre["power_thr"][i])
        mx, my = pre["mean2d"][2 * i:2 * i + 2].astype(np.float64)
        for ty in range(y0, y1):
            for tx in range(x0, x1):
                px = np.arange(tx * 16, tx * 16 + 16) + 0.5
                py = np.arange(ty * 16, ty * 16 + 16) + 0.5
                dx = mx - px[None, :]
                dy = my - py[:, None]
                pw = (0.5 * (a * dx * dx + c * dy * dy) + b * dx * dy).min()
                k = (ty * gw + tx, i) in kept
                if pw < 0.9 * pt - 0.05:
                    assert k, (i, tx, ty, pw, pt)
                    clear_in += 1
                elif pw > 1.1 * pt + 0.5:
                    assert not k, (i, tx, ty, pw, pt)
                    clear_out += 1
    assert clear_in > 200 and clear_out > 20, (clear_in, clear_out)


def test_fgs16_bin_sorted_and_complete(orc):
    s = _small(seed=13, n=2000)
    pre = orc.h_preprocess(s)
    bins = orc.h_bin(s, pre)
    t, p = bins["inst_tile"].astype(np.int64), bins["inst_prim"].astype(np.int64)
    assert np.all(np.diff(t) >= 0)
    d = pre["depth"][p].astype(np.float32).view(np.uint32).astype(np.int64)
    same = np.diff(t) == 0
    key = d * (s.n + 1) + p
    assert np.all(np.diff(key)[same] > 0)   # by depth, then index, inside a tile
    assert np.array_equal(np.bincount(p, minlength=s.n), pre["n_touched"])
    r = bins["ranges"].reshape(-1, 2)
    for tile in np.nonzero(r[:, 1] > r[:, 0])[0][:50]:
        assert np.all(t[r[tile, 0]:r[tile, 1]] == tile)


def _model_forward(scene, pre, bins, mean2d, conic, opac, rgb, weights=None):
    """float64 FGS16 blend: per pixel, the tile's depth-sorted list; alpha =
    min(o exp(-sigma), 0.99), no 1/255 cut; stop when T (1 - alpha) < 1e-4
    (not composited); count = Gaussians processed."""
    cam = scene.camera
    W, H = cam.width, cam.height
    gw, gh = cam.grid
    img = np.zeros((H, W, 3))
    nc = np.zeros((H, W), np.int64)
    ranges = bins["ranges"].reshape(-1, 2)
    for t in range(gw * gh):
        ty, tx = divmod(t, gw)
        ys = np.arange(ty * 16, min(ty * 16 + 16, H))
        xs = np.arange(tx * 16, min(tx * 16 + 16, W))
        if ys.size == 0 or xs.size == 0:
            continue
        X, Y = np.meshgrid(xs + 0.5, ys + 0.5)
        T = np.ones_like(X)
        C = np.zeros(X.shape + (3,))
        cnt = np.zeros(X.shape, np.int64)
        live = np.ones(X.shape, bool)
        for j in range(ranges[t, 0], ranges[t, 1]):
            q = bins["inst_prim"][j]
            dx = mean2d[q, 0] - X
            dy = mean2d[q, 1] - Y
            sig = 0.5 * (conic[q, 0] * dx * dx + conic[q, 2] * dy * dy) + conic[q, 1] * dx * dy
            al = np.minimum(opac[q] * np.exp(-sig), 0.99)
            nT = T * (1 - al)
            ok = live & (nT >= 1e-4)
            C += np.where(ok, T * al, 0.0)[..., None] * rgb[q][None, None, :]
            cnt += live
            T = np.where(ok, nT, T)
            live = ok
        img[ys[0]:ys[-1] + 1, xs[0]:xs[-1] + 1] = C
        nc[ys[0]:ys[-1] + 1, xs[0]:xs[-1] + 1] = cnt
    return img, nc


def _model_inputs(pre, n):
    return (pre["mean2d"].reshape(n, 2).astype(np.float64), _h(pre["conic"]).reshape(n, 3),
            _h(pre["opacity"]), pre["rgb"].reshape(n, 3).astype(np.float64) / 255.0)


def test_fgs16_blend_forward_against_float64_model(orc):
    s = scenes.config1(seed=7, n=500)
    pre, bins, fwd = orc.h_render(s)
    img, nc = _model_forward(s, pre, bins, *_model_inputs(pre, s.n))
    got = to_hwc(fwd["image"].view(np.float16).astype(np.float64), s.camera.shape)
    err = np.abs(got - img)
    print(f"[fgs16] half blend vs float64 model: max {err.max():.3e} mean {err.mean():.3e}")
    assert err.max() < 2.0 ** -8 and err.mean() < 2.0 ** -11
    idx = tiled_index(s.camera.shape)
    agree = fwd["n_contrib"][idx] == nc
    assert agree.mean() > 0.98, agree.mean()


def _fd_scene16(seed, n=10, size=32):
    rng = np.random.default_rng(seed)
    means = np.concatenate([rng.uniform(-0.5, 0.5, (n, 2)), rng.uniform(-0.3, 0.3, (n, 1))], 1).astype(np.float32)
    scales = rng.normal(-2.2, 0.2, (n, 3)).astype(np.float32)
    rots = rng.standard_normal((n, 4)).astype(np.float32)
    opac = rng.normal(-1.0, 0.4, n).astype(np.float32)   # no pixel reaches the transmittance stop
    sh0 = rng.uniform(0.2, 1.0, (n, 3)).astype(np.float32)
    w2c = scenes.look_at((0.3, -0.2, -3.0))
    cam = scenes.Camera(size, size, 40.0, 42.0, size / 2 + 0.3, size / 2 - 0.2, w2c)
    return scenes.Scene(means, scales, rots, opac, sh0, np.zeros((n, 15, 3), np.float32), 0, cam,
                        np.zeros(cam.shape.padded_size, np.float32))


@pytest.mark.parametrize("seed", [31, 32])
def test_fgs16_backward_against_finite_differences(orc, seed):
    s = _fd_scene16(seed)
    n = s.n
    shape = s.camera.shape
    pre, bins, fwd = orc.h_render(s)
    rng = np.random.default_rng(seed + 1)
    w_hwc = rng.uniform(-1, 1, (shape.height, shape.width, 3)).astype(np.float16).astype(np.float64)
    grad_img = np.zeros(shape.padded_size, np.float16)
    idx = tiled_index(shape)
    for c in range(3):
        grad_img[c * shape.channel_stride + idx] = w_hwc[..., c]
    ob = orc.h_blend_backward(s, pre, bins, fwd, grad_img.view(np.uint16))
    g = ob["g2d"]
    mean2d, conic, opac, rgb = _model_inputs(pre, n)
    logit = np.log(opac / (1 - opac))

    def loss(m=mean2d, cn=conic, lg=logit, cl=rgb):
        img, _ = _model_forward(s, pre, bins, m, cn, 1 / (1 + np.exp(-lg)), cl)
        return float((img * w_hwc).sum())

    fd = {k: np.zeros(v) for k, v in (("mean", (n, 2)), ("conic", (n, 3)), ("logit", n), ("color", (n, 3)))}
    h = 1e-4
    for q in range(n):
        for k in range(2):
            mp, mm = mean2d.copy(), mean2d.copy()
            mp[q, k] += h
            mm[q, k] -= h
            fd["mean"][q, k] = (loss(m=mp) - loss(m=mm)) / (2 * h)
        for k in range(3):
            cp, cm = conic.copy(), conic.copy()
            cp[q, k] += h * 1e-2
            cm[q, k] -= h * 1e-2
            fd["conic"][q, k] = (loss(cn=cp) - loss(cn=cm)) / (2 * h * 1e-2)
            lp, lm = rgb.copy(), rgb.copy()
            lp[q, k] += h
            lm[q, k] -= h
            fd["color"][q, k] = (loss(cl=lp) - loss(cl=lm)) / (2 * h)
        lp, lm = logit.copy(), logit.copy()
        lp[q] += h
        lm[q] -= h
        fd["logit"][q] = (loss(lg=lp) - loss(lg=lm)) / (2 * h)
    # the records' conic-b gradient is half of d/db (the fp32 path's convention,
    # which the 3D chain's dSigma2 formula expects)
    fd["conic"][:, 1] *= 0.5
    pairs = {"mean": g["grad_mean2d"].reshape(n, 2), "conic": g["grad_conic"].reshape(n, 3),
             "color": g["grad_color"].reshape(n, 3), "logit": g["grad_opacity"]}
    for k, an in pairs.items():
        e = np.abs(an - fd[k]).max() / np.abs(fd[k]).max()
        print(f"[fgs16] {k}: normwise {e:.2e}")
        assert e < 1.5e-2, (k, e)


def test_fgs16_reduce_records_correctly_rounded(orc):
    """Sums of random half records: the correctly rounded half of the exact
    sum (numpy's float64 -> float16 conversion of an exactly representable
    float64 sum), opacity as the float64 sum rounded to float."""
    import ctypes as C
    rng = np.random.default_rng(5)
    n, I = 200, 5000
    prim = rng.integers(0, n, I).astype(np.uint32)
    rec = np.zeros((I, 12), np.float32)
    rec[:, :10] = (rng.standard_normal((I, 10)) * np.exp(rng.uniform(-12, 6, (I, 10)))).astype(np.float16)
    rec[:, 10] = rng.standard_normal(I).astype(np.float32)
    has = (rng.random(I) < 0.9).astype(np.uint8)
    L = orc.lib()
    orc._declare_h(L)
    out = {k: np.zeros(m * n, np.float32) for k, m in
           (("grad_mean2d", 2), ("absgrad", 2), ("grad_conic", 3), ("grad_color", 3), ("grad_opacity", 1))}
    L.orc_h_reduce_records(n, I, prim, rec.reshape(-1), has, out["grad_mean2d"], out["absgrad"], out["grad_conic"],
                           out["grad_color"], out["grad_opacity"])
    sums = np.zeros((n, 10))
    op = np.zeros(n)
    for j in range(I):
        if has[j]:
            sums[prim[j]] += rec[j, :10].astype(np.float64)   # exact: few halves of bounded range
            op[prim[j]] += float(rec[j, 10])
    want = sums.astype(np.float16).astype(np.float32)
    got = np.concatenate([out["grad_mean2d"].reshape(n, 2), out["absgrad"].reshape(n, 2),
                          out["grad_conic"].reshape(n, 3), out["grad_color"].reshape(n, 3)], 1)
    assert np.array_equal(got, want)
    assert np.allclose(out["grad_opacity"], op.astype(np.float32), rtol=1e-6, atol=0)
    del C


def test_from_fixed_matches_numpy(orc):
    rng = np.random.default_rng(9)
    mag = rng.integers(0, 44, 1 << 16)
    s = (rng.integers(0, 1 << 62, 1 << 16) >> (62 - mag)) * rng.choice([-1, 1], 1 << 16)
    s = np.concatenate([s, [0, 1, -1, (65520 << 24) - 1, 65520 << 24, 3 << 23]]).astype(np.int64)
    got = orc.half_op(11, s)
    with np.errstate(over="ignore"):   # |s| < 2^53: exact doubles; beyond 65520 -> inf
        want = (s.astype(np.float64) * 2.0 ** -24).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want), np.count_nonzero(got != want)


def test_exp2_argument_one_multiply(orc):
    """The blend kernels scale the power by 16 RN(-log2 e) = -23.078125 in one
    multiply where the reference (and the oracle) multiply by 16, then by
    RN(-log2 e): the same half for every half input, and so the same exp2."""
    x = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    k = np.float16(-1.4426950409)
    big = (np.float16(16.0) * k).view(np.uint16)
    assert big == 0xcdc5 and float(np.float16(16.0) * k) == 16.0 * float(k)
    n = x.size
    two = orc.half_op(3, orc.half_op(3, x, np.full(n, np.float16(16.0).view(np.uint16))),
                      np.full(n, k.view(np.uint16)))
    one = orc.half_op(3, x, np.full(n, big, np.uint16))
    nan = (two & 0x7c00 == 0x7c00) & (two & 0x3ff != 0)
    assert np.array_equal(nan, (one & 0x7c00 == 0x7c00) & (one & 0x3ff != 0))
    assert np.array_equal(two[~nan], one[~nan])
    # and hence every exp2 the kernels evaluate
    assert np.array_equal(orc.half_op(0, two[~nan]), orc.half_op(0, one[~nan]))
