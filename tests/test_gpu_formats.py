"""PLY export / import and the image layout converters on the GPU against
the CPU restatement (oracle/formats.py): byte-exact files, bit-exact
parameters and pixels."""
import numpy as np
import pytest

from oracle import formats as FM

pytestmark = pytest.mark.gpu

F = np.float32


def _params(n, seed):
    g = np.random.default_rng(seed)
    p = {"means": g.normal(0, 1, (n, 3)).astype(F), "scales": g.normal(-4, 1, (n, 3)).astype(F),
         "rotations": g.normal(0, 1, (n, 4)).astype(F), "opacities": g.normal(0, 2, n).astype(F),
         "sh0": g.normal(0, 1.5, (n, 3)).astype(F), "sh_rest": g.normal(0, 0.2, (n, 45)).astype(F)}
    if n:
        p["sh0"][0] = [-10.0, 0.0, 10.0]
    return p


def _gaussians(p, sh_dtype):
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
    return g


def _stored(p, sh_dtype):
    """The parameters as stored (SH rounded to half in fp16 mode)."""
    q = dict(p)
    if sh_dtype == "float16":
        q["sh0"] = p["sh0"].astype(np.float16).astype(F)
        q["sh_rest"] = p["sh_rest"].astype(np.float16).astype(F)
    return q


def _bits(a):
    return np.ascontiguousarray(a, F).view(np.uint32)


@pytest.mark.parametrize("sh_dtype", ["float32", "float16"])
@pytest.mark.parametrize("n", [0, 1, 3, 1001])
def test_ply_save_matches_oracle_bytes(hip, tmp_path, sh_dtype, n):
    from tinygs_amd import io
    p = _params(n, n + 1)
    g = _gaussians(p, sh_dtype)
    for full in (False, True):
        f = tmp_path / f"g{int(full)}.ply"
        print(f"[ply_save] n={n} sh={sh_dtype} full={full}", flush=True)
        io.save_ply(str(f), g, full)
        assert f.read_bytes() == FM.ply_bytes(_stored(p, sh_dtype), full)


@pytest.mark.parametrize("sh_dtype", ["float32", "float16"])
def test_ply_round_trip_bit_exact(hip, tmp_path, sh_dtype):
    from tinygs_amd import io
    p = _params(4099, 7)
    g = _gaussians(p, sh_dtype)
    f = tmp_path / "full.ply"
    io.save_ply(str(f), g, True)
    info = io.ply_info(str(f))
    assert info["n_vertices"] == 4099 and info["has_gaussians"] and info["has_colors"]
    h = io.load_gaussians_ply(str(f), sh_dtype)
    for a, b in zip(g.tensors(), h.tensors()):
        assert a.dtype == b.dtype and a.shape == b.shape
        assert np.array_equal(a.cpu().numpy().view(np.uint8), b.cpu().numpy().view(np.uint8))
    part = tmp_path / "part.ply"
    io.save_ply(str(part), g, False)
    assert not io.ply_info(str(part))["has_gaussians"]
    with pytest.raises(RuntimeError, match="missing"):
        io.load_gaussians_ply(str(part))


@pytest.mark.parametrize("fmt", ["ascii", "binary_big_endian", "binary_little_endian"])
def test_ply_load_3dgs_names_any_order(hip, tmp_path, fmt):
    """A file with the common 3DGS names (f_dc_i, f_rest_i channel-major,
    rot_i), shuffled property order, double positions, extra properties and an
    element before the vertex element."""
    from tinygs_amd import io
    n = 257
    p = _params(n, 11)
    g = np.random.default_rng(12)
    cols = [("x", "double", p["means"][:, 0].astype(np.float64)), ("y", "double", p["means"][:, 1].astype(np.float64)),
            ("z", "float", p["means"][:, 2]), ("nx", "float", np.zeros(n, F)), ("opacity", "float", p["opacities"])]
    cols += [(f"scale_{k}", "float", p["scales"][:, k]) for k in range(3)]
    cols += [(f"rot_{k}", "float", p["rotations"][:, k]) for k in range(4)]
    cols += [(f"f_dc_{k}", "float", p["sh0"][:, k]) for k in range(3)]
    sh = p["sh_rest"].reshape(n, 15, 3)
    cols += [(f"f_rest_{c * 15 + k}", "float", sh[:, k, c]) for c in range(3) for k in range(15)]
    order = g.permutation(len(cols))
    f = tmp_path / "std.ply"
    FM.write_ply(str(f), [cols[i] for i in order], fmt, extra_elements=(("meta", 3, [("v", "uchar")]),))
    h = io.load_gaussians_ply(str(f))
    got = {"means": h.means(), "scales": h.scales(), "rotations": h.rotations(), "opacities": h.opacities(),
           "sh0": h.sh_coefficient_0(), "sh_rest": h.sh_coefficients_rest().reshape(n, 45)}
    for k, v in got.items():
        assert np.array_equal(_bits(v.cpu().numpy()), _bits(p[k].reshape(v.shape))), k


def _tiled(shape_hw, c, dtype):
    import torch
    w, h = shape_hw
    tw, th = (w + 7) // 8, (h + 7) // 8
    return torch.full((c * tw * th * 64,), 7, dtype=getattr(torch, dtype), device="cuda")


@pytest.mark.parametrize("wh", [(1, 1), (37, 21), (300, 17), (1920, 1080)])
@pytest.mark.parametrize("dtype", ["uint8", "float32", "float16"])
def test_image_converters_match_oracle(hip, wh, dtype):
    import torch
    from tinygs_amd import io
    from tinygs_amd.image import ImageShape
    w, h = wh
    rng = np.random.default_rng(w + h)
    for c, bgr in ((3, True), (3, False), (1, False), (4, False)):
        print(f"[image] {w}x{h} c={c} bgr={bgr} {dtype}", flush=True)
        shape = ImageShape(w, h, c)
        src = rng.integers(0, 256, (h, w, c)).astype(np.uint8)
        dst = _tiled(wh, c, dtype)
        io.from_cv2(dst, torch.from_numpy(src).cuda(), shape, bgr)
        want = FM.from_cv2(src, w, h, bgr, dtype)
        got = dst.cpu().numpy()
        assert got.dtype == want.dtype and np.array_equal(got.view(np.uint8), want.view(np.uint8))
        # back to HWC u8: exact for u8; for float / half the narrowing of the oracle
        out = torch.zeros((h, w, c), dtype=torch.uint8, device="cuda")
        io.to_cv2(out, dst, shape, bgr)
        assert np.array_equal(out.cpu().numpy(), FM.to_cv2(want, w, h, c, bgr))
        if dtype == "uint8":
            assert np.array_equal(out.cpu().numpy(), src)


def test_image_export_narrowing(hip):
    import torch
    from tinygs_amd import io
    from tinygs_amd.image import ImageShape
    w, h = 29, 11
    shape = ImageShape(w, h, 3)
    rng = np.random.default_rng(3)
    v = rng.uniform(-0.5, 1.5, shape.padded_size).astype(F)
    v[:5] = [np.nan, np.inf, -np.inf, 1.0, 0.999]
    src = torch.from_numpy(v).cuda()
    out = torch.zeros((h, w, 3), dtype=torch.uint8, device="cuda")
    io.to_cv2(out, src, shape)
    assert np.array_equal(out.cpu().numpy(), FM.to_cv2(v, w, h, 3, True))
    with pytest.raises(RuntimeError, match="3 channels"):
        io.to_cv2(torch.zeros((h, w, 4), dtype=torch.uint8, device="cuda"),
                  torch.zeros(ImageShape(w, h, 4).padded_size, device="cuda"), ImageShape(w, h, 4), bgr=True)


def test_convert_all_pairs(hip):
    import torch
    from tinygs_amd import io
    rng = np.random.default_rng(5)
    u8 = rng.integers(0, 256, 100003).astype(np.uint8)
    f32 = rng.uniform(-0.2, 1.2, 100003).astype(F)
    f32[:3] = [np.nan, 70000.0, 1e-8]   # 70000 overflows half to inf
    with np.errstate(over="ignore"):
        f16 = f32.astype(np.float16)
    host = {"uint8": u8, "float32": f32, "float16": f16}
    for s, a in host.items():
        for d in host:
            dst = torch.zeros(a.size, dtype=getattr(torch, d), device="cuda")
            io.convert(dst, torch.from_numpy(a).cuda())
            got = dst.cpu().numpy()
            if s == "uint8":
                want = FM.widen(a, d)
            elif d == "uint8":
                want = FM.narrow(a.astype(F))
            else:
                with np.errstate(over="ignore"):
                    want = a.astype(F).astype(np.float16 if d == "float16" else F)
            assert np.array_equal(got.view(np.uint8), want.view(np.uint8)) or \
                (np.array_equal(np.isnan(got.astype(F)), np.isnan(want.astype(F))) and
                 np.array_equal(np.nan_to_num(got.astype(F)), np.nan_to_num(want.astype(F)))), (s, d)
