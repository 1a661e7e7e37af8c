"""Shared helpers for the parity tests: run a scene through the HIP path (via
the C ABI) and through the CPU oracle, and compare with stated tolerances."""
from __future__ import annotations

import numpy as np

# Tolerances (north star: binning bit-exact, fp32 pixels within 1e-5 relative,
# gradients within 1e-4 relative).
PIXEL_RTOL = 1e-5
PIXEL_ATOL = 1e-7
GRAD_NORMWISE_RTOL = 1e-4      # max |gpu - cpu| <= 1e-4 * max |cpu| per parameter group


def gpu_render(scene, with_debug=True, densif=False):
    import torch
    from tinygs_amd.core import GPUGaussian3d, GPUBatchInput, Image, RasterizeContext
    from tinygs_amd.rasterizer import create_rasterizer
    g = GPUGaussian3d.from_scene(scene)
    r = create_rasterizer("fastgs")
    r.set_gaussians(g)
    ctx = RasterizeContext()
    ctx.fwd_input = GPUBatchInput.from_camera(scene.camera)
    ctx.fwd_output.image = Image.empty(scene.camera.shape)
    ctx.fwd_output.image.data.fill_(np.nan)   # padding must be written by the forward
    if densif:
        ctx.densification_info = torch.zeros((scene.n, 4), dtype=torch.float32, device="cuda")
    r.forward(ctx)
    torch.cuda.synchronize()
    out = {"r": r, "g": g, "ctx": ctx, "image": ctx.fwd_output.image.data.cpu().numpy()}
    if with_debug:
        dv = r.debug_view()
        out["dv"] = {k: (v.cpu().numpy() if hasattr(v, "cpu") else v) for k, v in dv.items()}
        out["n_contrib"] = r.debug_n_contrib(scene.camera.shape).cpu().numpy().view(np.uint32)
    return out


def gpu_backward(run, grad_image_np):
    import torch
    from tinygs_amd.core import Image
    ctx = run["ctx"]
    grads = run["g"].gradient_like()
    ctx.gaussians_grad = grads
    ctx.grad_output.image = Image(ctx.fwd_output.image.shape, "float32",
                                  torch.from_numpy(np.ascontiguousarray(grad_image_np, np.float32)).cuda())
    run["r"].backward(ctx)
    torch.cuda.synchronize()
    return {
        "means": grads.means().cpu().numpy().reshape(-1),
        "scales": grads.scales().cpu().numpy().reshape(-1),
        "rotations": grads.rotations().cpu().numpy().reshape(-1),
        "opacities": grads.opacities().cpu().numpy().reshape(-1),
        "sh0": grads.sh_coefficient_0().cpu().numpy().reshape(-1),
        "sh_rest": grads.sh_coefficients_rest().cpu().numpy().reshape(-1),
    }


def normwise_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.abs(b).max() if b.size else 0.0
    if scale == 0.0:
        return float(np.abs(a).max()) if a.size else 0.0
    return float(np.abs(a - b).max() / scale)


# Elementwise bar beside the normwise one: |gpu - cpu| <= 1e-4 |cpu| + atol_g
# per element, atol_g = GRAD_ELEM_ATOL_FRAC * max |cpu| of the group. The
# absolute part covers elements whose value is a sum with cancellation: the
# GPU sums each primitive's per-(primitive, bucket) records in the same fixed
# order as the oracle, but each record carries its own rounding (the hardware
# exp2 in the backward, another order of the pixel sums inside a bucket), and
# the absolute error of a cancelling sum scales with the group's largest
# terms, not with the (small) result. Measured worst cases: config 3 (1M,
# 1080p) log-scales, |d| = 3.7e-5 max|cpu| (one outlier Gaussian whose scale
# gradient sums ~1e5 cancelling pixel terms); config 2 (100k, 800x800)
# rotations, |d| up to 2.2e-5 max|cpu|. The p99 of the relative error over
# the elements above the floor is bounded as well (measured <= 1.4e-4).
GRAD_ELEM_RTOL = 1e-4
GRAD_ELEM_ATOL_FRAC = 6e-5
GRAD_P99_REL = 1e-3


def grad_error_stats(a, b, atol_frac=None):
    """normwise error, elementwise bar violations and the p99 / max relative
    error over elements with |ref| above the group's absolute floor."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.abs(b).max() if b.size else 0.0
    d = np.abs(a - b)
    atol = (GRAD_ELEM_ATOL_FRAC if atol_frac is None else atol_frac) * scale
    viol = int(np.count_nonzero(d > GRAD_ELEM_RTOL * np.abs(b) + atol))
    big = np.abs(b) > atol
    rel = d[big] / np.abs(b[big]) if big.any() else np.zeros(1)
    # the elements furthest over the relative part of the bar: (|d| / max|cpu|, |cpu| / max|cpu|)
    over = d - GRAD_ELEM_RTOL * np.abs(b)
    top = np.argsort(over)[-3:][::-1] if b.size else []
    worst = [(float(d[i] / scale) if scale else 0.0, float(abs(b[i]) / scale) if scale else 0.0) for i in top]
    return {"normwise": normwise_err(a, b), "violations": viol, "p99_rel": float(np.percentile(rel, 99)),
            "max_rel": float(rel.max()), "n": int(b.size), "worst": worst}


def assert_grads_close(gpu, ref, rtol=GRAD_NORMWISE_RTOL, groups=None, elementwise=True, atol_frac=None):
    """rtol: the normwise bar, a number or a per-group dict; atol_frac: the
    elementwise floor as a fraction of max |ref| (default GRAD_ELEM_ATOL_FRAC),
    a number or a per-group dict (groups it omits take the default)."""
    worst = {}
    for k in groups or gpu:
        st = grad_error_stats(gpu[k], ref[k], atol_frac.get(k) if isinstance(atol_frac, dict) else atol_frac)
        worst[k] = st["normwise"]
        print(f"[grads] {k}: normwise {st['normwise']:.2e}, p99 rel {st['p99_rel']:.2e}, max rel "
              f"{st['max_rel']:.2e}, elementwise violations {st['violations']} of {st['n']}; worst "
              f"(|d|, |ref|) / max|ref|: " + ", ".join(f"({x:.1e}, {y:.1e})" for x, y in st["worst"]), flush=True)
        bar = rtol[k] if isinstance(rtol, dict) else rtol
        assert st["normwise"] <= bar, (k, st, worst)
        if elementwise:
            assert st["violations"] == 0, (k, st)
            assert st["p99_rel"] <= GRAD_P99_REL, (k, st)
    return worst


def culled_group_scene():
    """160 Gaussians in five 32-primitive groups, built so that primitives the
    preprocess culls share a group with survivors:

    * group 0: survivors plus primitives behind the camera, beyond far, with
      opacity below 1/255, with |q|^2 below 1e-8 (radius still finite) and
      with q = 0 (radius NaN);
    * group 1: every primitive culled (behind the camera);
    * group 2: one survivor (index 80) among culled primitives;
    * group 3: unchanged;
    * group 4: one primitive at depth exactly 0.
    """
    from tinygs_amd import scenes
    s = scenes.config1(seed=9, n=160)
    means, rot, opac = s.means.copy(), s.rotations.copy(), s.opacities.copy()
    behind = [3, 7] + list(range(32, 64)) + [i for i in range(64, 96) if i % 2 == 0 and i != 80]
    means[behind, 2] = -4.0                       # depth -1
    opac[[11] + [i for i in range(64, 96) if i % 2 == 1 and i != 80]] = -9.0
    means[15, 2] = 197.0                           # depth 200 > far
    rot[19] = rot[19] * np.float32(1e-5)           # |q|^2 ~ 1e-10
    rot[23] = 0.0
    means[140, 2] = -3.0                           # depth exactly 0
    return scenes.Scene(means, s.scales, rot, opac, s.sh0, s.sh_rest, s.sh_degree, s.camera, s.target)


def screen_radius_double(scene, i):
    """ceil(3 sqrt(lambda_max)) of the dilated 2D covariance of primitive i, in
    double, with the reference's eigenvalue expression (kernels_forward.cuh:
    342-348) and its frustum clamp of the Jacobian (:298-307); None when the
    primitive's radius is not finite."""
    cam = scene.camera
    W = cam.w2c.astype(np.float64)
    t = W[:3, :3] @ scene.means[i].astype(np.float64) + W[:3, 3]
    q = scene.rotations[i].astype(np.float64)
    qn = float(q @ q)
    if qn == 0.0 or t[2] == 0.0:
        return None
    r, x, y, z = q / np.sqrt(qn)
    R = np.array([[1 - 2 * (y * y + z * z), 2 * (x * y - r * z), 2 * (x * z + r * y)],
                  [2 * (x * y + r * z), 1 - 2 * (x * x + z * z), 2 * (y * z - r * x)],
                  [2 * (x * z - r * y), 2 * (y * z + r * x), 1 - 2 * (x * x + y * y)]])
    S2 = np.diag(np.exp(2 * scene.scales[i].astype(np.float64)))
    Sig = R @ S2 @ R.T
    lx, rx = (-0.15 * cam.width - cam.cx) / cam.fx, (1.15 * cam.width - cam.cx) / cam.fx
    ty_, by_ = (-0.15 * cam.height - cam.cy) / cam.fy, (1.15 * cam.height - cam.cy) / cam.fy
    tx = min(max(t[0] / t[2], lx), rx)
    ty = min(max(t[1] / t[2], ty_), by_)
    J = np.array([[cam.fx / t[2], 0, -cam.fx / t[2] * tx], [0, cam.fy / t[2], -cam.fy / t[2] * ty]])
    c = J @ W[:3, :3] @ Sig @ W[:3, :3].T @ J.T + 0.3 * np.eye(2)
    det = c[0, 0] * c[1, 1] - c[0, 1] ** 2
    mid = 0.5 * (c[0, 0] + c[1, 1])
    l1 = mid + np.sqrt(max(0.1, mid * mid - det))
    l2 = mid - np.sqrt(max(0.1, mid * mid - det))
    lam = max(l1, l2)
    if not np.isfinite(lam) or lam < 0:
        return None
    return float(np.ceil(3 * np.sqrt(lam)))


def tile_centred_scene(k=12, seed=4):
    """k Gaussians per 16x16 tile of a 128x96 view, each projecting within
    3 px of its tile's centre with a footprint of a few pixels: every Gaussian
    lands in one tile, so the per-primitive sums of the fp32 blend backward
    have one record each and a training step is deterministic."""
    from tinygs_amd import scenes
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


def marked_slots(bits, masks, first_slot, n_instances):
    """Sorted record slots the fp32 backward marked: rank k < 32 of
    primitive p as bit k of masks[p] (slot first_slot[p] + k), the others as
    their slot's bit in bits."""
    I = int(n_instances)
    from_bits = np.nonzero(np.unpackbits(np.ascontiguousarray(bits, np.uint32).view(np.uint8),
                                         bitorder="little")[:I])[0].astype(np.int64)
    m = np.asarray(masks, np.uint32)
    p, k = np.nonzero((m[:, None] >> np.arange(32, dtype=np.uint32)) & 1)
    from_masks = first_slot[p].astype(np.int64) + k
    return np.sort(np.concatenate([from_bits, from_masks]))


def library_order_sums(records, bits, masks, first_slot, n_touched, n_instances):
    """The per-primitive sums of the 2D-gradient records (12 floats each) in
    the order the preprocess backward forms them on fp32 images: a
    primitive's marked slots (marked_slots) among [first_slot, first_slot +
    n_touched) in slot order; up to 16 records added one after another from
    0; above 16, the record at slot s = first_slot + k (rank k) goes to lane
    k mod 16 for k < 32 and otherwise to lane (s // 8 - (first_slot + 32) //
    8) mod 16, each lane adds its records in slot order from 0, and the lane
    sums are combined by an xor butterfly (partners 8, 4, 2, 1). Float32
    adds, so the result is bit-exact with the kernel's. Returns (n, 12)
    float32."""
    n = first_slot.size
    I = int(n_instances)
    out = np.zeros((n, 12), np.float32)
    if I == 0:
        return out
    marked = marked_slots(bits, masks, first_slot, I)
    if marked.size == 0:
        return out
    vis = np.nonzero(n_touched > 0)[0]
    order = vis[np.argsort(first_slot[vis].astype(np.int64), kind="stable")]
    starts = first_slot[order].astype(np.int64)
    owner = order[np.searchsorted(starts, marked, side="right") - 1]
    assert np.all(marked < first_slot[owner].astype(np.int64) + n_touched[owner]), "a mark outside its range"
    rec = records[marked].astype(np.float32)
    # marked slots ascend and each primitive's slots are contiguous: its marks form one run
    run_start = np.ones(marked.size, bool)
    run_start[1:] = owner[1:] != owner[:-1]
    first_idx = np.maximum.accumulate(np.where(run_start, np.arange(marked.size), 0))
    pos = np.arange(marked.size) - first_idx
    count = np.bincount(owner, minlength=n)
    light = count[owner] <= 16
    for q in range(16):
        sel = light & (pos == q)
        out[owner[sel]] += rec[sel]
    hv = ~light
    if hv.any():
        ho, hr = owner[hv], rec[hv]
        fs = first_slot[ho].astype(np.int64)
        k = marked[hv] - fs
        lane = np.where(k < 32, k, marked[hv] // 8 - (fs + 32) // 8) & 15
        heavy_ids, hid = np.unique(ho, return_inverse=True)
        key = hid * 16 + lane
        srt = np.argsort(key, kind="stable")          # slot order kept within a (primitive, lane)
        key, hr = key[srt], hr[srt]
        ks = np.ones(key.size, bool)
        ks[1:] = key[1:] != key[:-1]
        kpos = np.arange(key.size) - np.maximum.accumulate(np.where(ks, np.arange(key.size), 0))
        lanes = np.zeros((heavy_ids.size * 16, 12), np.float32)
        for q in range(int(kpos.max()) + 1):
            sel = kpos == q
            lanes[key[sel]] += hr[sel]
        v = lanes.reshape(-1, 16, 12)
        for m in (8, 4, 2, 1):
            v = v + v[:, np.arange(16) ^ m]
        out[heavy_ids] = v[:, 0]
    return out


def instance_ranks(inst_prim, n):
    """Each instance's rank among its primitive's instances, in instance order."""
    p = np.asarray(inst_prim, np.int64)
    if p.size == 0:
        return np.zeros(0, np.int64)
    srt = np.argsort(p, kind="stable")
    ps = p[srt]
    st = np.ones(ps.size, bool)
    st[1:] = ps[1:] != ps[:-1]
    r = np.arange(ps.size) - np.maximum.accumulate(np.where(st, np.arange(ps.size), 0))
    out = np.empty(p.size, np.int64)
    out[srt] = r
    return out
