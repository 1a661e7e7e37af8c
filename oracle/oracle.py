"""TEST INFRASTRUCTURE — ctypes front end of the CPU oracle (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product (tinygs_amd) never does.

``run_iteration`` chains the oracle stages the way tinygs's
Orchestrator::train_step does (tinygs/src/orchestrator.cu:335-439):
preprocess -> bin -> blend forward -> losses -> blend backward ->
preprocess backward -> SimpleAdam.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = C.CDLL(path)
        _declare(_LIB)
    return _LIB


def _declare(L):
    for pfx, rp in (("orc_f_", f32p), ("orc_d_", f64p)):
        R = C.c_float if pfx == "orc_f_" else C.c_double
        fn = getattr(L, pfx + "preprocess")
        fn.argtypes = [C.c_int64, rp, rp, rp, rp, rp, rp, C.c_int, rp, C.c_uint32, C.c_uint32,
                       u32p, u16p, rp, rp, rp, rp, rp, C.c_void_p]
        fn.restype = None
        fn = getattr(L, pfx + "bin")
        fn.argtypes = [C.c_int64, u32p, u16p, rp, rp, rp, rp, C.c_uint32, C.c_uint32, u32p,
                       C.POINTER(C.c_int64), u32p, u32p, C.c_int64, u32p]
        fn.restype = C.c_int64
        fn = getattr(L, pfx + "bucket_offsets")
        fn.argtypes = [C.c_uint32, C.c_uint32, u32p, u32p]
        fn.restype = C.c_int64
        fn = getattr(L, pfx + "blend_forward")
        fn.argtypes = [C.c_int, C.c_int, u32p, u32p, rp, rp, rp, rp, rp, u32p, u32p, u32p, C.c_void_p]
        fn.restype = None
        fn = getattr(L, pfx + "blend_backward")
        fn.argtypes = [C.c_int, C.c_int, u32p, u32p, rp, rp, rp, rp, rp, u32p, u32p, u32p, rp,
                       rp, rp, rp, rp, rp, C.c_int, C.c_int64, C.c_void_p]
        fn.restype = None
        fn = getattr(L, pfx + "preprocess_backward")
        fn.argtypes = [C.c_int64, rp, rp, rp, rp, C.c_int, rp, u32p, rp, rp, rp, rp,
                       rp, rp, rp, rp, rp, C.c_void_p, C.c_int, C.c_void_p]
        fn.restype = None
        fn = getattr(L, pfx + "l1")
        fn.argtypes = [C.c_int64, C.c_int64, rp, rp, C.c_void_p, C.c_void_p, R]
        fn.restype = None
        fn = getattr(L, pfx + "ssim")
        fn.argtypes = [C.c_int, C.c_int, rp, rp, C.c_void_p, C.c_void_p, R]
        fn.restype = None
        fn = getattr(L, pfx + "adam")
        fn.argtypes = [C.c_int64, rp, rp, rp, rp, R, R, R, R, R, R, R, R, C.c_int, C.c_int, R, C.c_int]
        fn.restype = None
    L.orc_half_op_array.argtypes = [C.c_int, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
    L.orc_half_op_array.restype = None
    L.orc_set_threads.argtypes = [C.c_int]
    L.orc_set_threads.restype = None
    L.orc_max_threads.argtypes = []
    L.orc_max_threads.restype = C.c_int
    for name, argt in (("orc_expf_array", [C.c_int64, f32p, f32p]), ("orc_exp2_core_array", [C.c_int64, f32p, f32p]),
                       ("orc_logf_array", [C.c_int64, f32p, f32p]),
                       ("orc_round_half_array", [C.c_int64, f32p, f32p]),
                       ("orc_half_bits_array", [C.c_int64, f32p, u16p])):
        getattr(L, name).argtypes = argt
        getattr(L, name).restype = None


def half_op(op, a, b=None, c=None):
    """The oracle's canonical half operation `op` (numbering of
    tgs_selftest_half) on uint16 bit-pattern arrays (float32 `a` for ops 7, 8,
    int64 for op 11)."""
    a = np.ascontiguousarray(a)
    n = a.size
    out = np.zeros(n, np.uint16)
    b = None if b is None else np.ascontiguousarray(b, np.uint16)
    c = None if c is None else np.ascontiguousarray(c, np.uint16)
    lib().orc_half_op_array(int(op), n, a.ctypes.data_as(C.c_void_p), _ptr(b), _ptr(c), out.ctypes.data_as(C.c_void_p))
    return out


def set_threads(n: int):
    """Threads of the oracle's parallel loops; results are identical for any count."""
    lib().orc_set_threads(int(n))


def max_threads() -> int:
    return int(lib().orc_max_threads())


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _dt(prec):
    return np.float32 if prec == "f" else np.float64


def expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_expf_array(x.size, x, y)
    return y


def exp2_core(x):
    """2^x for -150 <= x <= 0 (the blend forward's deterministic exp2)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_exp2_core_array(x.size, x, y)
    return y


def logf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_logf_array(x.size, x, y)
    return y


def half_bits(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_half_bits_array(x.size, x, y)
    return y


def round_half(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_round_half_array(x.size, x, y)
    return y


def cam_array(camera, prec="f"):
    a = camera.as_array().astype(np.float64)
    if prec == "d":
        a[6:18] = camera.w2c[:3, :].astype(np.float32).reshape(-1)
        a[18:21] = camera.cam_pos
    return np.ascontiguousarray(a, dtype=_dt(prec))


def params(scene, prec="f", overrides=None):
    dt = _dt(prec)
    p = {
        "means": scene.means, "scales": scene.scales, "rotations": scene.rotations,
        "opacities": scene.opacities, "sh0": scene.sh0, "sh_rest": scene.sh_rest,
    }
    if overrides:
        p.update(overrides)
    # always copies: Adam updates these arrays in place and must not touch the scene
    return {k: np.array(v, dtype=dt, copy=True).reshape(-1) for k, v in p.items()}


def preprocess(scene, prec="f", prm=None, cam=None, max_radii=None):
    L = lib()
    dt = _dt(prec)
    prm = prm or params(scene, prec)
    cam = cam if cam is not None else cam_array(scene.camera, prec)
    n = scene.n
    gw, gh = scene.camera.grid
    out = {
        "n_touched": np.zeros(n, np.uint32), "bounds": np.zeros(4 * n, np.uint16),
        "mean2d": np.zeros(2 * n, dt), "conic_opacity": np.zeros(4 * n, dt),
        "color": np.zeros(3 * n, dt), "power_thr": np.zeros(n, dt), "depth": np.zeros(n, dt),
    }
    bases = (scene.sh_degree + 1) ** 2
    getattr(L, f"orc_{prec}_preprocess")(
        n, prm["means"], prm["scales"], prm["rotations"], prm["opacities"], prm["sh0"], prm["sh_rest"],
        bases, cam, gw, gh, out["n_touched"], out["bounds"], out["mean2d"], out["conic_opacity"],
        out["color"], out["power_thr"], out["depth"], _ptr(max_radii))
    return out


def bin(scene, pre, prec="f"):
    L = lib()
    gw, gh = scene.camera.grid
    n = scene.n
    cap = int(pre["n_touched"].astype(np.int64).sum())
    out = {
        "sorted_prims": np.zeros(max(n, 1), np.uint32),
        "inst_tile": np.zeros(max(cap, 1), np.uint32), "inst_prim": np.zeros(max(cap, 1), np.uint32),
        "ranges": np.zeros(2 * gw * gh, np.uint32),
    }
    nv = C.c_int64(0)
    I = getattr(L, f"orc_{prec}_bin")(n, pre["n_touched"], pre["bounds"], pre["mean2d"], pre["conic_opacity"],
                                      pre["power_thr"], pre["depth"], gw, gh, out["sorted_prims"], C.byref(nv),
                                      out["inst_tile"], out["inst_prim"], cap, out["ranges"])
    assert I == cap, (I, cap)
    out["n_visible"] = nv.value
    out["n_instances"] = int(I)
    out["sorted_prims"] = out["sorted_prims"][: nv.value]
    out["inst_tile"] = out["inst_tile"][:I]
    out["inst_prim"] = out["inst_prim"][:I]
    return out


def blend_forward(scene, pre, bins, prec="f", with_ckpt=True):
    L = lib()
    dt = _dt(prec)
    cam = scene.camera
    gw, gh = cam.grid
    shape = cam.shape
    offs = np.zeros(gw * gh, np.uint32)
    nb = getattr(L, f"orc_{prec}_bucket_offsets")(gw, gh, bins["ranges"], offs)
    image = np.zeros(shape.padded_size, dt)
    ncontrib = np.zeros(shape.channel_stride, np.uint32)
    tmax = np.zeros(gw * gh, np.uint32)
    ckpt = np.zeros(max(nb, 1) * 256 * 4, dt) if with_ckpt else None
    getattr(L, f"orc_{prec}_blend_forward")(cam.width, cam.height, bins["ranges"], _u32(bins["inst_prim"]),
                                            pre["mean2d"], pre["conic_opacity"], pre["color"], pre["power_thr"],
                                            image, ncontrib, tmax, offs, _ptr(ckpt))
    return {"image": image, "n_contrib": ncontrib, "tile_max": tmax, "bucket_offsets": offs,
            "ckpt": ckpt, "n_buckets": int(nb)}


def _u32(a):
    return np.ascontiguousarray(a if a.size else np.zeros(1, np.uint32), dtype=np.uint32)


def first_slots(pre, bins) -> np.ndarray:
    """Each visible primitive's first instance slot: the exclusive scan of
    n_touched in depth order (the emission's offsets)."""
    n = pre["n_touched"].size
    fs = np.zeros(max(n, 1), np.uint32)
    order = np.asarray(bins["sorted_prims"], np.int64)
    nt = pre["n_touched"].astype(np.int64)[order]
    fs[order] = (np.cumsum(nt) - nt).astype(np.uint32)
    return fs


def blend_backward(scene, pre, bins, fwd, grad_image, prec="f", exact_grad=False, library_order=True):
    """library_order: each primitive's records summed in the library's fixed
    order (rank order up to 16 records, the 16-lane split by 8-slot bytes
    and xor butterfly above); otherwise in instance order."""
    L = lib()
    dt = _dt(prec)
    n = scene.n
    cam = scene.camera
    g = {k: np.zeros(m * n, dt) for k, m in
         (("grad_mean2d", 2), ("absgrad", 2), ("grad_conic", 3), ("grad_color", 3), ("grad_opacity", 1))}
    fs = first_slots(pre, bins) if library_order else None
    getattr(L, f"orc_{prec}_blend_backward")(
        cam.width, cam.height, bins["ranges"], _u32(bins["inst_prim"]), pre["mean2d"], pre["conic_opacity"],
        pre["color"], fwd["image"], np.ascontiguousarray(grad_image, dtype=dt), fwd["n_contrib"], fwd["tile_max"],
        fwd["bucket_offsets"], fwd["ckpt"], g["grad_mean2d"], g["absgrad"], g["grad_conic"], g["grad_color"],
        g["grad_opacity"], int(exact_grad), n, _ptr(fs))
    return g


def preprocess_backward(scene, pre, g2d, prec="f", prm=None, cam=None, exact_grad=False, densif=None,
                        grad_w2c=None):
    """grad_w2c: optional float array of 16 (column-major) that accumulates
    the pose gradient."""
    L = lib()
    dt = _dt(prec)
    n = scene.n
    prm = prm or params(scene, prec)
    cam = cam if cam is not None else cam_array(scene.camera, prec)
    out = {"means": np.zeros(3 * n, dt), "scales": np.zeros(3 * n, dt), "rotations": np.zeros(4 * n, dt),
           "sh0": np.zeros(3 * n, dt), "sh_rest": np.zeros(45 * n, dt)}
    bases = (scene.sh_degree + 1) ** 2
    getattr(L, f"orc_{prec}_preprocess_backward")(
        n, prm["means"], prm["scales"], prm["rotations"], prm["sh_rest"], bases, cam, pre["n_touched"],
        g2d["grad_mean2d"], g2d["grad_conic"], g2d["absgrad"], g2d["grad_color"],
        out["means"], out["scales"], out["rotations"], out["sh0"], out["sh_rest"], _ptr(densif), int(exact_grad),
        _ptr(grad_w2c))
    out["opacities"] = g2d["grad_opacity"].copy()
    return out


def l1(pred, target, shape, scale, loss=None, grad=None, prec="f"):
    dt = _dt(prec)
    loss = np.zeros(shape.padded_size, dt) if loss is None else loss
    grad = np.zeros(shape.padded_size, dt) if grad is None else grad
    getattr(lib(), f"orc_{prec}_l1")(shape.padded_size, shape.size(), np.ascontiguousarray(pred, dt),
                                     np.ascontiguousarray(target, dt), _ptr(loss), _ptr(grad), scale)
    return loss, grad


def ssim(pred, target, shape, scale, loss=None, grad=None, prec="f"):
    dt = _dt(prec)
    loss = np.zeros(shape.padded_size, dt) if loss is None else loss
    grad = np.zeros(shape.padded_size, dt) if grad is None else grad
    getattr(lib(), f"orc_{prec}_ssim")(shape.width, shape.height, np.ascontiguousarray(pred, dt),
                                       np.ascontiguousarray(target, dt), _ptr(loss), _ptr(grad), scale)
    return loss, grad


# SimpleAdam parameter groups in the order of simple_adam.cu:487-577:
# (name, lr attribute, lerp form, decay kind)
ADAM_GROUPS = (("means", "means", 0, 0), ("opacities", "opacities", 1, 1), ("rotations", "rotations", 0, 0),
               ("scales", "scales", 0, 2), ("sh0", "sh0", 0, 0), ("sh_rest", "sh_rest", 0, 0))


def adam_lrs(lr):
    """Per-group learning rates as SimpleAdam::step_adam forms them
    (simple_adam.cu:493,508,524,540,556,571): float products in that order."""
    f = np.float32
    g = f(lr.get("global", 1.0))
    return {
        "means": f(f(lr["means"]) * f(lr.get("scene_scale", 1.0))) * g,
        "opacities": f(lr["opacities"]) * g,
        "rotations": f(lr["rotations"]) * g,
        "scales": f(lr["scales"]) * g,
        "sh0": f(lr["shs"]) * g,
        "sh_rest": f(f(lr["shs"]) * f(0.05)) * g,
    }


def bias_corrections(step, beta1=0.9, beta2=0.999):
    b1 = float(np.float32(beta1))
    b2 = float(np.float32(beta2))
    return np.float32(1.0 - b1 ** step), np.float32(np.sqrt(1.0 - b2 ** step))


def adam_step(theta, grads, m1, m2, lr, step, grad_scale=1.0, beta1=0.9, beta2=0.999, eps=1e-15,
              max_grad=1.0, decay=None, sh_half=False):
    """In-place SimpleAdam step over the six groups (dicts of flat float32 arrays).
    sh_half: SH groups are stored as fp16 (results rounded to fp16)."""
    L = lib()
    bc1, bc2 = bias_corrections(step, beta1, beta2)
    lrs = adam_lrs(lr)
    decay = decay or {}
    for name, _, form, kind in ADAM_GROUPS:
        half = int(sh_half and name in ("sh0", "sh_rest"))
        L.orc_f_adam(theta[name].size, theta[name], np.ascontiguousarray(grads[name], np.float32), m1[name], m2[name],
                     lrs[name], beta1, beta2, eps, grad_scale, bc1, bc2, max_grad, form, kind,
                     float(decay.get(name, 0.0)), half)


def render(scene, prec="f", with_ckpt=True):
    pre = preprocess(scene, prec)
    bins = bin(scene, pre, prec)
    fwd = blend_forward(scene, pre, bins, prec, with_ckpt)
    return pre, bins, fwd


def run_iteration(scene, l1_w=0.8, ssim_w=0.2, grad_scaler=1.0, lr=None, step=1, adam_state=None,
                  eps=1e-15, max_grad=1.0):
    """One full training iteration on the CPU (float oracle). Returns a dict
    with the render, losses, gradients and the updated parameters."""
    shape = scene.camera.shape
    pre, bins, fwd = render(scene, "f")
    loss = np.zeros(shape.padded_size, np.float32)
    gimg = np.zeros(shape.padded_size, np.float32)
    if l1_w:
        l1(fwd["image"], scene.target, shape, np.float32(l1_w * grad_scaler), loss, gimg)
    if ssim_w:
        ssim(fwd["image"], scene.target, shape, np.float32(ssim_w * grad_scaler), loss, gimg)
    g2d = blend_backward(scene, pre, bins, fwd, gimg, "f")
    grads = preprocess_backward(scene, pre, g2d, "f")
    out = {"pre": pre, "bins": bins, "fwd": fwd, "loss": loss, "grad_image": gimg, "g2d": g2d, "grads": grads}
    if lr is not None:
        theta = params(scene, "f")
        st = adam_state or {k: (np.zeros_like(v), np.zeros_like(v)) for k, v in theta.items()}
        m1 = {k: v[0] for k, v in st.items()}
        m2 = {k: v[1] for k, v in st.items()}
        adam_step(theta, grads, m1, m2, lr, step, grad_scale=1.0 / grad_scaler, eps=eps, max_grad=max_grad,
                  sh_half=getattr(scene, "sh_dtype", "float32") == "float16")
        out["theta"], out["m1"], out["m2"] = theta, m1, m2
    return out


# ---------------------------------------------------------------- FGS16 (fp16 images)

u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")


def _declare_h(L):
    if getattr(L, "_h_declared", False):
        return
    L.orc_h_preprocess.argtypes = [C.c_int64, f32p, f32p, f32p, f32p, f32p, f32p, C.c_int, f32p, C.c_uint32,
                                   C.c_uint32, u32p, u16p, f32p, u16p, u16p, u8p, f32p, f32p, C.c_void_p]
    L.orc_h_preprocess.restype = None
    L.orc_h_bin.argtypes = [C.c_int64, u32p, u16p, f32p, u16p, f32p, f32p, C.c_uint32, C.c_uint32, u32p,
                            C.POINTER(C.c_int64), u32p, u32p, C.c_int64, u32p]
    L.orc_h_bin.restype = C.c_int64
    L.orc_h_blend_forward.argtypes = [C.c_int, C.c_int, u32p, u32p, f32p, u16p, u16p, u8p, u16p, u16p, u16p, u32p,
                                      C.c_void_p]
    L.orc_h_blend_forward.restype = None
    L.orc_h_blend_backward.argtypes = [C.c_int, C.c_int, u32p, u32p, f32p, u16p, u16p, u8p, u16p, u16p, u16p, u32p,
                                       u16p, f32p, u8p]
    L.orc_h_blend_backward.restype = None
    L.orc_h_reduce_records.argtypes = [C.c_int64, C.c_int64, u32p, f32p, u8p, f32p, f32p, f32p, f32p, f32p]
    L.orc_h_reduce_records.restype = None
    L._h_declared = True


def h_preprocess(scene, max_radii=None):
    """FGS16 preprocess (float inputs; SH in float)."""
    L = lib()
    _declare_h(L)
    prm = params(scene, "f")
    cam = cam_array(scene.camera, "f")
    n = scene.n
    gw, gh = scene.camera.grid
    out = {"n_touched": np.zeros(n, np.uint32), "bounds": np.zeros(4 * n, np.uint16),
           "mean2d": np.zeros(2 * n, np.float32), "conic": np.zeros(3 * n, np.uint16),
           "opacity": np.zeros(n, np.uint16), "rgb": np.zeros(3 * n, np.uint8),
           "power_thr": np.zeros(n, np.float32), "depth": np.zeros(n, np.float32)}
    L.orc_h_preprocess(n, prm["means"], prm["scales"], prm["rotations"], prm["opacities"], prm["sh0"],
                       prm["sh_rest"], (scene.sh_degree + 1) ** 2, cam, gw, gh, out["n_touched"], out["bounds"],
                       out["mean2d"], out["conic"], out["opacity"], out["rgb"], out["power_thr"], out["depth"],
                       _ptr(max_radii))
    return out


def h_bin(scene, pre):
    L = lib()
    _declare_h(L)
    gw, gh = scene.camera.grid
    n = scene.n
    cap = int(pre["n_touched"].astype(np.int64).sum())
    out = {"sorted_prims": np.zeros(max(n, 1), np.uint32), "inst_tile": np.zeros(max(cap, 1), np.uint32),
           "inst_prim": np.zeros(max(cap, 1), np.uint32), "ranges": np.zeros(2 * gw * gh, np.uint32)}
    nv = C.c_int64(0)
    I = L.orc_h_bin(n, pre["n_touched"], pre["bounds"], pre["mean2d"], pre["conic"], pre["power_thr"], pre["depth"],
                    gw, gh, out["sorted_prims"], C.byref(nv), out["inst_tile"], out["inst_prim"], cap, out["ranges"])
    assert I == cap, (I, cap)
    out["n_visible"] = nv.value
    out["n_instances"] = int(I)
    out["sorted_prims"] = out["sorted_prims"][: nv.value]
    out["inst_tile"] = out["inst_tile"][:I]
    out["inst_prim"] = out["inst_prim"][:I]
    return out


def h_blend_forward(scene, pre, bins):
    L = lib()
    _declare_h(L)
    cam = scene.camera
    gw, gh = cam.grid
    shape = cam.shape
    offs = np.zeros(gw * gh, np.uint32)
    nb = L.orc_f_bucket_offsets(gw, gh, bins["ranges"], offs)
    image = np.zeros(shape.padded_size, np.uint16)
    ncontrib = np.zeros(shape.channel_stride, np.uint16)
    tmax = np.zeros(gw * gh, np.uint16)
    ckpt = np.zeros(max(nb, 1) * 256 * 4, np.uint16)
    L.orc_h_blend_forward(cam.width, cam.height, bins["ranges"], _u32(bins["inst_prim"]), pre["mean2d"],
                          pre["conic"], pre["opacity"], pre["rgb"], image, ncontrib, tmax, offs,
                          ckpt.ctypes.data_as(C.c_void_p))
    return {"image": image, "n_contrib": ncontrib, "tile_max": tmax, "bucket_offsets": offs, "ckpt": ckpt,
            "n_buckets": int(nb)}


def h_render(scene):
    pre = h_preprocess(scene)
    bins = h_bin(scene, pre)
    return pre, bins, h_blend_forward(scene, pre, bins)


def h_blend_backward(scene, pre, bins, fwd, grad_image_h):
    """Per-instance records (12 floats; see orc_h_blend_backward) and their
    per-primitive reduction in the fp32 path's 2D-gradient layout."""
    L = lib()
    _declare_h(L)
    cam = scene.camera
    I = bins["n_instances"]
    rec = np.zeros(12 * max(I, 1), np.float32)
    has = np.zeros(max(I, 1), np.uint8)
    L.orc_h_blend_backward(cam.width, cam.height, bins["ranges"], _u32(bins["inst_prim"]), pre["mean2d"],
                           pre["conic"], pre["opacity"], pre["rgb"], fwd["image"],
                           np.ascontiguousarray(grad_image_h, np.uint16), fwd["tile_max"], fwd["bucket_offsets"],
                           fwd["ckpt"], rec, has)
    n = scene.n
    g = {k: np.zeros(m * n, np.float32) for k, m in
         (("grad_mean2d", 2), ("absgrad", 2), ("grad_conic", 3), ("grad_color", 3), ("grad_opacity", 1))}
    L.orc_h_reduce_records(n, I, _u32(bins["inst_prim"]), rec, has, g["grad_mean2d"], g["absgrad"],
                           g["grad_conic"], g["grad_color"], g["grad_opacity"])
    return {"records": rec[: 12 * I].reshape(I, 12) if I else rec[:0].reshape(0, 12), "has": has[:I], "g2d": g}


def h_preprocess_backward(scene, pre, g2d, densif=None):
    """The fp32 path's gradient chain (the reference's FGS16 preprocess
    backward is the same chain on half 2D gradients), with pre's fields as the
    chain reads them (n_touched only)."""
    return preprocess_backward(scene, {"n_touched": pre["n_touched"]}, g2d, "f", densif=densif)
