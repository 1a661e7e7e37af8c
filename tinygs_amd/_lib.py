"""ctypes binding of the C ABI declared in include/tinygs_amd.h.

The library must be built in-tree (``python -m tinygs_amd.build``). There is
no fallback: every entry point raises when libtinygs_amd.so is missing.
torch is imported first so that the library binds to the HIP runtime torch
already loaded (both carry the soname libamdhip64.so.7); streams and device
pointers from torch are then valid inside the library.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtinygs_amd.so")

TGS_DTYPE_FLOAT32 = 0
TGS_DTYPE_FLOAT16 = 1
TGS_DTYPE_UINT8 = 2
TGS_ADAM_DEVICE_STEP = 1
TGS_ADAM_ROWS_UNMARKED = 2
TGS_ADAM_ROWS_MARKED = 4
TGS_ADAM_SAME_STEP = 8
TGS_LOSS_ASSIGN = 1
TGS_BACKWARD_ASSIGN = 1
TGS_BACKWARD_SPARSE = 2
TGS_BACKWARD_POSE = 4
TGS_BACKWARD_KEEP_2D = 8
TGS_FORWARD_NO_SYNC = 1
TGS_OK = 0
TGS_ERR_INVALID = 1
TGS_ERR_HIP = 2
TGS_ERR_STATE = 3
TGS_ERR_UNSUPPORTED = 4
TGS_ERR_CAPACITY = 5

_lib = None
_hip = None


class tgs_gaussians(C.Structure):
    _fields_ = [("means", C.c_void_p), ("scales", C.c_void_p), ("rotations", C.c_void_p),
                ("opacities", C.c_void_p), ("sh0", C.c_void_p), ("sh_rest", C.c_void_p),
                ("n", C.c_int64), ("sh_degree", C.c_int32), ("sh_dtype", C.c_int32), ("scene_scale", C.c_float)]


class tgs_camera(C.Structure):
    _fields_ = [("width", C.c_uint32), ("height", C.c_uint32), ("near_plane", C.c_float),
                ("far_plane", C.c_float), ("K", C.c_float * 9), ("w2c", C.c_float * 16)]


class tgs_debug_view(C.Structure):
    _fields_ = [("n_touched", C.c_void_p), ("bounds", C.c_void_p), ("mean2d", C.c_void_p),
                ("conic_opacity", C.c_void_p), ("color", C.c_void_p), ("depth_sorted_keys", C.c_void_p),
                ("depth_sorted_prims", C.c_void_p), ("instance_tiles", C.c_void_p), ("instance_prims", C.c_void_p),
                ("tile_ranges", C.c_void_p), ("n_contrib", C.c_void_p), ("tile_max", C.c_void_p),
                ("grad2d", C.c_void_p), ("n_visible", C.c_int64), ("n_instances", C.c_int64),
                ("n_tiles", C.c_int64), ("depth_key_base", C.c_uint32), ("image_dtype", C.c_uint32),
                ("first_slot", C.c_void_p), ("records", C.c_void_p), ("instance_ranks", C.c_void_p),
                ("record_bits", C.c_void_p)]


class tgs_pcg32(C.Structure):
    _fields_ = [("state", C.c_uint64), ("inc", C.c_uint64)]


class tgs_loss_context(C.Structure):
    _fields_ = [("pred", C.c_void_p), ("target", C.c_void_p), ("loss", C.c_void_p), ("grad", C.c_void_p),
                ("width", C.c_uint32), ("height", C.c_uint32), ("channel", C.c_uint32), ("dtype", C.c_int32)]


class tgs_adam_params(C.Structure):
    _fields_ = [("beta1", C.c_float), ("beta2", C.c_float), ("epsilon", C.c_float), ("means_lr", C.c_float),
                ("shs_lr", C.c_float), ("opacities_lr", C.c_float), ("scales_lr", C.c_float),
                ("rotations_lr", C.c_float), ("max_grad_1", C.c_float), ("opacities_l1", C.c_float),
                ("scales_l1", C.c_float), ("decay_mean", C.c_int32)]


class tgs_ply_info(C.Structure):
    _fields_ = [("n_vertices", C.c_int64), ("format", C.c_int32), ("has_gaussians", C.c_int32),
                ("has_colors", C.c_int32)]


P = C.c_void_p
PP = C.POINTER(C.c_void_p)

SIGNATURES = {
    "tgs_last_error": ([], C.c_char_p),
    "tgs_version": ([], C.c_int),
    "tgs_rasterizer_create": ([C.c_char_p, PP], C.c_int),
    "tgs_rasterizer_destroy": ([P], C.c_int),
    "tgs_rasterizer_set_gaussians": ([P, C.POINTER(tgs_gaussians)], C.c_int),
    "tgs_rasterizer_forward": ([P, C.POINTER(tgs_camera), P, C.c_int32, P, P], C.c_int),
    "tgs_rasterizer_forward_ex": ([P, C.POINTER(tgs_camera), P, C.c_int32, P, C.c_int32, P], C.c_int),
    "tgs_rasterizer_reserve": ([P, C.c_int64, C.c_int32, P], C.c_int),
    "tgs_rasterizer_status": ([P, C.c_int32, P], C.c_int),
    "tgs_rasterizer_backward": ([P, P, P, C.POINTER(tgs_gaussians), P, P], C.c_int),
    "tgs_rasterizer_backward_ex": ([P, P, P, C.POINTER(tgs_gaussians), P, C.c_int32, P], C.c_int),
    "tgs_rasterizer_counts": ([P, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.POINTER(C.c_int64)], C.c_int),
    "tgs_rasterizer_debug_view": ([P, C.POINTER(tgs_debug_view)], C.c_int),
    "tgs_loss_create": ([C.c_char_p, PP], C.c_int),
    "tgs_loss_destroy": ([P], C.c_int),
    "tgs_loss_evaluate": ([P, C.POINTER(tgs_loss_context), C.c_float, P], C.c_int),
    "tgs_loss_l1_ssim": ([P, C.POINTER(tgs_loss_context), C.c_float, C.c_float, C.c_int32, P], C.c_int),
    "tgs_adam_create": ([C.POINTER(tgs_gaussians), C.POINTER(tgs_gaussians), PP], C.c_int),
    "tgs_adam_destroy": ([P], C.c_int),
    "tgs_adam_set_params": ([P, C.POINTER(tgs_adam_params)], C.c_int),
    "tgs_adam_get_params": ([P, C.POINTER(tgs_adam_params)], C.c_int),
    "tgs_adam_set_lr": ([P, C.c_float], C.c_int),
    "tgs_adam_get_lr": ([P], C.c_float),
    "tgs_adam_set_gaussians": ([P, C.POINTER(tgs_gaussians), C.POINTER(tgs_gaussians)], C.c_int),
    "tgs_adam_step": ([P, C.c_float, P], C.c_int),
    "tgs_adam_step_masked": ([P, C.c_float, P, P], C.c_int),
    "tgs_rasterizer_grad_row_mask": ([P, PP], C.c_int),
    "tgs_rasterizer_backward_rows": ([P, PP, P], C.c_int),
    "tgs_rasterizer_grad_w2c": ([P, C.POINTER(C.c_float), P], C.c_int),
    "tgs_adam_reset": ([P, P], C.c_int),
    "tgs_adam_global_steps": ([P], C.c_int64),
    "tgs_adam_moments": ([P, C.c_int32, C.POINTER(C.c_void_p), C.POINTER(C.c_void_p)], C.c_int),
    "tgs_adam_gather": ([P, P, C.c_int64, P], C.c_int),
    "tgs_adam_append": ([P, C.c_int64, P], C.c_int),
    "tgs_adam_reset_opacity": ([P, P], C.c_int),
    "tgs_adam_reset_rows": ([P, P, C.c_int64, P], C.c_int),
    "tgs_adam_reorder": ([P, P, P], C.c_int),
    "tgs_gaussians_reorder": ([C.POINTER(tgs_gaussians), P, P], C.c_int),
    "tgs_morton_order": ([P, C.c_int64, P, P], C.c_int),
    "tgs_densification_reorder": ([P, P, P, C.c_int64, P], C.c_int),
    "tgs_pcg32_seed": ([C.POINTER(tgs_pcg32), C.c_uint64, C.c_uint64], None),
    "tgs_pcg32_next_uint": ([C.POINTER(tgs_pcg32), C.c_uint32], C.c_uint32),
    "tgs_psnr": ([C.POINTER(tgs_loss_context), C.POINTER(C.c_float), P], C.c_int),
    "tgs_random_logistic": ([C.POINTER(tgs_pcg32), C.c_int64, P, C.c_float, C.c_float, P], C.c_int),
    "tgs_densify_select": ([C.POINTER(tgs_gaussians), P, C.c_float, C.c_float, C.c_int32, P, P,
                            C.POINTER(C.c_int64), C.POINTER(C.c_int64), P], C.c_int),
    "tgs_densify_apply": ([C.POINTER(tgs_gaussians), C.c_int64, P, C.c_int64, P, P, P], C.c_int),
    "tgs_prune_select": ([C.POINTER(tgs_gaussians), P, C.c_int64, C.c_float, C.c_float, C.c_float, C.c_int32, P, P,
                          C.POINTER(C.c_int64), P], C.c_int),
    "tgs_gaussians_gather": ([C.POINTER(tgs_gaussians), C.POINTER(tgs_gaussians), P, P], C.c_int),
    "tgs_flags_compact": ([P, C.c_int64, P, C.POINTER(C.c_int64), P], C.c_int),
    "tgs_flags_compact_noalloc": ([P, C.c_int64, P, C.POINTER(C.c_int64), P], C.c_int),
    "tgs_reset_opacity": ([C.POINTER(tgs_gaussians), C.c_float, P], C.c_int),
    "tgs_ply_save": ([C.c_char_p, C.POINTER(tgs_gaussians), C.c_int32, P], C.c_int),
    "tgs_ply_read_info": ([C.c_char_p, C.POINTER(tgs_ply_info)], C.c_int),
    "tgs_ply_load_gaussians": ([C.c_char_p, C.POINTER(tgs_gaussians), P], C.c_int),
    "tgs_point_cloud_load": ([C.c_char_p, C.POINTER(C.c_int64), P, P], C.c_int),
    "tgs_image_from_hwc_u8": ([P, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32, P, C.c_int32, P], C.c_int),
    "tgs_image_to_hwc_u8": ([P, C.c_int32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_int32, P, P], C.c_int),
    "tgs_convert": ([P, C.c_int32, P, C.c_int32, C.c_int64, P], C.c_int),
    "tgs_profiling_set": ([C.c_uint32], C.c_int),
    "tgs_profiling_read": ([C.c_int32, C.POINTER(C.c_double), C.POINTER(C.c_int64), C.c_int32], C.c_int),
    "tgs_stage_name": ([C.c_int32], C.c_char_p),
    "tgs_rasterizer_work_stats": ([P, C.POINTER(C.c_int64), C.POINTER(C.c_int64), C.c_int32], C.c_int),
    "tgs_selftest_detmath": ([C.c_int32, P, P, C.c_int64, P], C.c_int),
    "tgs_selftest_wave": ([P, P, P], C.c_int),
    "tgs_selftest_half": ([C.c_int32, P, P, P, P, C.c_int64, P], C.c_int),
    "tgs_selftest_half_div_exhaustive": ([P, P], C.c_int),
    "tgs_selftest_half_div_blend": ([P, C.c_uint32, C.c_uint32, P], C.c_int),
    "tgs_selftest_lookback_spins": ([C.c_uint32], C.c_int),
    "tgs_selftest_clock": ([C.POINTER(C.c_double), P], C.c_int),
    "tgs_adam_step_ex": ([P, C.c_float, P, C.c_int32, P], C.c_int),
    "tgs_adam_device_steps": ([P, C.POINTER(C.c_int64), P], C.c_int),
}


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def load(path: str | None = None):
    """Load libtinygs_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    path = path or LIB_PATH
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python -m tinygs_amd.build` "
                           "(the HIP path has no CPU fallback)")
    import torch  # noqa: F401  -- bind to torch's HIP runtime first
    lib = C.CDLL(path)
    for name, (argt, rest) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argt
        fn.restype = rest
    _lib = lib
    return lib


def check(rc: int, what: str = ""):
    if rc != 0:
        msg = load().tgs_last_error().decode(errors="replace")
        raise RuntimeError(f"{what}: {msg}" if what else msg)


def hip():
    """The HIP runtime torch loaded (for raw device copies in tests)."""
    global _hip
    if _hip is None:
        import torch  # noqa: F401
        _hip = C.CDLL("libamdhip64.so.7")
        _hip.hipMemcpy.argtypes = [P, P, C.c_size_t, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    return _hip


def copy_device(ptr: int, nbytes: int, out):
    """Synchronous device-to-device copy of nbytes from a raw pointer into tensor ``out``."""
    import torch
    if nbytes == 0:
        return out
    torch.cuda.synchronize()
    rc = hip().hipMemcpy(C.c_void_p(out.data_ptr()), C.c_void_p(ptr), C.c_size_t(nbytes), 3)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy failed ({rc})")
    return out
