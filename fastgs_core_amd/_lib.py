"""ctypes binding of libfastgs_hip.so (C ABI declared in include/fastgs_hip.h).

The structures below mirror the C structs field for field.  Every call
passes raw device pointers (``tensor.data_ptr()``) and the current HIP stream
of the tensors' device; the library never allocates or synchronises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_float, c_int32, c_int64, c_size_t, c_uint32, \
    c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libfastgs_hip.so")

FGS_OK = 0
FGS_ERR_INVALID_ARGUMENT = -1
FGS_ERR_LAUNCH = -2
FGS_ERR_UNSUPPORTED = -3
ABI_VERSION = 16


class PreprocessParams(Structure):
    _fields_ = [
        ("P", c_int32), ("degree", c_int32), ("max_sh_coeffs", c_int32),
        ("image_width", c_int32), ("image_height", c_int32), ("grid_x", c_int32),
        ("grid_y", c_int32), ("use_cov3d_precomp", c_int32), ("use_colors_precomp", c_int32),
        ("scale_modifier", c_float), ("mult", c_float), ("tan_fovx", c_float),
        ("tan_fovy", c_float),
    ]


class PreprocessFwdIO(Structure):
    _fields_ = [(n, c_void_p) for n in (
        "means3d", "dc", "sh", "colors_precomp", "opacities", "scales", "rotations",
        "cov3d_precomp", "viewmatrix", "projmatrix", "campos", "viewspace_in", "radii", "xys",
        "depths", "cov3d", "rgb", "conic_opacity", "tiles_touched", "clamped", "viewspace_out",
        "st_rec", "st_masks", "log_scales", "raw_rotations", "opacity_logits")]


class PreprocessBwdIO(Structure):
    _fields_ = [(n, c_void_p) for n in (
        "means3d", "scales", "rotations", "viewmatrix", "projmatrix", "campos", "sh",
        "cov3d_precomp", "cov3d_fwd", "radii", "clamped", "dL_dxys", "dL_drgb",
        "dL_dconic_opacity", "dL_dcov3d", "dL_dviewspace_out", "dL_dmeans3d", "dL_ddc", "dL_dsh",
        "dL_dcolors_precomp", "dL_dopacities", "dL_dscales", "dL_drotations",
        "dL_dviewspace_in", "quats_raw", "act_opacities", "dL_dlog_scales", "dL_dquats",
        "dL_dlogits", "log_scales", "opacity_logits")] + [("dL_dxys_stride", c_int64)]


class BinningIO(Structure):
    _fields_ = [
        ("P", c_int32), ("grid_x", c_int32), ("grid_y", c_int32), ("num_rendered", c_int64),
        ("mult", c_float),
    ] + [(n, c_void_p) for n in (
        "xys", "depths", "conic_opacity", "tiles_touched", "point_list_keys", "point_list",
        "ranges", "bucket_count", "bucket_offsets", "workspace", "depth_order", "st_rec",
        "st_masks", "wait_status", "host_result")]


class RasterParams(Structure):
    _fields_ = [
        ("image_width", c_int32), ("image_height", c_int32), ("num_channels", c_int32),
        ("num_tiles", c_int32), ("bucket_sum", c_int64), ("get_flag", c_int32),
        ("write_sampled", c_int32), ("num_points", c_int32), ("list_len", c_int64),
    ]


class RasterFwdIO(Structure):
    _fields_ = [(n, c_void_p) for n in (
        "ranges", "point_list", "bucket_offsets", "means2d", "colors", "conic_opacity",
        "background", "metric_map", "bucket_to_tile", "sampled_t", "sampled_ar", "final_t",
        "n_contrib", "max_contrib", "pixel_colors", "out_color", "metric_count", "n_iter")]


class RasterBwdIO(Structure):
    _fields_ = [(n, c_void_p) for n in (
        "ranges", "point_list", "means2d", "colors", "conic_opacity", "background", "final_t",
        "n_contrib", "max_contrib", "dL_dout_color", "dL_dmeans2d", "dL_dcolors",
        "dL_dconic_opacity", "dL_dviewspace", "tile_order")]


class AdamGroup(Structure):  # fgs_adam_group
    _fields_ = [("param", c_void_p), ("grad", c_void_p), ("exp_avg", c_void_p),
                ("exp_avg_sq", c_void_p), ("n", c_int64), ("lr", c_float), ("step", c_int32)]


class DensifyParams(Structure):
    _fields_ = [
        ("grad_thresh", c_float), ("grad_abs_thresh", c_float), ("clone_max_scale", c_float),
        ("importance_threshold", c_float), ("min_opacity", c_float), ("max_screen_size", c_float),
        ("world_max_scale", c_float), ("split_factor", c_int32),
    ]


class DensifyBuildIO(Structure):
    _fields_ = ([("P_new", c_int32), ("sh_row", c_int32), ("split_factor", c_int32),
                 ("reset_stats", c_int32), ("opacity_cap", c_float)]
                + [(n, c_void_p) for n in ("rows", "l2_src", "l2_kind", "l2_child", "normals",
                                           "means3d", "features_dc", "features_rest",
                                           "opacity_logits", "log_scales", "rotations")]
                + [("exp_avg", c_void_p * 6), ("exp_avg_sq", c_void_p * 6)]
                + [(n, c_void_p) for n in ("max_radii2d", "grad_accum", "grad_accum_abs", "denom",
                                           "tmp_radii", "d_means3d", "d_features_dc",
                                           "d_features_rest", "d_opacity_logits", "d_log_scales",
                                           "d_rotations")]
                + [("d_exp_avg", c_void_p * 6), ("d_exp_avg_sq", c_void_p * 6)]
                + [(n, c_void_p) for n in ("d_max_radii2d", "d_grad_accum", "d_grad_accum_abs",
                                           "d_denom", "d_tmp_radii")])


# Exported symbol -> (restype, argtypes).  The not-gpu test checks that the
# library exports every one of these and that include/fastgs_hip.h declares
# exactly this set.
SIGNATURES = {
    "fgs_last_error": (c_char_p, []),
    "fgs_abi_version": (c_int32, []),
    "fgs_preprocess_fwd": (c_int32, [POINTER(PreprocessParams), POINTER(PreprocessFwdIO), c_void_p]),
    "fgs_preprocess_bwd": (c_int32, [POINTER(PreprocessParams), POINTER(PreprocessBwdIO), c_void_p]),
    "fgs_preprocess_geometry_fwd": (c_int32, [POINTER(PreprocessParams), POINTER(PreprocessFwdIO),
                                              c_void_p]),
    "fgs_preprocess_colour_fwd": (c_int32, [POINTER(PreprocessParams), POINTER(PreprocessFwdIO),
                                            c_void_p]),
    "fgs_scan_workspace_bytes": (c_size_t, [c_int64]),
    "fgs_set_wait_spin_limit": (c_uint32, [c_uint32]),
    "fgs_set_launch_events": (c_int32, [c_char_p, c_void_p, c_void_p]),
    "fgs_inclusive_scan_u32": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p,
                                         c_void_p]),
    "fgs_inclusive_scan_u32_noalloc": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "fgs_duplicate_with_keys": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_float, c_int32, c_int32, c_int64, c_void_p,
                                          c_void_p, c_void_p]),
    "fgs_sort_workspace_bytes": (c_size_t, [c_int64]),
    "fgs_sort_pairs_u64": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32,
                                     c_int32, c_void_p, c_void_p, c_void_p]),
    "fgs_tile_ranges": (c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p]),
    "fgs_binning_workspace_bytes": (c_size_t, [c_int32, c_int64, c_int32]),
    "fgs_binning_sorted": (c_int32, [POINTER(BinningIO), c_void_p]),
    "fgs_depth_order_workspace_bytes": (c_size_t, [c_int32]),
    "fgs_depth_order": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fgs_rasterize_fwd": (c_int32, [POINTER(RasterParams), POINTER(RasterFwdIO), c_void_p]),
    "fgs_rasterize_bwd": (c_int32, [POINTER(RasterParams), POINTER(RasterBwdIO), c_void_p]),
    "fgs_fill_u32": (c_int32, [c_void_p, c_uint32, c_int64, c_void_p]),
    "fgs_l1_ssim_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "fgs_l1_ssim_fwd": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_float, c_float,
                                  c_void_p, c_void_p, c_void_p, c_void_p]),
    "fgs_l1_ssim_bwd": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                  c_int32, c_float, c_float, c_void_p, c_void_p]),
    "fgs_activations_fwd": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "fgs_activations_bwd": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fgs_adam_step": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_float, c_float,
                                c_float, c_float, c_int32, c_int32, c_void_p]),
    "fgs_adam_step_multi": (c_int32, [POINTER(AdamGroup), c_int32, c_float, c_float, c_float,
                                      c_int32, c_void_p]),
    "fgs_pointwise_loss_workspace_bytes": (c_size_t, [c_int64]),
    "fgs_pointwise_loss_fwd": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p,
                                         c_void_p, c_void_p]),
    "fgs_pointwise_loss_bwd": (c_int32, [c_void_p, c_void_p, c_int64, c_int32, c_void_p,
                                         c_void_p, c_void_p]),
    "fgs_densify_stats": (c_int32, [c_int32] + [c_void_p] * 7 + [c_void_p]),
    "fgs_densify_classify": (c_int32, [c_int32, POINTER(DensifyParams)] + [c_void_p] * 7
                             + [c_void_p]),
    "fgs_densify_layout": (c_int32, [c_int32, c_int32] + [c_void_p] * 5 + [c_void_p]),
    "fgs_densify_prune_keys": (c_int32, [c_int32, POINTER(DensifyParams), c_int32]
                               + [c_void_p] * 9 + [c_void_p]),
    "fgs_densify_select": (c_int32, [c_int32, c_int64, c_void_p, c_void_p, c_void_p]),
    "fgs_densify_keep_first": (c_int32, [c_int32, c_int64, c_void_p, c_void_p, c_void_p]),
    "fgs_invert_flags": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p]),
    "fgs_densify_compact": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fgs_densify_build": (c_int32, [POINTER(DensifyBuildIO), c_void_p]),
    "fgs_opacity_cap": (c_int32, [c_int32, c_float, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fgs_metric_map_workspace_bytes": (c_size_t, [c_int64]),
    "fgs_metric_map": (c_int32, [c_int32, c_int64, c_void_p, c_void_p, c_float, c_void_p,
                                 c_void_p, c_void_p, c_void_p]),
    "fgs_score_accumulate": (c_int32, [c_int32] + [c_void_p] * 4 + [c_void_p]),
    "fgs_score_finalize": (c_int32, [c_int32, c_int32] + [c_void_p] * 5 + [c_void_p]),
    "fgs_final_prune_mask": (c_int32, [c_int32, c_float, c_float] + [c_void_p] * 4
                             + [c_void_p]),
}

_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library (raises RuntimeError if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"fastgs_core_amd: HIP library not found at {path}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc, gfx950)")
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.fgs_abi_version() != ABI_VERSION:
        raise RuntimeError("fastgs_core_amd: libfastgs_hip.so ABI version mismatch; rebuild it")
    _lib = lib
    return lib


def check(code: int) -> None:
    """Map a C-ABI status code to the reference's exception classes."""
    if code == FGS_OK:
        return
    msg = (_lib.fgs_last_error() or b"").decode(errors="replace") if _lib else ""
    if code == FGS_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg or f"fastgs_core_amd: error {code}")
