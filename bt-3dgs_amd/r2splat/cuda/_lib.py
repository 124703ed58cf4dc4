"""ctypes bindings of ``libr2splat_hip.so`` (declarations in include/r2splat_hip.h)."""

from __future__ import annotations

import ctypes
import os

__all__ = ["LIB_PATH", "load", "SYMBOLS", "Column", "SplitGeometry"]

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib",
                        "libr2splat_hip.so")

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_u32 = ctypes.c_uint32
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the f32/f64 pairs share argument kinds.
_FLOAT_OPS = {
    "parameter_transform_fwd": [_p, _p, _f64, _f64, _p, _p, _i64, _p],
    "parameter_transform_bwd": [_p, _p, _f64, _f64, _p, _p, _p, _i64, _p],
    "prepare_gaussians": [_p, _p, _p, _f64, _f64, _p, _p, _p, _i64, _p],
    "opacity_bwd": [_p, _p, _p, _p, _i64, _i64, _p],
    "explicit_backward_tail": [_p, _p, _p, _p, _u32, _u32, _f64, _p, _p, _p, _p, _p, _p, _p, _p,
                               _p, _p, _f64, _f64, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _p],
    "world_to_image_projection_fwd": [_p, _p, _p, _p, _u32, _u32, _f32, _f32, _p, _p, _p,
                                      _i64, _i64, _p],
    "world_to_image_projection_bwd": [_p, _p, _p, _p, _u32, _u32, _p, _p, _p, _p, _i64, _i64, _p],
    "conics_mu_fwd": [_p, _f64, _p, _p, _i64, _p],
    "conics_mu_bwd": [_p, _f64, _p, _p, _p, _p, _p, _i64, _p],
    "project_gaussians_fwd": [_p, _p, _p, _p, _p, _u32, _u32, _f64, _f32, _p, _p, _p, _p, _p,
                              _p, _i64, _i64, _p],
    "project_pack_fwd": [_p, _p, _p, _p, _p, _u32, _u32, _f64, _f32, _p, _p, _p, _p, _p, _p,
                         _p, _p, _p, _p, _p, _p, _i64, _i64, _p],
    "project_gaussians_bwd": [_p, _p, _p, _p, _u32, _u32, _f64, _p, _p, _p, _p, _p, _p, _p, _p,
                              _i64, _i64, _p],
    "isect_count_2d": [_p, _p, _i32, _i64, _i64, _u32, _u32, _u32, _p, _p, _p, _sz, _p],
    "isect_emit_sort_2d": [_p, _p, _i32, _i64, _i64, _u32, _u32, _u32, _p, _i64, _u32, _p, _p,
                           _p, _p, _p, _p, _sz, _p],
    "isect_count_3d": [_p, _p, _i64, _u32, _u32, _u32, _u32, _p, _p, _p, _sz, _p],
    "isect_emit_sort_3d": [_p, _p, _i64, _u32, _u32, _u32, _u32, _p, _i64, _u32, _p, _p, _p,
                           _p, _p, _p, _sz, _p],
    "rasterize_fwd": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _u32, _u32, _u32, _u32, _u32,
                      _p, _p, _sz, _p],
    "rasterize_fwd_noalloc": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _u32, _u32, _u32, _u32,
                              _u32, _p, _p],
    "rasterize_bwd": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _u32, _u32, _u32, _u32,
                      _u32, _p, _p, _p, _p, _p, _p],
    "rasterize_bwd_emit": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _u32, _u32,
                           _u32, _u32, _u32, _p, _p, _p, _p, _p, _p, _sz, _p],
    "rasterize_bwd_rows": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _u32, _u32, _u32,
                           _u32, _u32, _i32, _p, _sz, _p],
    "rasterize_bwd_reduce": [_p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _p],
    "rasterize_pack": [_p, _p, _p, _p, _i64, _i64, _p, _p, _p, _p, _p, _p, _p],
    "rasterize_fwd_packed": [_p, _p, _p, _i64, _i64, _i64, _u32, _u32, _u32, _u32, _u32, _p, _p,
                             _sz, _p],
    "rasterize_bwd_packed": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _u32, _u32,
                             _u32, _u32, _u32, _p, _p, _p, _p, _p, _i32, _p, _sz, _p],
    "rasterize_bwd_rows_packed": [_p, _p, _p, _p, _p, _i64, _p, _i64, _i64, _u32, _u32, _u32,
                                  _u32, _u32, _i32, _p, _sz, _p],
    "world_to_volume_mapping_fwd": [_p, _p, _p, _p, _u32, _u32, _u32, _f64, _f64, _p, _p, _p,
                                    _i64, _p],
    "world_to_volume_mapping_bwd": [_p, _p, _p, _p, _u32, _u32, _u32, _f64, _p, _p, _p, _p,
                                    _i64, _p],
    "voxelize_fwd": [_p, _p, _p, _p, _p, _i64, _i64, _u32, _u32, _u32, _u32, _u32, _u32, _u32,
                     _p, _p],
    "voxelize_bwd": [_p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32, _u32, _u32, _u32,
                     _u32, _p, _p, _p, _p],
    "voxelize_bwd_rows": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32, _u32, _u32,
                          _u32, _u32, _p, _sz, _p],
    "voxelize_bwd_reduce": [_p, _p, _i64, _i64, _p, _p, _p, _p],
    "voxelize_bwd_emit": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32, _u32,
                          _u32, _u32, _u32, _p, _p, _p, _p, _sz, _p],
    "isect_layer_counts_3d": [_p, _p, _i64, _u32, _u32, _u32, _u32, _p, _p, _sz, _p],
    "isect_count_3d_slab": [_p, _p, _i64, _u32, _u32, _u32, _u32, _u32, _u32, _p, _p, _p, _sz,
                            _p],
    "isect_emit_sort_3d_slab": [_p, _p, _i64, _u32, _u32, _u32, _u32, _u32, _u32, _p, _i64, _u32,
                                _p, _p, _p, _p, _p, _p, _sz, _p],
    "voxelize_fwd_slab": [_p, _p, _p, _p, _p, _i64, _i64, _u32, _u32, _u32, _u32, _u32, _u32,
                          _u32, _u32, _p, _p],
    "voxelize_fwd_reach": [_p, _p, _p, _p, _p, _i64, _i64, _u32, _u32, _u32, _u32, _u32, _u32,
                           _u32, _p, _p, _p],
    "voxelize_bwd_rows_reach": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32,
                                _u32, _u32, _u32, _u32, _p, _p, _sz, _p],
    "voxelize_bwd_emit_reach": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32,
                                _u32, _u32, _u32, _u32, _p, _p, _p, _p, _p, _sz, _p],
    "voxelize_bwd_rows_slab": [_p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32, _u32,
                               _u32, _u32, _u32, _u32, _p, _sz, _p],
    "voxelize_bwd_emit_slab": [_p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _i64, _u32, _u32, _u32,
                               _u32, _u32, _u32, _u32, _u32, _p, _p, _p, _p, _sz, _p],
}

_PLAIN = {
    "r2s_last_error": (ctypes.c_char_p, []),
    "r2s_abi_version": (_i32, []),
    "r2s_isect_workspace_bytes": (_i64, [_i64, _i64, _u32]),
    "r2s_isect_offset_encode": (_i32, [_p, _i64, _i64, _p, _p]),
    "r2s_isect_keys_from_offsets": (_i32, [_p, _i64, _i64, _p, _p]),
    "r2s_rasterize_workspace_bytes": (_i64, [_i64, _i64, _u32, _i32]),
    "r2s_rasterize_bwd_workspace_bytes": (_i64, [_i64, _i64, _i32]),
    "r2s_rasterize_payload_bytes": (_i64, [_i64, _i32]),
    "r2s_voxelize_bwd_workspace_bytes": (_i64, [_i64, _i32]),
    "r2s_mask_workspace_bytes": (_i64, [_i64]),
    "r2s_mask_split": (_i32, [_p, _i64, _p, _p, _p, _sz, _p]),
    "r2s_densify_split": (_i32, [_p, _i64, _p, _i64, _i64, _p, _p, _i32, _p]),
    "r2s_densify_duplicate": (_i32, [_p, _i64, _p, _i64, _i64, _p, _i32, _p]),
    "r2s_densify_remove": (_i32, [_p, _i64, _p, _i32, _p]),
    "r2s_projection_loss_workspace_bytes": (_i64, [_i64, _i32, _i32]),
    "r2s_projection_loss_fwd_f32": (_i32, [_p, _p, _p, _p, _i64, _i32, _i32, _i32, _p, _p, _sz,
                                           _p]),
    "r2s_projection_loss_bwd_f32": (_i32, [_p, _p, _p, _p, _i64, _i32, _i32, _i32, _p, _p, _sz,
                                           _p, _p]),
    "r2s_tv_workspace_bytes": (_i64, []),
    "r2s_tv_fwd_f32": (_i32, [_p, _i32, _i32, _i32, _i32, _p, _p, _sz, _p]),
    "r2s_tv_bwd_f32": (_i32, [_p, _i32, _i32, _i32, _i32, _p, _p, _p]),
    "r2s_adam_step_f32": (_i32, [_p, _i32, _p]),
    "r2s_hierarchy_workspace_bytes": (_i64, [_i64]),
    "r2s_hierarchy_loss_fwd_f32": (_i32, [_p, _p, _i64, _p, _p, _p, _i64, _f32, _p, _p, _sz, _p]),
    "r2s_hierarchy_loss_bwd_f32": (_i32, [_i64, _p, _p, _p, _sz, _p, _p]),
}



class Column(ctypes.Structure):
    """r2s_column_t: one column of the Gaussian table for the densify calls."""

    _fields_ = [("src", _p), ("dst", _p), ("extra", _p), ("rows", _i64), ("width", _i32),
                ("role", _i32)]


class SplitGeometry(ctypes.Structure):
    """r2s_split_geometry_t: live quats / raw scales and the scale activation."""

    _fields_ = [("quats", _p), ("raw_scales", _p), ("scale_min", _f32 * 3),
                ("scale_max", _f32 * 3), ("scale_eps", _f32), ("sigmoid_scales", _i32)]


class AdamTensor(ctypes.Structure):
    """r2s_adam_tensor_t: one parameter tensor of an Adam step."""

    _fields_ = [("param", _p), ("grad", _p), ("exp_avg", _p), ("exp_avg_sq", _p), ("n", _i64),
                ("lerp_weight", _f32), ("beta2", _f32), ("one_minus_beta2", _f32),
                ("weight_decay", _f32), ("bias_correction2_sqrt", _f32), ("eps", _f32),
                ("step_size", _f32)]


# Column roles (R2S_COL_* in include/r2splat_hip.h).
COL_COPY, COL_ZERO_NEW, COL_MEANS, COL_RAW_SCALES, COL_RAW_OPACITIES, COL_PARENT, COL_LEVEL, \
    COL_HISTORY = range(8)
DENSIFY_MAX_WIDTH = 16

SYMBOLS = sorted(list(_PLAIN) + [f"r2s_{n}_{s}" for n in _FLOAT_OPS for s in ("f32", "f64")])

ABI_VERSION = 10


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """dlopen the library and attach the C signatures of every exported symbol."""
    lib = ctypes.CDLL(path)
    for name, (res, args) in _PLAIN.items():
        fn = getattr(lib, name)
        fn.restype, fn.argtypes = res, args
    for name, args in _FLOAT_OPS.items():
        for suffix in ("f32", "f64"):
            fn = getattr(lib, f"r2s_{name}_{suffix}")
            fn.restype, fn.argtypes = _i32, args
    if lib.r2s_abi_version() != ABI_VERSION:
        raise RuntimeError(f"{path}: ABI version {lib.r2s_abi_version()} != {ABI_VERSION}")
    return lib
