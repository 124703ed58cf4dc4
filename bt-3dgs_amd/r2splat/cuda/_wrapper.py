"""Name-forwarders to the HIP operators, as in r2splat/cuda/_wrapper.py:8-39.

The seventeen operator names and signatures of the reference are kept; the
extra names at the end are fused passes used by ``r2splat.ops``.
"""

from __future__ import annotations

from typing import Callable


def _make_cuda_func(name: str) -> Callable:
    def call_cuda(*args, **kwargs):
        from ._backend import _C

        return getattr(_C, name)(*args, **kwargs)

    call_cuda.__name__ = name
    return call_cuda


isect_tiles = _make_cuda_func("isect_tiles")
parameter_transform_fwd = _make_cuda_func("parameter_transform_fwd")
parameter_transform_bwd = _make_cuda_func("parameter_transform_bwd")
isect_offset_encode = _make_cuda_func("isect_offset_encode")
isect_tiles_3d = _make_cuda_func("isect_tiles_3d")
isect_offset_encode_3d = _make_cuda_func("isect_offset_encode_3d")
conics_mu_fwd = _make_cuda_func("conics_mu_fwd")
conics_mu_bwd = _make_cuda_func("conics_mu_bwd")
world_to_image_projection_fwd = _make_cuda_func("world_to_image_projection_fwd")
world_to_image_projection_bwd = _make_cuda_func("world_to_image_projection_bwd")
world_to_volume_mapping_fwd = _make_cuda_func("world_to_volume_mapping_fwd")
world_to_volume_mapping_bwd = _make_cuda_func("world_to_volume_mapping_bwd")
rasterize_to_pixels_fwd = _make_cuda_func("rasterize_to_pixels_fwd")
rasterize_to_pixels_bwd = _make_cuda_func("rasterize_to_pixels_bwd")
rasterize_to_pixels_bwd_per_gaussian = _make_cuda_func("rasterize_to_pixels_bwd_per_gaussian")
voxelize_to_voxels_fwd = _make_cuda_func("voxelize_to_voxels_fwd")
voxelize_to_voxels_bwd = _make_cuda_func("voxelize_to_voxels_bwd")
voxelize_to_voxels_bwd_per_gaussian = _make_cuda_func("voxelize_to_voxels_bwd_per_gaussian")

# Fused passes (no reference counterpart; same arithmetic as the ops above).
prepare_gaussians = _make_cuda_func("prepare_gaussians")
project_gaussians_fwd = _make_cuda_func("project_gaussians_fwd")
project_gaussians_bwd = _make_cuda_func("project_gaussians_bwd")
opacity_bwd = _make_cuda_func("opacity_bwd")
mask_split = _make_cuda_func("mask_split")
densify_split = _make_cuda_func("densify_split")
densify_duplicate = _make_cuda_func("densify_duplicate")
densify_remove = _make_cuda_func("densify_remove")
projection_loss_fwd = _make_cuda_func("projection_loss_fwd")
projection_loss_bwd = _make_cuda_func("projection_loss_bwd")
tv_fwd = _make_cuda_func("tv_fwd")
tv_bwd = _make_cuda_func("tv_bwd")
hierarchy_loss_fwd = _make_cuda_func("hierarchy_loss_fwd")
hierarchy_loss_bwd = _make_cuda_func("hierarchy_loss_bwd")


def is_cuda_extension_available() -> bool:
    try:
        from ._backend import is_cuda_available

        return is_cuda_available()
    except ImportError:
        return False


__all__ = [name for name in globals() if not name.startswith("_")]
