"""The r2splat.ops composition restated on the CPU oracle (test infrastructure only).

Follows r2splat/ops/direct.py:72-322 (forward passes) and
r2splat/ops/explicit.py:233-385 (explicit backward), calling the numpy and C
restatements of each operator.  All arrays are numpy, in the inputs' dtype.
"""

from __future__ import annotations

import numpy as np

from . import binning, native, ops


def prepare(quats, raw_scales, raw_opacities, scale_min, scale_max):
    """direct.py:72-96 -> (covars, max_scales, opacities)."""
    covars, max_scales = ops.parameter_transform_fwd(quats, raw_scales, scale_min, scale_max)
    return covars, max_scales, ops.softplus(raw_opacities)


def rasterize_forward(means, covars, opacities, viewmats, Ks, img_w, img_h, tile_size, eps2d,
                      radius_clip):
    """direct.py:117-198 -> dict of the ProjectionForwardBuffers fields."""
    means2d, cov2d, radii = ops.world_to_image_projection_fwd(
        means, covars, viewmats, Ks, img_w, img_h, eps2d, radius_clip)
    conics, mus = ops.conics_mu_fwd(cov2d, eps2d)
    C, N = viewmats.shape[0], means.shape[0]
    opacity = np.ascontiguousarray(np.broadcast_to(opacities, (C, N)))
    tw = (img_w + tile_size - 1) // tile_size
    th = (img_h + tile_size - 1) // tile_size
    _, isect_ids, flatten_ids = binning.isect_tiles(means2d, radii, tile_size, tw, th)
    tile_offsets = binning.isect_offset_encode(isect_ids, C, tw, th)
    image = native.raster_fwd(means2d, conics, opacity, mus, tile_offsets, flatten_ids, img_w,
                              img_h, tile_size)
    return dict(output=image, means2d=means2d, cov2d=cov2d, conics=conics, mus=mus,
                opacity=opacity, radii=radii, tile_offsets=tile_offsets,
                flatten_ids=flatten_ids, isect_ids=isect_ids, viewmats=viewmats, Ks=Ks,
                img_w=img_w, img_h=img_h, tile_size=tile_size, eps2d=eps2d)


def voxelize_forward(means, covars, opacities, ranges, centers, dim2, dim1, dim0, tile_size,
                     eps3d, radius_clip):
    """direct.py:233-322 -> dict of the VoxelForwardBuffers fields."""
    means3d, conics, radii = ops.world_to_volume_mapping_fwd(
        means, covars, ranges, centers, dim2, dim1, dim0, eps3d, radius_clip)
    n2 = (dim2 + tile_size - 1) // tile_size
    n1 = (dim1 + tile_size - 1) // tile_size
    n0 = (dim0 + tile_size - 1) // tile_size
    _, isect_ids, flatten_ids = binning.isect_tiles_3d(means3d, radii, tile_size, n2, n1, n0)
    tile_offsets = binning.isect_offset_encode_3d(isect_ids, n2, n1, n0)
    volume = native.voxel_fwd(means3d, conics, opacities, tile_offsets, flatten_ids, dim2, dim1,
                              dim0, tile_size)
    return dict(output=volume, means3d=means3d, conics=conics, opacity=opacities, radii=radii,
                tile_offsets=tile_offsets, flatten_ids=flatten_ids, isect_ids=isect_ids,
                ranges=ranges, centers=centers, dim2=dim2, dim1=dim1, dim0=dim0,
                tile_size=tile_size, eps3d=eps3d)


def explicit_backward(covars, proj, vox, means, quats, raw_scales, raw_opacities, scale_min,
                      scale_max, v_image, v_volume=None, absgrad=True):
    """explicit.py:233-385 -> dict of gradients (means, quats, raw_scales,
    raw_opacities, means2d, means2d_abs)."""
    dt = means.dtype
    v_means = np.zeros_like(means)
    v_covars = np.zeros_like(covars)
    v_opacity = np.zeros(means.shape[0], dt)
    v_abs, v_means2d, v_conics, v_opac_cn, v_mus = native.raster_bwd(
        proj["means2d"], proj["conics"], proj["opacity"], proj["mus"], proj["tile_offsets"],
        proj["flatten_ids"], v_image, proj["img_w"], proj["img_h"], proj["tile_size"], absgrad)
    v_cov2d = ops.conics_mu_bwd(proj["cov2d"], proj["eps2d"], proj["conics"], proj["mus"],
                                v_conics, v_mus)
    vm, vc = ops.world_to_image_projection_bwd(means, covars, proj["viewmats"], proj["Ks"],
                                               proj["img_w"], proj["img_h"], v_means2d, v_cov2d)
    v_means = v_means + vm
    v_covars = v_covars + vc
    v_opacity = v_opacity + v_opac_cn.sum(axis=0)
    if vox is not None and v_volume is not None:
        vm3, vc3, vo3 = native.voxel_bwd(vox["means3d"], vox["conics"], vox["opacity"],
                                         vox["tile_offsets"], vox["flatten_ids"], v_volume,
                                         vox["dim2"], vox["dim1"], vox["dim0"], vox["tile_size"])
        vm, vc = ops.world_to_volume_mapping_bwd(means, covars, vox["ranges"], vox["centers"],
                                                 vox["dim2"], vox["dim1"], vox["dim0"],
                                                 vox["eps3d"], vm3, vc3)
        v_means = v_means + vm
        v_covars = v_covars + vc
        v_opacity = v_opacity + vo3
    v_quats, v_raw_scales = ops.parameter_transform_bwd(quats, raw_scales, scale_min, scale_max,
                                                        v_covars)
    k = dt.type
    sig = k(1) / (k(1) + np.exp(-raw_opacities))
    return dict(means=v_means, quats=v_quats, raw_scales=v_raw_scales,
                raw_opacities=(v_opacity * sig).astype(dt), means2d=v_means2d,
                means2d_abs=v_abs)
