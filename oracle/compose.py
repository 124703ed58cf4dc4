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


def _cast(x, dt):
    if dt is None or not isinstance(x, np.ndarray) or x.dtype.kind != "f":
        return x
    return x.astype(dt)


def explicit_backward(covars, proj, vox, means, quats, raw_scales, raw_opacities, scale_min,
                      scale_max, v_image, v_volume=None, absgrad=True, dtype=None, eta=0.0,
                      raster_grads=None, voxel_grads=None):
    """explicit.py:233-385 -> dict of gradients (means, quats, raw_scales,
    raw_opacities, means2d, means2d_abs).

    ``dtype`` evaluates the whole backward in that precision on the given
    values (e.g. float64 over a float32 forward: the forward's geometry and
    tile lists stay those of the float32 run).  ``eta`` > 0 adds
    ``flagged``: a bool [N] marking the Gaussians whose raster or voxel sums
    hold a term within the flip bracket of an alpha cut-off (see
    r2s_oracle.c).  ``raster_grads`` / ``voxel_grads`` replace the raster /
    voxel VJPs by given values (the 5-tuple / 3-tuple of the ops), so that
    only the chain after them is evaluated."""
    dt = np.dtype(dtype) if dtype is not None else means.dtype
    P = {k: _cast(v, dt) for k, v in proj.items()}
    V = None if vox is None else {k: _cast(v, dt) for k, v in vox.items()}
    covars, means, quats, raw_scales, raw_opacities = (
        _cast(x, dt) for x in (covars, means, quats, raw_scales, raw_opacities))
    N = means.shape[0]
    flagged = np.zeros(N, bool)
    v_means = np.zeros_like(means)
    v_covars = np.zeros_like(covars)
    v_opacity = np.zeros(N, dt)
    if raster_grads is None:
        res = native.raster_bwd(P["means2d"], P["conics"], P["opacity"], P["mus"],
                                P["tile_offsets"], P["flatten_ids"], _cast(v_image, dt),
                                P["img_w"], P["img_h"], P["tile_size"], absgrad, eta=eta,
                                band=eta > 0)
        if eta > 0:
            res, bands = res
            for b in bands:
                if b is not None:
                    flagged |= (b.reshape(b.shape[0], N, -1) > 0).any(-1).any(0)
    else:
        res = tuple(None if g is None else _cast(np.asarray(g), dt) for g in raster_grads)
    v_abs, v_means2d, v_conics, v_opac_cn, v_mus = res
    v_cov2d = ops.conics_mu_bwd(P["cov2d"], P["eps2d"], P["conics"], P["mus"], v_conics, v_mus)
    vm, vc = ops.world_to_image_projection_bwd(means, covars, P["viewmats"], P["Ks"],
                                               P["img_w"], P["img_h"], v_means2d, v_cov2d)
    v_means = v_means + vm
    v_covars = v_covars + vc
    v_opacity = v_opacity + v_opac_cn.sum(axis=0)
    if V is not None and (v_volume is not None or voxel_grads is not None):
        if voxel_grads is None:
            r3 = native.voxel_bwd(V["means3d"], V["conics"], V["opacity"], V["tile_offsets"],
                                  V["flatten_ids"], _cast(v_volume, dt), V["dim2"], V["dim1"],
                                  V["dim0"], V["tile_size"], eta=eta, band=eta > 0)
            if eta > 0:
                r3, b3 = r3
                for b in b3:
                    flagged |= (b.reshape(N, -1) > 0).any(-1)
        else:
            r3 = tuple(_cast(np.asarray(g), dt) for g in voxel_grads)
        vm3, vc3, vo3 = r3
        vm, vc = ops.world_to_volume_mapping_bwd(means, covars, V["ranges"], V["centers"],
                                                 V["dim2"], V["dim1"], V["dim0"],
                                                 V["eps3d"], vm3, vc3)
        v_means = v_means + vm
        v_covars = v_covars + vc
        v_opacity = v_opacity + vo3
    v_quats, v_raw_scales = ops.parameter_transform_bwd(quats, raw_scales, scale_min, scale_max,
                                                        v_covars)
    k = dt.type
    sig = k(1) / (k(1) + np.exp(-raw_opacities))
    out = dict(means=v_means, quats=v_quats, raw_scales=v_raw_scales,
               raw_opacities=(v_opacity * sig).astype(dt), means2d=v_means2d,
               means2d_abs=v_abs)
    if eta > 0:
        out["flagged"] = flagged
    return out
