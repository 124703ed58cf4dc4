"""Forward passes that keep what their vector-Jacobian product needs.

Two pass types sit between the public API (``direct``, ``explicit``) and the
tensor operators of ``r2splat.cuda._ops``:

* :class:`ImagePass` -- cone-beam projection of the Gaussians into C views,
  tile binning and the X-ray line-integral rasterizer;
* :class:`VolumePass` -- the mapping into a voxel grid, brick binning and the
  voxelizer.

``ImagePass.run`` / ``VolumePass.run`` execute the forward and return the
pass; its ``vjp`` maps an upstream gradient of the image (volume) to
gradients of the Gaussians' world means, packed covariances and opacities.
The tile lists travel inside the pass together with their emission order
(:class:`r2splat.cuda._ops.TileLists`), so the backward always gets the
two-pass, atomic-free kernels.

The arithmetic is the reference's (r2splat/ops/direct.py:72-322 for the
forward composition, explicit.py:233-385 for the backward one); the fused
kernels change only how many launches it takes: the projection, conics/mu and
opacity broadcast run as one kernel, and so do their VJPs.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import NamedTuple, Optional, Tuple

import torch

Tensor = torch.Tensor

CUDA_REQUIRED = "Direct r2splat operators require CUDA tensors."
TILE_2D = "2D tile_size must be positive with tile_size**2 <= 1024."
TILE_3D = "3D tile_size must be positive with tile_size**3 <= 1024."


def _ops():
    # Deferred: importing r2splat.ops must not load the HIP library.
    from ..cuda._backend import _C

    return _C


def activate(quats: Tensor, raw_scales: Tensor, raw_opacities: Tensor, scale_min: float,
             scale_max: float) -> Tuple[Tensor, Tensor, Tensor]:
    """Raw parameters -> (covars [N,6], max_scales [N], opacities [N]) in one
    kernel: sigmoid-bounded scales, rotation, packed covariance and softplus
    opacity (direct.py:72-96, ParameterTransformFwd.cu:53-129)."""
    if not all(t.is_cuda for t in (quats, raw_scales, raw_opacities)):
        raise RuntimeError(CUDA_REQUIRED)
    return _ops().prepare_gaussians(quats.contiguous(), raw_scales.contiguous(),
                                    raw_opacities.contiguous(), float(scale_min),
                                    float(scale_max))


def _tiles_along(extent: int, tile: int) -> int:
    return -(-extent // tile)


class ImageVJP(NamedTuple):
    v_means: Tensor       # [N, 3]
    v_covars: Tensor      # [N, 6]
    v_weights: Tensor     # [C, N]: gradient of each view's opacity broadcast
    v_means2d: Tensor     # [C, N, 2]
    v_means2d_abs: Optional[Tensor]


class VolumeVJP(NamedTuple):
    v_means: Tensor       # [N, 3]
    v_covars: Tensor      # [N, 6]
    v_weights: Tensor     # [N]


class ParameterVJP(NamedTuple):
    v_means: Tensor          # [N, 3], image + volume
    v_quats: Tensor          # [N, 4]
    v_raw_scales: Tensor     # [N, 3]
    v_raw_opacities: Tensor  # [N]
    v_means2d: Tensor        # [C, N, 2]
    v_means2d_abs: Optional[Tensor]


@dataclass(eq=False)
class ImagePass:
    """Projection + rasterization of C views of N Gaussians.

    ``image`` is [C, height, width] (row = detector v, column = detector u).
    The per-view attributes are those the rasterizer consumed: ``means2d``
    [C,N,2] detector positions, ``cov2d`` [C,N,6] the projected 3x3
    covariances, ``conics`` [C,N,3] and ``mus`` [C,N] the line-integral
    conic and normaliser, ``weights`` [C,N] the opacities, ``radii`` [C,N,2].
    """

    width: int
    height: int
    tile_size: int
    eps2d: float
    viewmats: Tensor
    Ks: Tensor
    means2d: Tensor
    cov2d: Tensor
    conics: Tensor
    mus: Tensor
    weights: Tensor
    radii: Tensor
    tile_offsets: Tensor
    lists: object  # r2splat.cuda._ops.TileLists
    image: Tensor
    absgrad: bool = False
    # Tile sizes 8, 16 and 32 with records: the packed per-(view, Gaussian)
    # payload both raster passes read, and (for_backward) the raster
    # backward's outputs, zeroed by the launch that wrote it; handed to the
    # first vjp.
    payload: Optional[Tensor] = None
    zeroed_outputs: Optional[tuple] = None

    @classmethod
    @torch.no_grad()
    def run(cls, means: Tensor, covars: Tensor, opacities: Tensor, viewmats: Tensor, Ks: Tensor,
            *, img_w: int, img_h: int, tile_size: int, eps2d: float, radius_clip: float,
            absgrad: bool = False, for_backward: bool = False) -> "ImagePass":
        ts = int(tile_size)
        if ts <= 0 or ts * ts > 1024:
            raise ValueError(TILE_2D)
        width, height = int(img_w), int(img_h)
        ops = _ops()
        viewmats, Ks = viewmats.contiguous(), Ks.contiguous()
        # The payload depends on the projection only: the projection's launch
        # writes it (and, for the backward, zeros its outputs) from its own
        # results, before the binning, whose record count the host waits for.
        payload = zeroed = None
        if ts in ops.PACKED_TILE_SIZES:
            means2d, cov2d, radii, conics, mus, weights, payload, zeroed = ops.project_pack_fwd(
                means.contiguous(), covars.contiguous(), opacities.contiguous(), viewmats, Ks,
                width, height, float(eps2d), float(radius_clip), zero_outputs=for_backward,
                absgrad=absgrad)
        else:
            means2d, cov2d, radii, conics, mus, weights = ops.project_gaussians_fwd(
                means.contiguous(), covars.contiguous(), opacities.contiguous(), viewmats, Ks,
                width, height, float(eps2d), float(radius_clip))
        across, down = _tiles_along(width, ts), _tiles_along(height, ts)
        # The sorted int64 keys are not stored: the backward finds each
        # record's tile from the tile offsets (lists.isect_ids recovers them).
        lists = ops.bin_tiles_2d(means2d, radii, ts, across, down, keep_ids=False)
        tile_offsets = lists.tile_offsets
        if tile_offsets is None:  # no records
            tile_offsets = ops.isect_offset_encode(lists.isect_ids, int(viewmats.shape[0]),
                                                   across, down)
        if payload is not None and lists.flatten_ids.numel() > 0:
            image = ops.rasterize_packed(payload, tile_offsets, lists.flatten_ids,
                                         means2d.shape[0], means2d.shape[1], width, height, ts)
        else:
            image = ops.rasterize_to_pixels_fwd(means2d, conics, weights, mus, tile_offsets,
                                                lists.flatten_ids, width, height, ts)
        return cls(width, height, ts, float(eps2d), viewmats, Ks, means2d, cov2d, conics, mus,
                   weights, radii, tile_offsets, lists, image, bool(absgrad), payload, zeroed)

    def _raster_vjp(self, v_image: Tensor):
        """The rasterizer's VJP: (v_abs or None, v_means2d, v_conics, v_weights, v_mus)."""
        ops = _ops()
        if self.payload is None:
            return ops.raster_backward(self.means2d, self.conics, self.weights, self.mus,
                                       self.tile_offsets, self.lists, v_image.contiguous(),
                                       self.width, self.height, self.tile_size, self.absgrad)
        zeroed, self.zeroed_outputs = self.zeroed_outputs, None
        return ops.raster_backward_packed(self.payload, self.weights, self.mus,
                                          self.tile_offsets, self.lists, v_image.contiguous(),
                                          self.width, self.height, self.tile_size, self.absgrad,
                                          zeroed)

    @torch.no_grad()
    def vjp(self, v_image: Tensor, means: Tensor, covars: Tensor) -> ImageVJP:
        ops = _ops()
        v_abs, v_means2d, v_conics, v_weights, v_mus = self._raster_vjp(v_image)
        v_means, v_covars = ops.project_gaussians_bwd(
            means.contiguous(), covars, self.viewmats, self.Ks, self.width, self.height,
            self.eps2d, self.cov2d, self.conics, self.mus, v_means2d, v_conics, v_mus)
        return ImageVJP(v_means, v_covars, v_weights, v_means2d, v_abs)

    @torch.no_grad()
    def vjp_to_parameters(self, v_image: Tensor, means: Tensor, covars: Tensor,
                          volume: Optional["VolumeVJP"], quats: Tensor, raw_scales: Tensor,
                          scale_min: float, scale_max: float,
                          raw_opacities: Tensor) -> "ParameterVJP":
        """The image's VJP carried through to the raw parameters, with the
        volume pass's VJP (if any) added where the two meet: the raster
        backward, then one kernel for the projection, parameter-transform
        and opacity VJPs (bit-identical to vjp + parameter_transform_bwd +
        opacity_bwd with the world-space gradients summed image + volume)."""
        ops = _ops()
        v_abs, v_means2d, v_conics, v_weights, v_mus = self._raster_vjp(v_image)
        v_means, v_quats, v_raw_scales, v_raw_opac = ops.explicit_backward_tail(
            means.contiguous(), covars.contiguous(), self.viewmats, self.Ks, self.width,
            self.height, self.eps2d, self.cov2d, self.conics, self.mus, v_means2d, v_conics,
            v_mus, None if volume is None else volume.v_means.contiguous(),
            None if volume is None else volume.v_covars.contiguous(), quats.contiguous(),
            raw_scales.contiguous(), scale_min, scale_max, raw_opacities.contiguous(),
            v_weights, None if volume is None else volume.v_weights.contiguous())
        return ParameterVJP(v_means, v_quats, v_raw_scales, v_raw_opac, v_means2d, v_abs)


@dataclass(eq=False)
class VolumePass:
    """Mapping + voxelization of N Gaussians into a [dim0, dim1, dim2] grid
    spanning ``ranges`` around ``centers`` (x along dim2, y dim1, z dim0).
    ``means3d`` [N,3] and ``conics`` [N,6] are in voxel units.

    A volume whose brick list would hold more than ``_ops.SLAB_RECORDS``
    records (e.g. a 512^3 grid under needle-like Gaussians, whose bounding
    boxes span it: 7.5e9 records) is processed in z-slabs of brick layers:
    ``slabs`` lists their layer ranges, ``lists`` and ``tile_offsets`` are
    None, and the backward bins each slab again rather than keeping every
    slab's lists."""

    dim2: int
    dim1: int
    dim0: int
    tile_size: int
    eps3d: float
    ranges: Tensor
    centers: Tensor
    means3d: Tensor
    conics: Tensor
    weights: Tensor
    radii: Tensor
    tile_offsets: Optional[Tensor]
    lists: object  # r2splat.cuda._ops.TileLists, None for a slabbed volume
    volume: Tensor
    slabs: Tuple[Tuple[int, int], ...] = ()
    reach: Optional[Tensor] = None  # per-record reach masks (tile size 8) for the backward

    @classmethod
    @torch.no_grad()
    def run(cls, means: Tensor, covars: Tensor, max_scales: Tensor, opacities: Tensor,
            ranges: Tensor, centers: Tensor, *, dim2: int, dim1: int, dim0: int, tile_size: int,
            eps3d: float, radius_clip: float) -> "VolumePass":
        ts = int(tile_size)
        if ts <= 0 or ts ** 3 > 1024:
            raise ValueError(TILE_3D)
        d2, d1, d0 = int(dim2), int(dim1), int(dim0)
        ops = _ops()
        ranges, centers = ranges.contiguous(), centers.contiguous()
        means3d, conics, radii = ops.world_to_volume_mapping_fwd(
            means.contiguous(), covars.contiguous(), max_scales.contiguous(), ranges, centers,
            d2, d1, d0, float(eps3d), float(radius_clip))
        n2, n1, n0 = _tiles_along(d2, ts), _tiles_along(d1, ts), _tiles_along(d0, ts)
        weights = opacities.contiguous()
        lists = ops.bin_tiles_3d(means3d, radii, ts, n2, n1, n0, max_records=ops.SLAB_RECORDS,
                                 keep_ids=False)
        if lists is None:
            slabs = tuple(ops.plan_slabs(ops.layer_counts_3d(means3d, radii, ts, n2, n1, n0),
                                         ops.SLAB_RECORDS))
            volume = torch.empty((d0, d1, d2), dtype=means3d.dtype, device=means3d.device)
            for z0, z1 in slabs:
                slab_lists, slab_offsets = ops.bin_tiles_3d_slab(means3d, radii, ts, n2, n1, n0,
                                                                 z0, z1, keep_ids=False)
                ops.voxelize_slab(means3d, conics, weights, slab_offsets, slab_lists, volume, ts,
                                  z0)
                del slab_lists, slab_offsets
            return cls(d2, d1, d0, ts, float(eps3d), ranges, centers, means3d, conics, weights,
                       radii, None, None, volume, slabs)
        tile_offsets = lists.tile_offsets
        if tile_offsets is None:  # no records
            tile_offsets = ops.isect_offset_encode_3d(lists.isect_ids, n2, n1, n0)
        reach = None
        if ts == 8:  # the backward reuses the forward's culling
            volume, reach = ops.voxelize_with_reach(means3d, conics, weights, tile_offsets,
                                                    lists.flatten_ids, d2, d1, d0)
        else:
            volume = ops.voxelize_to_voxels_fwd(means3d, conics, weights, tile_offsets,
                                                lists.flatten_ids, d2, d1, d0, ts)
        return cls(d2, d1, d0, ts, float(eps3d), ranges, centers, means3d, conics, weights,
                   radii, tile_offsets, lists, volume, reach=reach)

    @torch.no_grad()
    def vjp(self, v_volume: Tensor, means: Tensor, covars: Tensor) -> VolumeVJP:
        ops = _ops()
        v_volume = v_volume.contiguous()
        if self.slabs:
            ts = self.tile_size
            n2, n1, n0 = (_tiles_along(d, ts) for d in (self.dim2, self.dim1, self.dim0))
            total = None
            for z0, z1 in self.slabs:
                slab_lists, slab_offsets = ops.bin_tiles_3d_slab(self.means3d, self.radii, ts,
                                                                 n2, n1, n0, z0, z1,
                                                                 keep_ids=False)
                part = ops.voxel_backward_slab(self.means3d, self.conics, self.weights,
                                               slab_offsets, slab_lists, v_volume, ts, z0)
                total = list(part) if total is None else [a.add_(b) for a, b in zip(total, part)]
                del slab_lists, slab_offsets, part
            v_means3d, v_conics, v_weights = total
        else:
            v_means3d, v_conics, v_weights = ops.voxel_backward(
                self.means3d, self.conics, self.weights, self.tile_offsets, self.lists,
                v_volume, self.dim2, self.dim1, self.dim0, self.tile_size, reach=self.reach)
        v_means, v_covars = ops.world_to_volume_mapping_bwd(
            means.contiguous(), covars, self.ranges, self.centers, self.dim2, self.dim1,
            self.dim0, self.eps3d, v_means3d, v_conics)
        return VolumeVJP(v_means, v_covars, v_weights)
