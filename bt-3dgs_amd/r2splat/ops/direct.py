"""Forward-only Gaussian CT splatting on the HIP backend.

Public surface of the reference's ``r2splat/ops/direct.py`` (names, keyword
arguments, result dataclasses, error types and messages): an
:class:`InferenceGaussianState` is prepared once and can be rendered and
voxelized any number of times; nothing is kept for a backward pass.  The
passes themselves live in ``r2splat.ops._passes``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ._passes import ImagePass, VolumePass, activate


@dataclass(frozen=True)
class InferenceGaussianState:
    """Reusable transformed Gaussian parameters for forward-only rendering."""

    covars: torch.Tensor
    max_scales: torch.Tensor
    opacities: torch.Tensor


@dataclass
class ProjectionRasterizationResult:
    """Rendered projections [C, img_h, img_w], detector means [C, N, 2] and
    per-axis pixel radii [C, N, 2] (int32)."""

    image: torch.Tensor
    means2d: torch.Tensor
    radii: torch.Tensor


@dataclass
class MappingVoxelizationResult:
    """Volume [dim0, dim1, dim2], voxel-space means [N, 3] and per-axis voxel
    radii [N, 3] (int32)."""

    volume: torch.Tensor
    means3d: torch.Tensor
    radii: torch.Tensor


def prepare_inference_gaussians(
    quats: torch.Tensor,
    raw_scales: torch.Tensor,
    raw_opacities: torch.Tensor,
    *,
    scale_min: float,
    scale_max: float,
) -> InferenceGaussianState:
    """Transform raw parameters once for reusable forward-only evaluation.

    Raises ``RuntimeError`` unless every input is a device tensor."""
    with torch.no_grad():
        covars, max_scales, opacities = activate(quats, raw_scales, raw_opacities, scale_min,
                                                 scale_max)
    return InferenceGaussianState(covars=covars, max_scales=max_scales, opacities=opacities)


def inference_rasterize(
    state: InferenceGaussianState,
    means: torch.Tensor,
    viewmats: torch.Tensor,
    Ks: torch.Tensor,
    *,
    img_w: int,
    img_h: int,
    tile_size: int,
    eps2d: float,
    radius_clip: float,
) -> ProjectionRasterizationResult:
    """Rasterize without building or retaining any backward state.

    ``tile_size**2`` must not exceed 1024 (``ValueError``)."""
    image_pass = ImagePass.run(means, state.covars, state.opacities, viewmats, Ks, img_w=img_w,
                               img_h=img_h, tile_size=tile_size, eps2d=eps2d,
                               radius_clip=radius_clip)
    return ProjectionRasterizationResult(image=image_pass.image, means2d=image_pass.means2d,
                                         radii=image_pass.radii)


def inference_voxelize(
    state: InferenceGaussianState,
    means: torch.Tensor,
    ranges: torch.Tensor,
    centers: torch.Tensor,
    *,
    dim2: int,
    dim1: int,
    dim0: int,
    tile_size: int,
    eps3d: float,
    radius_clip: float,
) -> MappingVoxelizationResult:
    """Voxelize without building or retaining any backward state.

    ``tile_size**3`` must not exceed 1024 (``ValueError``)."""
    volume_pass = VolumePass.run(means, state.covars, state.max_scales, state.opacities, ranges,
                                 centers, dim2=dim2, dim1=dim1, dim0=dim0, tile_size=tile_size,
                                 eps3d=eps3d, radius_clip=radius_clip)
    return MappingVoxelizationResult(volume=volume_pass.volume, means3d=volume_pass.means3d,
                                     radii=volume_pass.radii)


__all__ = [
    "InferenceGaussianState",
    "MappingVoxelizationResult",
    "ProjectionRasterizationResult",
    "inference_rasterize",
    "inference_voxelize",
    "prepare_inference_gaussians",
]
