"""Explicit first-order Gaussian CT splatting on the HIP backend.

Public surface of the reference's ``r2splat/ops/explicit.py`` (names, keyword
arguments, the :class:`ExplicitGaussianState` fields, one-shot rules, error
types and messages).  A training step runs

    state = prepare_explicit_gaussians(quats, raw_scales, raw_opacities, ...)
    proj = explicit_rasterize(state, means, viewmats, Ks, ...)   # at most once
    vol = explicit_voxelize(state, means, ranges, centers, ...)   # optional, once
    loss(proj.image, vol.volume).backward()                     # any torch loss
    explicit_backward(state, means, quats, raw_scales, raw_opacities)  # once

The forwards run outside autograd.  ``proj.image``, ``proj.means2d`` and
``vol.volume`` are returned as leaf tensors that require grad, so any loss
can fill their ``.grad``; :func:`explicit_backward` then maps those gradients
to the four raw parameters and adds them to their ``.grad``, and sets
``means2d.grad`` (and ``means2d.absgrad`` when ``absgrad`` was requested),
which the densification strategy reads.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from ._passes import ImagePass, VolumePass, activate
from .direct import MappingVoxelizationResult, ProjectionRasterizationResult

BACKWARD_MODES = ("pixel", "primitive")


def _backward_mode(value) -> str:
    mode = str(value).lower()
    if mode not in BACKWARD_MODES:
        raise ValueError("backward_mode must be 'pixel' or 'primitive'.")
    return mode


@dataclass
class ExplicitGaussianState:
    """One-shot context shared by projection and voxelization for one step.

    ``projection`` / ``voxel`` hold the forward passes (``r2splat.ops._passes``
    ImagePass / VolumePass) once they have run.  Both backward modes run the
    same atomic-free kernels here; ``backward_mode`` is kept for callers."""

    covars: torch.Tensor
    max_scales: torch.Tensor
    opacities: torch.Tensor
    scale_min: float
    scale_max: float
    backward_mode: str
    projection: Optional[ImagePass] = None
    voxel: Optional[VolumePass] = None
    backward_called: bool = False


def prepare_explicit_gaussians(
    quats: torch.Tensor,
    raw_scales: torch.Tensor,
    raw_opacities: torch.Tensor,
    *,
    scale_min: float,
    scale_max: float,
    backward_mode: str = "primitive",
) -> ExplicitGaussianState:
    """Activate raw parameters without constructing a renderer autograd graph."""
    mode = _backward_mode(backward_mode)
    with torch.no_grad():
        covars, max_scales, opacities = activate(quats, raw_scales, raw_opacities, scale_min,
                                                 scale_max)
    return ExplicitGaussianState(covars=covars, max_scales=max_scales, opacities=opacities,
                                 scale_min=float(scale_min), scale_max=float(scale_max),
                                 backward_mode=mode)


def _leaf(t: torch.Tensor) -> torch.Tensor:
    return t.detach().requires_grad_(True)


def explicit_rasterize(
    state: ExplicitGaussianState,
    means: torch.Tensor,
    viewmats: torch.Tensor,
    Ks: torch.Tensor,
    *,
    img_w: int,
    img_h: int,
    tile_size: int,
    eps2d: float,
    radius_clip: float,
    absgrad: bool,
) -> ProjectionRasterizationResult:
    """Project and rasterize once for this state; the image and the detector
    means are returned as grad-requiring leaves."""
    if state.projection is not None:
        raise RuntimeError("An explicit Gaussian state can only be rasterized once.")
    image_pass = ImagePass.run(means, state.covars, state.opacities, viewmats, Ks, img_w=img_w,
                               img_h=img_h, tile_size=tile_size, eps2d=eps2d,
                               radius_clip=radius_clip, absgrad=bool(absgrad), for_backward=True)
    image_pass.image = _leaf(image_pass.image)
    image_pass.means2d = _leaf(image_pass.means2d)
    image_pass.absgrad = bool(absgrad)
    state.projection = image_pass
    return ProjectionRasterizationResult(image=image_pass.image, means2d=image_pass.means2d,
                                         radii=image_pass.radii)


def explicit_voxelize(
    state: ExplicitGaussianState,
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
    """Map and voxelize once for this state; the volume is returned as a
    grad-requiring leaf."""
    if state.voxel is not None:
        raise RuntimeError("An explicit Gaussian state can only be voxelized once.")
    volume_pass = VolumePass.run(means, state.covars, state.max_scales, state.opacities, ranges,
                                 centers, dim2=dim2, dim1=dim1, dim0=dim0, tile_size=tile_size,
                                 eps3d=eps3d, radius_clip=radius_clip)
    volume_pass.volume = _leaf(volume_pass.volume)
    state.voxel = volume_pass
    return MappingVoxelizationResult(volume=volume_pass.volume, means3d=volume_pass.means3d,
                                     radii=volume_pass.radii)


class _Sum:
    """Running sum of optional gradient tensors of one shape."""

    def __init__(self, like: torch.Tensor) -> None:
        self.like = like
        self.value: Optional[torch.Tensor] = None

    def add(self, t: torch.Tensor) -> None:
        self.value = t if self.value is None else self.value + t

    def get(self) -> torch.Tensor:
        return torch.zeros_like(self.like) if self.value is None else self.value


def _add_to_grad(parameter: torch.Tensor, g: torch.Tensor) -> None:
    if parameter.grad is None:
        parameter.grad = g.detach()
    else:
        parameter.grad.add_(g.detach())


@torch.no_grad()
def explicit_backward(
    state: ExplicitGaussianState,
    means: torch.Tensor,
    quats: torch.Tensor,
    raw_scales: torch.Tensor,
    raw_opacities: torch.Tensor,
) -> None:
    """Map the image / volume gradients to the raw parameters, once per state.

    The projection must have run; the volume's gradient is used when the
    voxelization ran and its volume received one.  A projection whose image
    received no gradient contributes nothing, and ``means2d.grad`` is zero."""
    if state.backward_called:
        raise RuntimeError("Explicit first-order backward can only run once per state.")
    image_pass = state.projection
    if image_pass is None:
        raise RuntimeError("Explicit backward requires a projection forward pass.")
    from ..cuda._backend import _C

    volume_pass = state.voxel
    g3 = None
    if volume_pass is not None and volume_pass.volume.grad is not None:
        g3 = volume_pass.vjp(volume_pass.volume.grad, means, state.covars)

    if image_pass.image.grad is not None:
        # The raster backward, then one kernel for the projection, parameter
        # transform and opacity VJPs with the volume's gradients added where
        # the world-space gradients meet (image + volume).
        gp = image_pass.vjp_to_parameters(image_pass.image.grad, means, state.covars, g3,
                                          quats, raw_scales, state.scale_min, state.scale_max,
                                          raw_opacities)
        image_pass.means2d.grad = gp.v_means2d
        if image_pass.absgrad:
            image_pass.means2d.absgrad = gp.v_means2d_abs
        v_means, v_quats = gp.v_means, gp.v_quats
        v_raw_scales, v_raw_opacities = gp.v_raw_scales, gp.v_raw_opacities
    else:
        image_pass.means2d.grad = torch.zeros_like(image_pass.means2d)
        if image_pass.absgrad:
            image_pass.means2d.absgrad = torch.zeros_like(image_pass.means2d)
        world_means = _Sum(means)
        world_covars = _Sum(state.covars)
        volume_weights = None
        if g3 is not None:
            world_means.add(g3.v_means)
            world_covars.add(g3.v_covars)
            volume_weights = g3.v_weights
        # Covariance -> (quaternion, raw scale) VJP; opacity: the volume's
        # gradient times softplus' = sigmoid.
        v_quats, v_raw_scales = _C.parameter_transform_bwd(
            quats.contiguous(), raw_scales.contiguous(), state.scale_min, state.scale_max,
            world_covars.get().contiguous())
        v_raw_opacities = _C.opacity_bwd(raw_opacities.contiguous(), None, volume_weights)
        v_means = world_means.get()

    _add_to_grad(means, v_means)
    _add_to_grad(quats, v_quats)
    _add_to_grad(raw_scales, v_raw_scales)
    _add_to_grad(raw_opacities, v_raw_opacities)
    state.backward_called = True


__all__ = [
    "ExplicitGaussianState",
    "explicit_backward",
    "explicit_rasterize",
    "explicit_voxelize",
    "prepare_explicit_gaussians",
]
