"""Seeded synthetic Gaussian scenes with the reference model's parameterisation.

Raw parameters are produced exactly as BT-3DGS's ``GaussianModel`` stores
them (``src/models/gaussian_model.py:248-274, 680-684``): bounded-sigmoid raw
scales, softplus raw opacities and (w, x, y, z) quaternions.  Everything is
drawn on the CPU from one ``torch.Generator`` in a fixed order (means,
log-scales, quaternions, densities, then whatever the caller draws next), so
a device run and the CPU oracle see identical bits.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = ["RawGaussians", "SCALE_MIN", "SCALE_MAX", "SCALE_EPS", "activate_scale",
           "inverse_activate_scale", "inverse_softplus", "random_gaussians",
           "binary_tree_gaussians", "stress_gaussians"]

# configs/model/binary_tree.yaml:6-8
SCALE_MIN = 0.0005
SCALE_MAX = 1.0
SCALE_EPS = 1.0e-5


@dataclass
class RawGaussians:
    means: torch.Tensor          # [N, 3]
    quats: torch.Tensor          # [N, 4] (w, x, y, z), not normalised
    raw_scales: torch.Tensor     # [N, 3]
    raw_opacities: torch.Tensor  # [N]

    def to(self, device) -> "RawGaussians":
        return RawGaussians(*(t.to(device).contiguous() for t in
                              (self.means, self.quats, self.raw_scales, self.raw_opacities)))

    @property
    def n(self) -> int:
        return int(self.means.shape[0])


def activate_scale(raw: torch.Tensor) -> torch.Tensor:
    """gaussian_model.py:254-260: min + (max - min) * sigmoid(raw)."""
    return SCALE_MIN + (SCALE_MAX - SCALE_MIN) * torch.sigmoid(raw)


def inverse_activate_scale(scales: torch.Tensor) -> torch.Tensor:
    """gaussian_model.py:262-270: clamp inside the bounds by eps, then logit."""
    clamped = scales.clamp(min=SCALE_MIN + SCALE_EPS, max=SCALE_MAX - SCALE_EPS)
    sigma = ((clamped - SCALE_MIN) / (SCALE_MAX - SCALE_MIN)).clamp(min=1e-6, max=1.0 - 1e-6)
    return torch.logit(sigma)


def inverse_softplus(y: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """gaussian_model.py:680-684: log(expm1(max(y, 0) + eps))."""
    return torch.log(torch.expm1(y.clamp_min(0.0) + eps))


def random_gaussians(n: int, generator: torch.Generator, log_scale_mu: float = -4.0,
                     log_scale_sigma: float = 0.5, extent: float = 1.0) -> RawGaussians:
    """Config-style Gaussians: means U[-e,e]^3, log-scales N(mu, sigma),
    normalised N(0,1) quaternions, densities U[0,1] (in that draw order)."""
    g = generator
    means = (torch.rand(n, 3, generator=g) * 2.0 - 1.0) * extent
    log_scales = torch.randn(n, 3, generator=g) * log_scale_sigma + log_scale_mu
    quats = torch.nn.functional.normalize(torch.randn(n, 4, generator=g), dim=-1)
    density = torch.rand(n, generator=g)
    return RawGaussians(means.float(), quats.float(),
                        inverse_activate_scale(torch.exp(log_scales)).float(),
                        inverse_softplus(density).float())


def stress_gaussians(n: int, generator: torch.Generator, needle_fraction: float = 0.05,
                     needle_log_ratio: float = math.log(50.0)) -> RawGaussians:
    """Config 5: log-scale N(-5, 1) per axis; a fraction of needles whose long
    axis exceeds the larger other axis by at least ``needle_log_ratio``."""
    g = generator
    means = torch.rand(n, 3, generator=g) * 2.0 - 1.0
    log_scales = torch.randn(n, 3, generator=g) * 1.0 - 5.0
    quats = torch.nn.functional.normalize(torch.randn(n, 4, generator=g), dim=-1)
    density = torch.rand(n, generator=g)
    needle = torch.rand(n, generator=g) < needle_fraction
    axis = torch.randint(0, 3, (n,), generator=g)
    extra = torch.rand(n, generator=g) * 0.5
    others = log_scales.clone()
    others[torch.arange(n), axis] = -float("inf")
    long_axis = others.max(dim=-1).values + needle_log_ratio + extra
    ls = log_scales.clone()
    ls[needle, axis[needle]] = long_axis[needle]
    return RawGaussians(means.float(), quats.float(),
                        inverse_activate_scale(torch.exp(ls)).float(),
                        inverse_softplus(density).float())


def _rotmat(q: torch.Tensor) -> torch.Tensor:
    # src/utils/math.py:35-53 normalized_quat_to_rotmat
    w, x, y, z = torch.unbind(q, dim=-1)
    m = torch.stack([1 - 2 * (y ** 2 + z ** 2), 2 * (x * y - w * z), 2 * (x * z + w * y),
                     2 * (x * y + w * z), 1 - 2 * (x ** 2 + z ** 2), 2 * (y * z - w * x),
                     2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x ** 2 + y ** 2)], -1)
    return m.reshape(q.shape[:-1] + (3, 3))


def _split(means, quats, raw_scales, raw_opac, mask, revised_opacity):
    """src/strategies/binary_tree.py:93-148 split(): children [all +off; all -off]."""
    sel = torch.where(mask)[0]
    rest = torch.where(~mask)[0]
    scales = activate_scale(raw_scales[sel])
    rot = _rotmat(torch.nn.functional.normalize(quats[sel], dim=-1))
    longest = scales.argmax(dim=-1)
    axis_mask = torch.zeros_like(scales)
    axis_mask.scatter_(1, longest.unsqueeze(1), 1.0)
    offset = torch.einsum("nij,nj->ni", rot, scales * axis_mask)
    samples = torch.stack([offset, -offset], dim=0)
    new_means = (means[sel] + samples).reshape(-1, 3)
    target = scales.clone()
    target.scatter_(1, longest.unsqueeze(1),
                    (scales.gather(1, longest.unsqueeze(1)) / 1.6).clamp_min(1e-12))
    new_raw_scales = inverse_activate_scale(target).repeat(2, 1)
    if revised_opacity:
        base = torch.nn.functional.softplus(raw_opac[sel]).clamp(max=0.9999)
        new_raw_opac = torch.log(torch.expm1(1.0 - torch.sqrt(1.0 - base))).repeat(2)
    else:
        new_raw_opac = raw_opac[sel].repeat(2)
    cat = lambda p, q: torch.cat([p[rest], q])  # noqa: E731
    return (cat(means, new_means), cat(quats, quats[sel].repeat(2, 1)),
            cat(raw_scales, new_raw_scales), cat(raw_opac, new_raw_opac))


def binary_tree_gaussians(n: int, generator: torch.Generator | None = None,
                          opacity: str = "uniform", root_scale: float = 1.0,
                          root_opacity: float = 0.1) -> RawGaussians:
    """Config 4: ``n`` leaves grown from one root by the reference split.

    The root sits at the origin with isotropic scale ``root_scale``, identity
    rotation and opacity ``root_opacity`` (trainers/binary_tree.py:73-90,
    binary_tree_gaussian_model.py:115-150).  All leaves are split level by
    level, then the first leaves in index order until ``n`` is reached.

    ``opacity="revised"`` applies the strategy's revised opacity at each split
    (1 - sqrt(1 - o), configs/strategy/binary_tree.yaml:15); after 18 levels
    that leaves o ~ 4e-7, below the rasterizer's 1e-5 alpha cut-off
    everywhere.  ``opacity="uniform"`` (default) instead redraws the leaf
    densities U[0,1] from ``generator`` so the image is not identically zero.
    """
    means = torch.zeros(1, 3)
    quats = torch.tensor([[1.0, 0.0, 0.0, 0.0]])
    raw_scales = inverse_activate_scale(torch.full((1, 3), float(root_scale)))
    raw_opac = inverse_softplus(torch.tensor([root_opacity]).clamp(1e-6, 0.99))
    revised = opacity == "revised"
    while means.shape[0] < n:
        m = means.shape[0]
        mask = torch.zeros(m, dtype=torch.bool)
        mask[: min(m, n - m)] = True
        means, quats, raw_scales, raw_opac = _split(means, quats, raw_scales, raw_opac,
                                                    mask, revised)
    if opacity == "uniform":
        gen = generator if generator is not None else torch.Generator().manual_seed(0)
        raw_opac = inverse_softplus(torch.rand(n, generator=gen))
    elif opacity != "revised":
        raise ValueError("opacity must be 'uniform' or 'revised'")
    return RawGaussians(means.float().contiguous(), quats.float().contiguous(),
                        raw_scales.float().contiguous(), raw_opac.float().contiguous())
