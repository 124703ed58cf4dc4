"""Cone-beam CT view construction (caller-side inputs of the projection).

Restates the scanner geometry that BT-3DGS's dataset builds before calling the
backend: the intrinsic matrix (``src/data/ctproj.py:137-159``), the orbit pose
(``src/data/ctproj.py:161-267``) and the rigid inverse that turns it into a
world-to-camera matrix (``src/utils/math.py:5-32``).  Host-side torch code;
the results are copied to the device as ``viewmats`` / ``Ks``.
"""

from __future__ import annotations

import math
from typing import Sequence

import torch

__all__ = ["cone_beam_K", "cone_beam_camtoworld", "invert_rigid_transform", "cone_beam_views"]


def cone_beam_K(n_detector: Sequence[int], s_detector: Sequence[float], dsd: float,
                off_detector: Sequence[float] = (0.0, 0.0)) -> torch.Tensor:
    """Intrinsics of a flat-panel detector, ``ctproj.py:137-159``.

    ``n_detector``, ``s_detector`` and ``off_detector`` are in [v, u] order
    (rows, columns), as in the reference scanner JSON.
    """
    width, height = n_detector[1], n_detector[0]
    pixel_x = s_detector[1] / n_detector[1]
    pixel_y = s_detector[0] / n_detector[0]
    fx, fy = dsd / pixel_x, dsd / pixel_y
    cx = width / 2 + off_detector[1] / pixel_x
    cy = height / 2 + off_detector[0] / pixel_y
    return torch.tensor([[fx, 0.0, cx], [0.0, fy, cy], [0.0, 0.0, 1.0]], dtype=torch.float32)


def cone_beam_camtoworld(angle: float, dso: float, yaw: float = 0.0,
                         roll: float = 0.0) -> torch.Tensor:
    """Camera-to-world pose on the source orbit, ``ctproj.py:161-267``.

    rot = Rz(angle) Ry(yaw) Rx(roll) R_base, with R_base mapping camera x to
    world +y, camera y to world -z and camera z (the look direction) to -x;
    the source sits at dso * (cos yaw cos a, cos yaw sin a, -sin yaw).
    """
    r_base = torch.tensor([[0.0, 0.0, -1.0], [1.0, 0.0, 0.0], [0.0, -1.0, 0.0]],
                          dtype=torch.float64)
    cr, sr = math.cos(roll), math.sin(roll)
    cyw, syw = math.cos(yaw), math.sin(yaw)
    ca, sa = math.cos(angle), math.sin(angle)
    r_roll = torch.tensor([[1.0, 0.0, 0.0], [0.0, cr, -sr], [0.0, sr, cr]], dtype=torch.float64)
    r_yaw = torch.tensor([[cyw, 0.0, syw], [0.0, 1.0, 0.0], [-syw, 0.0, cyw]], dtype=torch.float64)
    r_angle = torch.tensor([[ca, -sa, 0.0], [sa, ca, 0.0], [0.0, 0.0, 1.0]], dtype=torch.float64)
    rot = r_angle @ r_yaw @ r_roll @ r_base
    trans = torch.tensor([dso * cyw * ca, dso * cyw * sa, -dso * syw], dtype=torch.float64)
    pose = torch.eye(4, dtype=torch.float32)
    pose[:3, :3] = rot.float()
    pose[:3, 3] = trans.float()
    return pose


def invert_rigid_transform(transform: torch.Tensor) -> torch.Tensor:
    """[R | t] -> [R^T | -R^T t] for [..., 4, 4] poses, ``src/utils/math.py:5-32``."""
    if transform.shape[-2:] != (4, 4):
        raise ValueError(f"Expected transform shape [..., 4, 4], got {tuple(transform.shape)}")
    rot_t = transform[..., :3, :3].transpose(-1, -2)
    trans = transform[..., :3, 3]
    inv_t = -torch.matmul(rot_t, trans.unsqueeze(-1)).squeeze(-1)
    top = torch.cat((rot_t, inv_t.unsqueeze(-1)), dim=-1)
    bottom = torch.zeros(transform.shape[:-2] + (1, 4), dtype=transform.dtype,
                         device=transform.device)
    bottom[..., 0, 3] = 1
    return torch.cat((top, bottom), dim=-2).contiguous()


def cone_beam_views(angles: Sequence[float], n_detector: int, s_detector: float = 3.0,
                    dso: float = 1.0, dsd: float = 1.5):
    """(viewmats [C,4,4], Ks [C,3,3]) float32 for a square detector at the given angles."""
    K = cone_beam_K((n_detector, n_detector), (s_detector, s_detector), dsd)
    poses = torch.stack([cone_beam_camtoworld(a, dso) for a in angles])
    viewmats = invert_rigid_transform(poses)
    Ks = K.unsqueeze(0).expand(len(angles), 3, 3).contiguous()
    return viewmats, Ks
