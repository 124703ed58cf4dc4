"""Densify / prune index compaction on the GPU.

The binary-tree strategy selects Gaussians with ``torch.where(mask)[0]`` and
keeps the rest with ``torch.where(~mask)[0]``
(src/strategies/binary_tree.py:68, 101-102, 158).  ``split_indices`` returns
both lists from one HIP pass (wave ballot + prefix scan) with a single host
read-back of the selected count; ``where_indices`` is the drop-in for
``torch.where(mask)[0]``.  Both return ascending int64 indices on the mask's
device.
"""

from __future__ import annotations

from typing import Tuple

import torch

__all__ = ["split_indices", "where_indices"]


def split_indices(mask: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """(torch.where(mask)[0], torch.where(~mask)[0]) for a 1-D CUDA mask."""
    from ..cuda._wrapper import mask_split

    if not mask.is_cuda:
        raise RuntimeError("Direct r2splat operators require CUDA tensors.")
    if mask.dim() != 1:
        raise ValueError("mask must be 1-D")
    out, n_true = mask_split(mask)
    return out[:n_true], out[n_true:]


def where_indices(mask: torch.Tensor) -> torch.Tensor:
    """torch.where(mask)[0] for a 1-D CUDA mask."""
    return split_indices(mask)[0]
