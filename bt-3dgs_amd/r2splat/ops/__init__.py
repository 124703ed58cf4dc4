"""Direct Gaussian CT splatting interfaces."""

from .compact import split_indices, where_indices
from .direct import (
    InferenceGaussianState,
    MappingVoxelizationResult,
    ProjectionRasterizationResult,
    inference_rasterize,
    inference_voxelize,
    prepare_inference_gaussians,
)
from .explicit import ExplicitGaussianState

__all__ = [
    "ExplicitGaussianState",
    "InferenceGaussianState",
    "MappingVoxelizationResult",
    "ProjectionRasterizationResult",
    "inference_rasterize",
    "inference_voxelize",
    "prepare_inference_gaussians",
    "split_indices",
    "where_indices",
]
