"""Gaussian-only CT splatting operators for AMD MI355X (gfx950).

Drop-in for the ``r2splat`` package of BT-3DGS: same ``r2splat.ops`` API,
backed by hand-written HIP kernels in ``libr2splat_hip.so``.
"""

__version__ = "0.1.0"

from .ops import ExplicitGaussianState, InferenceGaussianState

__all__ = ["__version__", "ExplicitGaussianState", "InferenceGaussianState"]
