"""BASELINE configs 1 and 2 end to end on the GPU against the oracle.

* Config 1 (the CPU-reference case): seed 0, 4,096 Gaussians (means
  U[-1,1]^3, log-scales N(-4, 0.5), random unit quaternions, densities
  U[0,1]), one cone-beam view at an angle drawn from the same generator, a
  64^2 detector and a 64^3 voxelization over [-1,1]^3, upstream gradients
  N(0,1); the image, the volume, every raster / voxel gradient and the four
  parameter gradients.
* Config 2: 50,000 Gaussians of the same distributions, a 256^2 detector,
  one view per call at angles k 2 pi / 64; all 64 angles are checked
  (projection fwd+bwd only, dL/d means, raw scales, quats, raw opacities),
  each on its own explicit state as the trainer calls it.

The check is tests/pipeline_check.py's: fp64-anchored, alpha flips counted.
"""

import math

import pytest
import torch

from pipeline_check import check_against_oracle, run
from r2splat import geometry, scenes

pytestmark = pytest.mark.gpu


def test_config1_end_to_end():
    g = torch.Generator().manual_seed(0)
    raw = scenes.random_gaussians(4096, g, -4.0, 0.5)
    angle = float(torch.rand(1, generator=g)) * 2.0 * math.pi
    viewmats, Ks = geometry.cone_beam_views([angle], 64)
    v_image = torch.randn(1, 64, 64, generator=g)
    v_volume = torch.randn(64, 64, 64, generator=g)
    out = run(raw, viewmats, Ks, 64, 64, (64, 64, 64), v_image=v_image, v_volume=v_volume)
    assert out["state"].projection.lists.isect_ids.numel() > 2000
    assert out["state"].voxel.lists.isect_ids.numel() > 2000
    check_against_oracle(out, raw, viewmats, Ks, 64, 64, (64, 64, 64))


@pytest.fixture(scope="module")
def config2_scene():
    g = torch.Generator().manual_seed(2)
    return scenes.random_gaussians(50_000, g, -4.0, 0.5), g


@pytest.mark.parametrize("k", list(range(64)))
def test_config2_view(config2_scene, k):
    raw, _ = config2_scene
    viewmats, Ks = geometry.cone_beam_views([k * 2.0 * math.pi / 64], 256)
    v_image = torch.randn(1, 256, 256, generator=torch.Generator().manual_seed(100 + k))
    out = run(raw, viewmats, Ks, 256, 256, v_image=v_image)
    assert out["state"].projection.lists.isect_ids.numel() > 50_000
    check_against_oracle(out, raw, viewmats, Ks, 256, 256)
