"""Cone-beam view construction and the seeded scene generators (CPU)."""

import math

import numpy as np
import torch

from r2splat import geometry, scenes


def test_K_matches_scanner_formula():
    # src/data/ctproj.py:137-159 with nDetector [v,u] = [48, 64], sDetector [1.5, 3.0].
    K = geometry.cone_beam_K((48, 64), (1.5, 3.0), 1.5, (0.1, -0.2))
    fx, fy = 1.5 / (3.0 / 64), 1.5 / (1.5 / 48)
    np.testing.assert_allclose(K.numpy(), [[fx, 0, 32 + -0.2 / (3.0 / 64)],
                                           [0, fy, 24 + 0.1 / (1.5 / 48)], [0, 0, 1]], rtol=1e-6)


def test_orbit_pose_and_inverse():
    for a in (0.0, 0.7, math.pi / 2, 3.0):
        pose = geometry.cone_beam_camtoworld(a, 1.0)
        # The source sits on the orbit and looks at the origin.
        np.testing.assert_allclose(pose[:3, 3].numpy(), [math.cos(a), math.sin(a), 0.0], atol=1e-6)
        np.testing.assert_allclose((pose[:3, :3] @ torch.tensor([0, 0, 1.0])).numpy(),
                                   [-math.cos(a), -math.sin(a), 0.0], atol=1e-6)
        view = geometry.invert_rigid_transform(pose)
        np.testing.assert_allclose((view @ pose).numpy(), np.eye(4), atol=1e-6)
        # The origin lies on the optical axis at depth DSO.
        np.testing.assert_allclose((view @ torch.tensor([0, 0, 0, 1.0]))[:3].numpy(),
                                   [0, 0, 1.0], atol=1e-6)
    vm, Ks = geometry.cone_beam_views([0.0, 1.0], 512)
    assert vm.shape == (2, 4, 4) and Ks.shape == (2, 3, 3)
    np.testing.assert_allclose(Ks[0, 0, 0].item(), 1.5 / (3.0 / 512), rtol=1e-6)


def test_scale_and_opacity_inverses():
    s = torch.tensor([1e-3, 0.01, 0.5, 0.99])
    np.testing.assert_allclose(scenes.activate_scale(scenes.inverse_activate_scale(s)).numpy(),
                               s.numpy(), rtol=1e-4)
    d = torch.tensor([0.0, 0.2, 0.9])
    np.testing.assert_allclose(torch.nn.functional.softplus(scenes.inverse_softplus(d)).numpy(),
                               (d + 1e-6).numpy(), rtol=1e-5, atol=1e-7)


def test_random_gaussians_are_seeded():
    a = scenes.random_gaussians(100, torch.Generator().manual_seed(3))
    b = scenes.random_gaussians(100, torch.Generator().manual_seed(3))
    assert all(torch.equal(x, y) for x, y in zip(
        (a.means, a.quats, a.raw_scales, a.raw_opacities),
        (b.means, b.quats, b.raw_scales, b.raw_opacities)))
    assert a.means.abs().max() <= 1.0


def test_binary_tree_follows_split_semantics():
    # src/strategies/binary_tree.py:93-148: children [all +off; all -off] along
    # the longest axis, that axis' scale divided by 1.6.
    t1 = scenes.binary_tree_gaussians(2, opacity="revised")
    s1 = scenes.activate_scale(t1.raw_scales)
    np.testing.assert_allclose(t1.means.numpy(), [[1 - 1e-5, 0, 0], [-(1 - 1e-5), 0, 0]],
                               rtol=1e-4)
    np.testing.assert_allclose(s1[0].numpy(), [(1 - 1e-5) / 1.6, 1 - 1e-5, 1 - 1e-5], rtol=1e-4)
    # Revised opacity: o' = 1 - sqrt(1 - o) from the root's 0.1.
    o1 = torch.nn.functional.softplus(t1.raw_opacities)
    np.testing.assert_allclose(o1.numpy(), [1 - math.sqrt(0.9)] * 2, rtol=1e-4)
    t = scenes.binary_tree_gaussians(500_000)
    assert t.n == 500_000
    assert t.means.abs().max() < 2.7
    levels = torch.log(scenes.activate_scale(t.raw_scales).prod(-1)) / math.log(1 / 1.6)
    assert 18 <= levels.round().min() and levels.round().max() <= 19
