"""Shared helpers of the test suite."""

from __future__ import annotations

import math

import numpy as np
import torch

from r2splat import geometry, scenes

# Parity bar for floating-point outputs (float32): rel 1e-4 / abs 1e-5.
RTOL = 1e-4
ATOL = 1e-5


def make_scene(n, seed, n_det=64, n_views=1, log_mu=-4.0, log_sigma=0.5, extent=1.0):
    """Seeded Gaussians + cone-beam views (DSO 1.0, DSD 1.5, sDetector 3.0)."""
    g = torch.Generator().manual_seed(seed)
    raw = scenes.random_gaussians(n, g, log_mu, log_sigma, extent)
    angles = (torch.rand(n_views, generator=g) * 2 * math.pi).tolist()
    viewmats, Ks = geometry.cone_beam_views(angles, n_det)
    return raw, viewmats, Ks, g


def np32(t):
    return t.detach().cpu().numpy()


def assert_close(actual, expected, name, rtol=RTOL, atol=ATOL, max_outliers=0,
                 outlier_atol=None):
    """Elementwise |a - e| <= atol + rtol |e|.

    ``max_outliers`` entries may exceed that bound, but never ``outlier_atol``:
    used where a value within a few ulp of an alpha cut-off can be counted on
    one side by the kernel's exp and on the other by the oracle's.
    """
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    if a.size == 0:
        return
    assert np.array_equal(np.isnan(a), np.isnan(e)), f"{name}: NaN pattern differs"
    finite = ~np.isnan(e)
    err = np.abs(a - e)
    bad = (err > atol + rtol * np.abs(e)) & finite
    nbad = int(bad.sum())
    if nbad:
        worst = np.unravel_index(np.argmax(np.where(bad, err, -1)), a.shape)
        msg = (f"{name}: {nbad}/{a.size} outside rtol={rtol} atol={atol}; worst at {worst}: "
               f"actual={a[worst]!r} expected={e[worst]!r}")
        assert nbad <= max_outliers, msg
        if outlier_atol is not None:
            assert float(err[bad].max()) <= outlier_atol, msg


def assert_equal(actual, expected, name):
    a, e = np.asarray(actual), np.asarray(expected)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    diff = a != e
    if a.dtype.kind == "f":
        diff &= ~(np.isnan(a) & np.isnan(e))
    n = int(diff.sum())
    if n:
        idx = np.argwhere(diff)[0]
        raise AssertionError(f"{name}: {n}/{a.size} entries differ; first at {tuple(idx)}: "
                             f"{a[tuple(idx)]!r} vs {e[tuple(idx)]!r}")
