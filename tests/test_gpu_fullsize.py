"""Size-independent properties at BASELINE's full sizes (config 4 and 3).

The oracle's rasterizer and voxelizer need minutes at these sizes, so parity
here rests on properties that hold exactly or up to summation order:

* the tile lists equal the cover of the oracle's per-Gaussian rectangles /
  boxes (count per Gaussian, membership of every record, no duplicates,
  (key, id) order, offsets = lower bounds) -- bit-exact;
* renders are additive over a split of the Gaussians;
* the backward is linear in the upstream gradient;
* the two backward orders (atomic one-pass, two-pass) agree, and the
  two-pass result is identical run to run.
"""

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, np32
from oracle import binning
from r2splat import geometry, scenes
from r2splat.cuda import _wrapper as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
SMIN, SMAX = 5e-4, 1.0


@pytest.fixture(scope="module")
def config4():
    g = torch.Generator().manual_seed(0)
    raw = scenes.binary_tree_gaussians(500_000, g, opacity="uniform")
    vm, Ks = geometry.cone_beam_views([math.radians(37.0)], 512)
    covars, _, opac = W.prepare_gaussians(raw.quats.to(DEV), raw.raw_scales.to(DEV),
                                          raw.raw_opacities.to(DEV), SMIN, SMAX)
    m2, cov2d, radii, conics, mus, op = W.project_gaussians_fwd(
        raw.means.to(DEV), covars, opac, vm.to(DEV), Ks.to(DEV), 512, 512, 1e-8, 3.0)
    v = torch.randn((2, 1, 512, 512), generator=g).to(DEV)
    return dict(m2=m2, radii=radii, conics=conics, mus=mus, op=op, v=v)


def _bin2d(d, idx=None):
    sel = (lambda t: t) if idx is None else (lambda t: t[:, idx].contiguous())
    m2, r = sel(d["m2"]), sel(d["radii"])
    tpg, ids, fl = W.isect_tiles(m2, r, 16, 32, 32)
    off = W.isect_offset_encode(ids, 1, 32, 32)
    return sel, tpg, ids, fl, off


def test_config4_tile_lists_equal_the_rectangle_cover(config4):
    _, tpg, ids, fl, off = _bin2d(config4)
    n = ids.numel()
    assert n > 1_000_000
    x0, x1, y0, y1, count = binning.tile_rects_2d(np32(config4["m2"]), np32(config4["radii"]),
                                                  16, 32, 32)
    assert np.array_equal(np32(tpg).reshape(-1), count)
    assert n == int(count.sum())
    ids_n, fl_n = np32(ids), np32(fl).astype(np.int64)
    assert np.all((ids_n[1:] > ids_n[:-1]) | ((ids_n[1:] == ids_n[:-1]) & (fl_n[1:] > fl_n[:-1])))
    tx, ty = ids_n % 32, ids_n // 32
    assert np.all((tx >= x0[fl_n]) & (tx < x1[fl_n]) & (ty >= y0[fl_n]) & (ty < y1[fl_n]))
    assert np.array_equal(np.bincount(fl_n, minlength=count.size), count)
    assert np.array_equal(np32(off).reshape(-1), np.searchsorted(ids_n, np.arange(1024), "left"))


def _raster(d, idx=None):
    sel, _, ids, fl, off = _bin2d(d, idx)
    img = W.rasterize_to_pixels_fwd(sel(d["m2"]), sel(d["conics"]), sel(d["op"]), sel(d["mus"]),
                                    off, fl, 512, 512, 16)
    return img, (sel, ids, fl, off)


def test_config4_render_is_additive(config4):
    whole, _ = _raster(config4)
    n = config4["m2"].shape[1]
    even = torch.arange(0, n, 2, device=DEV)
    odd = torch.arange(1, n, 2, device=DEV)
    parts = _raster(config4, even)[0] + _raster(config4, odd)[0]
    scale = float(whole.abs().max())
    assert scale > 0
    assert_close(np32(parts), np32(whole), "image(A) + image(B)", rtol=1e-4,
                 atol=max(1e-5, 1e-6 * scale), max_outliers=whole.numel() // 10_000,
                 outlier_atol=3e-5)


def _raster_bwd(d, lists, v, clone=False):
    sel, ids, fl, off = lists
    fl = fl.clone() if clone else fl
    return W.rasterize_to_pixels_bwd_per_gaussian(sel(d["m2"]), sel(d["conics"]), sel(d["op"]),
                                                  sel(d["mus"]), off, ids, fl, v, 512, 512, 16,
                                                  True)


RASTER_GRADS = ("v_means2d_abs", "v_means2d", "v_conics", "v_opacities", "v_mus")


def _close_grads(a, b, what, names=RASTER_GRADS):
    for x, y, n in zip(a, b, names):
        e = np32(y)
        scale = float(np.abs(e).max()) + 1e-30
        assert_close(np32(x), e, f"{what} {n}", rtol=1e-4, atol=max(1e-5, 3e-6 * scale),
                     max_outliers=e.size // 10_000, outlier_atol=1e-4 * scale)


def test_config4_backward_orders_agree_and_two_pass_is_deterministic(config4):
    _, lists = _raster(config4)
    v = config4["v"][0]
    two = _raster_bwd(config4, lists, v)
    again = _raster_bwd(config4, lists, v)
    for a, b in zip(two, again):
        assert torch.equal(a, b)
    one = _raster_bwd(config4, lists, v, clone=True)
    _close_grads(one, two, "one-pass vs two-pass")


def test_config4_backward_is_linear_in_the_upstream_gradient(config4):
    _, lists = _raster(config4)
    v1, v2 = config4["v"][0], config4["v"][1]
    g1, g2 = _raster_bwd(config4, lists, v1), _raster_bwd(config4, lists, v2)
    g12 = _raster_bwd(config4, lists, v1 + v2)
    # The absolute-value partials are not linear; the other four are.
    _close_grads(g12[1:], [b + c for b, c in zip(g1[1:], g2[1:])], "g(v1+v2) vs g(v1)+g(v2)",
                 RASTER_GRADS[1:])


@pytest.fixture(scope="module")
def config3():
    g = torch.Generator().manual_seed(1)
    raw = scenes.random_gaussians(200_000, g, -4.5, 0.6)
    covars, max_scales, opac = W.prepare_gaussians(raw.quats.to(DEV), raw.raw_scales.to(DEV),
                                                   raw.raw_opacities.to(DEV), SMIN, SMAX)
    m3, con, r3 = W.world_to_volume_mapping_fwd(
        raw.means.to(DEV), covars, max_scales, torch.full((3,), 2.0, device=DEV),
        torch.zeros(3, device=DEV), 256, 256, 256, 1e-8, 3.0)
    v = torch.randn((256, 256, 256), generator=g).to(DEV)
    return dict(m3=m3, con=con, r3=r3, op=opac, v=v)


def _voxel(d, idx=None):
    sel = (lambda t: t) if idx is None else (lambda t: t[idx].contiguous())
    tpg, ids, fl = W.isect_tiles_3d(sel(d["m3"]), sel(d["r3"]), 8, 32, 32, 32)
    off = W.isect_offset_encode_3d(ids, 32, 32, 32)
    vol = W.voxelize_to_voxels_fwd(sel(d["m3"]), sel(d["con"]), sel(d["op"]), off, fl, 256, 256,
                                   256, 8)
    return vol, (sel, tpg, ids, fl, off)


def test_config3_brick_lists_equal_the_box_cover(config3):
    _, (_, tpg, ids, fl, off) = _voxel(config3)
    ids_n, fl_n = np32(ids), np32(fl).astype(np.int64)
    assert ids_n.size > 1_000_000
    lo, hi, count = binning.tile_boxes_3d(np32(config3["m3"]), np32(config3["r3"]), 8, 32, 32, 32)
    assert np.array_equal(np32(tpg), count)
    assert np.all((ids_n[1:] > ids_n[:-1]) | ((ids_n[1:] == ids_n[:-1]) & (fl_n[1:] > fl_n[:-1])))
    b2, b1, b0 = ids_n % 32, (ids_n // 32) % 32, ids_n // 1024
    for axis, b in enumerate((b2, b1, b0)):
        assert np.all((b >= lo[axis][fl_n]) & (b < hi[axis][fl_n]))
    assert np.array_equal(np.bincount(fl_n, minlength=count.size), count)
    assert np.array_equal(np32(off).reshape(-1),
                          np.searchsorted(ids_n, np.arange(32 ** 3), "left"))


def test_config3_volume_is_additive(config3):
    whole, _ = _voxel(config3)
    n = config3["m3"].shape[0]
    parts = (_voxel(config3, torch.arange(0, n, 2, device=DEV))[0] +
             _voxel(config3, torch.arange(1, n, 2, device=DEV))[0])
    scale = float(whole.abs().max())
    assert scale > 0
    assert_close(np32(parts), np32(whole), "volume(A) + volume(B)", rtol=1e-4,
                 atol=max(1e-5, 1e-6 * scale), max_outliers=whole.numel() // 10_000,
                 outlier_atol=3e-6)


def test_config3_backward_orders_agree_and_two_pass_is_deterministic(config3):
    _, (sel, _, ids, fl, off) = _voxel(config3)
    d = config3

    def bwd(f):
        return W.voxelize_to_voxels_bwd_per_gaussian(d["m3"], d["con"], d["op"], off, ids, f,
                                                     d["v"], 256, 256, 256, 8)

    two, again, one = bwd(fl), bwd(fl), bwd(fl.clone())
    for a, b in zip(two, again):
        assert torch.equal(a, b)
    for x, y, n in zip(one, two, ("v_means3d", "v_conics", "v_opacities")):
        e = np32(y)
        scale = float(np.abs(e).max()) + 1e-30
        assert_close(np32(x), e, f"one-pass vs two-pass {n}", rtol=1e-4,
                     atol=max(1e-5, 3e-6 * scale), max_outliers=e.size // 10_000,
                     outlier_atol=1e-4 * scale)
