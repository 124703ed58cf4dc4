"""Config 5 (stress): 2M Gaussians, log-scales N(-5, 1) with needles, a
1024^2 detector and a 512^3 volume.  Size-independent properties, as at
configs 3 and 4: the tile and brick lists equal the oracle's rectangle / box
cover bit-exactly, renders are additive over a split of the Gaussians, and
the two-pass backward is deterministic and agrees with the one-pass kernels.

With 5 % needles the 512^3 volume needs 7.46e9 brick records (the needles'
bounding boxes span the volume), beyond the int32 tile offsets of the
reference and of this library: that case must fail cleanly before allocating.
The volume properties are checked with 0.05 % needles (2.5e8 records)."""

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
N5, DET5, VOX5 = 2_000_000, 1024, 512


def _config5(needle_fraction):
    g = torch.Generator().manual_seed(5)
    raw = scenes.stress_gaussians(N5, g, needle_fraction=needle_fraction)
    covars, max_scales, opac = W.prepare_gaussians(raw.quats.to(DEV), raw.raw_scales.to(DEV),
                                                   raw.raw_opacities.to(DEV), 5e-4, 1.0)
    return dict(means=raw.means.to(DEV), covars=covars, max_scales=max_scales, opac=opac, g=g)


@pytest.fixture(scope="module")
def config5():
    return _config5(0.05)


def _map(d):
    return W.world_to_volume_mapping_fwd(
        d["means"], d["covars"], d["max_scales"], torch.full((3,), 2.0, device=DEV),
        torch.zeros(3, device=DEV), VOX5, VOX5, VOX5, 1e-8, 3.0)


def test_config5_volume_beyond_the_record_range_fails_cleanly(config5):
    m3, _, r3 = _map(config5)
    nb = VOX5 // 8
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    with pytest.raises(RuntimeError, match="exceed the int32 offset range"):
        W.isect_tiles_3d(m3, r3, 8, nb, nb, nb)
    assert torch.cuda.memory_allocated() - before < 2 ** 30


def _project(d):
    vm, Ks = geometry.cone_beam_views([math.radians(123.0)], DET5)
    return W.project_gaussians_fwd(d["means"], d["covars"], d["opac"], vm.to(DEV), Ks.to(DEV),
                                   DET5, DET5, 1e-8, 3.0)


def test_config5_projection_lists_render_and_backward(config5):
    m2, _, radii, con, mu, op = _project(config5)
    nt = DET5 // 16
    tpg, ids, fl = W.isect_tiles(m2, radii, 16, nt, nt)
    off = W.isect_offset_encode(ids, 1, nt, nt)
    n = ids.numel()
    assert n > 2_000_000
    x0, x1, y0, y1, count = binning.tile_rects_2d(np32(m2), np32(radii), 16, nt, nt)
    assert np.array_equal(np32(tpg).reshape(-1), count) and n == int(count.sum())
    ids_n, fl_n = np32(ids), np32(fl).astype(np.int64)
    assert np.all((ids_n[1:] > ids_n[:-1]) | ((ids_n[1:] == ids_n[:-1]) & (fl_n[1:] > fl_n[:-1])))
    tx, ty = ids_n % nt, ids_n // nt
    assert np.all((tx >= x0[fl_n]) & (tx < x1[fl_n]) & (ty >= y0[fl_n]) & (ty < y1[fl_n]))
    assert np.array_equal(np32(off).reshape(-1), np.searchsorted(ids_n, np.arange(nt * nt), "left"))

    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, DET5, DET5, 16)
    parts = []
    for half in (torch.arange(0, N5, 2, device=DEV), torch.arange(1, N5, 2, device=DEV)):
        sel = lambda t: t[:, half].contiguous()  # noqa: E731
        _, i2, f2 = W.isect_tiles(sel(m2), sel(radii), 16, nt, nt)
        o2 = W.isect_offset_encode(i2, 1, nt, nt)
        parts.append(W.rasterize_to_pixels_fwd(sel(m2), sel(con), sel(op), sel(mu), o2, f2, DET5,
                                               DET5, 16))
    scale = float(img.abs().max())
    assert scale > 0
    assert_close(np32(parts[0] + parts[1]), np32(img), "image(A) + image(B)", rtol=1e-4,
                 atol=max(1e-5, 1e-6 * scale), max_outliers=img.numel() // 10_000,
                 outlier_atol=3e-5)

    v = torch.randn((1, DET5, DET5), generator=config5["g"]).to(DEV)
    two = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v, DET5, DET5, 16,
                                                 True)
    again = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v, DET5, DET5,
                                                   16, True)
    for a, b in zip(two, again):
        assert torch.equal(a, b)
    one = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl.clone(), v, DET5,
                                                 DET5, 16, True)
    for x, y, name in zip(one, two, ("abs", "xy", "conic", "opac", "mu")):
        e = np32(y)
        s = float(np.abs(e).max()) + 1e-30
        assert_close(np32(x), e, f"one-pass vs two-pass {name}", rtol=1e-4,
                     atol=max(1e-5, 3e-6 * s), max_outliers=e.size // 10_000,
                     outlier_atol=1e-4 * s)


def test_config5_voxel_lists_volume_and_backward():
    d = _config5(0.0005)
    m3, con, r3 = _map(d)
    nb = VOX5 // 8
    tpg, ids, fl = W.isect_tiles_3d(m3, r3, 8, nb, nb, nb)
    off = W.isect_offset_encode_3d(ids, nb, nb, nb)
    ids_n, fl_n = np32(ids), np32(fl).astype(np.int64)
    assert ids_n.size > 200_000_000
    lo, hi, count = binning.tile_boxes_3d(np32(m3), np32(r3), 8, nb, nb, nb)
    assert np.array_equal(np32(tpg), count)
    assert np.all((ids_n[1:] > ids_n[:-1]) | ((ids_n[1:] == ids_n[:-1]) & (fl_n[1:] > fl_n[:-1])))
    b2, b1, b0 = ids_n % nb, (ids_n // nb) % nb, ids_n // (nb * nb)
    for axis, b in enumerate((b2, b1, b0)):
        assert np.all((b >= lo[axis][fl_n]) & (b < hi[axis][fl_n]))
    del ids_n, fl_n, b0, b1, b2

    vol = W.voxelize_to_voxels_fwd(m3, con, d["opac"], off, fl, VOX5, VOX5, VOX5, 8)
    assert vol.shape == (VOX5, VOX5, VOX5) and bool(torch.isfinite(vol).all())
    assert float(vol.abs().max()) > 0
    v = torch.randn((VOX5, VOX5, VOX5), generator=d["g"]).to(DEV)
    two = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, d["opac"], off, ids, fl, v, VOX5, VOX5,
                                                VOX5, 8)
    again = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, d["opac"], off, ids, fl, v, VOX5,
                                                  VOX5, VOX5, 8)
    for a, b in zip(two, again):
        assert torch.equal(a, b)
    one = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, d["opac"], off, ids, fl.clone(), v,
                                                VOX5, VOX5, VOX5, 8)
    for x, y, name in zip(one, two, ("v_means3d", "v_conics", "v_opacities")):
        e = np32(y)
        s = float(np.abs(e).max()) + 1e-30
        assert_close(np32(x), e, f"one-pass vs two-pass {name}", rtol=1e-4,
                     atol=max(1e-5, 3e-6 * s), max_outliers=e.size // 10_000,
                     outlier_atol=1e-4 * s)
