"""Config 5 (stress): 2M Gaussians, log-scales N(-5, 1) with needles, a
1024^2 detector and a 512^3 volume.

The lists are too long for the whole oracle (2.2e8 tile records), so parity
is checked on a sample of tiles / bricks (the most loaded one and random
others): their pixels / voxels, and the per-record partials of their records
as the two-pass backward stores them, against the oracle one precision up
(helpers.check_raster_sampled).  The whole tile / brick lists equal the
oracle's rectangle / box cover bit for bit, and the two-pass backward is
deterministic.

With 5 % needles the 512^3 volume needs 7.46e9 brick records (the needles'
bounding boxes span the volume), beyond the int32 tile offsets of the
reference and of its operator signature: isect_tiles_3d must fail cleanly
before allocating (r2splat.ops voxelizes that volume in z-slabs, checked in
test_gpu_slabs.py).  The volume with 0.05 % needles (2.5e8 records) runs as
one list.
"""

import math

import numpy as np
import pytest
import torch

from helpers import (RASTER_ROW_SLOTS, VOXEL_ROW_SLOTS, check_raster_sampled, check_voxel_sampled,
                     np32, sample_keys)
from oracle import binning
from r2splat import geometry, scenes
from r2splat.cuda import _backend, _ops
from r2splat.cuda import _wrapper as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
N5, DET5, VOX5 = 2_000_000, 1024, 512

# Needle-like footprints (axis ratio above 50, conic eigenvalue ratio above
# 2500) make sigma's terms cancel: any float32 evaluation of sigma errs by
# about u S, with S (the sum of |sigma's terms|) up to ~1e4, i.e. beyond the
# bar's 1e-4 relative, so such elements need the conditioning term (with
# err / (u |terms|) at most 1.6 measured).  Measured fractions of the
# conditioning + flip classes: projection record partials 1.5e-3, the 0.05 %
# needle volume's sampled voxels 1.1e-3.  The cap is about twice that.
NEEDLE_FRAC = 3e-3


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


def _project(d, degrees=123.0):
    vm, Ks = geometry.cone_beam_views([math.radians(degrees)], DET5)
    return W.project_gaussians_fwd(d["means"], d["covars"], d["opac"], vm.to(DEV), Ks.to(DEV),
                                   DET5, DET5, 1e-8, 3.0)


def _raster_rows(m2, con, op, mu, off, lists, v, W_, H_, ts):
    lib, P = _backend.library(), _ops._ptr
    n, C, N = lists.flatten_ids.numel(), m2.shape[0], m2.shape[1]
    rows = torch.empty(lib.r2s_rasterize_bwd_workspace_bytes(n, C * N, 4), dtype=torch.uint8,
                       device=DEV)
    tw, th = off.shape[2], off.shape[1]
    rc = lib.r2s_rasterize_bwd_rows_f32(P(m2), P(con), P(op), P(mu), P(off), P(lists.isect_ids),
                                        P(lists.flatten_ids), P(lists.isect_src), n, P(v), C, N,
                                        W_, H_, ts, tw, th, 1, P(rows), rows.numel(),
                                        torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.r2s_last_error()
    return rows.view(torch.float32)


def _sampled_rows(rows, lists, keys, off, slots):
    """Rows of the sampled tiles' records only (the whole table is GBs):
    (rows [n_sampled * slots], index of each list position's row in them)."""
    o = np32(off).reshape(-1).astype(np.int64)
    n = lists.flatten_ids.numel()
    pos = np.concatenate([np.arange(o[k], o[k + 1] if k + 1 < o.size else n) for k in keys])
    src = lists.isect_src[torch.from_numpy(pos).to(DEV)].long()
    sub = rows.view(-1, slots)[src].cpu().numpy()
    lookup = np.full(n, -1, np.int64)
    lookup[pos] = np.arange(pos.size)
    return sub.reshape(-1), lookup


@pytest.mark.parametrize("degrees", [123.0, 0.0, 90.0, 237.0])
def test_config5_projection_lists_render_and_backward(config5, degrees):
    # Four views: the sampled tiles' pixels and record partials at each; the
    # whole-list checks (numpy over 2e8 records) at the first.
    m2, _, radii, con, mu, op = _project(config5, degrees)
    nt = DET5 // 16
    lists = _ops.bin_tiles_2d(m2, radii, 16, nt, nt)
    ids, fl = lists.isect_ids, lists.flatten_ids
    off = W.isect_offset_encode(ids, 1, nt, nt)
    n = ids.numel()
    assert n > 2_000_000
    x0, x1, y0, y1, count = binning.tile_rects_2d(np32(m2), np32(radii), 16, nt, nt)
    assert np.array_equal(np32(lists.tiles_per_gauss).reshape(-1), count) and n == int(count.sum())
    print(f"{degrees} degrees: {n} tile records", flush=True)
    if degrees == 123.0:
        ids_n, fl_n = np32(ids), np32(fl).astype(np.int64)
        assert np.all((ids_n[1:] > ids_n[:-1])
                      | ((ids_n[1:] == ids_n[:-1]) & (fl_n[1:] > fl_n[:-1])))
        tx, ty = ids_n % nt, ids_n // nt
        assert np.all((tx >= x0[fl_n]) & (tx < x1[fl_n]) & (ty >= y0[fl_n]) & (ty < y1[fl_n]))
        assert np.array_equal(np32(off).reshape(-1),
                              np.searchsorted(ids_n, np.arange(nt * nt), "left"))
        del ids_n, fl_n, tx, ty

    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, DET5, DET5, 16)
    v = torch.randn((1, DET5, DET5), generator=torch.Generator().manual_seed(int(degrees))).to(DEV)
    rows = _raster_rows(m2, con, op, mu, off, lists, v, DET5, DET5, 16)
    keys = sample_keys(np32(off), n, 24, seed=5 + int(degrees))
    table, lookup = _sampled_rows(rows, lists, keys, off, RASTER_ROW_SLOTS)
    del rows
    reps = check_raster_sampled(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl),
                                np32(v), DET5, DET5, 16, keys, image=np32(img), rows=table,
                                isect_src=lookup, max_frac=NEEDLE_FRAC)
    for k, r in reps.items():
        print(k, r, flush=True)
    if degrees == 123.0:
        two = _ops.raster_backward(m2, con, op, mu, off, lists, v, DET5, DET5, 16, True)
        again = _ops.raster_backward(m2, con, op, mu, off, lists, v, DET5, DET5, 16, True)
        for a, b in zip(two, again):
            assert torch.equal(a, b)


def _voxel_rows(m3, con, op, off, lists, v, nb, key_offset=0):
    lib, P = _backend.library(), _ops._ptr
    n, N = lists.flatten_ids.numel(), m3.shape[0]
    rows = torch.empty(lib.r2s_voxelize_bwd_workspace_bytes(n, 4), dtype=torch.uint8,
                       device=DEV)
    n0 = off.shape[0]
    rc = lib.r2s_voxelize_bwd_rows_f32(P(m3), P(con), P(op), P(off), None, P(lists.flatten_ids),
                                       P(lists.isect_src), n, P(v), N, VOX5, VOX5, VOX5, 8, nb,
                                       nb, n0, P(rows), rows.numel(),
                                       torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.r2s_last_error()
    return rows.view(torch.float32)


def test_config5_voxel_lists_volume_and_backward():
    d = _config5(0.0005)
    m3, con, r3 = _map(d)
    nb = VOX5 // 8
    lists = _ops.bin_tiles_3d(m3, r3, 8, nb, nb, nb)
    ids, fl = lists.isect_ids, lists.flatten_ids
    off = W.isect_offset_encode_3d(ids, nb, nb, nb)
    ids_n, fl_n = np32(ids), np32(fl).astype(np.int64)
    n = ids_n.size
    assert n > 200_000_000
    lo, hi, count = binning.tile_boxes_3d(np32(m3), np32(r3), 8, nb, nb, nb)
    assert np.array_equal(np32(lists.tiles_per_gauss), count)
    assert np.all((ids_n[1:] > ids_n[:-1]) | ((ids_n[1:] == ids_n[:-1]) & (fl_n[1:] > fl_n[:-1])))
    b2, b1, b0 = ids_n % nb, (ids_n // nb) % nb, ids_n // (nb * nb)
    for axis, b in enumerate((b2, b1, b0)):
        assert np.all((b >= lo[axis][fl_n]) & (b < hi[axis][fl_n]))
    del ids_n, fl_n, b0, b1, b2

    vol = W.voxelize_to_voxels_fwd(m3, con, d["opac"], off, fl, VOX5, VOX5, VOX5, 8)
    v = torch.randn((VOX5, VOX5, VOX5), generator=d["g"]).to(DEV)
    rows = _voxel_rows(m3, con, d["opac"], off, lists, v, nb)
    keys = sample_keys(np32(off), n, 24, seed=6)
    table, lookup = _sampled_rows(rows, lists, keys, off, VOXEL_ROW_SLOTS)
    del rows
    reps = check_voxel_sampled(np32(m3), np32(con), np32(d["opac"]), np32(off), np32(fl),
                               np32(v), VOX5, VOX5, VOX5, 8, keys, volume=np32(vol), rows=table,
                               isect_src=lookup, max_frac=NEEDLE_FRAC)
    for k, r in reps.items():
        print(k, r, flush=True)
    two = _ops.voxel_backward(m3, con, d["opac"], off, lists, v, VOX5, VOX5, VOX5, 8)
    again = _ops.voxel_backward(m3, con, d["opac"], off, lists, v, VOX5, VOX5, VOX5, 8)
    for a, b in zip(two, again):
        assert torch.equal(a, b)
