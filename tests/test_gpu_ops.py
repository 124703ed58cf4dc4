"""HIP operators vs the CPU oracle on seeded inputs (op level).

Bit-exact where the kernel has no transcendental function (projection,
conics/mu, volume mapping, their VJPs, binning, offsets, compaction).
Otherwise every output is checked against the oracle one precision up with
helpers.assert_parity: rel 1e-4 / abs 1e-5 in float32 (rel 1e-9 / abs
1e-12 in float64), or within twice the reference order's own error, plus
the flip band of terms at an alpha cut-off (flips are counted).  Every call
goes through the C ABI via r2splat.cuda._wrapper or r2splat.cuda._ops.
"""

import numpy as np
import pytest
import torch

from helpers import (assert_close, assert_equal, assert_parity, check_raster, check_voxel,
                     make_scene, np32, raster_references, voxel_references)
from oracle import binning, native, ops
from r2splat.cuda import _ops
from r2splat.cuda import _wrapper as W

pytestmark = pytest.mark.gpu


def fl_keys(tile_offsets):
    """Number of tile / brick keys of a tile_offsets tensor."""
    return tile_offsets.numel()

DEV = "cuda"


def _prepared(n, seed, dtype=torch.float32, **kw):
    raw, viewmats, Ks, g = make_scene(n, seed, **kw)
    covars, max_scales = ops.parameter_transform_fwd(
        raw.quats.double().numpy(), raw.raw_scales.double().numpy(), 5e-4, 1.0)
    t = lambda a: torch.as_tensor(a, dtype=dtype, device=DEV).contiguous()  # noqa: E731
    return dict(raw=raw, means=t(raw.means.numpy()), covars=t(covars), viewmats=t(viewmats),
                Ks=t(Ks), opac=t(ops.softplus(raw.raw_opacities.double().numpy())), gen=g)


def test_library_loaded():
    assert W.is_cuda_extension_available(), "libr2splat_hip.so failed to load"


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_parameter_transform(dtype):
    raw, _, _, g = make_scene(3000, 1)
    q = raw.quats.to(dtype) * 0.7
    s = raw.raw_scales.to(dtype)
    o = raw.raw_opacities.to(dtype)
    qd, sd, od = q.to(DEV), s.to(DEV), o.to(DEV)
    cov, ms = W.parameter_transform_fwd(qd, sd, 5e-4, 1.0)
    hi = np.float64 if dtype == torch.float32 else np.longdouble
    cov_o, ms_o = ops.parameter_transform_fwd(q.numpy(), s.numpy(), 5e-4, 1.0)
    cov_a, ms_a = ops.parameter_transform_fwd(q.numpy().astype(hi), s.numpy().astype(hi), 5e-4,
                                              1.0)
    assert_parity(np32(cov), cov_a, cov_o, None, "covars")
    assert_parity(np32(ms), ms_a, ms_o, None, "max_scales")
    cov2, ms2, op2 = W.prepare_gaussians(qd, sd, od, 5e-4, 1.0)
    assert_equal(np32(cov2), np32(cov), "fused covars")
    assert_equal(np32(ms2), np32(ms), "fused max_scales")
    assert_parity(np32(op2), ops.softplus(o.numpy().astype(hi)), ops.softplus(o.numpy()), None,
                  "softplus")
    v = torch.randn(3000, 6, generator=g, dtype=dtype)
    vq, vs = W.parameter_transform_bwd(qd, sd, 5e-4, 1.0, v.to(DEV))
    vq_o, vs_o = ops.parameter_transform_bwd(q.numpy(), s.numpy(), 5e-4, 1.0, v.numpy())
    vq_a, vs_a = ops.parameter_transform_bwd(q.numpy().astype(hi), s.numpy().astype(hi), 5e-4,
                                             1.0, v.numpy().astype(hi))
    assert_parity(np32(vq), vq_a, vq_o, None, "v_quats")
    assert_parity(np32(vs), vs_a, vs_o, None, "v_raw_scales")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n_views", [1, 3])
def test_projection_bit_exact(dtype, n_views):
    d = _prepared(4000, 2, dtype, n_det=96, n_views=n_views)
    m2, c2, r = W.world_to_image_projection_fwd(d["means"], d["covars"], d["viewmats"], d["Ks"],
                                                96, 96, 1e-8, 3.0)
    m2o, c2o, ro = ops.world_to_image_projection_fwd(np32(d["means"]), np32(d["covars"]),
                                                     np32(d["viewmats"]), np32(d["Ks"]), 96, 96,
                                                     1e-8, 3.0)
    assert_equal(np32(m2), m2o, "means2d")
    assert_equal(np32(c2), c2o, "cov2d")
    assert_equal(np32(r), ro, "radii")
    assert int((ro > 0).any(-1).sum()) > 100
    con, mu = W.conics_mu_fwd(c2, 1e-8)
    cono, muo = ops.conics_mu_fwd(c2o, 1e-8)
    assert_equal(np32(con), cono, "conics")
    assert_equal(np32(mu), muo, "mus")
    # Fused forward = the three separate passes.
    fm2, fc2, fr, fcon, fmu, fop = W.project_gaussians_fwd(
        d["means"], d["covars"], d["opac"], d["viewmats"], d["Ks"], 96, 96, 1e-8, 3.0)
    for a, b, n in ((fm2, m2, "means2d"), (fc2, c2, "cov2d"), (fr, r, "radii"),
                    (fcon, con, "conics"), (fmu, mu, "mus")):
        assert_equal(np32(a), np32(b), f"fused {n}")
    assert_equal(np32(fop), np.broadcast_to(np32(d["opac"]), fop.shape), "opacity[C,N]")
    # VJPs.
    g = d["gen"]
    C, N = n_views, 4000
    vm2 = torch.randn(C, N, 2, generator=g, dtype=dtype)
    vcon = torch.randn(C, N, 3, generator=g, dtype=dtype)
    vmu = torch.randn(C, N, generator=g, dtype=dtype)
    vcov = W.conics_mu_bwd(c2, 1e-8, con, mu, vcon.to(DEV), vmu.to(DEV))
    vcovo = ops.conics_mu_bwd(c2o, 1e-8, cono, muo, vcon.numpy(), vmu.numpy())
    assert_equal(np32(vcov), vcovo, "v_cov2d")
    vmean, vcovar = W.world_to_image_projection_bwd(d["means"], d["covars"], d["viewmats"],
                                                    d["Ks"], 96, 96, vm2.to(DEV), vcov)
    vmeano, vcovaro = ops.world_to_image_projection_bwd(
        np32(d["means"]), np32(d["covars"]), np32(d["viewmats"]), np32(d["Ks"]), 96, 96,
        vm2.numpy(), vcovo)
    assert_equal(np32(vmean), vmeano, "v_means")
    assert_equal(np32(vcovar), vcovaro, "v_covars")
    fvm, fvc = W.project_gaussians_bwd(d["means"], d["covars"], d["viewmats"], d["Ks"], 96, 96,
                                       1e-8, c2, con, mu, vm2.to(DEV), vcon.to(DEV), vmu.to(DEV))
    assert_equal(np32(fvm), vmeano, "fused v_means")
    assert_equal(np32(fvc), vcovaro, "fused v_covars")


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n_views", [1, 3])
@pytest.mark.parametrize("with_volume", [False, True])
def test_explicit_backward_tail_equals_the_three_ops(dtype, n_views, with_volume):
    # One kernel for project_gaussians_bwd (+ the volume's world-space
    # gradients), parameter_transform_bwd and opacity_bwd: bit-identical to
    # the three ops in turn, with v_covars = image + volume.
    d = _prepared(4000, 5, dtype, n_det=96, n_views=n_views)
    raw = d["raw"]
    quats = raw.quats.to(dtype).to(DEV).contiguous()
    scales = raw.raw_scales.to(dtype).to(DEV).contiguous()
    ropac = raw.raw_opacities.to(dtype).to(DEV).contiguous()
    m2, c2, r, con, mu, op = W.project_gaussians_fwd(d["means"], d["covars"], d["opac"],
                                                     d["viewmats"], d["Ks"], 96, 96, 1e-8, 3.0)
    g = torch.Generator().manual_seed(17)
    C, N = n_views, 4000
    rnd = lambda *shape: torch.randn(*shape, generator=g, dtype=dtype).to(DEV)  # noqa: E731
    vm2, vcon, vmu, vop = rnd(C, N, 2), rnd(C, N, 3), rnd(C, N), rnd(C, N)
    add_m, add_c, vop3 = (rnd(N, 3), rnd(N, 6), rnd(N)) if with_volume else (None, None, None)
    got = _ops.explicit_backward_tail(d["means"], d["covars"], d["viewmats"], d["Ks"], 96, 96,
                                      1e-8, c2, con, mu, vm2, vcon, vmu, add_m, add_c, quats,
                                      scales, 5e-4, 1.0, ropac, vop, vop3)
    vm, vc = _ops.project_gaussians_bwd(d["means"], d["covars"], d["viewmats"], d["Ks"], 96, 96,
                                        1e-8, c2, con, mu, vm2, vcon, vmu)
    if with_volume:
        vm, vc = vm + add_m, vc + add_c
    vq, vs = _ops.parameter_transform_bwd(quats, scales, 5e-4, 1.0, vc)
    vo = _ops.opacity_bwd(ropac, vop, vop3)
    for a, b, n in zip(got, (vm, vq, vs, vo), ("v_means", "v_quats", "v_raw_scales", "v_raw_opac")):
        assert torch.equal(a, b), n
    assert float(vq.abs().max()) > 0 and float(vo.abs().max()) > 0


@pytest.mark.parametrize("rect", [True, False])
@pytest.mark.parametrize("n_views", [1, 2])
def test_isect_tiles_bit_exact(rect, n_views):
    d = _prepared(6000, 3, n_det=100, n_views=n_views, log_mu=-3.5)
    m2, _, r, _, _, _ = W.project_gaussians_fwd(d["means"], d["covars"], d["opac"],
                                                d["viewmats"], d["Ks"], 100, 100, 1e-8, 3.0)
    radii = r if rect else r.amax(-1).contiguous()
    tw = th = 7
    tpg, ids, fl = W.isect_tiles(m2, radii, 16, tw, th)
    tpg_o, ids_o, fl_o = binning.isect_tiles(np32(m2), np32(radii), 16, tw, th)
    assert ids_o.size > 1000
    assert_equal(np32(tpg), tpg_o, "tiles_per_gauss")
    assert_equal(np32(ids), ids_o, "isect_ids")
    assert_equal(np32(fl), fl_o, "flatten_ids")
    off = W.isect_offset_encode(ids, n_views, tw, th)
    assert_equal(np32(off), binning.isect_offset_encode(ids_o, n_views, tw, th), "tile_offsets")
    # The offsets the sort writes itself (r2splat.ops uses them).
    lists = _ops.bin_tiles_2d(m2, radii, 16, tw, th)
    assert_equal(np32(lists.tile_offsets), binning.isect_offset_encode(ids_o, n_views, tw, th),
                 "sort tile_offsets")


def test_isect_tiles_large_footprints_and_degenerate():
    # Huge radii, non-finite means and zero radii: the emit loop and clamps.
    g = torch.Generator().manual_seed(4)
    N = 5000
    m2 = (torch.rand(1, N, 2, generator=g) * 1400 - 200).float()
    r = torch.randint(0, 400, (1, N, 2), generator=g).int()
    m2[0, :7, 0] = float("nan")
    m2[0, 7:14, 1] = float("inf")
    r[0, 14:40] = 0
    m2d, rd = m2.to(DEV), r.to(DEV)
    tpg, ids, fl = W.isect_tiles(m2d, rd, 16, 64, 64)
    tpg_o, ids_o, fl_o = binning.isect_tiles(m2.numpy(), r.numpy(), 16, 64, 64)
    assert ids_o.size > 1_000_000
    assert_equal(np32(tpg), tpg_o, "tiles_per_gauss")
    assert_equal(np32(ids), ids_o, "isect_ids")
    assert_equal(np32(fl), fl_o, "flatten_ids")


def test_isect_tiles_empty():
    m2 = torch.zeros(1, 10, 2, device=DEV)
    r = torch.zeros(1, 10, 2, dtype=torch.int32, device=DEV)
    tpg, ids, fl = W.isect_tiles(m2, r, 16, 4, 4)
    assert ids.numel() == 0 and fl.numel() == 0 and int(tpg.abs().sum()) == 0
    off = W.isect_offset_encode(ids, 1, 4, 4)
    assert off.shape == (1, 4, 4) and int(off.abs().sum()) == 0
    tpg, ids, fl = W.isect_tiles(torch.zeros(1, 0, 2, device=DEV),
                                 torch.zeros(1, 0, 2, dtype=torch.int32, device=DEV), 16, 4, 4)
    assert tpg.shape == (1, 0) and ids.numel() == 0


def test_isect_tiles_3d_bit_exact():
    d = _prepared(5000, 5, log_mu=-3.0)
    ranges = torch.full((3,), 2.0, device=DEV)
    centers = torch.zeros(3, device=DEV)
    m3, con, r3 = W.world_to_volume_mapping_fwd(d["means"], d["covars"], d["opac"], ranges,
                                                centers, 40, 36, 44, 1e-8, 3.0)
    n2, n1, n0 = 5, 5, 6
    tpg, ids, fl = W.isect_tiles_3d(m3, r3, 8, n2, n1, n0)
    tpg_o, ids_o, fl_o = binning.isect_tiles_3d(np32(m3), np32(r3), 8, n2, n1, n0)
    assert ids_o.size > 5000
    assert_equal(np32(tpg), tpg_o, "tiles_per_gauss")
    assert_equal(np32(ids), ids_o, "isect_ids")
    assert_equal(np32(fl), fl_o, "flatten_ids")
    off = W.isect_offset_encode_3d(ids, n2, n1, n0)
    assert_equal(np32(off), binning.isect_offset_encode_3d(ids_o, n2, n1, n0), "tile_offsets")
    lists = _ops.bin_tiles_3d(m3, r3, 8, n2, n1, n0)
    assert_equal(np32(lists.tile_offsets), binning.isect_offset_encode_3d(ids_o, n2, n1, n0),
                 "sort tile_offsets")


@pytest.mark.parametrize("tiles,views", [((1, 1), 1), ((32, 32), 2), ((45, 46), 1)])
def test_isect_tiles_sort_widths(tiles, views):
    # Key widths 0 bits (one tile), 11 bits (2048 keys, the widest one-pass
    # sort) and 12 bits (two passes).
    tw, th = tiles
    g = torch.Generator().manual_seed(11 + tw)
    N = 4000
    m2 = (torch.rand(views, N, 2, generator=g) * torch.tensor([16.0 * tw, 16.0 * th])).float()
    r = torch.randint(0, 40, (views, N, 2), generator=g).int()
    tpg, ids, fl = W.isect_tiles(m2.to(DEV), r.to(DEV), 16, tw, th)
    tpg_o, ids_o, fl_o = binning.isect_tiles(m2.numpy(), r.numpy(), 16, tw, th)
    assert ids_o.size > 3000
    assert_equal(np32(tpg), tpg_o, "tiles_per_gauss")
    assert_equal(np32(ids), ids_o, "isect_ids")
    assert_equal(np32(fl), fl_o, "flatten_ids")
    off = W.isect_offset_encode(ids, views, tw, th)
    assert_equal(np32(off), binning.isect_offset_encode(ids_o, views, tw, th), "tile_offsets")
    # From the one pass's digit offsets (1 and 2048 keys) or, with two
    # passes, searched after the sort.
    lists = _ops.bin_tiles_2d(m2.to(DEV), r.to(DEV), 16, tw, th)
    assert_equal(np32(lists.tile_offsets), binning.isect_offset_encode(ids_o, views, tw, th),
                 "sort tile_offsets")


def test_isect_tiles_capacity_guess():
    # Later calls with the same sizes allocate from the recent record counts
    # and launch the emit + sort before reading their count back; a count
    # above the guess relaunches with exact sizes.  Every result equals the
    # oracle's, and the backward reads the leading-record views correctly.
    _ops._COUNT_HISTORY.clear()
    g = torch.Generator().manual_seed(21)
    N = 3000
    m2 = (torch.rand(1, N, 2, generator=g) * 512).float()
    con = torch.tensor([0.02, 0.003, 0.03]).repeat(1, N, 1)
    op = torch.rand(1, N, generator=g) + 0.1
    mu = torch.rand(1, N, generator=g)
    v = torch.randn(1, 512, 512, generator=g).to(DEV)
    guessed = []
    for scale in (20, 10, 60, 60, 5):
        r = torch.randint(0, scale, (1, N, 2), generator=g).int()
        # isect_tiles' own steps, keeping the lists for their tile offsets.
        binned = _ops.bin_tiles_2d(m2.to(DEV), r.to(DEV), 16, 32, 32)
        _ops._remember_emission(binned, 1024)
        tpg, ids, fl = binned.tiles_per_gauss, binned.isect_ids, binned.flatten_ids
        tpg_o, ids_o, fl_o = binning.isect_tiles(m2.numpy(), r.numpy(), 16, 32, 32)
        assert_equal(np32(tpg), tpg_o, "tiles_per_gauss")
        assert_equal(np32(ids), ids_o, "isect_ids")
        assert_equal(np32(fl), fl_o, "flatten_ids")
        guessed.append(ids.untyped_storage().nbytes() > 8 * ids.numel())
        off = W.isect_offset_encode(ids, 1, 32, 32)
        assert torch.equal(binned.tile_offsets, off)
        args = (m2.to(DEV), con.to(DEV), op.to(DEV), mu.to(DEV), off)
        got = W.rasterize_to_pixels_bwd_per_gaussian(*args, ids, fl, v, 512, 512, 16, True)
        # The same records in exact-size tensors, with the same emission order.
        emit_ids, src = _ops.emission_order(fl, 1024)
        lists = _ops.TileLists(tpg, ids.clone(), fl.clone(), emit_ids.clone(), src.clone())
        want = _ops.raster_backward(*args, lists, v, 512, 512, 16, True)
        for a, b in zip(got, want):
            assert torch.equal(a, b)
    # First call exact; the third (60 > the guess from 20 and 10) relaunched.
    assert guessed == [False, True, False, True, True]


@pytest.mark.parametrize("n_tiles", [(32, 32), (64, 48)])
def test_isect_emit_sort_guessed_capacity_without_records(n_tiles):
    # A capacity guessed before the count is known, and no records on the
    # device: the emit + sort entry must still write the tile offsets that
    # r2s_isect_offset_encode gives for an empty list (all zeros), with one
    # sort pass (1024 tiles) and with two (3072 tiles).
    tw, th = n_tiles
    lib = _ops._lib()
    C, N, cap = 1, 2000, 5000
    m2 = torch.rand(1, N, 2, device=DEV) * 512
    radii = torch.zeros(1, N, 2, dtype=torch.int32, device=DEV)
    st = _ops._stream(torch.device(DEV))
    tpg = torch.empty(C * N, dtype=torch.int32, device=DEV)
    offsets = torch.empty(C * N + 1, dtype=torch.int64, device=DEV)
    ws = _ops._workspace(lib.r2s_isect_workspace_bytes(C * N, 0, 0), m2.device)
    _ops._call("r2s_isect_count_2d_f32", _ops._ptr(m2), _ops._ptr(radii), 1, C, N, 16, tw, th,
               _ops._ptr(tpg), _ops._ptr(offsets), _ops._ptr(ws), ws.numel(), st)
    end_bit = _ops._end_bit(C * tw * th)
    outs = [torch.empty(cap, dtype=d, device=DEV)
            for d in (torch.int64, torch.int32, torch.int32, torch.int32)]
    tile_offsets = torch.full((C, th, tw), -7, dtype=torch.int32, device=DEV)
    ws2 = _ops._workspace(lib.r2s_isect_workspace_bytes(0, cap, end_bit), m2.device)
    _ops._call("r2s_isect_emit_sort_2d_f32", _ops._ptr(m2), _ops._ptr(radii), 1, C, N, 16, tw, th,
               _ops._ptr(offsets), cap, end_bit, *[_ops._ptr(t) for t in outs],
               _ops._ptr(tile_offsets), _ops._ptr(ws2), ws2.numel(), st)
    empty = W.isect_offset_encode(torch.empty(0, dtype=torch.int64, device=DEV), C, tw, th)
    torch.cuda.synchronize()
    assert int(offsets[-1]) == 0
    assert torch.equal(tile_offsets, empty) and not empty.any()


@pytest.mark.parametrize("bricks", [(13, 13, 13), (256, 256, 160)])
def test_isect_tiles_3d_sort_widths(bricks):
    # 2197 bricks: two 6-bit passes; 10.5 M bricks (24-bit keys): three passes.
    n2, n1, n0 = bricks
    g = torch.Generator().manual_seed(n0)
    N = 3000
    ext = torch.tensor([8.0 * n2, 8.0 * n1, 8.0 * n0])
    m3 = (torch.rand(N, 3, generator=g) * (ext + 40) - 20).float()
    r3 = torch.randint(0, 20, (N, 3), generator=g).int()
    tpg, ids, fl = W.isect_tiles_3d(m3.to(DEV), r3.to(DEV), 8, n2, n1, n0)
    tpg_o, ids_o, fl_o = binning.isect_tiles_3d(m3.numpy(), r3.numpy(), 8, n2, n1, n0)
    assert ids_o.size > 3000 and ids_o.max() >= n2 * n1 * n0 // 2
    assert_equal(np32(tpg), tpg_o, "tiles_per_gauss")
    assert_equal(np32(ids), ids_o, "isect_ids")
    assert_equal(np32(fl), fl_o, "flatten_ids")
    # Two or three passes: the sort searches its sorted keys for the offsets.
    lists = _ops.bin_tiles_3d(m3.to(DEV), r3.to(DEV), 8, n2, n1, n0)
    assert_equal(np32(lists.tile_offsets), binning.isect_offset_encode_3d(ids_o, n2, n1, n0),
                 "sort tile_offsets")


def _windows_past_empty_keys(tile_offsets, n, walk=4):
    """Whether some 64-record window of a list of n records holds more than
    `walk` keys whose first index lies inside it after its first record's
    key (empty keys count: they share their successor's first index), so
    that the backward's key search bisects per lane there."""
    o = np32(tile_offsets).reshape(-1).astype(np.int64)
    rb = np.arange(0, n, 64)
    lo = np.searchsorted(o, rb, side="right") - 1
    hi = np.searchsorted(o, np.minimum(rb + 63, n - 1), side="right") - 1
    return bool(((hi - lo) > walk).any())


@pytest.mark.parametrize("views", [1, 3])
def test_lists_without_keys(views):
    # r2splat.ops bins without storing the sorted int64 keys: the sort writes
    # none (1024 tiles: one pass; 3072: two passes, the tile offsets searched
    # in the sort's own 32-bit keys) and the backward finds each record's tile
    # from the tile offsets.  Footprints clustered in a few tiles leave runs of
    # empty tiles inside 64-record windows, where that search bisects per
    # lane.  Everything equals the lists binned with their keys, bit for bit.
    g = torch.Generator().manual_seed(41 + views)
    N, W_img, H_img, ts = 3000, 512, 512, 16
    tw, th = W_img // ts, H_img // ts
    cells = torch.randint(0, tw * th, (views, N // 20), generator=g)
    pick = torch.gather(cells, 1, torch.randint(0, N // 20, (views, N), generator=g))
    centre = torch.stack([(pick % tw).float(), (pick // tw).float()], -1) * ts + ts / 2
    m2 = centre + (torch.rand(views, N, 2, generator=g) - 0.5) * 12
    a = 0.05 + 0.1 * torch.rand(views, N, generator=g)
    c = 0.05 + 0.1 * torch.rand(views, N, generator=g)
    b = (torch.rand(views, N, generator=g) - 0.5) * 0.5 * (a * c).sqrt()
    con = torch.stack([a, b, c], -1)
    op = 0.2 + 0.8 * torch.rand(views, N, generator=g)
    mu = 0.5 + torch.rand(views, N, generator=g)
    r = torch.randint(2, 10, (views, N, 2), generator=g).int()
    m2, con, op, mu, r = (t.to(DEV) for t in (m2, con, op, mu, r))
    with_ids = _ops.bin_tiles_2d(m2, r, ts, tw, th)
    without = _ops.bin_tiles_2d(m2, r, ts, tw, th, keep_ids=False)
    assert without.keys is None and with_ids.keys is not None
    for name in ("tiles_per_gauss", "flatten_ids", "emit_ids", "isect_src", "tile_offsets"):
        assert torch.equal(getattr(without, name), getattr(with_ids, name)), name
    assert torch.equal(without.isect_ids, with_ids.keys)
    n = with_ids.flatten_ids.numel()
    off = with_ids.tile_offsets
    assert n > 3000 and _windows_past_empty_keys(off, n)
    v = torch.randn(views, H_img, W_img, generator=g).to(DEV)
    payload, _ = _ops.raster_pack(m2, con, op, mu)
    for absgrad in (True, False):
        want = _ops.raster_backward(m2, con, op, mu, off, with_ids, v, W_img, H_img, ts, absgrad)
        got = _ops.raster_backward(m2, con, op, mu, off, without, v, W_img, H_img, ts, absgrad)
        _same_grads(got, want, exact=True)
        got = _ops.raster_backward_packed(payload, op, mu, off, without, v, W_img, H_img, ts,
                                          absgrad)
        _same_grads(got, want, exact=True)
        # Tile order (one-pass kernels, atomics): keys from the offsets too.
        one = _ops.TileLists(None, None, with_ids.flatten_ids.clone(), None, None, off)
        got = _ops.raster_backward(m2, con, op, mu, off, one, v, W_img, H_img, ts, absgrad)
        _same_grads(got, want, exact=False)


@pytest.mark.parametrize("bricks", [(8, 8, 8), (16, 16, 16), (40, 36, 32), (256, 256, 160)])
def test_volume_lists_without_keys(bricks):
    # As test_lists_without_keys for brick lists: 512 bricks (one sort pass),
    # 4096 and 46080 (two passes) and 10.5 M (three passes; lists only), and
    # the slab lists of a large volume's z-slabs.  Gaussians in a few
    # clusters; the backward in its two emission-order forms (with and
    # without the forward's reach masks).
    n2, n1, n0 = bricks
    dims = (8 * n2, 8 * n1, 8 * n0)
    d = _prepared(3000, 43, log_mu=-4.0)
    g = d["gen"]
    centres = torch.rand(30, 3, generator=g) * 1.8 - 0.9
    means = centres[torch.randint(0, 30, (3000,), generator=g)]
    means = (means + 0.02 * torch.randn(3000, 3, generator=g)).to(DEV)
    m3, con, r3 = W.world_to_volume_mapping_fwd(means, d["covars"], d["opac"],
                                                torch.full((3,), 2.0, device=DEV),
                                                torch.zeros(3, device=DEV), *dims, 1e-8, 3.0)
    op = d["opac"]
    with_ids = _ops.bin_tiles_3d(m3, r3, 8, n2, n1, n0)
    without = _ops.bin_tiles_3d(m3, r3, 8, n2, n1, n0, keep_ids=False)
    assert without.keys is None
    for name in ("tiles_per_gauss", "flatten_ids", "emit_ids", "isect_src", "tile_offsets"):
        assert torch.equal(getattr(without, name), getattr(with_ids, name)), name
    assert torch.equal(without.isect_ids, with_ids.keys)
    n = with_ids.flatten_ids.numel()
    off = with_ids.tile_offsets
    assert n > 3000 and _windows_past_empty_keys(off, n)
    z0, z1 = n0 // 4, n0 // 2 + 1
    sl_k, off_k = _ops.bin_tiles_3d_slab(m3, r3, 8, n2, n1, n0, z0, z1)
    sl_n, off_n = _ops.bin_tiles_3d_slab(m3, r3, 8, n2, n1, n0, z0, z1, keep_ids=False)
    assert sl_n.keys is None and torch.equal(off_n, off_k)
    assert torch.equal(sl_n.flatten_ids, sl_k.flatten_ids)
    assert torch.equal(sl_n.isect_ids, sl_k.keys)
    if n2 * n1 * n0 > 50_000:
        return
    d2, d1, d0 = dims
    vol, reach = _ops.voxelize_with_reach(m3, con, op, off, with_ids.flatten_ids, d2, d1, d0)
    v = torch.randn(vol.shape, generator=g).to(DEV)
    for rc in (reach, None):
        want = _ops.voxel_backward(m3, con, op, off, with_ids, v, d2, d1, d0, 8, reach=rc)
        got = _ops.voxel_backward(m3, con, op, off, without, v, d2, d1, d0, 8, reach=rc)
        _same_grads(got, want, exact=True)
    want = _ops.voxel_backward_slab(m3, con, op, off_k, sl_k, v, 8, z0)
    got = _ops.voxel_backward_slab(m3, con, op, off_n, sl_n, v, 8, z0)
    _same_grads(got, want, exact=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_volume_mapping_bit_exact(dtype):
    d = _prepared(4000, 6, dtype, log_mu=-3.0)
    ranges = torch.tensor([2.0, 1.5, 2.5], dtype=dtype, device=DEV)
    centers = torch.tensor([0.1, -0.2, 0.0], dtype=dtype, device=DEV)
    m3, con, r3 = W.world_to_volume_mapping_fwd(d["means"], d["covars"], d["opac"], ranges,
                                                centers, 48, 40, 56, 1e-8, 3.0)
    m3o, cono, r3o = ops.world_to_volume_mapping_fwd(np32(d["means"]), np32(d["covars"]),
                                                     np32(ranges), np32(centers), 48, 40, 56,
                                                     1e-8, 3.0)
    assert_equal(np32(m3), m3o, "means3d")
    assert_equal(np32(con), cono, "conics3d")
    assert_equal(np32(r3), r3o, "radii3d")
    g = d["gen"]
    vm3 = torch.randn(4000, 3, generator=g, dtype=dtype)
    vc3 = torch.randn(4000, 6, generator=g, dtype=dtype)
    vm, vc = W.world_to_volume_mapping_bwd(d["means"], d["covars"], ranges, centers, 48, 40, 56,
                                           1e-8, vm3.to(DEV), vc3.to(DEV))
    vmo, vco = ops.world_to_volume_mapping_bwd(np32(d["means"]), np32(d["covars"]), np32(ranges),
                                               np32(centers), 48, 40, 56, 1e-8, vm3.numpy(),
                                               vc3.numpy())
    assert_equal(np32(vm), vmo, "v_means (volume)")
    assert_equal(np32(vc), vco, "v_covars (volume)")


def _raster_case(n, seed, W_img, H_img, ts, n_views=1, dtype=torch.float32, log_mu=-3.6):
    d = _prepared(n, seed, dtype, n_det=max(W_img, H_img), n_views=n_views, log_mu=log_mu)
    Ks = d["Ks"].clone()
    Ks[:, 0, 2] = W_img / 2
    Ks[:, 1, 2] = H_img / 2
    m2, c2, r, con, mu, op = W.project_gaussians_fwd(d["means"], d["covars"], d["opac"],
                                                     d["viewmats"], Ks, W_img, H_img, 1e-8, 3.0)
    tw, th = -(-W_img // ts), -(-H_img // ts)
    _, ids, fl = W.isect_tiles(m2, r, ts, tw, th)
    off = W.isect_offset_encode(ids, n_views, tw, th)
    return d, m2, con, mu, op, ids, fl, off


@pytest.mark.parametrize("order", ["emission", "tile"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", [(64, 64, 16), (70, 45, 16), (40, 40, 8), (50, 38, 12),
                                   (66, 40, 20), (96, 72, 32)])
def test_rasterize_fwd_bwd(dtype, shape, order):
    W_img, H_img, ts = shape
    d, m2, con, mu, op, ids, fl, off = _raster_case(3000, 7, W_img, H_img, ts, 2, dtype)
    assert fl.numel() > 500
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, ts)
    v = torch.randn(img.shape, generator=d["gen"], dtype=dtype)
    refs = raster_references(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl),
                             W_img, H_img, ts, v_image=v.numpy())
    print("image", check_raster(refs, image=np32(img)))
    if order == "tile":
        fl = fl.clone()  # no emission-order records: the tile-order kernels run
    assert (_ops.emission_order(fl, fl_keys(off)) is not None) == (order == "emission")
    for mode in ("primitive", "pixel"):
        if mode == "primitive":
            got = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl,
                                                         v.to(DEV), W_img, H_img, ts, True)
        else:
            got = W.rasterize_to_pixels_bwd(m2, con, op, mu, off, fl, v.to(DEV), W_img, H_img,
                                            ts, True)
        for n, r in check_raster(refs, grads=[np32(t) for t in got], tag=f"{mode} ").items():
            print(mode, n, r)
    no_abs = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v.to(DEV),
                                                    W_img, H_img, ts, False)
    assert no_abs[0] is None


@pytest.mark.parametrize("ts", [8, 16, 32])
def test_rasterize_fwd_small_gaussians(ts):
    """Sub-pixel footprints (conic entries 20..80) anywhere along a lane's row
    of pixels: where sigma is small the exponent's terms in dx are large, so
    an evaluation that loses that cancellation (e.g. a quadratic in the
    column offset from the row start) errs by 1e-4..1e-3 relative."""
    g = torch.Generator().manual_seed(31)
    N, W_img, H_img = 4000, 64, 64
    m2 = torch.rand(1, N, 2, generator=g) * torch.tensor([W_img, H_img])
    a = 20 + 60 * torch.rand(1, N, generator=g)
    c = 20 + 60 * torch.rand(1, N, generator=g)
    b = (torch.rand(1, N, generator=g) - 0.5) * (a * c).sqrt()
    con = torch.stack([a, b, c], -1)
    op = 0.2 + 0.8 * torch.rand(1, N, generator=g)
    mu = torch.ones(1, N)
    r = torch.full((1, N, 2), 2, dtype=torch.int32)
    m2, con, op, mu, r = (t.to(DEV) for t in (m2, con, op, mu, r))
    tw, th = -(-W_img // ts), -(-H_img // ts)
    _, ids, fl = W.isect_tiles(m2, r, ts, tw, th)
    off = W.isect_offset_encode(ids, 1, tw, th)
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, ts)
    refs = raster_references(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl),
                             W_img, H_img, ts)
    print(check_raster(refs, image=np32(img)))


def test_raster_backward_with_many_gaussians_per_reduce_wave():
    # Footprints of one or two tiles: a 256-row wave of the row reduce holds
    # well over 128 Gaussians, so it stages and stores its totals in more
    # than one round.
    g = torch.Generator().manual_seed(33)
    N, W_img, H_img, ts = 6000, 128, 128, 16
    m2 = torch.rand(1, N, 2, generator=g) * torch.tensor([W_img, H_img])
    a = 0.5 + 0.5 * torch.rand(1, N, generator=g)
    c = 0.5 + 0.5 * torch.rand(1, N, generator=g)
    b = (torch.rand(1, N, generator=g) - 0.5) * 0.5 * (a * c).sqrt()
    con = torch.stack([a, b, c], -1)
    op = 0.2 + 0.8 * torch.rand(1, N, generator=g)
    mu = 0.5 + torch.rand(1, N, generator=g)
    r = torch.full((1, N, 2), 3, dtype=torch.int32)
    m2, con, op, mu, r = (t.to(DEV) for t in (m2, con, op, mu, r))
    tw, th = W_img // ts, H_img // ts
    _, ids, fl = W.isect_tiles(m2, r, ts, tw, th)
    off = W.isect_offset_encode(ids, 1, tw, th)
    emit_ids, _ = _ops.emission_order(fl, tw * th)
    e = np32(emit_ids)
    heads = max(int(np.unique(e[i:i + 256]).size) for i in range(0, e.size, 256))
    assert heads > 128, heads
    v = torch.randn(1, H_img, W_img, generator=g)
    refs = raster_references(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl),
                             W_img, H_img, ts, v_image=v.numpy())
    got = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v.to(DEV),
                                                 W_img, H_img, ts, True)
    print(check_raster(refs, grads=[np32(t) for t in got]))


@pytest.mark.parametrize("dims,ts", [((32, 32, 32), 8), ((30, 20, 40), 10)])
def test_voxelize_fwd_small_gaussians(dims, ts):
    """Sub-voxel footprints anywhere along a thread's x-row (see
    test_rasterize_fwd_small_gaussians)."""
    d, m3, con, ids, fl, off = _voxel_case(6000, 22, dims, ts, log_mu=-5.0)
    assert float(con[..., 0].max()) > 10.0
    d2, d1, d0 = dims
    vol = W.voxelize_to_voxels_fwd(m3, con, d["opac"], off, fl, d2, d1, d0, ts)
    refs = voxel_references(np32(m3), np32(con), np32(d["opac"]), np32(off), np32(fl), d2, d1,
                            d0, ts)
    print(check_voxel(refs, volume=np32(vol)))


def _one_sign(p, q, dxa, dya, span=15.0, margin=1.0 / 64):
    """(p, q) . d keeps one sign over a tile's pixel centres, with margin."""
    t = np.stack([p * (dxa + i) + q * (dya + j) for i in (0.0, span) for j in (0.0, span)], 1)
    scale = (np.abs(p) * np.maximum(np.abs(dxa), np.abs(dxa + span))
             + np.abs(q) * np.maximum(np.abs(dya), np.abs(dya + span)))
    return (t.min(1) >= margin * scale) | (t.max(1) <= -margin * scale)


@pytest.mark.parametrize("dtype,shape", [(torch.float32, (128, 128)),
                                         (torch.float64, (128, 128)),
                                         (torch.float32, (96, 72))])
def test_absgrad_sign_split_backward(dtype, shape):
    """The tile-size-16 absolute-gradient backward partitions each block's
    records: waves whose records keep one sign of (P d)_x and (P d)_y over
    their tile sum |w| moments instead of per-pixel absolute values.  The
    scene has large Gaussians so that both kinds of waves run (and, at 96 x
    72, records of tiles cut by the image edge, which never qualify); every
    output is checked against the oracle."""
    W_img, H_img = shape
    d, m2, con, mu, op, ids, fl, off = _raster_case(1500, 11, W_img, H_img, 16, 1, dtype,
                                                     log_mu=-2.0)
    tw, th = -(-W_img // 16), -(-H_img // 16)
    keys, g = np32(ids).astype(np.int64), np32(fl).astype(np.int64)
    t = keys % (tw * th)
    ox, oy = (t % tw) * 16.0, (t // tw) * 16.0
    m2n, cn = np32(m2).reshape(-1, 2).astype(np.float64), np32(con).reshape(-1, 3)
    a, b, c = cn[g, 0], cn[g, 1], cn[g, 2]
    dxa, dya = ox + 0.5 - m2n[g, 0], oy + 0.5 - m2n[g, 1]
    fast = _one_sign(a, b, dxa, dya) & _one_sign(b, c, dxa, dya)
    fast &= (ox + 16 <= W_img) & (oy + 16 <= H_img)
    n_blk = fast.size // 256
    per_block = fast[:n_blk * 256].reshape(n_blk, 256).sum(1)
    assert (per_block >= 64).any() and (per_block < 256).any(), per_block
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, 16)
    v = torch.randn(img.shape, generator=d["gen"], dtype=dtype)
    refs = raster_references(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl),
                             W_img, H_img, 16, v_image=v.numpy())
    got = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v.to(DEV),
                                                 W_img, H_img, 16, True)
    for n, r in check_raster(refs, grads=[np32(t) for t in got]).items():
        print(n, r)


def _same_grads(a, b, exact):
    for x, y in zip(a, b):
        if x is None:
            assert y is None
            continue
        assert bool(torch.isfinite(x).all())
        if exact:
            assert torch.equal(x, y)
        else:  # one-pass forms: device atomics add in any order
            torch.testing.assert_close(x, y, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("order", ["emission", "tile"])
def test_non_finite_upstream_gradient_where_nothing_passes(order):
    # The reference skips a (record, pixel / voxel) pair that fails the alpha
    # test before it reads the upstream gradient there, so an inf or NaN
    # gradient where no record passes changes nothing.  The kernels add exact
    # zeros for failing pairs: the gradients equal those with zeros there,
    # bit for bit in the two-pass forms.
    # Sparse small Gaussians: tiles with records hold pixels no record passes.
    d, m2, con, mu, op, ids, fl, off = _raster_case(150, 21, 64, 64, 16, 1, torch.float32,
                                                    log_mu=-4.3)
    assert fl.numel() > 50
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, 64, 64, 16)
    v = torch.randn(img.shape, generator=d["gen"]).to(DEV)
    dead = img == 0  # no record passes there: a passing alpha is at least 1e-5
    starts = off.reshape(-1).long()
    ends = torch.cat([starts[1:], torch.tensor([fl.numel()], device=DEV)])
    live = (ends > starts).reshape(4, 4).repeat_interleave(16, 0).repeat_interleave(16, 1)
    assert int((dead.reshape(64, 64) & live).sum()) > 20  # inside tiles the kernels walk
    v_zero = torch.where(dead, torch.zeros_like(v), v)
    fl_run = fl if order == "emission" else fl.clone()
    for bad in (float("inf"), float("nan")):
        v_bad = torch.where(dead, torch.full_like(v, bad), v)
        for absgrad in (True, False):
            a = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl_run, v_bad,
                                                       64, 64, 16, absgrad)
            b = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl_run, v_zero,
                                                       64, 64, 16, absgrad)
            _same_grads(a, b, exact=order == "emission")
    d3, m3, con3, ids3, fl3, off3 = _voxel_case(300, 8, (32, 32, 32), 8)
    assert fl3.numel() > 100
    op3 = d3["opac"]
    vol = W.voxelize_to_voxels_fwd(m3, con3, op3, off3, fl3, 32, 32, 32, 8)
    v3 = torch.randn(vol.shape, generator=d3["gen"]).to(DEV)
    dead3 = vol == 0
    starts3 = off3.reshape(-1).long()
    ends3 = torch.cat([starts3[1:], torch.tensor([fl3.numel()], device=DEV)])
    live3 = (ends3 > starts3).reshape(4, 4, 4)
    live3 = live3.repeat_interleave(8, 0).repeat_interleave(8, 1).repeat_interleave(8, 2)
    assert int((dead3 & live3).sum()) > 100  # inside bricks the kernels walk
    v3_zero = torch.where(dead3, torch.zeros_like(v3), v3)
    fl3_run = fl3 if order == "emission" else fl3.clone()
    lists = _ops.bin_tiles_3d(m3, W.world_to_volume_mapping_fwd(
        d3["means"], d3["covars"], op3, torch.full((3,), 2.0, device=DEV),
        torch.zeros(3, device=DEV), 32, 32, 32, 1e-8, 3.0)[2], 8, 4, 4, 4)
    _, reach = _ops.voxelize_with_reach(m3, con3, op3, off3, lists.flatten_ids, 32, 32, 32)
    for bad in (float("inf"), float("nan")):
        v3_bad = torch.where(dead3, torch.full_like(v3, bad), v3)
        a = W.voxelize_to_voxels_bwd_per_gaussian(m3, con3, op3, off3, ids3, fl3_run, v3_bad, 32,
                                                  32, 32, 8)
        b = W.voxelize_to_voxels_bwd_per_gaussian(m3, con3, op3, off3, ids3, fl3_run, v3_zero,
                                                  32, 32, 32, 8)
        _same_grads(a, b, exact=order == "emission")
        if order == "emission":  # the chunked walk given the forward's reach masks
            a = _ops.voxel_backward(m3, con3, op3, off3, lists, v3_bad, 32, 32, 32, 8,
                                    reach=reach)
            b = _ops.voxel_backward(m3, con3, op3, off3, lists, v3_zero, 32, 32, 32, 8,
                                    reach=reach)
            _same_grads(a, b, exact=True)


@pytest.mark.parametrize("order", ["emission", "tile"])
def test_nan_opacity_propagates_as_in_the_reference(order):
    # A NaN alpha is not below the cut-off, so the reference does not skip it:
    # the pixels / voxels of a NaN-opacity Gaussian's tiles turn NaN, and so do
    # that Gaussian's gradients that carry its opacity.  The NaN patterns must
    # match the oracle's exactly, the finite values the parity bar.
    d, m2, con, mu, op, ids, fl, off = _raster_case(3000, 17, 64, 64, 16, 1, torch.float32)
    g = int(fl[fl.numel() // 2])
    op = op.clone()
    op[0, g] = float("nan")
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, 64, 64, 16)
    v = torch.randn(img.shape, generator=d["gen"])
    refs = raster_references(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl), 64,
                             64, 16, v_image=v.numpy())
    assert np.isnan(refs["fwd"][0]).any() and not np.isnan(refs["fwd"][0]).all()
    check_raster(refs, image=np32(img))
    fl_run = fl if order == "emission" else fl.clone()
    got = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl_run, v.to(DEV),
                                                 64, 64, 16, True)
    check_raster(refs, grads=[np32(t) for t in got])
    assert np.isnan(refs["bwd"][1][0]).any()
    d3, m3, con3, ids3, fl3, off3 = _voxel_case(2500, 18, (32, 32, 32), 8)
    g3 = int(fl3[fl3.numel() // 2])
    op3 = d3["opac"].clone()
    op3[g3] = float("nan")
    vol = W.voxelize_to_voxels_fwd(m3, con3, op3, off3, fl3, 32, 32, 32, 8)
    v3 = torch.randn(vol.shape, generator=d3["gen"])
    refs3 = voxel_references(np32(m3), np32(con3), np32(op3), np32(off3), np32(fl3), 32, 32, 32,
                             8, v_volume=v3.numpy())
    assert np.isnan(refs3["fwd"][0]).any() and not np.isnan(refs3["fwd"][0]).all()
    check_voxel(refs3, volume=np32(vol))
    fl3_run = fl3 if order == "emission" else fl3.clone()
    got3 = W.voxelize_to_voxels_bwd_per_gaussian(m3, con3, op3, off3, ids3, fl3_run, v3.to(DEV),
                                                 32, 32, 32, 8)
    check_voxel(refs3, grads=[np32(t) for t in got3])
    assert np.isnan(refs3["bwd"][0][0]).any()


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape", [(32, 32, 16), (48, 40, 8)])
def test_rasterize_fwd_splits_heavy_tiles(dtype, shape):
    """Many large Gaussians on a small detector: thousands of records per tile,
    so each tile is summed by several blocks and their partials combined."""
    from r2splat.cuda import _backend

    W_img, H_img, ts = shape
    d, m2, con, mu, op, ids, fl, off = _raster_case(6000, 11, W_img, H_img, ts, 2, dtype,
                                                    log_mu=-2.0)
    n_keys = off.numel()
    lib = _backend.library()
    assert lib.r2s_rasterize_workspace_bytes(n_keys, fl.numel(), ts, 4) > 0  # split path
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, ts)
    refs = raster_references(np32(m2), np32(con), np32(op), np32(mu), np32(off), np32(fl),
                             W_img, H_img, ts)
    print(check_raster(refs, image=np32(img)))
    again = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, ts)
    assert torch.equal(img, again)


def test_rasterize_empty():
    m2 = torch.zeros(1, 3, 2, device=DEV)
    z3 = torch.zeros(1, 3, 3, device=DEV)
    z = torch.zeros(1, 3, device=DEV)
    off = torch.zeros(1, 2, 2, dtype=torch.int32, device=DEV)
    fl = torch.zeros(0, dtype=torch.int32, device=DEV)
    img = W.rasterize_to_pixels_fwd(m2, z3, z, z, off, fl, 30, 20, 16)
    assert img.shape == (1, 20, 30) and float(img.abs().sum()) == 0.0
    g = W.rasterize_to_pixels_bwd(m2, z3, z, z, off, fl, torch.ones(1, 20, 30, device=DEV), 30,
                                  20, 16, True)
    assert all(float(t.abs().sum()) == 0.0 for t in g)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("shape,log_mu", [((64, 64, 16), -4.0), ((70, 45, 16), -4.0),
                                          ((40, 40, 8), -4.0), ((96, 72, 32), -4.0),
                                          ((32, 32, 16), -2.0)])
def test_packed_rasterizer_equals_the_array_form(dtype, shape, log_mu):
    """The packed payload's forward and two-pass backward (r2splat.ops' path)
    against the four-array forward and the two-pass backward with its own
    pack: bit for bit, absgrad on and off, with the outputs zeroed by the
    pack launch and without; heavy tiles (log_mu -2) take the split
    forward."""
    W_img, H_img, ts = shape
    d, m2, con, mu, op, ids, fl, off = _raster_case(3000, 17, W_img, H_img, ts, 2, dtype,
                                                    log_mu=log_mu)
    C, N = m2.shape[:2]
    lists = _ops.TileLists(None, ids, fl, *_ops.emission_order(fl, fl_keys(off)))
    want_img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, ts)
    # Non-finite records (a NaN opacity, infinite and huge conic entries) take
    # the alpha limit's non-finite branch in both forms.
    listed = torch.unique(fl.long())
    g0, g1, g2 = (int(listed[k]) for k in (3, len(listed) // 2, -4))
    bad_op, bad_con = op.clone(), con.clone()
    bad_op.view(-1)[g0] = float("nan")
    bad_con.view(-1, 3)[g1, 1] = float("inf")
    bad_con.view(-1, 3)[g2, 1] = torch.finfo(dtype).max  # finite; log2(e) times it is not
    bad_want = W.rasterize_to_pixels_fwd(m2, bad_con, bad_op, mu, off, fl, W_img, H_img, ts)
    bad_payload, _ = _ops.raster_pack(m2, bad_con, bad_op, mu)
    bad_img = _ops.rasterize_packed(bad_payload, off, fl, C, N, W_img, H_img, ts)
    assert bad_img.isnan().any() and torch.equal(bad_img.isnan(), bad_want.isnan())
    assert torch.equal(bad_img.nan_to_num(0.0), bad_want.nan_to_num(0.0))
    v = torch.randn(want_img.shape, generator=d["gen"], dtype=dtype).to(DEV)
    for absgrad in (True, False):
        payload, zeroed = _ops.raster_pack(m2, con, op, mu, zero_outputs=True, absgrad=absgrad)
        assert payload.numel() == C * N * 8 and (zeroed[0] is None) == (not absgrad)
        assert all(t is None or not t.any() for t in zeroed)
        img = _ops.rasterize_packed(payload, off, fl, C, N, W_img, H_img, ts)
        assert torch.equal(img, want_img)
        want = _ops.raster_backward(m2, con, op, mu, off, lists, v, W_img, H_img, ts, absgrad)
        in_place = _ops.raster_backward_packed(payload, op, mu, off, lists, v, W_img, H_img, ts,
                                               absgrad, zeroed)
        assert in_place[1].data_ptr() == zeroed[1].data_ptr()  # the zeroed outputs, filled
        fresh = _ops.raster_backward_packed(payload, op, mu, off, lists, v, W_img, H_img, ts,
                                            absgrad)
        for got in (in_place, fresh):
            for a, b in zip(got, want):
                assert (a is None and b is None) or torch.equal(a, b)


def test_packed_rasterizer_rejects_other_tile_sizes_and_empty_lists():
    d, m2, con, mu, op, ids, fl, off = _raster_case(500, 3, 50, 38, 12, 1, torch.float32)
    payload, _ = _ops.raster_pack(m2, con, op, mu)
    with pytest.raises(RuntimeError, match="tile sizes 8, 16 and 32"):
        _ops.rasterize_packed(payload, off, fl, 1, m2.shape[1], 50, 38, 12)
    empty = torch.zeros(0, dtype=torch.int32, device=DEV)
    off16 = torch.zeros(1, 3, 4, dtype=torch.int32, device=DEV)
    img = _ops.rasterize_packed(payload, off16, empty, 1, m2.shape[1], 50, 38, 16)
    assert img.shape == (1, 38, 50) and not img.any()
    lists = _ops.TileLists(None, torch.zeros(0, dtype=torch.int64, device=DEV), empty, None, None)
    _, zeroed = _ops.raster_pack(m2, con, op, mu, zero_outputs=True, absgrad=True)
    got = _ops.raster_backward_packed(payload, op, mu, off16, lists,
                                      torch.ones(1, 38, 50, device=DEV), 50, 38, 16, True, zeroed)
    assert all(not t.any() for t in got)
    got = _ops.raster_backward_packed(payload, op, mu, off16, lists,
                                      torch.ones(1, 38, 50, device=DEV), 50, 38, 16, True)
    assert all(not t.any() for t in got)


def _bits(t):
    """The tensor's bit patterns (NaNs compare equal to themselves)."""
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    if t.dtype == torch.float64:
        return t.view(torch.int64)
    return t


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n_views,log_mu", [(1, -3.6), (3, -3.6), (2, -2.0)])
def test_fused_projection_pack_equals_projection_then_pack(dtype, n_views, log_mu):
    """r2s_project_pack_fwd_* against r2s_project_gaussians_fwd_* followed by
    r2s_rasterize_pack_* on its outputs: the six projection outputs, the
    payload and the zeroed raster backward outputs bit for bit, with and
    without the zeros and with absgrad on and off; a NaN opacity and an
    infinite covariance entry take the same non-finite branches in both."""
    d = _prepared(3000, 23, dtype, n_det=64, n_views=n_views, log_mu=log_mu)
    opac, covars = d["opac"].clone(), d["covars"].clone()
    opac[5] = float("nan")
    covars[9, 1] = float("inf")
    args = (d["means"], covars, opac, d["viewmats"], d["Ks"], 64, 64, 1e-8, 3.0)
    want = _ops.project_gaussians_fwd(*args)
    m2, _, _, con, mu, op = want
    want_payload, _ = _ops.raster_pack(m2, con, op, mu)
    assert want_payload.isnan().any() and (want_payload.view(-1, 8)[:, 7] > 0).any()
    for zero, absgrad in ((False, False), (True, False), (True, True)):
        got = _ops.project_pack_fwd(*args, zero_outputs=zero, absgrad=absgrad)
        for a, b in zip(got[:6], want):
            assert a.shape == b.shape and torch.equal(_bits(a), _bits(b))
        assert torch.equal(_bits(got[6]), _bits(want_payload))
        outs = got[7]
        if not zero:
            assert outs is None
            continue
        assert (outs[0] is None) == (not absgrad)
        assert all(t is None or (t.numel() > 0 and not t.any()) for t in outs)


def _voxel_case(n, seed, dims, ts, dtype=torch.float32, log_mu=-3.2):
    d = _prepared(n, seed, dtype, log_mu=log_mu)
    ranges = torch.full((3,), 2.0, dtype=dtype, device=DEV)
    centers = torch.zeros(3, dtype=dtype, device=DEV)
    d2, d1, d0 = dims
    m3, con, r3 = W.world_to_volume_mapping_fwd(d["means"], d["covars"], d["opac"], ranges,
                                                centers, d2, d1, d0, 1e-8, 3.0)
    n2, n1, n0 = (-(-x // ts) for x in dims)
    _, ids, fl = W.isect_tiles_3d(m3, r3, ts, n2, n1, n0)
    off = W.isect_offset_encode_3d(ids, n2, n1, n0)
    return d, m3, con, ids, fl, off


@pytest.mark.parametrize("order", ["emission", "tile"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("dims,ts", [((32, 32, 32), 8), ((30, 20, 26), 8), ((24, 24, 24), 4),
                                     ((20, 18, 22), 6), ((21, 22, 20), 10)])
def test_voxelize_fwd_bwd(dtype, dims, ts, order):
    d, m3, con, ids, fl, off = _voxel_case(2500, 8, dims, ts, dtype)
    d2, d1, d0 = dims
    assert fl.numel() > 500
    op = d["opac"]
    vol = W.voxelize_to_voxels_fwd(m3, con, op, off, fl, d2, d1, d0, ts)
    v = torch.randn(vol.shape, generator=d["gen"], dtype=dtype)
    refs = voxel_references(np32(m3), np32(con), np32(op), np32(off), np32(fl), d2, d1, d0, ts,
                            v_volume=v.numpy())
    print("volume", check_voxel(refs, volume=np32(vol)))
    if order == "tile":
        fl = fl.clone()  # no emission-order records: the tile-order kernels run
    assert (_ops.emission_order(fl, fl_keys(off)) is not None) == (order == "emission")
    for mode in ("primitive", "pixel"):
        if mode == "primitive":
            got = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, op, off, ids, fl, v.to(DEV), d2,
                                                        d1, d0, ts)
        else:
            got = W.voxelize_to_voxels_bwd(m3, con, op, off, fl, v.to(DEV), d2, d1, d0, ts)
        for n, r in check_voxel(refs, grads=[np32(t) for t in got], tag=f"{mode} ").items():
            print(mode, n, r)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n,band", [(4500, (192, 384)), (8000, (384, 10 ** 9))])
def test_voxelize_fwd_long_lists(dtype, n, band):
    """Brick lists long enough that the forward shares each brick between 2 (mean 192-383
    records per brick) or 4 waves (384 and more) and adds their partial bricks in wave
    order: the volume against the oracle at the usual bar."""
    dims = (32, 32, 32)
    d, m3, con, ids, fl, off = _voxel_case(n, 8, dims, 8, dtype)
    mean = fl.numel() / 64
    assert band[0] <= mean < band[1], mean
    vol = W.voxelize_to_voxels_fwd(m3, con, d["opac"], off, fl, *dims, 8)
    refs = voxel_references(np32(m3), np32(con), np32(d["opac"]), np32(off), np32(fl), *dims, 8)
    print("volume", check_voxel(refs, volume=np32(vol)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n,log_mu,dims", [(1500, -3.2, (32, 32, 40)), (1500, -1.6, (32, 32, 40)),
                                           (8000, -3.2, (32, 32, 32))])
def test_voxel_backward_reuses_the_forward_reach_masks(dtype, n, log_mu, dims):
    """voxelize_with_reach stores each record's reach mask; the two-pass backward given them
    skips its own culling and returns exactly what it computes without them (chunked waves,
    dense waves, and lists long enough for 4 forward waves per brick), and the volume equals
    the plain forward's."""
    d = _prepared(n, 13, dtype, log_mu=log_mu)
    ranges = torch.full((3,), 2.0, dtype=dtype, device=DEV)
    centers = torch.zeros(3, dtype=dtype, device=DEV)
    m3, con, r3 = W.world_to_volume_mapping_fwd(d["means"], d["covars"], d["opac"], ranges,
                                                centers, *dims, 1e-8, 3.0)
    n2, n1, n0 = (-(-x // 8) for x in dims)
    lists = _ops.bin_tiles_3d(m3, r3, 8, n2, n1, n0)
    off = W.isect_offset_encode_3d(lists.isect_ids, n2, n1, n0)
    op = d["opac"]
    vol = W.voxelize_to_voxels_fwd(m3, con, op, off, lists.flatten_ids, *dims, 8)
    vol_r, reach = _ops.voxelize_with_reach(m3, con, op, off, lists.flatten_ids, *dims)
    assert reach.numel() == lists.flatten_ids.numel() and bool((reach != 0).any())
    assert torch.equal(vol, vol_r)
    v = torch.randn(vol.shape, generator=d["gen"], dtype=dtype).to(DEV)
    plain = _ops.voxel_backward(m3, con, op, off, lists, v, *dims, 8)
    given = _ops.voxel_backward(m3, con, op, off, lists, v, *dims, 8, reach=reach)
    for a, b in zip(plain, given):
        assert torch.equal(a, b)


def _voxel_row_reach(m3, con, op, ids, fl, dims, ts):
    """Rows (of 64) of its brick that each record's alpha-test ellipsoid reaches."""
    d2, d1, d0 = dims
    n2, n1 = -(-d2 // ts), -(-d1 // ts)
    g = fl.astype(np.int64)
    k = ids.astype(np.int64)
    bi, rem = k // (n1 * n2), k % (n1 * n2)
    bj, bk = rem // n2, rem % n2
    q = con.reshape(-1, 6).astype(np.float64)[g]
    p00, p01, p02, p11, p12, p22 = q.T
    # Schur complement of the x block: sigma_min(y, z) = 1/2 [y z] S [y z]^T.
    s11, s12, s22 = p11 - p01 * p01 / p00, p12 - p01 * p02 / p00, p22 - p02 * p02 / p00
    s_max = np.log(np.maximum(np.abs(op.astype(np.float64)[g]), 1e-300) / 1e-6)
    m = m3.reshape(-1, 3).astype(np.float64)[g]
    out = np.zeros(g.size)
    for li in range(ts):
        dz = bi * ts + li + 0.5 - m[:, 2]
        for lj in range(ts):
            dy = bj * ts + lj + 0.5 - m[:, 1]
            sig = 0.5 * (s11 * dy * dy + 2 * s12 * dy * dz + s22 * dz * dz)
            out += (sig <= s_max)
    return out


@pytest.mark.parametrize("log_mu,dense", [(-3.2, False), (-1.6, True)])
def test_voxelize_bwd_chunked_and_dense_waves(log_mu, dense):
    """Brick size 8 with every brick inside the volume runs the chunked
    backward: small footprints take the chunked walk over the reached rows,
    large ones (most rows of every brick reached) the dense walk.  Both
    against the oracle, in both backward modes."""
    dims = (32, 32, 40)
    d, m3, con, ids, fl, off = _voxel_case(1500, 13, dims, 8, log_mu=log_mu)
    d2, d1, d0 = dims
    op = d["opac"]
    # Share of the kernel's waves (64 records in list order) whose records
    # reach more than 3072 of their 64 x 64 (record, row) pairs: a row is
    # reached when the smallest sigma over x on its centre line is within
    # ln(|o| / 1e-6).
    reach = _voxel_row_reach(np32(m3), np32(con), np32(op), np32(ids), np32(fl), dims, 8)
    n_w = reach.size // 64
    dense_waves = (reach[:n_w * 64].reshape(n_w, 64).sum(1) > 3072).mean()
    assert (dense_waves > 0.5) == dense, dense_waves
    vol = W.voxelize_to_voxels_fwd(m3, con, op, off, fl, d2, d1, d0, 8)
    v = torch.randn(vol.shape, generator=d["gen"])
    refs = voxel_references(np32(m3), np32(con), np32(op), np32(off), np32(fl), d2, d1, d0, 8,
                            v_volume=v.numpy())
    check_voxel(refs, volume=np32(vol))
    for mode in ("primitive", "pixel"):
        if mode == "primitive":
            got = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, op, off, ids, fl, v.to(DEV), d2,
                                                        d1, d0, 8)
        else:
            got = W.voxelize_to_voxels_bwd(m3, con, op, off, fl, v.to(DEV), d2, d1, d0, 8)
        for n, r in check_voxel(refs, grads=[np32(t) for t in got], tag=f"{mode} ").items():
            print(mode, n, r)


@pytest.mark.parametrize("n", [0, 1, 63, 64, 65, 4095, 4096, 4097, 100_003, 2_000_000])
def test_mask_split_matches_torch_where(n):
    g = torch.Generator().manual_seed(n)
    for p in (0.0, 0.3, 1.0):
        mask = (torch.rand(n, generator=g) < p).to(DEV)
        out, n_true = W.mask_split(mask)
        sel, rest = torch.where(mask)[0], torch.where(~mask)[0]
        assert n_true == sel.numel()
        assert torch.equal(out[:n_true], sel) and torch.equal(out[n_true:], rest)


@pytest.mark.parametrize("n", [4_194_304, 4_194_305, 9_000_001])
def test_count_scan_beyond_one_level(n):
    # More than 1024 scan blocks of 4096 items: the block sums are scanned
    # one level down.  Offsets must equal the int64 cumsum of the counts.
    from r2splat.cuda import _backend

    lib, P = _backend.library(), _ops._ptr
    g = torch.Generator().manual_seed(n)
    m2 = (torch.rand((1, n, 2), generator=g) * 256).to(DEV)
    radii = torch.randint(0, 24, (1, n, 2), generator=g, dtype=torch.int32).to(DEV)
    counts = torch.empty(n, dtype=torch.int32, device=DEV)
    offsets = torch.empty(n + 1, dtype=torch.int64, device=DEV)
    ws = torch.empty(lib.r2s_isect_workspace_bytes(n, 0, 0), dtype=torch.uint8, device=DEV)
    rc = lib.r2s_isect_count_2d_f32(P(m2), P(radii), 1, 1, n, 16, 16, 16, P(counts), P(offsets),
                                    P(ws), ws.numel(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.r2s_last_error()
    c = counts.cpu().numpy().astype(np.int64)
    assert c.sum() > n
    want = np.concatenate([[0], np.cumsum(c)])
    assert np.array_equal(offsets.cpu().numpy(), want)


def test_emission_order_backward_is_deterministic():
    d, m2, con, mu, op, ids, fl, off = _raster_case(3000, 9, 64, 64, 16, 2, torch.float32)
    v = torch.randn((2, 64, 64), generator=d["gen"]).to(DEV)
    runs = [W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v, 64, 64, 16,
                                                   True) for _ in range(3)]
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
    for a, b in zip(runs[0], runs[2]):
        assert torch.equal(a, b)
    d, m3, con3, ids3, fl3, off3 = _voxel_case(2500, 10, (32, 32, 32), 8)
    v3 = torch.randn((32, 32, 32), generator=d["gen"]).to(DEV)
    runs = [W.voxelize_to_voxels_bwd(m3, con3, d["opac"], off3, fl3, v3, 32, 32, 32, 8)
            for _ in range(2)]
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("seed", [0, 1])
def test_row_reduction_stores_every_id(seed):
    # Hand-built emission orders: ids ascending, gaps before the first and
    # after the last record and between records, segments longer than a
    # wave; integer rows, so every summation order gives the same sums.
    from r2splat.cuda import _backend

    lib, P = _backend.library(), _ops._ptr
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(seed)
    N = 700
    ids = torch.sort(torch.randperm(N - 20, generator=g)[:300] + 7).values
    ids = ids[(ids < 150) | (ids > 400)]  # one long run of ids without records
    counts = torch.randint(1, 9, (ids.numel(),), generator=g)
    counts[::25] = torch.randint(60, 200, (counts[::25].numel(),), generator=g)
    emit_ids = torch.repeat_interleave(ids, counts).int()
    n = emit_ids.numel()
    # Rows (v_xy 2, v_conic 3, T0, v_xy_abs 2); small integers and integer
    # opacities / mus, so the sums and the T0 products are exact.
    rows = torch.randint(-8, 9, (n, 8), generator=g).float()
    sums = torch.zeros(N, 8).index_add_(0, emit_ids.long(), rows)
    opac = torch.randint(1, 5, (1, N), generator=g).float()
    mus = torch.randint(1, 5, (1, N), generator=g).float()
    want = torch.cat([sums[:, :5], mus.reshape(N, 1) * sums[:, 5:6],
                      opac.reshape(N, 1) * sums[:, 5:6], sums[:, 6:8]], 1)
    outs = [torch.full((1, N, k), float("nan"), device=DEV) for k in (2, 3)]
    outs += [torch.full((1, N), float("nan"), device=DEV) for _ in range(2)]
    outs.insert(0, torch.full((1, N, 2), float("nan"), device=DEV))  # absgrad
    rows_d, emit_d = rows.to(DEV), emit_ids.to(DEV)
    op_d, mu_d = opac.to(DEV), mus.to(DEV)
    assert lib.r2s_rasterize_bwd_reduce_f32(P(rows_d), P(emit_d), n, 1, N, P(op_d), P(mu_d),
                                            *[P(t) for t in outs], st) == 0
    v_abs, v_xy, v_con, v_op, v_mu = (t.cpu().reshape(N, -1) for t in outs)
    got = torch.cat([v_xy, v_con, v_op, v_mu, v_abs], 1)
    assert torch.equal(got, want)
    assert int(emit_ids[0]) > 0 and int(emit_ids[-1]) < N - 1
    # No records at all: every output is still stored (zeros).
    for t in outs:
        t.fill_(float("nan"))
    assert lib.r2s_rasterize_bwd_reduce_f32(None, None, 0, 1, N, None, None,
                                            *[P(t) for t in outs], st) == 0
    assert all(int(torch.count_nonzero(t)) == 0 for t in outs)


def test_backward_stage_entry_points_match_the_two_pass_op():
    from r2splat.cuda import _backend

    lib, P = _backend.library(), _ops._ptr
    st = torch.cuda.current_stream().cuda_stream
    d, m2, con, mu, op, ids, fl, off = _raster_case(3000, 13, 64, 48, 16, 2, torch.float32)
    v = torch.randn((2, 48, 64), generator=d["gen"]).to(DEV)
    want = W.rasterize_to_pixels_bwd_per_gaussian(m2, con, op, mu, off, ids, fl, v, 64, 48, 16,
                                                  True)
    emit_ids, src = _ops.emission_order(fl, off.numel())
    n, N = fl.numel(), m2.shape[1]
    rows = torch.empty(lib.r2s_rasterize_bwd_workspace_bytes(n, 2 * N, 4), dtype=torch.uint8,
                       device=DEV)
    assert lib.r2s_rasterize_bwd_rows_f32(P(m2), P(con), P(op), P(mu), P(off), P(ids), P(fl),
                                          P(src), n, P(v), 2, N, 64, 48, 16, 4, 3, 1, P(rows),
                                          rows.numel(), st) == 0
    # NaN on entry: the reduction stores every output, zero without records.
    got = [torch.full_like(t, float("nan")) for t in want]
    assert lib.r2s_rasterize_bwd_reduce_f32(P(rows), P(emit_ids), n, 2, N, P(op), P(mu),
                                            *[P(t) for t in got], st) == 0
    for a, b in zip(got, want):
        assert torch.equal(a, b)
    untouched = torch.ones(2 * N, dtype=torch.bool, device=DEV)
    untouched[fl.long()] = False
    assert int(untouched.sum()) > 0
    assert int(got[1].reshape(2 * N, 2)[untouched].abs().sum()) == 0
    d3, m3, con3, ids3, fl3, off3 = _voxel_case(2500, 14, (32, 24, 16), 8)
    v3 = torch.randn((16, 24, 32), generator=d3["gen"]).to(DEV)
    want3 = W.voxelize_to_voxels_bwd(m3, con3, d3["opac"], off3, fl3, v3, 32, 24, 16, 8)
    emit3, src3 = _ops.emission_order(fl3, off3.numel())
    n3, N3 = fl3.numel(), m3.shape[0]
    rows3 = torch.empty(lib.r2s_voxelize_bwd_workspace_bytes(n3, 4), dtype=torch.uint8,
                        device=DEV)
    assert lib.r2s_voxelize_bwd_rows_f32(P(m3), P(con3), P(d3["opac"]), P(off3), None, P(fl3),
                                         P(src3), n3, P(v3), N3, 32, 24, 16, 8, 4, 3, 2,
                                         P(rows3), rows3.numel(), st) == 0
    got3 = [torch.full_like(t, float("nan")) for t in want3]
    assert lib.r2s_voxelize_bwd_reduce_f32(P(rows3), P(emit3), n3, N3, *[P(t) for t in got3],
                                           st) == 0
    for a, b in zip(got3, want3):
        assert torch.equal(a, b)


def test_one_pass_fallback_is_counted_and_warned():
    """The wrapper-level backward finds the emission order only on the very
    flatten_ids tensor isect_tiles returned; any other tensor runs the
    one-pass kernels, which is counted and warned about (once per process).
    The explicit TileLists path needs no lookup."""
    d, m2, con, mu, op, ids, fl, off = _raster_case(2000, 19, 64, 64, 16, 1, torch.float32)
    v = torch.randn(1, 64, 64, generator=d["gen"]).to(DEV)
    args = (m2, con, op, mu, off)
    _ops._WARNED_ONE_PASS = False
    c0 = dict(_ops.PATH_COUNTS)
    fast = W.rasterize_to_pixels_bwd_per_gaussian(*args, ids, fl, v, 64, 64, 16, True)
    assert _ops.PATH_COUNTS["two_pass"] == c0["two_pass"] + 1
    with pytest.warns(_ops.OnePassBackwardWarning, match="one-pass"):
        slow = W.rasterize_to_pixels_bwd_per_gaussian(*args, ids, fl.clone(), v, 64, 64, 16, True)
    assert _ops.PATH_COUNTS["one_pass"] == c0["one_pass"] + 1
    fl.add_(0)  # an in-place change invalidates the attached order
    assert _ops.emission_order(fl, off.numel()) is None
    lists = _ops.bin_tiles_2d(m2, _raster_radii(m2, d), 16, 4, 4)
    assert lists.emission is not None and torch.equal(lists.flatten_ids, fl)
    c1 = dict(_ops.PATH_COUNTS)
    explicit = _ops.raster_backward(*args, lists, v, 64, 64, 16, True)
    assert _ops.PATH_COUNTS == dict(c1, two_pass=c1["two_pass"] + 1)
    for a, b, c in zip(fast, slow, explicit):
        assert torch.equal(a, c)
        assert_close(np32(b), np32(a), "one-pass vs two-pass", rtol=1e-4, atol=1e-5)


def _raster_radii(m2, d):
    Ks = d["Ks"].clone()
    Ks[:, 0, 2] = 32
    Ks[:, 1, 2] = 32
    return W.project_gaussians_fwd(d["means"], d["covars"], d["opac"], d["viewmats"], Ks, 64, 64,
                                   1e-8, 3.0)[2]
