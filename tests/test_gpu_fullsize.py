"""Oracle parity at BASELINE's full sizes: config 4 (500k binary-tree
Gaussians, 512^2 detector, views 0 and 180 degrees, and the trainer's 128^3
volume of the same tree) and config 3 (200k Gaussians, 256^3 volume).

* Projection outputs (means2d, cov2d, conics, mus, radii) of all 500k
  Gaussians and the tile / brick lists and offsets equal the oracle's bit for
  bit (given the kernel's covariances; the parameter transform's exp is
  checked within the parity bar).
* The image / volume and every raster / voxel gradient meet
  helpers.assert_parity against the oracle one precision up, in both
  backward forms (the two-pass emission-order kernels of the explicit path
  and the one-pass kernels the wrapper runs without emission order).

The C oracle shares tiles out over OMP_NUM_THREADS threads (bit-identical to
its sequential loops): on 16 host threads each config takes about 15 s.
"""


import numpy as np
import pytest
import torch

from helpers import (assert_equal, assert_parity, check_raster, check_voxel, np32,
                     raster_references, voxel_references)
from oracle import binning, ops
from r2splat import geometry, scenes
from r2splat.cuda import _ops
from r2splat.cuda import _wrapper as W

pytestmark = pytest.mark.gpu

DEV = "cuda"
SMIN, SMAX = 5e-4, 1.0


def _grads(ts):
    return [None if t is None else np32(t) for t in ts]


def _report(tag, reps):
    for k, r in reps.items():
        print(tag, k, r, flush=True)


# ---------------------------------------------------------------- config 4 --

@pytest.fixture(scope="module")
def config4():
    g = torch.Generator().manual_seed(0)
    raw = scenes.binary_tree_gaussians(500_000, g, opacity="uniform")
    vm, Ks = geometry.cone_beam_views([0.0], 512)
    q, s, o = raw.quats.to(DEV), raw.raw_scales.to(DEV), raw.raw_opacities.to(DEV)
    covars, max_scales, opac = W.prepare_gaussians(q, s, o, SMIN, SMAX)
    means = raw.means.to(DEV)
    m2, cov2d, radii, conics, mus, op = W.project_gaussians_fwd(
        means, covars, opac, vm.to(DEV), Ks.to(DEV), 512, 512, 1e-8, 3.0)
    lists = _ops.bin_tiles_2d(m2, radii, 16, 32, 32)
    off = W.isect_offset_encode(lists.isect_ids, 1, 32, 32)
    v = torch.randn((1, 512, 512), generator=g)
    print(f"config 4: {lists.isect_ids.numel()} tile records", flush=True)
    return dict(raw=raw, vm=vm, Ks=Ks, covars=covars, max_scales=max_scales, opac=opac,
                means=means, m2=m2, cov2d=cov2d, radii=radii, conics=conics, mus=mus, op=op,
                lists=lists, off=off, v=v)


@pytest.fixture(scope="module")
def config4_refs(config4):
    d = config4
    refs = raster_references(np32(d["m2"]), np32(d["conics"]), np32(d["op"]), np32(d["mus"]),
                             np32(d["off"]), np32(d["lists"].flatten_ids), 512, 512, 16,
                             v_image=d["v"].numpy())
    print("config 4 oracle done", flush=True)
    return refs


def test_config4_parameter_transform_and_projection(config4):
    d = config4
    raw = d["raw"]
    q, s = raw.quats.numpy(), raw.raw_scales.numpy()
    cov32, ms32 = ops.parameter_transform_fwd(q, s, SMIN, SMAX)
    cov64, ms64 = ops.parameter_transform_fwd(q.astype(np.float64), s.astype(np.float64), SMIN,
                                              SMAX)
    assert_parity(np32(d["covars"]), cov64, cov32, None, "covars")
    assert_parity(np32(d["max_scales"]), ms64, ms32, None, "max_scales")
    # Projection of all 500k Gaussians, bit-exact on the kernel's covariances.
    m2, c2, r = ops.world_to_image_projection_fwd(raw.means.numpy(), np32(d["covars"]),
                                                  d["vm"].numpy(), d["Ks"].numpy(), 512, 512,
                                                  1e-8, 3.0)
    con, mu = ops.conics_mu_fwd(c2, 1e-8)
    for got, want, n in ((d["m2"], m2, "means2d"), (d["cov2d"], c2, "cov2d"),
                         (d["radii"], r, "radii"), (d["conics"], con, "conics"),
                         (d["mus"], mu, "mus")):
        assert_equal(np32(got), want, n)
    assert int((r > 0).any(-1).sum()) > 100_000


def test_config4_tile_lists_bit_exact(config4):
    d = config4
    tpg, ids, fl = binning.isect_tiles(np32(d["m2"]), np32(d["radii"]), 16, 32, 32)
    assert ids.size > 4_000_000
    assert_equal(np32(d["lists"].tiles_per_gauss), tpg, "tiles_per_gauss")
    assert_equal(np32(d["lists"].isect_ids), ids, "isect_ids")
    assert_equal(np32(d["lists"].flatten_ids), fl, "flatten_ids")
    assert_equal(np32(d["off"]), binning.isect_offset_encode(ids, 1, 32, 32), "tile_offsets")
    # The emission order is a permutation: record r was emitted at isect_src[r].
    src = np32(d["lists"].isect_src).astype(np.int64)
    assert np.array_equal(np.sort(src), np.arange(ids.size))
    assert np.array_equal(np32(d["lists"].emit_ids)[src], fl)


def test_config4_raster_forward_and_backward(config4, config4_refs):
    d = config4
    img = W.rasterize_to_pixels_fwd(d["m2"], d["conics"], d["op"], d["mus"], d["off"],
                                    d["lists"].flatten_ids, 512, 512, 16)
    _report("fwd", check_raster(config4_refs, image=np32(img)))
    got = _ops.raster_backward(d["m2"], d["conics"], d["op"], d["mus"], d["off"], d["lists"],
                               d["v"].to(DEV), 512, 512, 16, True)
    _report("two-pass", check_raster(config4_refs, grads=_grads(got)))


def test_config4_one_pass_backward(config4, config4_refs):
    d = config4
    one = _ops.TileLists(*d["lists"][:3], None, None)
    got = _ops.raster_backward(d["m2"], d["conics"], d["op"], d["mus"], d["off"], one,
                               d["v"].to(DEV), 512, 512, 16, True)
    _report("one-pass", check_raster(config4_refs, grads=_grads(got)))


def test_config4_second_view_full_size(config4):
    """The 500k tree from the opposite side (180 degrees, where the tree's
    footprints differ from view 0's): projection and lists bit-exact, the
    image and both backward forms' gradients against the oracle."""
    d = config4
    vm, Ks = geometry.cone_beam_views([np.pi], 512)
    m2, cov2d, radii, conics, mus, op = W.project_gaussians_fwd(
        d["means"], d["covars"], d["opac"], vm.to(DEV), Ks.to(DEV), 512, 512, 1e-8, 3.0)
    pm2, pc2, pr = ops.world_to_image_projection_fwd(d["raw"].means.numpy(), np32(d["covars"]),
                                                     vm.numpy(), Ks.numpy(), 512, 512, 1e-8,
                                                     3.0)
    pcon, pmu = ops.conics_mu_fwd(pc2, 1e-8)
    for got, want, n in ((m2, pm2, "means2d"), (cov2d, pc2, "cov2d"), (radii, pr, "radii"),
                         (conics, pcon, "conics"), (mus, pmu, "mus")):
        assert_equal(np32(got), want, n)
    lists = _ops.bin_tiles_2d(m2, radii, 16, 32, 32)
    off = W.isect_offset_encode(lists.isect_ids, 1, 32, 32)
    tpg, ids, fl = binning.isect_tiles(pm2, pr, 16, 32, 32)
    assert ids.size > 4_000_000 and ids.size != d["lists"].isect_ids.numel()
    assert_equal(np32(lists.isect_ids), ids, "isect_ids")
    assert_equal(np32(lists.flatten_ids), fl, "flatten_ids")
    assert_equal(np32(off), binning.isect_offset_encode(ids, 1, 32, 32), "tile_offsets")
    print(f"config 4 at 180 degrees: {ids.size} tile records", flush=True)
    v = torch.randn((1, 512, 512), generator=torch.Generator().manual_seed(180))
    refs = raster_references(np32(m2), np32(conics), np32(op), np32(mus), np32(off), fl, 512,
                             512, 16, v_image=v.numpy())
    img = W.rasterize_to_pixels_fwd(m2, conics, op, mus, off, lists.flatten_ids, 512, 512, 16)
    _report("180 fwd", check_raster(refs, image=np32(img)))
    got = _ops.raster_backward(m2, conics, op, mus, off, lists, v.to(DEV), 512, 512, 16, True)
    _report("180 two-pass", check_raster(refs, grads=_grads(got)))
    one = _ops.TileLists(*lists[:3], None, None)
    got1 = _ops.raster_backward(m2, conics, op, mus, off, one, v.to(DEV), 512, 512, 16, True)
    _report("180 one-pass", check_raster(refs, grads=_grads(got1)))


def test_config4_volume_regulariser_voxelization(config4):
    """The trainer's 128^3 volume of the 500k tree over [-1, 1]^3 (large,
    near-source footprints: the chunked backward's dense-wave path)."""
    d = config4
    rng, ctr = torch.full((3,), 2.0, device=DEV), torch.zeros(3, device=DEV)
    m3, con, r3 = W.world_to_volume_mapping_fwd(d["means"], d["covars"], d["max_scales"], rng,
                                                ctr, 128, 128, 128, 1e-8, 3.0)
    lists = _ops.bin_tiles_3d(m3, r3, 8, 16, 16, 16)
    off = W.isect_offset_encode_3d(lists.isect_ids, 16, 16, 16)
    tpg, ids, fl = binning.isect_tiles_3d(np32(m3), np32(r3), 8, 16, 16, 16)
    assert ids.size > 1_000_000
    assert_equal(np32(lists.isect_ids), ids, "isect_ids 3d")
    assert_equal(np32(lists.flatten_ids), fl, "flatten_ids 3d")
    vol = W.voxelize_to_voxels_fwd(m3, con, d["opac"], off, lists.flatten_ids, 128, 128, 128, 8)
    v = torch.randn((128, 128, 128), generator=torch.Generator().manual_seed(7))
    refs = voxel_references(np32(m3), np32(con), np32(d["opac"]), np32(off), fl, 128, 128, 128,
                            8, v_volume=v.numpy())
    _report("tree 128^3 fwd", check_voxel(refs, volume=np32(vol)))
    got = _ops.voxel_backward(m3, con, d["opac"], off, lists, v.to(DEV), 128, 128, 128, 8)
    _report("tree 128^3 bwd", check_voxel(refs, grads=_grads(got)))
    # The forward's reach masks given to the backward: the same outputs.
    vol_r, reach = _ops.voxelize_with_reach(m3, con, d["opac"], off, lists.flatten_ids, 128, 128,
                                            128)
    assert torch.equal(vol_r, vol)
    given = _ops.voxel_backward(m3, con, d["opac"], off, lists, v.to(DEV), 128, 128, 128, 8,
                                reach=reach)
    for a, b in zip(got, given):
        assert torch.equal(a, b)


# ---------------------------------------------------------------- config 3 --

@pytest.fixture(scope="module")
def config3():
    g = torch.Generator().manual_seed(1)
    raw = scenes.random_gaussians(200_000, g, -4.5, 0.6)
    covars, max_scales, opac = W.prepare_gaussians(raw.quats.to(DEV), raw.raw_scales.to(DEV),
                                                   raw.raw_opacities.to(DEV), SMIN, SMAX)
    rng, ctr = torch.full((3,), 2.0, device=DEV), torch.zeros(3, device=DEV)
    means = raw.means.to(DEV)
    m3, con, r3 = W.world_to_volume_mapping_fwd(means, covars, max_scales, rng, ctr, 256, 256,
                                                256, 1e-8, 3.0)
    lists = _ops.bin_tiles_3d(m3, r3, 8, 32, 32, 32)
    off = W.isect_offset_encode_3d(lists.isect_ids, 32, 32, 32)
    v = torch.randn((256, 256, 256), generator=g)
    print(f"config 3: {lists.isect_ids.numel()} brick records", flush=True)
    return dict(means=means, covars=covars, m3=m3, con=con, r3=r3, op=opac, lists=lists,
                off=off, v=v)


@pytest.fixture(scope="module")
def config3_refs(config3):
    d = config3
    refs = voxel_references(np32(d["m3"]), np32(d["con"]), np32(d["op"]), np32(d["off"]),
                            np32(d["lists"].flatten_ids), 256, 256, 256, 8,
                            v_volume=d["v"].numpy())
    print("config 3 oracle done", flush=True)
    return refs


def test_config3_mapping_and_brick_lists_bit_exact(config3):
    d = config3
    m3, con, r3 = ops.world_to_volume_mapping_fwd(
        np32(d["means"]), np32(d["covars"]), np.full(3, 2.0, np.float32),
        np.zeros(3, np.float32), 256, 256, 256, 1e-8, 3.0)
    assert_equal(np32(d["m3"]), m3, "means3d")
    assert_equal(np32(d["con"]), con, "conics3d")
    assert_equal(np32(d["r3"]), r3, "radii3d")
    tpg, ids, fl = binning.isect_tiles_3d(m3, r3, 8, 32, 32, 32)
    assert ids.size > 3_000_000
    assert_equal(np32(d["lists"].tiles_per_gauss), tpg, "tiles_per_gauss")
    assert_equal(np32(d["lists"].isect_ids), ids, "isect_ids")
    assert_equal(np32(d["lists"].flatten_ids), fl, "flatten_ids")
    assert_equal(np32(d["off"]), binning.isect_offset_encode_3d(ids, 32, 32, 32), "offsets")


def test_config3_voxel_forward_and_backward(config3, config3_refs):
    d = config3
    vol = W.voxelize_to_voxels_fwd(d["m3"], d["con"], d["op"], d["off"],
                                   d["lists"].flatten_ids, 256, 256, 256, 8)
    _report("fwd", check_voxel(config3_refs, volume=np32(vol)))
    got = _ops.voxel_backward(d["m3"], d["con"], d["op"], d["off"], d["lists"], d["v"].to(DEV),
                              256, 256, 256, 8)
    _report("two-pass", check_voxel(config3_refs, grads=_grads(got)))
    again = _ops.voxel_backward(d["m3"], d["con"], d["op"], d["off"], d["lists"],
                                d["v"].to(DEV), 256, 256, 256, 8)
    for a, b in zip(got, again):
        assert torch.equal(a, b)
    vol_r, reach = _ops.voxelize_with_reach(d["m3"], d["con"], d["op"], d["off"],
                                            d["lists"].flatten_ids, 256, 256, 256)
    assert torch.equal(vol_r, vol)
    given = _ops.voxel_backward(d["m3"], d["con"], d["op"], d["off"], d["lists"],
                                d["v"].to(DEV), 256, 256, 256, 8, reach=reach)
    for a, b in zip(got, given):
        assert torch.equal(a, b)


def test_config3_one_pass_backward(config3, config3_refs):
    d = config3
    one = _ops.TileLists(*d["lists"][:3], None, None)
    got = _ops.voxel_backward(d["m3"], d["con"], d["op"], d["off"], one, d["v"].to(DEV), 256,
                              256, 256, 8)
    _report("one-pass", check_voxel(config3_refs, grads=_grads(got)))
