"""HIP operators against the committed golden fixtures (tests/golden/).

Given the fixture's covariances, the projection, conics/mu, volume mapping,
tile lists, offsets and the compaction must equal the fixture bit for bit.
Operators that evaluate exp (the sigmoid / softplus of the parameter
transform, the rasterizer, the voxelizer) and the composed gradients meet the
parity bar of helpers.assert_parity with the fixture as the reference-order
float32 result and the oracle one precision up as the anchor.
"""

import os

import numpy as np
import pytest
import torch

from helpers import (assert_equal, assert_parity, check_parameter_gradients, check_raster,
                     check_voxel, np32, raster_references, voxel_references)
from oracle import compose, ops
from r2splat.cuda import _ops
from r2splat.cuda import _wrapper as W
from r2splat.ops import compact, explicit

pytestmark = pytest.mark.gpu

DEV = "cuda"
HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(HERE, name)))


def _t(a, dtype=None):
    t = torch.as_tensor(a).to(DEV)
    return t if dtype is None else t.to(dtype)


def test_projection_ops_fixture():
    f = _load("projection_small.npz")
    m2, cov2d, radii, conics, mus, op = W.project_gaussians_fwd(
        _t(f["means"]), _t(f["covars"]), _t(f["opacities"]), _t(f["viewmats"]), _t(f["Ks"]), 48,
        48, 1e-8, 3.0)
    assert_equal(np32(m2), f["means2d"], "means2d")
    assert_equal(np32(cov2d), f["cov2d"], "cov2d")
    assert_equal(np32(radii), f["radii"], "radii")
    assert_equal(np32(conics), f["conics"], "conics")
    assert_equal(np32(mus), f["mus"], "mus")
    _, ids, fl = W.isect_tiles(m2, radii, 16, 3, 3)
    off = W.isect_offset_encode(ids, 1, 3, 3)
    assert_equal(np32(ids), f["isect_ids"], "isect_ids")
    assert_equal(np32(fl), f["flatten_ids"], "flatten_ids")
    assert_equal(np32(off), f["tile_offsets"], "tile_offsets")
    img = W.rasterize_to_pixels_fwd(m2, conics, op, mus, off, fl, 48, 48, 16)
    refs = raster_references(f["means2d"], f["conics"], np32(op), f["mus"], f["tile_offsets"],
                             f["flatten_ids"], 48, 48, 16)
    assert_equal(refs["fwd"][1], f["image"], "oracle image = fixture")
    check_raster(refs, image=np32(img))


def test_projection_pipeline_fixture():
    f = _load("projection_small.npz")
    params = [torch.nn.Parameter(_t(f[k]).clone())
              for k in ("means", "quats", "raw_scales", "raw_opacities")]
    means, quats, scales, opac = params
    state = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=5e-4,
                                                scale_max=1.0)
    hi = lambda k: f[k].astype(np.float64)  # noqa: E731
    cov64, _ = ops.parameter_transform_fwd(hi("quats"), hi("raw_scales"), 5e-4, 1.0)
    assert_parity(np32(state.covars), cov64, f["covars"], None, "covars")
    assert_parity(np32(state.opacities), ops.softplus(hi("raw_opacities")), f["opacities"], None,
                  "opacities")
    res = explicit.explicit_rasterize(state, means, _t(f["viewmats"]), _t(f["Ks"]), img_w=48,
                                      img_h=48, tile_size=16, eps2d=1e-8, radius_clip=3.0,
                                      absgrad=True)
    res.image.backward(_t(f["v_image"]))
    explicit.explicit_backward(state, means, quats, scales, opac)
    # The fixture's chain ran on its own covariances; the GPU's differ in the
    # last ulp (exp), so the composition is re-evaluated on the GPU's forward
    # (bit-exact geometry and lists) and the fixture pins the oracle itself.
    gc, go = np32(state.covars), np32(state.opacities)
    proj = compose.rasterize_forward(f["means"], gc, go, f["viewmats"], f["Ks"], 48, 48, 16,
                                     1e-8, 3.0)
    assert_equal(np32(state.projection.lists.flatten_ids), proj["flatten_ids"], "flatten_ids")
    refs = raster_references(proj["means2d"], proj["conics"], proj["opacity"], proj["mus"],
                             proj["tile_offsets"], proj["flatten_ids"], 48, 48, 16,
                             v_image=f["v_image"])
    check_raster(refs, image=np32(res.image))
    p = state.projection
    rg = [np32(t) for t in _ops.raster_backward(p.means2d.detach(), p.conics, p.weights, p.mus,
                                                p.tile_offsets, p.lists, p.image.grad, 48, 48,
                                                16, True)]
    check_raster(refs, grads=rg)
    assert np.array_equal(rg[1], np32(res.means2d.grad))
    assert np.array_equal(rg[0], np32(res.means2d.absgrad))
    args = (gc, proj, None, f["means"], f["quats"], f["raw_scales"], f["raw_opacities"], 5e-4,
            1.0, f["v_image"])
    got = dict(means=np32(means.grad), quats=np32(quats.grad), raw_scales=np32(scales.grad),
               raw_opacities=np32(opac.grad))
    reps, plain = check_parameter_gradients(got, args, rg)
    print(reps, plain)
    # The fixture's gradients are the oracle's on the fixture's covariances.
    fix = compose.explicit_backward(f["covars"], compose.rasterize_forward(
        f["means"], f["covars"], f["opacities"], f["viewmats"], f["Ks"], 48, 48, 16, 1e-8, 3.0),
        None, f["means"], f["quats"], f["raw_scales"], f["raw_opacities"], 5e-4, 1.0,
        f["v_image"])
    for name in ("means", "quats", "raw_scales", "raw_opacities", "means2d", "means2d_abs"):
        assert_equal(fix[name], f[f"grad_{name}"], f"oracle grad {name} = fixture")


def test_voxel_fixture():
    f = _load("voxel_small.npz")
    covars, opac = _t(f["covars"]), _t(f["opacities"])
    means = _t(f["means"])
    m3, con, r3 = W.world_to_volume_mapping_fwd(means, covars, opac, _t(f["ranges"]),
                                                _t(f["centers"]), 16, 12, 20, 1e-8, 3.0)
    assert_equal(np32(m3), f["vox_means3d"], "means3d")
    assert_equal(np32(con), f["vox_conics"], "conics3d")
    assert_equal(np32(r3), f["vox_radii"], "radii3d")
    _, ids, fl = W.isect_tiles_3d(m3, r3, 8, 2, 2, 3)
    off = W.isect_offset_encode_3d(ids, 2, 2, 3)
    assert_equal(np32(ids), f["vox_isect_ids"], "isect_ids3d")
    assert_equal(np32(fl), f["vox_flatten_ids"], "flatten_ids3d")
    assert_equal(np32(off), f["vox_tile_offsets"], "tile_offsets3d")
    vol = W.voxelize_to_voxels_fwd(m3, con, opac, off, fl, 16, 12, 20, 8)
    vm3, vc3, vo3 = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, opac, off, ids, fl,
                                                          _t(f["v_volume"]), 16, 12, 20, 8)
    refs = voxel_references(f["vox_means3d"], f["vox_conics"], f["opacities"],
                            f["vox_tile_offsets"], f["vox_flatten_ids"], 16, 12, 20, 8,
                            v_volume=f["v_volume"])
    assert_equal(refs["fwd"][1], f["volume"], "oracle volume = fixture")
    for (_, lo, _, _), name in zip(refs["bwd"], ("vox_v_means3d", "vox_v_conics",
                                              "vox_v_opacities")):
        assert_equal(lo, f[name], f"oracle {name} = fixture")
    print(check_voxel(refs, volume=np32(vol), grads=[np32(t) for t in (vm3, vc3, vo3)]))
    vm, vc = W.world_to_volume_mapping_bwd(means, covars, _t(f["ranges"]), _t(f["centers"]),
                                           16, 12, 20, 1e-8, _t(f["vox_v_means3d"]),
                                           _t(f["vox_v_conics"]))
    assert_equal(np32(vm), f["vox_v_means"], "mapping v_means")
    assert_equal(np32(vc), f["vox_v_covars"], "mapping v_covars")


def test_compaction_fixture():
    f = _load("compaction.npz")
    sel, rest = compact.split_indices(_t(f["mask"]))
    assert_equal(np32(sel), f["sel"], "sel")
    assert_equal(np32(rest), f["rest"], "rest")
