"""HIP operators against the committed golden fixtures (tests/golden/).

Given the fixture's covariances, the projection, conics/mu, volume mapping,
tile lists, offsets and the compaction must equal the fixture bit for bit.
Operators that evaluate exp (the sigmoid / softplus of the parameter
transform, the rasterizer, the voxelizer) and the composed gradients match
within rel 1e-4 / abs 1e-5 (fp32), with the alpha cut-off allowance of
tests/helpers.py.
"""

import os

import numpy as np
import pytest
import torch

from helpers import assert_close, assert_equal, np32
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
    assert_close(np32(img), f["image"], "image", max_outliers=2, outlier_atol=3e-5)


def test_projection_pipeline_fixture():
    f = _load("projection_small.npz")
    params = [torch.nn.Parameter(_t(f[k]).clone())
              for k in ("means", "quats", "raw_scales", "raw_opacities")]
    means, quats, scales, opac = params
    state = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=5e-4,
                                                scale_max=1.0)
    assert_close(np32(state.covars), f["covars"], "covars", atol=1e-9)
    assert_close(np32(state.opacities), f["opacities"], "opacities")
    res = explicit.explicit_rasterize(state, means, _t(f["viewmats"]), _t(f["Ks"]), img_w=48,
                                      img_h=48, tile_size=16, eps2d=1e-8, radius_clip=3.0,
                                      absgrad=True)
    assert_close(np32(res.image), f["image"], "image", max_outliers=2, outlier_atol=3e-5)
    res.image.backward(_t(f["v_image"]))
    explicit.explicit_backward(state, means, quats, scales, opac)
    for name, got in (("means", means.grad), ("quats", quats.grad), ("raw_scales", scales.grad),
                      ("raw_opacities", opac.grad), ("means2d", res.means2d.grad),
                      ("means2d_abs", res.means2d.absgrad)):
        e = f[f"grad_{name}"]
        scale = float(np.abs(e).max())
        # The covariances enter through exp (sigmoid), so the composed
        # gradients carry their ulp-level differences: same allowance as the
        # end-to-end pipeline test.
        assert_close(np32(got), e, f"grad {name}", atol=max(1e-5, 1e-5 * scale),
                     max_outliers=e.size // 200, outlier_atol=1e-3 * scale)


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
    assert_close(np32(vol), f["volume"], "volume", max_outliers=2, outlier_atol=3e-6)
    vm3, vc3, vo3 = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, opac, off, ids, fl,
                                                          _t(f["v_volume"]), 16, 12, 20, 8)
    for name, got in (("vox_v_means3d", vm3), ("vox_v_conics", vc3), ("vox_v_opacities", vo3)):
        e = f[name]
        scale = float(np.abs(e).max())
        assert_close(np32(got), e, name, atol=max(1e-5, 3e-6 * scale), max_outliers=2,
                     outlier_atol=2e-4 * scale)
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
