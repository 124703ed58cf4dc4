"""r2splat.ops end to end on the GPU vs the oracle composition.

prepare -> explicit_rasterize -> explicit_voxelize -> losses' upstream
gradients -> explicit_backward, compared with oracle/compose.py on the same
seeded inputs; plus the API's one-shot guards and mode equivalences.
"""

import numpy as np
import pytest
import torch

from helpers import assert_close, assert_equal, make_scene, np32
from oracle import compose
from r2splat.ops import direct, explicit

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMIN, SMAX = 5e-4, 1.0


def _params(raw):
    return [torch.nn.Parameter(t.clone().to(DEV)) for t in
            (raw.means, raw.quats, raw.raw_scales, raw.raw_opacities)]


def _run(raw, viewmats, Ks, W_img, dims, mode="primitive", absgrad=True, seed=0):
    means, quats, scales, opac = _params(raw)
    state = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN,
                                                scale_max=SMAX, backward_mode=mode)
    res = explicit.explicit_rasterize(state, means, viewmats.to(DEV), Ks.to(DEV), img_w=W_img,
                                      img_h=W_img, tile_size=16, eps2d=1e-8, radius_clip=3.0,
                                      absgrad=absgrad)
    ranges = torch.full((3,), 2.0, device=DEV)
    centers = torch.zeros(3, device=DEV)
    vox = explicit.explicit_voxelize(state, means, ranges, centers, dim2=dims[0], dim1=dims[1],
                                     dim0=dims[2], tile_size=8, eps3d=1e-8, radius_clip=3.0)
    g = torch.Generator().manual_seed(seed)
    v_img = torch.randn(res.image.shape, generator=g)
    v_vol = torch.randn(vox.volume.shape, generator=g)
    ((res.image * v_img.to(DEV)).sum() + (vox.volume * v_vol.to(DEV)).sum()).backward()
    explicit.explicit_backward(state, means, quats, scales, opac)
    return dict(state=state, res=res, vox=vox, means=means, quats=quats, scales=scales,
                opac=opac, v_img=v_img, v_vol=v_vol)


def test_explicit_pipeline_matches_oracle():
    raw, viewmats, Ks, _ = make_scene(3000, 11, n_det=64, log_mu=-3.6)
    out = _run(raw, viewmats, Ks, 64, (32, 32, 32))
    r = {k: v.double().numpy() if False else v.numpy() for k, v in
         dict(means=raw.means, quats=raw.quats, scales=raw.raw_scales,
              opac=raw.raw_opacities).items()}
    covars, _, opac = compose.prepare(r["quats"], r["scales"], r["opac"], SMIN, SMAX)
    assert_close(np32(out["state"].covars), covars, "covars")
    proj = compose.rasterize_forward(r["means"], np32(out["state"].covars),
                                     np32(out["state"].opacities), viewmats.numpy(), Ks.numpy(),
                                     64, 64, 16, 1e-8, 3.0)
    # Binning is a pure function of (means2d, radii): same inputs, same list.
    assert_equal(np32(out["res"].means2d), proj["means2d"], "means2d")
    assert_equal(np32(out["res"].radii), proj["radii"], "radii")
    assert_equal(np32(out["state"].projection.isect_ids), proj["isect_ids"], "isect_ids")
    assert_equal(np32(out["state"].projection.flatten_ids), proj["flatten_ids"], "flatten_ids")
    assert_close(np32(out["res"].image), proj["output"], "image", max_outliers=4,
                 outlier_atol=3e-5)
    vox = compose.voxelize_forward(r["means"], np32(out["state"].covars),
                                   np32(out["state"].opacities), np.full(3, 2.0, np.float32),
                                   np.zeros(3, np.float32), 32, 32, 32, 8, 1e-8, 3.0)
    assert_equal(np32(out["state"].voxel.isect_ids), vox["isect_ids"], "isect_ids 3d")
    assert_close(np32(out["vox"].volume), vox["output"], "volume", max_outliers=30,
                 outlier_atol=3e-6)
    grads = compose.explicit_backward(np32(out["state"].covars), proj, vox, r["means"],
                                      r["quats"], r["scales"], r["opac"], SMIN, SMAX,
                                      out["v_img"].numpy(), out["v_vol"].numpy())
    for name, param in (("means", "means"), ("quats", "quats"), ("raw_scales", "scales"),
                        ("raw_opacities", "opac")):
        e = grads[name]
        scale = float(np.abs(e).max())
        assert_close(np32(out[param].grad), e, f"grad {name}", atol=max(1e-5, 1e-5 * scale),
                     max_outliers=e.size // 200, outlier_atol=1e-3 * scale)
    scale = float(np.abs(grads["means2d"]).max())
    assert_close(np32(out["res"].means2d.grad), grads["means2d"], "means2d.grad",
                 atol=max(1e-5, 1e-5 * scale), max_outliers=20, outlier_atol=1e-3 * scale)
    assert_close(np32(out["res"].means2d.absgrad), grads["means2d_abs"], "means2d.absgrad",
                 atol=max(1e-5, 1e-5 * scale), max_outliers=20, outlier_atol=1e-3 * scale)


def test_inference_equals_explicit_forward_and_is_reusable():
    raw, viewmats, Ks, _ = make_scene(2000, 12, n_det=48)
    means, quats, scales, opac = _params(raw)
    st = direct.prepare_inference_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    kw = dict(img_w=48, img_h=48, tile_size=16, eps2d=1e-8, radius_clip=3.0)
    a = direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), **kw)
    b = direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), **kw)
    assert not a.image.requires_grad
    assert torch.equal(a.image, b.image)
    ex = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    c = explicit.explicit_rasterize(ex, means, viewmats.to(DEV), Ks.to(DEV), absgrad=False, **kw)
    assert torch.equal(a.image, c.image.detach())
    with pytest.raises(RuntimeError, match="rasterized once"):
        explicit.explicit_rasterize(ex, means, viewmats.to(DEV), Ks.to(DEV), absgrad=False, **kw)
    vkw = dict(dim2=16, dim1=16, dim0=16, tile_size=8, eps3d=1e-8, radius_clip=3.0)
    rng, ctr = torch.full((3,), 2.0, device=DEV), torch.zeros(3, device=DEV)
    v1 = direct.inference_voxelize(st, means, rng, ctr, **vkw)
    v2 = explicit.explicit_voxelize(ex, means, rng, ctr, **vkw)
    assert torch.equal(v1.volume, v2.volume.detach())
    with pytest.raises(RuntimeError, match="voxelized once"):
        explicit.explicit_voxelize(ex, means, rng, ctr, **vkw)
    # No image gradient: zero means2d grad, parameters still receive grads.
    explicit.explicit_backward(ex, means, quats, scales, opac)
    assert float(c.means2d.grad.abs().sum()) == 0.0
    with pytest.raises(RuntimeError, match="only run once"):
        explicit.explicit_backward(ex, means, quats, scales, opac)


def test_pixel_and_primitive_backward_agree():
    raw, viewmats, Ks, _ = make_scene(2000, 13, n_det=64, log_mu=-3.6)
    a = _run(raw, viewmats, Ks, 64, (24, 24, 24), mode="primitive")
    b = _run(raw, viewmats, Ks, 64, (24, 24, 24), mode="pixel")
    for k in ("means", "quats", "scales", "opac"):
        e = np32(a[k].grad)
        assert_close(np32(b[k].grad), e, f"{k} pixel vs primitive",
                     atol=1e-5 * (float(np.abs(e).max()) + 1))


def test_guards():
    raw, viewmats, Ks, _ = make_scene(10, 14)
    with pytest.raises(RuntimeError, match="require CUDA tensors"):
        direct.prepare_inference_gaussians(raw.quats, raw.raw_scales, raw.raw_opacities,
                                           scale_min=SMIN, scale_max=SMAX)
    means, quats, scales, opac = _params(raw)
    st = direct.prepare_inference_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    with pytest.raises(ValueError, match="tile_size"):
        direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), img_w=16, img_h=16,
                                   tile_size=33, eps2d=1e-8, radius_clip=3.0)
    with pytest.raises(ValueError, match="tile_size"):
        direct.inference_voxelize(st, means, torch.ones(3, device=DEV), torch.zeros(3, device=DEV),
                                  dim2=8, dim1=8, dim0=8, tile_size=11, eps3d=1e-8,
                                  radius_clip=3.0)
    with pytest.raises(ValueError, match="backward_mode"):
        explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX,
                                            backward_mode="bogus")
    ex = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    with pytest.raises(RuntimeError, match="projection forward"):
        explicit.explicit_backward(ex, means, quats, scales, opac)
