"""r2splat.ops end to end on the GPU vs the oracle composition.

prepare -> explicit_rasterize -> explicit_voxelize -> losses' upstream
gradients -> explicit_backward, compared with oracle/compose.py on the same
seeded inputs; plus the API's one-shot guards and mode equivalences.

Parity of every output, up to the composed parameter gradients, is checked
by tests/pipeline_check.py (fp64-anchored, alpha flips counted).

The API cases drive the operators the way src/models/gaussian_model.py does
(:375-416, :443-480): a [C, H, W] image handed on as renders [C, W, H, 1],
and volume_shape (W, D, H) as dim2 = W, dim1 = D, dim0 = H with ranges and
centres from a bounding box.  With W != H and W != D != H, a swap of the
image axes or of dim2 / dim0 anywhere in r2splat.ops fails them.
"""

import numpy as np
import pytest
import torch

from helpers import make_scene
from pipeline_check import DEV, SMAX, SMIN, check_against_oracle, detector_views, params_of, run
from r2splat.ops import direct, explicit

pytestmark = pytest.mark.gpu


def test_explicit_pipeline_matches_oracle():
    raw, viewmats, Ks, _ = make_scene(3000, 11, n_det=64, log_mu=-3.6)
    out = run(raw, viewmats, Ks, 64, 64, (32, 32, 32))
    check_against_oracle(out, raw, viewmats, Ks, 64, 64, (32, 32, 32))


@pytest.mark.parametrize("width,height,volume_shape", [(80, 48, (24, 16, 40)),
                                                      (40, 72, (36, 28, 12))])
def test_model_argument_mapping_non_square(width, height, volume_shape):
    """W != H detector and a W x D x H volume through the model's mapping, two
    views, against the oracle (image rows = detector v, volume axes z, y, x)."""
    raw, _, _, g = make_scene(2500, 21, log_mu=-3.5)
    viewmats, Ks = detector_views([0.4, 2.1], width, height)
    bbox = ((-1.0, -0.8, -1.2), (1.0, 1.1, 0.9))
    out = run(raw, viewmats, Ks, width, height, volume_shape, bbox=bbox, seed=5)
    assert int(out["state"].projection.lists.isect_ids.numel()) > 1000
    check_against_oracle(out, raw, viewmats, Ks, width, height, volume_shape)


def test_swapped_axes_are_caught():
    """The composition at the transposed shapes differs from the correct one:
    a W/H or dim2/dim0 swap would fail the checks above."""
    raw, _, _, _ = make_scene(800, 22, log_mu=-3.5)
    viewmats, Ks = detector_views([0.4], 80, 48)
    means, quats, scales, opac = params_of(raw)
    st = direct.prepare_inference_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    kw = dict(tile_size=16, eps2d=1e-8, radius_clip=3.0)
    good = direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), img_w=80,
                                      img_h=48, **kw)
    bad = direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), img_w=48,
                                     img_h=80, **kw)
    assert good.image.shape == (1, 48, 80) and bad.image.shape == (1, 80, 48)
    assert not torch.equal(good.image[:, :48, :48], bad.image[:, :48, :48])
    rng = torch.tensor([2.0, 1.9, 2.1], device=DEV)
    ctr = torch.tensor([0.0, 0.15, -0.15], device=DEV)
    vk = dict(tile_size=8, eps3d=1e-8, radius_clip=3.0)
    a = direct.inference_voxelize(st, means, rng, ctr, dim2=24, dim1=16, dim0=40, **vk)
    b = direct.inference_voxelize(st, means, rng, ctr, dim2=40, dim1=16, dim0=24, **vk)
    assert a.volume.shape == (40, 16, 24)
    assert not torch.equal(a.volume.permute(2, 1, 0), b.volume)


def test_inference_equals_explicit_forward_and_is_reusable():
    raw, viewmats, Ks, _ = make_scene(2000, 12, n_det=48)
    means, quats, scales, opac = params_of(raw)
    st = direct.prepare_inference_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    kw = dict(img_w=48, img_h=48, tile_size=16, eps2d=1e-8, radius_clip=3.0)
    a = direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), **kw)
    b = direct.inference_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), **kw)
    assert not a.image.requires_grad
    assert torch.equal(a.image, b.image)
    ex = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN, scale_max=SMAX)
    c = explicit.explicit_rasterize(ex, means, viewmats.to(DEV), Ks.to(DEV), absgrad=False, **kw)
    assert c.image.requires_grad and c.image.is_leaf and c.means2d.is_leaf
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
    assert not hasattr(c.means2d, "absgrad")
    assert means.grad is not None and float(means.grad.abs().sum()) == 0.0
    with pytest.raises(RuntimeError, match="only run once"):
        explicit.explicit_backward(ex, means, quats, scales, opac)


def test_backward_accumulates_into_existing_grads():
    raw, viewmats, Ks, _ = make_scene(1500, 15, n_det=48, log_mu=-3.6)
    outs = []
    for pre in (False, True):
        means, quats, scales, opac = params_of(raw)
        if pre:
            for t in (means, quats, scales, opac):
                t.grad = torch.ones_like(t)
        st = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN,
                                                 scale_max=SMAX)
        res = explicit.explicit_rasterize(st, means, viewmats.to(DEV), Ks.to(DEV), img_w=48,
                                          img_h=48, tile_size=16, eps2d=1e-8, radius_clip=3.0,
                                          absgrad=True)
        res.image.square().sum().backward()
        explicit.explicit_backward(st, means, quats, scales, opac)
        outs.append([t.grad.clone() for t in (means, quats, scales, opac)])
    for a, b in zip(*outs):
        assert torch.equal(a + 1, b)


def test_pixel_and_primitive_backward_agree():
    raw, viewmats, Ks, _ = make_scene(2000, 13, n_det=64, log_mu=-3.6)
    a = run(raw, viewmats, Ks, 64, 64, (24, 24, 24), mode="primitive")
    b = run(raw, viewmats, Ks, 64, 64, (24, 24, 24), mode="pixel")
    # Both modes run the same deterministic kernels here.
    for k in ("means", "quats", "scales", "opac"):
        assert torch.equal(a[k].grad, b[k].grad), k


def test_guards():
    raw, viewmats, Ks, _ = make_scene(10, 14)
    with pytest.raises(RuntimeError, match="require CUDA tensors"):
        direct.prepare_inference_gaussians(raw.quats, raw.raw_scales, raw.raw_opacities,
                                           scale_min=SMIN, scale_max=SMAX)
    means, quats, scales, opac = params_of(raw)
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
