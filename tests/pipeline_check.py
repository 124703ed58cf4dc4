"""One explicit training step through r2splat.ops, driven with the argument
mapping of src/models/gaussian_model.py, and its check against the oracle
composition (shared by the GPU pipeline and config tests; not collected).

Every output meets helpers.assert_parity against the oracle one precision
up: the covariances and opacities, the image and volume, every raster and
voxel VJP output (the sums: alpha flips counted), and -- compositionally --
the four parameter gradients, whose chain after the raster / voxel VJPs is
checked on the kernels' own VJP outputs (helpers.check_parameter_gradients).
"""

import numpy as np
import torch

from helpers import (ETA, PARAM_GRADS, assert_equal, assert_parity, check_parameter_gradients,
                     check_raster, check_voxel, np32, raster_references, voxel_references)
from oracle import compose, native
from r2splat import geometry
from r2splat.cuda import _ops
from r2splat.ops import explicit

DEV = "cuda"
SMIN, SMAX = 5e-4, 1.0
ETA32 = ETA[np.dtype(np.float32)]


def params_of(raw):
    return [torch.nn.Parameter(t.clone().to(DEV)) for t in
            (raw.means, raw.quats, raw.raw_scales, raw.raw_opacities)]


def detector_views(angles, width, height, s_detector=3.0):
    """Views of a width x height detector of square pixels (ctproj.py:137-159)."""
    K = geometry.cone_beam_K((height, width), (s_detector * height / width, s_detector), 1.5)
    poses = torch.stack([geometry.cone_beam_camtoworld(a, 1.0) for a in angles])
    viewmats = geometry.invert_rigid_transform(poses)
    return viewmats, K.unsqueeze(0).expand(len(angles), 3, 3).contiguous()


class ModelGlue:
    """The argument mapping of GaussianModel.rasterize / .voxelize
    (src/models/gaussian_model.py:375-416, 443-480)."""

    img_tile_size, vol_tile_size = 16, 8
    eps2d = eps3d = 1e-8
    img_radius_clip = vol_radius_clip = 3.0

    def __init__(self, means):
        self.means = means

    def rasterize(self, state, viewmats, Ks, width, height, absgrad=True):
        res = explicit.explicit_rasterize(
            state, self.means, viewmats, Ks, img_w=width, img_h=height,
            tile_size=self.img_tile_size, eps2d=self.eps2d, radius_clip=self.img_radius_clip,
            absgrad=absgrad)
        return res.image.transpose(1, 2).unsqueeze(-1).contiguous(), res

    def voxelize(self, state, volume_shape, bbox):
        width, depth, height = volume_shape
        ranges = bbox[1] - bbox[0]
        centers = (bbox[0] + bbox[1]) / 2.0
        res = explicit.explicit_voxelize(
            state, self.means, ranges, centers, dim2=width, dim1=depth, dim0=height,
            tile_size=self.vol_tile_size, eps3d=self.eps3d, radius_clip=self.vol_radius_clip)
        return res.volume.unsqueeze(-1).contiguous(), res


def run(raw, viewmats, Ks, width, height, volume_shape=None, mode="primitive", seed=0,
        bbox=((-1.0, -1.0, -1.0), (1.0, 1.0, 1.0)), v_image=None, v_volume=None):
    """One explicit training step through the model's argument mapping, with
    upstream gradients N(0, 1) from `seed` (or the given [C, H, W] / volume
    ones).  Without volume_shape the step has no voxelization."""
    means, quats, scales, opac = params_of(raw)
    state = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN,
                                                scale_max=SMAX, backward_mode=mode)
    glue = ModelGlue(means)
    renders, res = glue.rasterize(state, viewmats.to(DEV), Ks.to(DEV), width, height)
    assert renders.shape == (viewmats.shape[0], width, height, 1)
    g = torch.Generator().manual_seed(seed)
    v_ren = (torch.randn(renders.shape, generator=g) if v_image is None
             else v_image.transpose(1, 2).unsqueeze(-1).contiguous())
    loss = (renders * v_ren.to(DEV)).sum()
    vox = v_vol = None
    if volume_shape is not None:
        bb = torch.tensor(bbox, device=DEV)
        volume, vox = glue.voxelize(state, volume_shape, bb)
        W_, D_, H_ = volume_shape
        assert volume.shape == (H_, D_, W_, 1)
        v_vol = (torch.randn(volume.shape, generator=g) if v_volume is None
                 else v_volume.unsqueeze(-1).contiguous())
        loss = loss + (volume * v_vol.to(DEV)).sum()
    loss.backward()
    c0 = _ops.PATH_COUNTS["one_pass"]
    explicit.explicit_backward(state, means, quats, scales, opac)
    assert _ops.PATH_COUNTS["one_pass"] == c0, "the explicit path fell back to one pass"
    return dict(state=state, res=res, vox=vox, means=means, quats=quats, scales=scales,
                opac=opac, bbox=np.asarray(bbox, np.float32),
                v_img=v_ren[..., 0].transpose(1, 2).contiguous(),  # image layout [C, H, W]
                v_vol=None if v_vol is None else v_vol[..., 0].contiguous())


def _slab_lists(v):
    """(lists, tile offsets, first layer) of each z-slab of a slabbed VolumePass."""
    n2, n1, n0 = (-(-d // v.tile_size) for d in (v.dim2, v.dim1, v.dim0))
    for z0, z1 in v.slabs:
        lists, off = _ops.bin_tiles_3d_slab(v.means3d, v.radii, v.tile_size, n2, n1, n0, z0, z1)
        yield lists, off, z0


def _voxel_lists(v):
    """A VolumePass's whole brick list (isect_ids, flatten_ids) as numpy; a
    slabbed pass's slab lists are concatenated with their keys made absolute."""
    if not v.slabs:
        return np32(v.lists.isect_ids), np32(v.lists.flatten_ids)
    plane = (-(-v.dim2 // v.tile_size)) * (-(-v.dim1 // v.tile_size))
    parts = [(np32(lists.isect_ids) + z0 * plane, np32(lists.flatten_ids))
             for lists, _, z0 in _slab_lists(v)]
    return np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])


def _voxel_vjp(v, v_volume):
    """The kernels' voxel VJP outputs for a VolumePass, the slabs' partials
    added in slab order as VolumePass.vjp adds them."""
    if not v.slabs:
        return _ops.voxel_backward(v.means3d, v.conics, v.weights, v.tile_offsets, v.lists,
                                   v_volume, v.dim2, v.dim1, v.dim0, v.tile_size)
    total = None
    for lists, off, z0 in _slab_lists(v):
        part = _ops.voxel_backward_slab(v.means3d, v.conics, v.weights, off, lists,
                                        v_volume.contiguous(), v.tile_size, z0)
        total = list(part) if total is None else [a.add_(b) for a, b in zip(total, part)]
    return total


def check_against_oracle(out, raw, viewmats, Ks, width, height, volume_shape=None):
    """Every output of a run() step against the oracle (see module docstring)."""
    st = out["state"]
    r = dict(means=raw.means.numpy(), quats=raw.quats.numpy(), scales=raw.raw_scales.numpy(),
             opac=raw.raw_opacities.numpy())
    covars, _, opac = compose.prepare(r["quats"], r["scales"], r["opac"], SMIN, SMAX)
    cov64, _, opac64 = compose.prepare(*(r[k].astype(np.float64) for k in
                                         ("quats", "scales", "opac")), SMIN, SMAX)
    assert_parity(np32(st.covars), cov64, covars, None, "covars")
    assert_parity(np32(st.opacities), opac64, opac, None, "opacities")
    # The composition runs on the GPU's covariances / opacities (their exp
    # differs in the last ulp), so its forward geometry is the GPU's.
    gc, go = np32(st.covars), np32(st.opacities)
    proj = compose.rasterize_forward(r["means"], gc, go, viewmats.numpy(), Ks.numpy(), width,
                                     height, 16, 1e-8, 3.0)
    assert_equal(np32(out["res"].means2d), proj["means2d"], "means2d")
    assert_equal(np32(out["res"].radii), proj["radii"], "radii")
    assert_equal(np32(st.projection.lists.isect_ids), proj["isect_ids"], "isect_ids")
    assert_equal(np32(st.projection.lists.flatten_ids), proj["flatten_ids"], "flatten_ids")
    assert out["res"].image.shape == (viewmats.shape[0], height, width)
    pin = [proj[k].astype(np.float64) for k in ("means2d", "conics", "opacity", "mus")]
    img_a, img_b, img_m = native.raster_fwd(*pin, proj["tile_offsets"], proj["flatten_ids"],
                                            width, height, 16, eta=ETA32, band=True, mag=True)
    print("image", assert_parity(np32(out["res"].image), img_a, proj["output"], img_b, "image",
                                 mag=img_m))
    vox = None
    if volume_shape is not None:
        W_, D_, H_ = volume_shape
        lo, hi = out["bbox"]
        vox = compose.voxelize_forward(r["means"], gc, go, hi - lo, (lo + hi) / 2, W_, D_, H_, 8,
                                       1e-8, 3.0)
        ids3, fl3 = _voxel_lists(st.voxel)
        assert_equal(ids3, vox["isect_ids"], "isect_ids 3d")
        assert_equal(fl3, vox["flatten_ids"], "flatten_ids 3d")
        vin = [vox[k].astype(np.float64) for k in ("means3d", "conics", "opacity")]
        vol_a, vol_b, vol_m = native.voxel_fwd(*vin, vox["tile_offsets"], vox["flatten_ids"],
                                               W_, D_, H_, 8, eta=ETA32, band=True, mag=True)
        print("volume", assert_parity(np32(out["vox"].volume), vol_a, vox["output"], vol_b,
                                      "volume", mag=vol_m))

    # The kernels' own raster / voxel gradients (deterministic: the same
    # values explicit_backward used), checked with their flip bands...
    p, v = st.projection, st.voxel
    rg = _ops.raster_backward(p.means2d.detach(), p.conics, p.weights, p.mus, p.tile_offsets,
                              p.lists, p.image.grad, p.width, p.height, p.tile_size, True)
    rg = [np32(t) for t in rg]
    assert np.array_equal(rg[1], np32(p.means2d.grad))
    assert np.array_equal(rg[0], np32(p.means2d.absgrad))
    refs = raster_references(proj["means2d"], proj["conics"], proj["opacity"], proj["mus"],
                             proj["tile_offsets"], proj["flatten_ids"], width, height, 16,
                             v_image=out["v_img"].numpy())
    reports = {f"raster {k}": r for k, r in check_raster(refs, grads=rg).items()}
    vg = None
    if vox is not None:
        vg = [np32(t) for t in _voxel_vjp(v, v.volume.grad)]
        vrefs = voxel_references(vox["means3d"], vox["conics"], vox["opacity"],
                                 vox["tile_offsets"], vox["flatten_ids"], W_, D_, H_, 8,
                                 v_volume=out["v_vol"].numpy())
        reports.update({f"voxel {k}": r for k, r in check_voxel(vrefs, grads=vg).items()})
    # ...and the parameter gradients composed from them.
    args = (gc, proj, vox, r["means"], r["quats"], r["scales"], r["opac"], SMIN, SMAX,
            out["v_img"].numpy(), None if vox is None else out["v_vol"].numpy())
    got = {k: np32(out[p_].grad) for k, p_ in zip(PARAM_GRADS, ("means", "quats", "scales",
                                                               "opac"))}
    prep, plain = check_parameter_gradients(got, args, rg, vg)
    reports.update({f"{k} (chain)": r for k, r in prep.items()})
    for k, rep in reports.items():
        print(k, rep)
    print("end to end within rel 1e-4 / abs 1e-5 of the float64 composition:", plain)
    return reports
