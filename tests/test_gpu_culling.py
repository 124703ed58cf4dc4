"""Rasterizer and voxelizer on hard footprints vs the CPU oracle.

The kernels visit only the pixels / voxels inside the alpha-test ellipse of
each record; the oracle evaluates every element of the tile.  These cases
stress that culling: conic eigenvalues spread over many decades (needle and
pancake footprints, sub-pixel and multi-tile), conics that are not positive
definite (the kernels must fall back to the whole tile), negative weights,
weights just above and below the alpha threshold, and means outside the
image / volume.
"""

import numpy as np
import pytest
import torch

from helpers import check_raster, check_voxel, np32, raster_references, voxel_references
from r2splat.cuda import _ops
from r2splat.cuda import _wrapper as W

pytestmark = pytest.mark.gpu


def fl_keys(tile_offsets):
    """Number of tile / brick keys of a tile_offsets tensor."""
    return tile_offsets.numel()

DEV = "cuda"


def _spd(rng, n, d, log_lo, log_hi):
    """n random d x d matrices with eigenvalues exp(U(log_lo, log_hi))."""
    q, _ = np.linalg.qr(rng.normal(size=(n, d, d)))
    ev = np.exp(rng.uniform(log_lo, log_hi, size=(n, d)))
    return np.einsum("nij,nj,nkj->nik", q, ev, q), ev


def _weights(rng, n, thr):
    w = np.exp(rng.uniform(np.log(0.3 * thr), np.log(2.0), size=n)) * rng.choice([-1.0, 1.0], n)
    w[: n // 20] = thr * (1.0 + rng.uniform(-1e-3, 1e-3, size=n // 20))  # at the cut-off
    return w


def _radius(ev_conic, w, thr):
    s = np.log(np.maximum(np.abs(w) / thr, 1.0))
    return np.ceil(np.sqrt(2.0 * s / ev_conic.min(axis=1))) + 1.0


# Conic eigenvalue ranges (log).  fp32 evaluates sigma of a strongly
# anisotropic conic with cancellation, whatever the summation order (the
# reference's included), so the float32 cases keep the spread moderate; the
# float64 cases cover the extreme shapes.
_LOG_EV = {torch.float32: (-4.5, 1.5), torch.float64: (-7.0, 3.0)}


def _raster_case(seed, n, W_img, H_img, dtype):
    rng = np.random.default_rng(seed)
    P, ev = _spd(rng, n, 2, *_LOG_EV[dtype])
    bad = rng.random(n) < 0.1  # indefinite conics
    P[bad, 1, 1] = -np.abs(P[bad, 1, 1])
    conics = np.stack([P[:, 0, 0], P[:, 0, 1], P[:, 1, 1]], -1)[None]
    opac = rng.uniform(-1.0, 1.5, size=n)
    mus = _weights(rng, n, 1e-5) / np.where(opac == 0, 1.0, opac)
    means = np.stack([rng.uniform(-10, W_img + 10, n), rng.uniform(-10, H_img + 10, n)], -1)[None]
    rad = np.where(bad, 6.0, np.minimum(_radius(ev, opac * mus, 1e-5), 4 * max(W_img, H_img)))
    t = lambda a: torch.as_tensor(a, dtype=dtype, device=DEV).contiguous()  # noqa: E731
    radii = torch.as_tensor(np.stack([rad, rad], -1)[None], dtype=torch.int32, device=DEV)
    return t(means), t(conics), t(opac[None]), t(mus[None]), radii


@pytest.mark.parametrize("order", ["emission", "tile"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("W_img,H_img,ts", [(96, 80, 16), (50, 37, 8)])
def test_rasterize_hard_footprints(dtype, W_img, H_img, ts, order):
    m2, con, op, mu, radii = _raster_case(11, 1500, W_img, H_img, dtype)
    tw, th = -(-W_img // ts), -(-H_img // ts)
    _, ids, fl = W.isect_tiles(m2, radii, ts, tw, th)
    off = W.isect_offset_encode(ids, 1, tw, th)
    assert fl.numel() > 1000
    img = W.rasterize_to_pixels_fwd(m2, con, op, mu, off, fl, W_img, H_img, ts)
    v = torch.randn(img.shape, generator=torch.Generator().manual_seed(3), dtype=dtype)
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


def _voxel_case(seed, n, dims, dtype):
    rng = np.random.default_rng(seed)
    P, ev = _spd(rng, n, 3, *_LOG_EV[dtype])
    bad = rng.random(n) < 0.1
    P[bad, 2, 2] = -np.abs(P[bad, 2, 2])
    conics = np.stack([P[:, 0, 0], P[:, 0, 1], P[:, 0, 2], P[:, 1, 1], P[:, 1, 2], P[:, 2, 2]], -1)
    opac = _weights(rng, n, 1e-6)
    d2, d1, d0 = dims
    means = np.stack([rng.uniform(-6, d + 6, n) for d in (d2, d1, d0)], -1)
    rad = np.where(bad, 5.0, np.minimum(_radius(ev, opac, 1e-6), 2 * max(dims)))
    t = lambda a: torch.as_tensor(a, dtype=dtype, device=DEV).contiguous()  # noqa: E731
    radii = torch.as_tensor(np.stack([rad] * 3, -1), dtype=torch.int32, device=DEV)
    return t(means), t(conics), t(opac), radii


@pytest.mark.parametrize("order", ["emission", "tile"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("dims,ts", [((40, 36, 28), 8), ((21, 19, 23), 4)])
def test_voxelize_hard_footprints(dtype, dims, ts, order):
    m3, con, op, radii = _voxel_case(12, 1200, dims, dtype)
    d2, d1, d0 = dims
    n2, n1, n0 = (-(-x // ts) for x in dims)
    _, ids, fl = W.isect_tiles_3d(m3, radii, ts, n2, n1, n0)
    off = W.isect_offset_encode_3d(ids, n2, n1, n0)
    assert fl.numel() > 1000
    vol = W.voxelize_to_voxels_fwd(m3, con, op, off, fl, d2, d1, d0, ts)
    v = torch.randn(vol.shape, generator=torch.Generator().manual_seed(4), dtype=dtype)
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
