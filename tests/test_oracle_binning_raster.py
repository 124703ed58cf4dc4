"""Pins the oracle's binning, rasterizer, voxelizer and compaction on the CPU.

* Binning: a brute-force double loop over (Gaussian, tile) using the geometric
  characterisation of the reference's floor/ceil bounds -- tile [t*ts, (t+1)*ts)
  is listed iff it meets the open interval (m - r, m + r) and lies on the
  grid -- on dyadic inputs where float arithmetic is exact; plus the list
  invariants (sorted keys, ascending ids within a key, lower-bound offsets).
* Rasterizer / voxelizer: the reference tests' literal two-Gaussian cases and
  random scenes against the dense formulation of tests/test_cuda_gaussian_ops.py
  (float64, masked by each Gaussian's tile cover) and its autograd gradients.
* Compaction: torch.where.
"""

import numpy as np
import pytest
import torch

from oracle import binning, native



@pytest.fixture(autouse=True)
def _float64_default():
    # Dense references in this module are float64; restore the global default.
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _brute_2d(means2d, radii, ts, tw, th):
    pairs = []
    C, N = means2d.shape[:2]
    for c in range(C):
        for g in range(N):
            mx, my = means2d[c, g]
            rx, ry = radii[c, g] if radii.ndim == 3 else (radii[c, g], radii[c, g])
            if rx <= 0 or ry <= 0 or not (np.isfinite(mx) and np.isfinite(my)):
                continue
            for ty in range(th):
                for tx in range(tw):
                    if (mx - rx < (tx + 1) * ts and tx * ts < mx + rx
                            and my - ry < (ty + 1) * ts and ty * ts < my + ry):
                        pairs.append((c * tw * th + ty * tw + tx, c * N + g))
    return sorted(pairs)


@pytest.mark.parametrize("rect", [True, False])
def test_isect_tiles_brute_force(rect):
    r = np.random.default_rng(0)
    C, N, ts, tw, th = 2, 300, 16, 6, 5
    means2d = (np.round(r.uniform(-40, 140, size=(C, N, 2)) * 8) / 8).astype(np.float32)
    radii = r.integers(0, 40, size=(C, N, 2) if rect else (C, N)).astype(np.int32)
    means2d[0, :3, 0] = np.nan
    means2d[1, 3:6, 1] = np.inf
    tpg, keys, ids = binning.isect_tiles(means2d, radii, ts, tw, th)
    pairs = _brute_2d(means2d.astype(np.float64), radii, ts, tw, th)
    assert len(pairs) > 1000
    assert list(zip(keys.tolist(), ids.tolist())) == pairs
    # Counts per record and list invariants.
    cnt = np.bincount(ids, minlength=C * N)
    np.testing.assert_array_equal(tpg.reshape(-1), cnt)
    assert (np.diff(keys) >= 0).all()
    same = np.diff(keys) == 0
    assert (np.diff(ids)[same] > 0).all()
    off = binning.isect_offset_encode(keys, C, tw, th).reshape(-1)
    for k in range(C * tw * th):
        assert off[k] == sum(1 for kk in keys if kk < k)


def test_isect_tiles_3d_brute_force():
    r = np.random.default_rng(1)
    N, ts, n2, n1, n0 = 200, 8, 4, 3, 5
    m3 = (np.round(r.uniform(-12, 44, size=(N, 3)) * 4) / 4).astype(np.float32)
    rad = r.integers(0, 12, size=(N, 3)).astype(np.int32)
    tpg, keys, ids = binning.isect_tiles_3d(m3, rad, ts, n2, n1, n0)
    pairs = []
    grid = (n2, n1, n0)
    for g in range(N):
        if (rad[g] <= 0).any():
            continue
        # Brick b along an axis is listed iff it lies on the grid and meets
        # the open interval (m - r, m + r).
        ok = [[b for b in range(grid[a])
               if m3[g, a] - rad[g, a] < (b + 1) * ts and b * ts < m3[g, a] + rad[g, a]]
              for a in range(3)]
        for b0 in ok[2]:
            for b1 in ok[1]:
                for b2 in ok[0]:
                    pairs.append((b0 * n1 * n2 + b1 * n2 + b2, g))
    pairs.sort()
    assert len(pairs) > 300
    assert list(zip(keys.tolist(), ids.tolist())) == pairs
    np.testing.assert_array_equal(tpg, np.bincount(ids, minlength=N))
    off = binning.isect_offset_encode_3d(keys, n2, n1, n0).reshape(-1)
    np.testing.assert_array_equal(off, [np.searchsorted(keys, k) for k in range(n0 * n1 * n2)])


def test_end_bit_and_empty():
    assert binning.end_bit(1024) == 11 and binning.end_bit(32768) == 16
    assert binning.end_bit(256) == 9 and binning.end_bit(262144) == 19
    tpg, k, i = binning.isect_tiles(np.zeros((1, 4, 2), np.float32),
                                    np.zeros((1, 4, 2), np.int32), 16, 2, 2)
    assert k.size == 0 and (tpg == 0).all()
    assert (binning.isect_offset_encode(k, 1, 2, 2) == 0).all()


# --------------------------------------------------------------- rasterizer --

def _dense_raster(means2d, conics, opac, mus, H, W, mask=None):
    # tests/test_cuda_gaussian_ops.py:200-215, optionally masked by tile cover.
    py, px = torch.meshgrid(torch.arange(H) + 0.5, torch.arange(W) + 0.5, indexing="ij")
    dx = px[None, None] - means2d[..., 0, None, None]
    dy = py[None, None] - means2d[..., 1, None, None]
    sigma = (0.5 * conics[..., 0, None, None] * dx.square() + conics[..., 1, None, None] * dx * dy
             + 0.5 * conics[..., 2, None, None] * dy.square())
    alpha = opac[..., None, None] * mus[..., None, None] * torch.exp(-sigma)
    keep = (sigma >= 0) & (alpha.abs() >= 1e-5)
    if mask is not None:
        keep = keep & mask
    return torch.where(keep, alpha, 0.0).sum(dim=1)


def _pixel_mean_grads(means2d, conics, opac, mus, v, H, W, mask=None):
    """[C, N, H, W, 2]: the gradient of v_p alpha_p with respect to the mean, for
    every pixel p on its own.  Each pixel evaluates alpha with a private copy of
    the mean, so autograd of the summed dense formulation returns the per-pixel
    gradients in those copies' slots."""
    C, N = means2d.shape[:2]
    m = means2d.detach()[:, :, None, None, :].expand(C, N, H, W, 2).clone().requires_grad_(True)
    py, px = torch.meshgrid(torch.arange(H) + 0.5, torch.arange(W) + 0.5, indexing="ij")
    dx, dy = px - m[..., 0], py - m[..., 1]
    con = conics.detach()
    sigma = (0.5 * con[..., 0, None, None] * dx.square() + con[..., 1, None, None] * dx * dy
             + 0.5 * con[..., 2, None, None] * dy.square())
    alpha = (opac.detach() * mus.detach())[..., None, None] * torch.exp(-sigma)
    keep = (sigma >= 0) & (alpha.abs() >= 1e-5)
    if mask is not None:
        keep = keep & mask
    terms = torch.where(keep, alpha, 0.0) * torch.as_tensor(v)[:, None]
    (g,) = torch.autograd.grad(terms.sum(), m)
    return g


def _tile_parts(g, ts, part):
    """Sum the per-pixel gradients over each (tile, part) group: part(local index)
    gives the group of a pixel inside its tile.  Returns [C, N, groups, 2]."""
    C, N, H, W, _ = g.shape
    th, tw = -(-H // ts), -(-W // ts)
    pad = torch.zeros(C, N, th * ts, tw * ts, 2, dtype=g.dtype)
    pad[:, :, :H, :W] = g
    t = pad.reshape(C, N, th, ts, tw, ts, 2).permute(0, 1, 2, 4, 3, 5, 6)
    t = t.reshape(C, N, th * tw, ts * ts, 2)
    lab = torch.tensor([part(k) for k in range(ts * ts)])
    n_lab = int(lab.max()) + 1
    out = torch.zeros(C, N, th * tw, n_lab, 2, dtype=g.dtype)
    out.index_add_(3, lab, t)
    return out.reshape(C, N, -1, 2)


def _check_absgrad(got_abs, t, v, H, W, ts, mask=None):
    """The oracle's absgrad against sum_p |d(v_p alpha_p)/d mean|
    (RasterizeToPixelsBwd.cu:444-445 per record, :218 in pixel mode), and two
    planted mistakes that this comparison must reject: |.| taken after a lane's
    strided pixel sum (lane l of 32 holds pixels l, l + 32, ...), and after the
    record's whole-tile sum (after the warp sum)."""
    g = _pixel_mean_grads(*t, v, H, W, mask)
    want = g.abs().sum(dim=(2, 3)).numpy()
    assert (want > 1e-6).mean() > 0.5
    np.testing.assert_allclose(got_abs, want, rtol=1e-11, atol=1e-14)
    for part in (lambda k: k % 32, lambda k: 0):
        planted = _tile_parts(g, ts, part).abs().sum(dim=2).numpy()
        assert not np.allclose(planted, want, rtol=1e-6, atol=1e-10)


def test_raster_reference_kat():
    # tests/test_cuda_gaussian_ops.py:244-253 (two Gaussians, one 16x16 tile)
    means = np.array([[[5.2, 6.1], [10.0, 9.3]]])
    conics = np.array([[[0.18, 0.01, 0.15], [0.12, -0.015, 0.2]]])
    opac = np.array([[0.7, 0.4]])
    mus = np.array([[1.2, 0.8]])
    off = np.zeros((1, 1, 1), np.int32)
    fl = np.arange(2, dtype=np.int32)
    img = native.raster_fwd(means, conics, opac, mus, off, fl, 16, 16, 16)
    t = [torch.tensor(a, requires_grad=True) for a in (means, conics, opac, mus)]
    ref = _dense_raster(*t, 16, 16)
    np.testing.assert_allclose(img, ref.detach().numpy(), rtol=1e-13, atol=1e-15)
    w = torch.linspace(0.1, 1.0, 256).reshape(1, 16, 16)
    got = native.raster_bwd(means, conics, opac, mus, off, fl, w.numpy(), 16, 16, 16)
    exp = torch.autograd.grad((ref * w).sum(), t)
    for a, e in zip(got[1:], exp):
        np.testing.assert_allclose(a, e.numpy(), rtol=1e-11, atol=1e-13)
    _check_absgrad(got[0], t, w.numpy(), 16, 16, 16)
    # float32 build of the same case within the parity bar.
    img32 = native.raster_fwd(*(a.astype(np.float32) for a in (means, conics, opac, mus)), off, fl,
                              16, 16, 16)
    np.testing.assert_allclose(img32, img, rtol=1e-5, atol=1e-6)


def _tile_mask(means2d, radii, ts, tw, th, H, W):
    x0, x1, y0, y1, cnt = binning.tile_rects_2d(means2d, radii, ts, tw, th)
    tyx = np.arange(H)[:, None] // ts, np.arange(W)[None, :] // ts
    m = ((tyx[1][None] >= x0[:, None, None]) & (tyx[1][None] < x1[:, None, None])
         & (tyx[0][None] >= y0[:, None, None]) & (tyx[0][None] < y1[:, None, None])
         & (cnt[:, None, None] > 0))
    return torch.tensor(m)[None]


def test_raster_random_scene_matches_masked_dense():
    r = np.random.default_rng(3)
    N, W, H, ts = 150, 40, 37, 16
    tw, th = 3, 3
    means2d = r.uniform(-5, 45, size=(1, N, 2))
    A = r.normal(size=(N, 2, 2)) * 2
    cov = A @ A.transpose(0, 2, 1) + np.eye(2)
    inv = np.linalg.inv(cov)
    conics = np.stack([inv[:, 0, 0], inv[:, 0, 1], inv[:, 1, 1]], -1)[None]
    radii = np.ceil(3 * np.sqrt(np.stack([cov[:, 0, 0], cov[:, 1, 1]], -1))).astype(np.int32)[None]
    opac = r.uniform(0.05, 1, size=(1, N))
    mus = r.uniform(0.5, 2, size=(1, N))
    _, keys, ids = binning.isect_tiles(means2d, radii, ts, tw, th)
    off = binning.isect_offset_encode(keys, 1, tw, th)
    img = native.raster_fwd(means2d, conics, opac, mus, off, ids, W, H, ts)
    mask = _tile_mask(means2d, radii, ts, tw, th, H, W)
    t = [torch.tensor(a, requires_grad=True) for a in (means2d, conics, opac, mus)]
    ref = _dense_raster(*t, H, W, mask)
    np.testing.assert_allclose(img, ref.detach().numpy(), rtol=1e-12, atol=1e-14)
    v = r.normal(size=img.shape)
    got = native.raster_bwd(means2d, conics, opac, mus, off, ids, v, W, H, ts)
    exp = torch.autograd.grad((ref * torch.tensor(v)).sum(), t)
    for a, e in zip(got[1:], exp):
        np.testing.assert_allclose(a, e.numpy(), rtol=1e-9, atol=1e-12)
    # absgrad: every pixel's own mean gradient by autograd, |.| per pixel,
    # summed (RasterizeToPixelsBwd.cu:444-445); never below |gradient|.
    _check_absgrad(got[0], t, v, H, W, ts, mask)
    assert (got[0] >= np.abs(got[1]) - 1e-12).all()
    # Linear in opacity and mu once every alpha clears the cut-off.
    # Doubling opacity doubles every kept alpha; only alphas in [5e-6, 1e-5)
    # newly clear the cut-off, each adding at most 2e-5.
    img2 = native.raster_fwd(means2d, conics, 2 * opac, mus, off, ids, W, H, ts)
    assert (img > 1e-3).sum() > 100
    assert (img2 >= 2 * img - 1e-12).all()
    assert (img2 - 2 * img).max() <= 2e-5 * N


# ---------------------------------------------------------------- voxelizer --

def _dense_voxel(means3d, conics, opac, d0, d1, d2, mask=None):
    # tests/test_cuda_gaussian_ops.py:218-238, optionally masked by brick cover.
    pz, py, px = torch.meshgrid(torch.arange(d0) + 0.5, torch.arange(d1) + 0.5,
                                torch.arange(d2) + 0.5, indexing="ij")
    dx = px[None] - means3d[:, 0, None, None, None]
    dy = py[None] - means3d[:, 1, None, None, None]
    dz = pz[None] - means3d[:, 2, None, None, None]
    c = conics
    sigma = (0.5 * c[:, 0, None, None, None] * dx.square() + c[:, 1, None, None, None] * dx * dy
             + c[:, 2, None, None, None] * dx * dz + 0.5 * c[:, 3, None, None, None] * dy.square()
             + c[:, 4, None, None, None] * dy * dz + 0.5 * c[:, 5, None, None, None] * dz.square())
    alpha = opac[:, None, None, None] * torch.exp(-sigma)
    keep = (sigma >= 0) & (alpha.abs() >= 1e-6)
    if mask is not None:
        keep = keep & mask
    return torch.where(keep, alpha, 0.0).sum(dim=0)


def test_voxel_reference_kat():
    # tests/test_cuda_gaussian_ops.py:315-328 (two Gaussians, one 8^3 brick)
    means = np.array([[2.5, 3.1, 4.0], [5.2, 4.6, 3.3]])
    conics = np.array([[0.3, 0.01, 0.0, 0.25, -0.01, 0.2], [0.22, 0.0, 0.01, 0.28, 0.0, 0.24]])
    opac = np.array([0.8, 0.5])
    off = np.zeros((1, 1, 1), np.int32)
    fl = np.arange(2, dtype=np.int32)
    vol = native.voxel_fwd(means, conics, opac, off, fl, 8, 8, 8, 8)
    t = [torch.tensor(a, requires_grad=True) for a in (means, conics, opac)]
    ref = _dense_voxel(*t, 8, 8, 8)
    np.testing.assert_allclose(vol, ref.detach().numpy(), rtol=1e-13, atol=1e-15)
    w = torch.linspace(0.1, 1.0, 512).reshape(8, 8, 8)
    got = native.voxel_bwd(means, conics, opac, off, fl, w.numpy(), 8, 8, 8, 8)
    exp = torch.autograd.grad((ref * w).sum(), t)
    for a, e in zip(got, exp):
        np.testing.assert_allclose(a, e.numpy(), rtol=1e-11, atol=1e-13)


def test_voxel_random_scene_matches_masked_dense():
    r = np.random.default_rng(4)
    N, dims, ts = 80, (20, 17, 22), 8
    d2, d1, d0 = dims
    n2, n1, n0 = 3, 3, 3
    m3 = r.uniform(-2, 24, size=(N, 3))
    A = r.normal(size=(N, 3, 3)) * 1.2
    cov = A @ A.transpose(0, 2, 1) + 0.8 * np.eye(3)
    P = np.linalg.inv(cov)
    conics = P[:, [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]]
    rad = np.ceil(3 * np.sqrt(np.diagonal(cov, axis1=1, axis2=2))).astype(np.int32)
    opac = r.uniform(0.01, 1, size=N)
    lo, hi, cnt = binning.tile_boxes_3d(m3, rad, ts, n2, n1, n0)
    _, keys, ids = binning.isect_tiles_3d(m3, rad, ts, n2, n1, n0)
    off = binning.isect_offset_encode_3d(keys, n2, n1, n0)
    vol = native.voxel_fwd(m3, conics, opac, off, ids, d2, d1, d0, ts)
    b = [np.arange(d)[None, :] // ts for d in (d0, d1, d2)]
    inz = (b[0] >= lo[2][:, None]) & (b[0] < hi[2][:, None])
    iny = (b[1] >= lo[1][:, None]) & (b[1] < hi[1][:, None])
    inx = (b[2] >= lo[0][:, None]) & (b[2] < hi[0][:, None])
    mask = torch.tensor(inz[:, :, None, None] & iny[:, None, :, None] & inx[:, None, None, :]
                        & (cnt > 0)[:, None, None, None])
    t = [torch.tensor(a, requires_grad=True) for a in (m3, conics, opac)]
    ref = _dense_voxel(*t, d0, d1, d2, mask)
    np.testing.assert_allclose(vol, ref.detach().numpy(), rtol=1e-12, atol=1e-14)
    v = r.normal(size=vol.shape)
    got = native.voxel_bwd(m3, conics, opac, off, ids, v, d2, d1, d0, ts)
    exp = torch.autograd.grad((ref * torch.tensor(v)).sum(), t)
    for a, e in zip(got, exp):
        np.testing.assert_allclose(a, e.numpy(), rtol=1e-9, atol=1e-12)


# --------------------------------------------------------------- compaction --

def test_where_split_matches_torch():
    r = np.random.default_rng(5)
    for n in (0, 1, 7, 1000, 100_003):
        m = r.random(n) < 0.37
        sel, rest = binning.where_split(m)
        np.testing.assert_array_equal(sel, torch.where(torch.tensor(m))[0].numpy())
        np.testing.assert_array_equal(rest, torch.where(~torch.tensor(m))[0].numpy())
        assert sel.size + rest.size == n
