"""The reference's dense PyTorch formulation of the r2splat path -- TEST AND
BASELINE INFRASTRUCTURE ONLY (imported by ``tests/`` and ``bench.py``'s CPU
baseline leg, never by the ``r2splat`` package).

Every Gaussian is evaluated at every pixel (voxel) of the detector (grid) as
one broadcast torch expression, and torch autograd supplies the backward --
the formulation of the reference's own dense checks
(tests/test_cuda_gaussian_ops.py:200-238), extended with the element-wise
preprocessing so that a call runs from the raw parameters:

* ``activate``        ParameterTransformFwd.cu:53-129 and direct.py:91
                      (sigmoid-bounded scales, quaternion rotation, packed
                      covariance, softplus opacity);
* ``project``         WorldToImageProjectionFwd.cu:74-283 (cone-beam
                      perspective, the field-of-view clamp, radii);
* ``conics_mu``       ConicsMuFwd.cu:36-100;
* ``volume_mapping``  WorldToVolumeMappingFwd.cu:90-189;
* ``raster`` / ``voxel``  the alpha sums, masked by the tiles (bricks) that
                      the binning lists for each Gaussian
                      (IsectTilesKernel.cu:57-113, IsectTiles3DKernel.cu:49-104),
                      so that they equal the tiled kernels' sums.

``config1_call`` is one forward + backward of BASELINE config 1 (one view
rasterized and a volume voxelized from the same Gaussians, upstream
gradients given), the voxel sums chunked over Gaussians to bound memory.
How the formulation is pinned: tests/test_oracle_dense.py compares it with
the numpy / C oracle (values and the composed parameter gradients).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

Tensor = torch.Tensor


def activate(quats: Tensor, raw_scales: Tensor, raw_opacities: Tensor, scale_min: float,
             scale_max: float):
    """-> (covars [N,6] packed 00,01,02,11,12,22, max_scales [N], opacities [N])."""
    q = quats / torch.clamp(quats.norm(dim=-1, keepdim=True), min=1e-12)
    w, x, y, z = q.unbind(-1)
    R = torch.stack([
        torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)], -1),
        torch.stack([2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)], -1),
        torch.stack([2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)], -1),
    ], -2)
    s = torch.sigmoid(raw_scales) * (scale_max - scale_min) + scale_min
    cov = (R * (s * s)[:, None, :]) @ R.transpose(1, 2)
    iu = ([0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2])
    return cov[:, iu[0], iu[1]], s.max(dim=-1).values, F.softplus(raw_opacities)


def _sym(packed: Tensor) -> Tensor:
    a, b, c, d, e, f = packed.unbind(-1)
    return torch.stack([torch.stack([a, b, c], -1), torch.stack([b, d, e], -1),
                        torch.stack([c, e, f], -1)], -2)


def project(means: Tensor, covars: Tensor, viewmat: Tensor, K: Tensor, width: int, height: int,
            eps2d: float, radius_clip: float):
    """One view -> (means2d [N,2], cov2d [N,6], radii [N,2] int32, no gradient)."""
    R, t = viewmat[:3, :3], viewmat[:3, 3]
    fx, fy, cx, cy = K[0, 0], K[1, 1], K[0, 2], K[1, 2]
    pc = means @ R.T + t
    x, y, z = pc.unbind(-1)
    keep = z > 0.01
    rz = 1.0 / z
    mx, my = fx * x * rz + cx, fy * y * rz + cy
    tan_x, tan_y = 0.5 * width / fx, 0.5 * height / fy
    lxp, lxn = (width - cx) / fx + 0.3 * tan_x, cx / fx + 0.3 * tan_x
    lyp, lyn = (height - cy) / fy + 0.3 * tan_y, cy / fy + 0.3 * tan_y
    tx = z * torch.minimum(torch.maximum(x * rz, -lxn), lxp)
    ty = z * torch.minimum(torch.maximum(y * rz, -lyn), lyp)
    rl = 1.0 / torch.sqrt(tx * tx + ty * ty + z * z)
    zero = torch.zeros_like(z)
    J = torch.stack([torch.stack([fx * rz, zero, -fx * tx * rz * rz], -1),
                     torch.stack([zero, fy * rz, -fy * ty * rz * rz], -1),
                     torch.stack([tx * rl, ty * rl, z * rl], -1)], -2)
    M = J @ R
    C = M @ _sym(covars) @ M.transpose(1, 2)
    iu = ([0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2])
    cov2d = C[:, iu[0], iu[1]]
    with torch.no_grad():
        a, d, b = cov2d[:, 0] + eps2d, cov2d[:, 3] + eps2d, cov2d[:, 1]
        rx = torch.ceil(radius_clip * torch.sqrt(torch.clamp(a, min=0)))
        ry = torch.ceil(radius_clip * torch.sqrt(torch.clamp(d, min=0)))
        ok = keep & (a * d - b * b > 0) & torch.isfinite(rx) & torch.isfinite(ry)
        ok &= (rx > 0) & (ry > 0)
        ok &= ~((mx + rx <= 0) | (mx - rx >= width) | (my + ry <= 0) | (my - ry >= height))
        radii = torch.stack([torch.where(ok, rx, 0), torch.where(ok, ry, 0)], -1).to(torch.int32)
    means2d = torch.where(keep[:, None], torch.stack([mx, my], -1), 0.0)
    return means2d, torch.where(keep[:, None], cov2d, 0.0), radii


def conics_mu(cov2d: Tensor, eps: float):
    """-> (conics [N,3] of the blurred 2x2 block, mus [N] = sqrt(2 pi det3 / det2))."""
    a, b, c, d, e, f = cov2d.unbind(-1)
    ab, db, fb = a + eps, d + eps, f + eps
    d2 = ab * db - b * b
    d3 = ab * db * fb - ab * e * e - b * b * fb + 2 * b * c * e - c * c * db
    valid = d2 > 1e-9
    safe = torch.where(valid, d2, torch.ones_like(d2))
    conics = torch.stack([db / safe, -b / safe, ab / safe], -1)
    ratio = d3 / safe
    pos = valid & (ratio > 0)
    mus = torch.sqrt(2.0 * math.pi * torch.where(pos, ratio, torch.ones_like(ratio)))
    return (torch.where(valid[:, None], conics, 0.0), torch.where(pos, mus, 0.0))


def volume_mapping(means: Tensor, covars: Tensor, ranges: Tensor, centers: Tensor, dim2: int,
                   dim1: int, dim0: int, eps3d: float, radius_clip: float):
    """-> (means3d [N,3] in voxel units, conics [N,6] of the inverse, radii [N,3])."""
    r = torch.stack([dim2 / ranges[0], dim1 / ranges[1], dim0 / ranges[2]])
    half = torch.tensor([dim2, dim1, dim0], dtype=means.dtype) * 0.5
    m3 = (means - centers) * r + half
    Sv = _sym(covars) * (r[:, None] * r[None, :]) + eps3d * torch.eye(3, dtype=means.dtype)
    det = torch.linalg.det(Sv)
    ok = det.abs() >= 1e-12
    inv = torch.linalg.inv(torch.where(ok[:, None, None], Sv,
                                       torch.eye(3, dtype=means.dtype).expand_as(Sv)))
    iu = ([0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2])
    conics = torch.where(ok[:, None], inv[:, iu[0], iu[1]], 0.0)
    with torch.no_grad():
        diag = torch.diagonal(Sv, dim1=1, dim2=2)
        rad = torch.ceil(radius_clip * torch.sqrt(torch.clamp(diag, min=0)))
        good = ok & torch.isfinite(rad).all(-1) & (rad > 0).all(-1)
        radii = torch.where(good[:, None], rad, 0).to(torch.int32)
    return m3, conics, radii


def _tile_bound(v: Tensor, upper: int) -> Tensor:
    # IsectTilesKernel.cu:30-40: non-finite or <= 0 -> 0, >= upper -> upper, else truncate.
    v = torch.where(torch.isfinite(v) & (v > 0), v, torch.zeros_like(v))
    return torch.clamp(v, max=float(upper)).floor()


def cover_2d(means2d: Tensor, radii: Tensor, ts: int, h: int, w: int) -> Tensor:
    """[N, H, W] mask of the pixels in the tiles listed for each Gaussian."""
    tw, th = -(-w // ts), -(-h // ts)
    rx, ry = radii[:, 0].to(means2d.dtype), radii[:, 1].to(means2d.dtype)
    mx, my = means2d[:, 0], means2d[:, 1]
    ok = (rx > 0) & (ry > 0) & torch.isfinite(mx) & torch.isfinite(my)
    x0 = _tile_bound(torch.floor(mx / ts - rx / ts), tw)
    x1 = _tile_bound(torch.ceil(mx / ts + rx / ts), tw)
    y0 = _tile_bound(torch.floor(my / ts - ry / ts), th)
    y1 = _tile_bound(torch.ceil(my / ts + ry / ts), th)
    tj = (torch.arange(w) // ts).to(means2d.dtype)
    ti = (torch.arange(h) // ts).to(means2d.dtype)
    cx = (tj[None] >= x0[:, None]) & (tj[None] < x1[:, None])
    cy = (ti[None] >= y0[:, None]) & (ti[None] < y1[:, None])
    return ok[:, None, None] & cy[:, :, None] & cx[:, None, :]


def cover_3d(means3d: Tensor, radii: Tensor, ts: int, d2: int, d1: int, d0: int) -> Tensor:
    """[N, d0, d1, d2] mask of the voxels in the bricks listed for each Gaussian."""
    ok = (radii > 0).all(-1)
    lo, hi = [], []
    for a, d in enumerate((d2, d1, d0)):
        n = -(-d // ts)
        c, r = means3d[:, a] / ts, radii[:, a].to(means3d.dtype) / ts
        lo.append(_tile_bound(torch.floor(c - r), n))
        hi.append(_tile_bound(torch.ceil(c + r), n))
    axes = [(torch.arange(d) // ts).to(means3d.dtype) for d in (d2, d1, d0)]
    cx, cy, cz = ((t[None] >= lo[a][:, None]) & (t[None] < hi[a][:, None])
                  for a, t in enumerate(axes))
    return (ok[:, None, None, None] & cz[:, :, None, None] & cy[:, None, :, None]
            & cx[:, None, None, :])


def raster(means2d: Tensor, conics: Tensor, om: Tensor, cover: Tensor) -> Tensor:
    """[N] Gaussians -> [H, W]: sum of om exp(-sigma) over the cover, skipping
    sigma < 0 and |alpha| < 1e-5 (RasterizeToPixelsFwd.cu:150-170).  The
    offsets broadcast per axis (dx [N,1,W], dy [N,H,1])."""
    h, w = cover.shape[1:]
    dx = (torch.arange(w, dtype=means2d.dtype) + 0.5)[None, None, :] - means2d[:, 0, None, None]
    dy = (torch.arange(h, dtype=means2d.dtype) + 0.5)[None, :, None] - means2d[:, 1, None, None]
    a, b, c = (conics[:, i, None, None] for i in range(3))
    sigma = (0.5 * a * dx.square() + b * dx * dy) + 0.5 * c * dy.square()
    alpha = om[:, None, None] * torch.exp(-sigma)
    keep = cover & (sigma >= 0) & (alpha.abs() >= 1e-5)
    return torch.where(keep, alpha, torch.zeros_like(alpha)).sum(0)


def voxel(means3d: Tensor, conics: Tensor, opac: Tensor, cover: Tensor) -> Tensor:
    """[N] Gaussians -> [d0, d1, d2]: sum of opac exp(-sigma) over the cover,
    skipping sigma < 0 and |alpha| < 1e-6 (VoxelizeToVoxelsFwd.cu).  The
    offsets broadcast per axis (dx [N,1,1,d2], dy [N,1,d1,1], dz [N,d0,1,1]),
    so only the pair terms and the sums are full [N,d0,d1,d2] tensors."""
    d0, d1, d2 = cover.shape[1:]
    t = means3d.dtype
    dx = (torch.arange(d2, dtype=t) + 0.5)[None, None, None, :] - means3d[:, 0, None, None, None]
    dy = (torch.arange(d1, dtype=t) + 0.5)[None, None, :, None] - means3d[:, 1, None, None, None]
    dz = (torch.arange(d0, dtype=t) + 0.5)[None, :, None, None] - means3d[:, 2, None, None, None]
    q = [conics[:, i, None, None, None] for i in range(6)]
    # The 2D part (x, y) is [N,1,d1,d2]; z enters through the [N,d0,1,*] terms.
    sxy = (0.5 * q[0] * dx.square() + q[1] * dx * dy) + 0.5 * q[3] * dy.square()
    sigma = sxy + dz * (q[2] * dx + q[4] * dy + 0.5 * q[5] * dz)
    alpha = opac[:, None, None, None] * torch.exp(-sigma)
    keep = cover & (sigma >= 0) & (alpha.abs() >= 1e-6)
    return torch.where(keep, alpha, torch.zeros_like(alpha)).sum(0)


def config1_call(params, viewmat: Tensor, K: Tensor, width: int, height: int, v_image: Tensor,
                 dims, v_volume: Tensor, *, scale_min=5e-4, scale_max=1.0, eps=1e-8,
                 radius_clip=3.0, tile_2d=16, tile_3d=8, chunk=256):
    """One forward + backward from the raw parameters (means, quats,
    raw_scales, raw_opacities; leaf tensors with requires_grad): one view
    rasterized against ``v_image`` [H,W] and, when ``dims`` = (d2, d1, d0),
    a volume over [-1,1]^3 voxelized against ``v_volume`` [d0,d1,d2].
    Leaves .grad on the parameters; returns (image, volume).  The voxel sums
    run ``chunk`` Gaussians at a time: each chunk's VJP is taken at detached
    copies of its mapped attributes, and the collected gradients go through
    the mapping and the parameter transform in one final backward."""
    means, quats, scales, opac = params
    covars, _, op = activate(quats, scales, opac, scale_min, scale_max)
    m2, cov2d, r2 = project(means, covars, viewmat, K, width, height, eps, radius_clip)
    con, mu = conics_mu(cov2d, eps)
    image = raster(m2, con, op * mu, cover_2d(m2.detach(), r2, tile_2d, height, width))
    outs, grads = [(image * v_image).sum()], [None]
    volume = None
    if dims is not None:
        d2, d1, d0 = dims
        rng = torch.full((3,), 2.0, dtype=means.dtype)
        ctr = torch.zeros(3, dtype=means.dtype)
        m3, con3, r3 = volume_mapping(means, covars, rng, ctr, d2, d1, d0, eps, radius_clip)
        g3 = [torch.zeros_like(m3), torch.zeros_like(con3), torch.zeros_like(op)]
        volume = torch.zeros((d0, d1, d2), dtype=means.dtype)
        for s in range(0, m3.shape[0], chunk):
            x, c, o = (t[s:s + chunk].detach().requires_grad_(True) for t in (m3, con3, op))
            part = voxel(x, c, o, cover_3d(x.detach(), r3[s:s + chunk], tile_3d, d2, d1, d0))
            (part * v_volume).sum().backward()
            volume += part.detach()
            for acc, leaf in zip(g3, (x, c, o)):
                acc[s:s + chunk] = leaf.grad
        outs += [m3, con3, op]
        grads += g3
    torch.autograd.backward(outs, grads)
    return image.detach(), volume
