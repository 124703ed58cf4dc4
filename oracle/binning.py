"""Tile binning and index compaction restated in numpy (test infrastructure only).

The reference emits intersection records per Gaussian in index order, tiles
row-major (2D) or z->y->x (3D), then stable-radix-sorts them by key
(IsectTilesKernel.cu:138-217, 398-445; IsectTiles3DKernel.cu:125-200,
364-409).  Because emission is in ascending record id and the sort is stable,
the result is the lexicographic (key, id) order; numpy's stable argsort of the
emitted keys reproduces it exactly.
"""

from __future__ import annotations

import math

import numpy as np

__all__ = [
    "tile_rects_2d",
    "isect_tiles",
    "isect_offset_encode",
    "tile_boxes_3d",
    "isect_tiles_3d",
    "isect_offset_encode_3d",
    "end_bit",
    "where_split",
]


def end_bit(n_keys: int) -> int:
    """IsectTiles.cpp:146-147 / IsectTiles3D.cpp:140: ceil(log2(n_keys + 1))."""
    return int(math.ceil(math.log2(float(n_keys + 1))))


def _clamp_tile_bound(value, upper):
    # IsectTilesKernel.cu:30-40: non-finite or <= 0 -> 0; >= upper -> upper
    out = np.zeros(value.shape, np.int64)
    with np.errstate(invalid="ignore"):
        pos = np.isfinite(value) & (value > 0)
        big = pos & (value >= value.dtype.type(upper))
        mid = pos & ~big
    out[big] = upper
    out[mid] = value[mid].astype(np.int64)
    return out


def tile_rects_2d(means2d, radii, tile_size, n_tiles_w, n_tiles_h):
    """IsectTilesKernel.cu:57-113: per (camera, Gaussian) tile rectangle and count.

    Returns (x0, x1, y0, y1, count) as int64 arrays of shape [C*N]; the
    rectangle is [x0, x1) x [y0, y1) and count is 0 where the reference emits
    nothing.
    """
    m = means2d.reshape(-1, 2)
    dt = m.dtype.type
    if radii.ndim == 3:
        r = radii.reshape(-1, 2)
        rx, ry = r[:, 0], r[:, 1]
    else:
        rx = ry = radii.reshape(-1)
    rxf, ryf = rx.astype(m.dtype), ry.astype(m.dtype)
    mx, my = m[:, 0], m[:, 1]
    ts = dt(tile_size)
    with np.errstate(all="ignore"):
        valid = (rxf > 0) & (ryf > 0) & np.isfinite(mx) & np.isfinite(my)
        trx, tyr = rxf / ts, ryf / ts
        tx, ty = mx / ts, my / ts
        x0 = _clamp_tile_bound(np.floor(tx - trx), n_tiles_w)
        y0 = _clamp_tile_bound(np.floor(ty - tyr), n_tiles_h)
        x1 = _clamp_tile_bound(np.ceil(tx + trx), n_tiles_w)
        y1 = _clamp_tile_bound(np.ceil(ty + tyr), n_tiles_h)
    valid &= (x1 > x0) & (y1 > y0)
    count = np.where(valid, (y1 - y0) * (x1 - x0), 0)
    return x0, x1, y0, y1, count


def isect_tiles(means2d, radii, tile_size, n_tiles_w, n_tiles_h):
    """IsectTiles.cpp:31-170 -> (tiles_per_gauss [C,N] i32, isect_ids i64, flatten_ids i32)."""
    C, N = means2d.shape[0], means2d.shape[1]
    n_tiles = n_tiles_w * n_tiles_h
    x0, x1, y0, y1, count = tile_rects_2d(means2d, radii, tile_size, n_tiles_w, n_tiles_h)
    tiles_per_gauss = count.astype(np.int32).reshape(C, N)
    total = int(count.sum())
    if total == 0:
        return tiles_per_gauss, np.zeros(0, np.int64), np.zeros(0, np.int32)
    # Emission in record order, rows then columns (IsectTilesKernel.cu:193-216).
    idx = np.repeat(np.arange(C * N, dtype=np.int64), count)
    starts = np.cumsum(count) - count
    local = np.arange(total, dtype=np.int64) - np.repeat(starts, count)
    width = np.repeat(x1 - x0, count)
    ty = np.repeat(y0, count) + local // width
    tx = np.repeat(x0, count) + local % width
    cid = idx // N
    keys = cid * n_tiles + ty * n_tiles_w + tx
    order = np.argsort(keys, kind="stable")
    return tiles_per_gauss, keys[order], idx[order].astype(np.int32)


def isect_offset_encode(isect_ids, n_cameras, n_tiles_w, n_tiles_h):
    """IsectTilesKernel.cu:234-273 -> tile_offsets [C, th, tw] (lower_bound of each key)."""
    n_keys = n_cameras * n_tiles_w * n_tiles_h
    if isect_ids.size == 0:
        off = np.zeros(n_keys, np.int32)
    else:
        off = np.searchsorted(isect_ids, np.arange(n_keys, dtype=np.int64), "left")
    return off.astype(np.int32).reshape(n_cameras, n_tiles_h, n_tiles_w)


def _sat_u32(value):
    # CUDA float->uint32 conversion saturates: NaN and negatives -> 0.
    out = np.zeros(value.shape, np.int64)
    with np.errstate(invalid="ignore"):
        pos = np.isfinite(value) & (value > 0)
        big = (value >= 4294967295.0) & ~np.isnan(value)
    out[pos & ~big] = value[pos & ~big].astype(np.int64)
    out[big] = 4294967295
    return out


def tile_boxes_3d(means3d, radii, tile_size, n2, n1, n0):
    """IsectTiles3DKernel.cu:49-104: per Gaussian brick box and count.

    Bounds are min(max(0, u32(floor/ceil(.))), n) with the saturating cast;
    there is no finite-mean test (a non-finite mean collapses the box).
    """
    m = means3d.reshape(-1, 3)
    r = radii.reshape(-1, 3)
    dt = m.dtype.type
    ts = dt(tile_size)
    rf = r.astype(m.dtype)
    with np.errstate(all="ignore"):
        valid = (rf[:, 0] > 0) & (rf[:, 1] > 0) & (rf[:, 2] > 0)
        lo, hi = [], []
        for axis, n in ((0, n2), (1, n1), (2, n0)):
            c = m[:, axis] / ts
            rr = rf[:, axis] / ts
            lo.append(np.minimum(_sat_u32(np.floor(c - rr)), n))
            hi.append(np.minimum(_sat_u32(np.ceil(c + rr)), n))
    ext = [np.maximum(h - l, 0) for l, h in zip(lo, hi)]
    count = np.where(valid, ext[0] * ext[1] * ext[2], 0)
    return lo, hi, count


def isect_tiles_3d(means3d, radii, tile_size, n2, n1, n0):
    """IsectTiles3D.cpp:31-162 -> (tiles_per_gauss [N] i32, isect_ids i64, flatten_ids i32)."""
    N = means3d.shape[0]
    lo, hi, count = tile_boxes_3d(means3d, radii, tile_size, n2, n1, n0)
    tiles_per_gauss = count.astype(np.int32)
    total = int(count.sum())
    if total == 0:
        return tiles_per_gauss, np.zeros(0, np.int64), np.zeros(0, np.int32)
    # Emission z (dim0) -> y (dim1) -> x (dim2), IsectTiles3DKernel.cu:182-199.
    idx = np.repeat(np.arange(N, dtype=np.int64), count)
    starts = np.cumsum(count) - count
    local = np.arange(total, dtype=np.int64) - np.repeat(starts, count)
    e2 = np.repeat(hi[0] - lo[0], count)
    e1 = np.repeat(hi[1] - lo[1], count)
    t2 = np.repeat(lo[0], count) + local % e2
    t1 = np.repeat(lo[1], count) + (local // e2) % e1
    t0 = np.repeat(lo[2], count) + local // (e2 * e1)
    keys = t0 * (n1 * n2) + t1 * n2 + t2
    order = np.argsort(keys, kind="stable")
    return tiles_per_gauss, keys[order], idx[order].astype(np.int32)


def isect_offset_encode_3d(isect_ids, n2, n1, n0):
    """IsectTiles3DKernel.cu:212-249 -> tile_offsets [n0, n1, n2]."""
    n_keys = n0 * n1 * n2
    if isect_ids.size == 0:
        off = np.zeros(n_keys, np.int32)
    else:
        off = np.searchsorted(isect_ids, np.arange(n_keys, dtype=np.int64), "left")
    return off.astype(np.int32).reshape(n0, n1, n2)


def where_split(mask):
    """src/strategies/binary_tree.py:68,101-102,158: (torch.where(mask)[0], torch.where(~mask)[0])."""
    mask = np.asarray(mask).astype(bool).reshape(-1)
    return np.flatnonzero(mask).astype(np.int64), np.flatnonzero(~mask).astype(np.int64)
