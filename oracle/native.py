"""ctypes bindings of the sequential C oracle (test infrastructure only).

``oracle/c/r2s_oracle.c`` restates the rasterizer and voxelizer loops of the
reference (RasterizeToPixelsFwd.cu, RasterizeToPixelsBwd.cu,
VoxelizeToVoxelsFwd.cu, VoxelizeToVoxelsBwd.cu); it is built by
``oracle/Makefile`` into ``oracle/_build/libr2s_oracle.so``.  Tiles are shared
out over OpenMP threads (OMP_NUM_THREADS) with results bit-identical to the
sequential loops.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libr2s_oracle.so")
SRC = os.path.join(HERE, "c", "r2s_oracle.c")

_lib = None


def build(force: bool = False) -> str:
    if force or not os.path.exists(LIB) or os.path.getmtime(LIB) < os.path.getmtime(SRC):
        subprocess.run(["make", "-s", "-C", HERE] + (["-B"] if force else [])
                       + ["_build/libr2s_oracle.so"], check=True)
    return LIB


def _load():
    global _lib
    if _lib is None:
        build()
        _lib = ctypes.CDLL(LIB)
    return _lib


THR_2D = 1e-5  # RasterizeToPixelsFwd.cu / Bwd.cu alpha cut-off
THR_3D = 1e-6  # VoxelizeToVoxelsFwd.cu / Bwd.cu alpha cut-off

_SUFFIX = {np.dtype(np.float32): "f32", np.dtype(np.float64): "f64",
           np.dtype(np.longdouble): "f80"}
_CTYPE = {"f32": ctypes.c_float, "f64": ctypes.c_double, "f80": ctypes.c_longdouble}


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _sfx(dt):
    return _SUFFIX[np.dtype(dt)]


def _c(a, dt=None):
    return np.ascontiguousarray(a if dt is None else a.astype(dt, copy=False))


def _ok(rc):
    if rc != 0:
        raise MemoryError("oracle: no memory for the per-record partials")


def _scalars(dt, thr, eta):
    k = _CTYPE[_sfx(dt)]
    return k(thr), k(eta)


def _extras(out, bnd, mg, band, mag):
    if mag:
        return out, bnd, mg
    return (out, bnd) if band else out


def _keys(keys):
    if keys is None:
        return None, 0
    k = np.ascontiguousarray(np.asarray(keys, np.int64))
    return k, k.size


def raster_fwd(means2d, conics, opac, mus, tile_offsets, flatten_ids, width, height, tile_size,
               thr=THR_2D, eta=0.0, band=False, mag=False, keys=None):
    """RasterizeToPixelsFwd.cu:57-186 -> image [C, H, W] in means2d's dtype
    (float32, float64 or longdouble).  band=True adds the flip band [C, H, W]
    of every pixel for bracket eta, mag=True the sum of |terms| per pixel
    (see r2s_oracle.c): (image, band) or (image, band or None, mag).  With
    ``keys`` only those tiles' pixels are computed (the rest stay zero)."""
    dt = means2d.dtype
    C = means2d.shape[0]
    th, tw = tile_offsets.shape[1], tile_offsets.shape[2]
    out = np.zeros((C, height, width), dt)
    bnd = np.zeros((C, height, width), dt) if band else None
    mg = np.zeros((C, height, width), dt) if mag else None
    kk, n_sel = _keys(keys)
    if flatten_ids.size and means2d.shape[1]:
        args = [_c(means2d), _c(conics, dt), _c(opac, dt), _c(mus, dt),
                _c(tile_offsets, np.int32), _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_raster_fwd_{_sfx(dt)}")
        fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), ctypes.c_int64(C),
           ctypes.c_uint32(width), ctypes.c_uint32(height), ctypes.c_uint32(tile_size),
           ctypes.c_uint32(tw), ctypes.c_uint32(th), _p(kk), ctypes.c_int64(n_sel),
           *_scalars(dt, thr, eta), _p(out), _p(bnd), _p(mg))
    return _extras(out, bnd, mg, band, mag)


def raster_bwd(means2d, conics, opac, mus, tile_offsets, flatten_ids, v_image, width, height,
               tile_size, absgrad=True, thr=THR_2D, eta=0.0, band=False, mag=False):
    """RasterizeToPixelsBwd.cu:350-480 -> (v_abs|None, v_means2d, v_conics, v_opac, v_mus);
    band=True adds a second tuple of the same shapes with each output's flip
    band, mag=True a third (band tuple None unless band) with each output's
    sum of |terms|."""
    dt = means2d.dtype
    C = means2d.shape[0]
    th, tw = tile_offsets.shape[1], tile_offsets.shape[2]
    v_xy = np.zeros_like(means2d)
    v_abs = np.zeros_like(means2d)
    v_con = np.zeros(conics.shape, dt)
    v_o = np.zeros(opac.shape, dt)
    v_mu = np.zeros(mus.shape, dt)
    bnd = np.zeros(means2d.shape[:2] + (9,), dt) if band else None
    mg = np.zeros(means2d.shape[:2] + (9,), dt) if mag else None
    if flatten_ids.size:
        args = [_c(means2d), _c(conics, dt), _c(opac, dt), _c(mus, dt),
                _c(tile_offsets, np.int32), _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_raster_bwd_{_sfx(dt)}")
        _ok(fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), _p(_c(v_image, dt)),
           ctypes.c_int64(C), ctypes.c_uint32(width), ctypes.c_uint32(height),
           ctypes.c_uint32(tile_size), ctypes.c_uint32(tw), ctypes.c_uint32(th),
           *_scalars(dt, thr, eta), _p(v_abs), _p(v_xy), _p(v_con), _p(v_o), _p(v_mu), _p(bnd),
           _p(mg)))
    grads = ((v_abs if absgrad else None), v_xy, v_con, v_o, v_mu)

    def split(a):
        if a is None:
            return None
        return ((a[..., 0:2] if absgrad else None), a[..., 2:4], a[..., 4:7], a[..., 7],
                a[..., 8])

    if mag:
        return grads, split(bnd), split(mg)
    return (grads, split(bnd)) if band else grads


def voxel_fwd(means3d, conics, opac, tile_offsets, flatten_ids, dim2, dim1, dim0, tile_size,
              thr=THR_3D, eta=0.0, band=False, mag=False, keys=None, key_offset=0):
    """VoxelizeToVoxelsFwd.cu:69-221 -> volume [dim0, dim1, dim2]; band / mag
    / keys as in raster_fwd.  ``key_offset``: the lists (tile_offsets [n0,
    n1, n2]) are those of the brick layers from key_offset / (n1 n2) on of
    the whole volume's grid (one z-slab's lists)."""
    dt = means3d.dtype
    n0, n1, n2 = tile_offsets.shape
    out = np.zeros((dim0, dim1, dim2), dt)
    bnd = np.zeros((dim0, dim1, dim2), dt) if band else None
    mg = np.zeros((dim0, dim1, dim2), dt) if mag else None
    kk, n_sel = _keys(keys)
    if flatten_ids.size and means3d.shape[0]:
        args = [_c(means3d), _c(conics, dt), _c(opac, dt), _c(tile_offsets, np.int32),
                _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_voxel_fwd_{_sfx(dt)}")
        fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), ctypes.c_uint32(dim2),
           ctypes.c_uint32(dim1), ctypes.c_uint32(dim0), ctypes.c_uint32(tile_size),
           ctypes.c_uint32(n2), ctypes.c_uint32(n1), ctypes.c_uint32(n0),
           ctypes.c_int64(key_offset), _p(kk), ctypes.c_int64(n_sel), *_scalars(dt, thr, eta),
           _p(out), _p(bnd), _p(mg))
    return _extras(out, bnd, mg, band, mag)


def voxel_bwd(means3d, conics, opac, tile_offsets, flatten_ids, v_volume, dim2, dim1, dim0,
              tile_size, thr=THR_3D, eta=0.0, band=False, mag=False):
    """VoxelizeToVoxelsBwd.cu:322-441 -> (v_means3d, v_conics, v_opac); band /
    mag add tuples of the same shapes as in raster_bwd."""
    dt = means3d.dtype
    n0, n1, n2 = tile_offsets.shape
    v_m = np.zeros(means3d.shape, dt)
    v_c = np.zeros(conics.shape, dt)
    v_o = np.zeros(opac.shape, dt)
    bnd = np.zeros((means3d.shape[0], 10), dt) if band else None
    mg = np.zeros((means3d.shape[0], 10), dt) if mag else None
    if flatten_ids.size:
        args = [_c(means3d), _c(conics, dt), _c(opac, dt), _c(tile_offsets, np.int32),
                _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_voxel_bwd_{_sfx(dt)}")
        _ok(fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), _p(_c(v_volume, dt)),
           ctypes.c_uint32(dim2), ctypes.c_uint32(dim1), ctypes.c_uint32(dim0),
           ctypes.c_uint32(tile_size), ctypes.c_uint32(n2), ctypes.c_uint32(n1),
           ctypes.c_uint32(n0), *_scalars(dt, thr, eta), _p(v_m), _p(v_c), _p(v_o), _p(bnd),
           _p(mg)))
    grads = (v_m, v_c, v_o)

    def split(a):
        return None if a is None else (a[:, 0:3], a[:, 3:9], a[:, 9])

    if mag:
        return grads, split(bnd), split(mg)
    return (grads, split(bnd)) if band else grads


def _selected(tile_offsets, n_isects, keys):
    """(keys, first row of each key's records in the output, records' list
    positions) for the listed keys."""
    off = np.asarray(tile_offsets).reshape(-1).astype(np.int64)
    k = np.ascontiguousarray(np.asarray(keys, np.int64))
    start = off[k]
    end = np.where(k == off.size - 1, n_isects, off[np.minimum(k + 1, off.size - 1)])
    cnt = end - start
    first = np.ascontiguousarray(np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.int64))
    rec = (np.concatenate([np.arange(a, b) for a, b in zip(start, end)]) if k.size
           else np.zeros(0, np.int64))
    return k, first, rec.astype(np.int64)


def raster_records(means2d, conics, opac, mus, tile_offsets, flatten_ids, v_image, width,
                   height, tile_size, keys, thr=THR_2D, eta=0.0):
    """Per-record partials of the listed tiles' records (RasterizeToPixelsBwd.cu
    :412-452): (positions r in the sorted list, values [n, 9] in the order
    v_xy_abs x, y, v_xy x, y, v_conic 0..2, v_opacity, v_mu, their flip bands
    [n, 9] for bracket eta, their sums of |terms| [n, 9])."""
    dt = means2d.dtype
    C = means2d.shape[0]
    th, tw = tile_offsets.shape[1], tile_offsets.shape[2]
    k, first, rec = _selected(tile_offsets, flatten_ids.size, keys)
    part = np.zeros((rec.size, 27), dt)
    if rec.size:
        args = [_c(means2d), _c(conics, dt), _c(opac, dt), _c(mus, dt),
                _c(tile_offsets, np.int32), _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_raster_records_{_sfx(dt)}")
        _ok(fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), _p(_c(v_image, dt)),
               ctypes.c_int64(C), ctypes.c_uint32(width), ctypes.c_uint32(height),
               ctypes.c_uint32(tile_size), ctypes.c_uint32(tw), ctypes.c_uint32(th), _p(k),
               ctypes.c_int64(k.size), _p(first), *_scalars(dt, thr, eta), _p(part)))
    return rec, part[:, 0:9], part[:, 9:18], part[:, 18:27]


def voxel_records(means3d, conics, opac, tile_offsets, flatten_ids, v_volume, dim2, dim1, dim0,
                  tile_size, keys, thr=THR_3D, eta=0.0, key_offset=0):
    """Per-record partials of the listed bricks' records (VoxelizeToVoxelsBwd.cu
    :382-422): (positions, values [n, 10] in the order v_means 0..2,
    v_conics 0..5, v_opacity, bands [n, 10], sums of |terms| [n, 10])."""
    dt = means3d.dtype
    n0, n1, n2 = tile_offsets.shape
    k, first, rec = _selected(tile_offsets, flatten_ids.size, keys)
    part = np.zeros((rec.size, 30), dt)
    if rec.size:
        args = [_c(means3d), _c(conics, dt), _c(opac, dt), _c(tile_offsets, np.int32),
                _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_voxel_records_{_sfx(dt)}")
        _ok(fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), _p(_c(v_volume, dt)),
               ctypes.c_uint32(dim2), ctypes.c_uint32(dim1), ctypes.c_uint32(dim0),
               ctypes.c_uint32(tile_size), ctypes.c_uint32(n2), ctypes.c_uint32(n1),
               ctypes.c_uint32(n0), ctypes.c_int64(key_offset), _p(k), ctypes.c_int64(k.size),
               _p(first), *_scalars(dt, thr, eta), _p(part)))
    return rec, part[:, 0:10], part[:, 10:20], part[:, 20:30]
