"""ctypes bindings of the sequential C oracle (test infrastructure only).

``oracle/c/r2s_oracle.c`` restates the rasterizer and voxelizer loops of the
reference (RasterizeToPixelsFwd.cu, RasterizeToPixelsBwd.cu,
VoxelizeToVoxelsFwd.cu, VoxelizeToVoxelsBwd.cu); it is built by
``oracle/Makefile`` into ``oracle/_build/libr2s_oracle.so``.
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


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def _sfx(dt):
    return "f32" if np.dtype(dt) == np.float32 else "f64"


def _c(a, dt=None):
    return np.ascontiguousarray(a if dt is None else a.astype(dt, copy=False))


def raster_fwd(means2d, conics, opac, mus, tile_offsets, flatten_ids, width, height, tile_size):
    """RasterizeToPixelsFwd.cu:57-186 -> image [C, H, W]."""
    dt = means2d.dtype
    C = means2d.shape[0]
    th, tw = tile_offsets.shape[1], tile_offsets.shape[2]
    out = np.zeros((C, height, width), dt)
    if flatten_ids.size == 0 or means2d.shape[1] == 0:
        return out
    args = [_c(means2d), _c(conics, dt), _c(opac, dt), _c(mus, dt),
            _c(tile_offsets, np.int32), _c(flatten_ids, np.int32)]
    fn = getattr(_load(), f"orc_raster_fwd_{_sfx(dt)}")
    fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), ctypes.c_int64(C),
       ctypes.c_uint32(width), ctypes.c_uint32(height), ctypes.c_uint32(tile_size),
       ctypes.c_uint32(tw), ctypes.c_uint32(th), _p(out))
    return out


def raster_bwd(means2d, conics, opac, mus, tile_offsets, flatten_ids, v_image, width, height,
               tile_size, absgrad=True):
    """RasterizeToPixelsBwd.cu:350-480 -> (v_abs|None, v_means2d, v_conics, v_opac, v_mus)."""
    dt = means2d.dtype
    C = means2d.shape[0]
    th, tw = tile_offsets.shape[1], tile_offsets.shape[2]
    v_xy = np.zeros_like(means2d)
    v_abs = np.zeros_like(means2d)
    v_con = np.zeros(conics.shape, dt)
    v_o = np.zeros(opac.shape, dt)
    v_mu = np.zeros(mus.shape, dt)
    if flatten_ids.size:
        args = [_c(means2d), _c(conics, dt), _c(opac, dt), _c(mus, dt),
                _c(tile_offsets, np.int32), _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_raster_bwd_{_sfx(dt)}")
        fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), _p(_c(v_image, dt)),
           ctypes.c_int64(C), ctypes.c_uint32(width), ctypes.c_uint32(height),
           ctypes.c_uint32(tile_size), ctypes.c_uint32(tw), ctypes.c_uint32(th), _p(v_abs),
           _p(v_xy), _p(v_con), _p(v_o), _p(v_mu))
    return (v_abs if absgrad else None), v_xy, v_con, v_o, v_mu


def voxel_fwd(means3d, conics, opac, tile_offsets, flatten_ids, dim2, dim1, dim0, tile_size):
    """VoxelizeToVoxelsFwd.cu:69-221 -> volume [dim0, dim1, dim2]."""
    dt = means3d.dtype
    n0, n1, n2 = tile_offsets.shape
    out = np.zeros((dim0, dim1, dim2), dt)
    if flatten_ids.size == 0 or means3d.shape[0] == 0:
        return out
    args = [_c(means3d), _c(conics, dt), _c(opac, dt), _c(tile_offsets, np.int32),
            _c(flatten_ids, np.int32)]
    fn = getattr(_load(), f"orc_voxel_fwd_{_sfx(dt)}")
    fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), ctypes.c_uint32(dim2),
       ctypes.c_uint32(dim1), ctypes.c_uint32(dim0), ctypes.c_uint32(tile_size),
       ctypes.c_uint32(n2), ctypes.c_uint32(n1), ctypes.c_uint32(n0), _p(out))
    return out


def voxel_bwd(means3d, conics, opac, tile_offsets, flatten_ids, v_volume, dim2, dim1, dim0,
              tile_size):
    """VoxelizeToVoxelsBwd.cu:322-441 -> (v_means3d, v_conics, v_opac)."""
    dt = means3d.dtype
    n0, n1, n2 = tile_offsets.shape
    v_m = np.zeros(means3d.shape, dt)
    v_c = np.zeros(conics.shape, dt)
    v_o = np.zeros(opac.shape, dt)
    if flatten_ids.size:
        args = [_c(means3d), _c(conics, dt), _c(opac, dt), _c(tile_offsets, np.int32),
                _c(flatten_ids, np.int32)]
        fn = getattr(_load(), f"orc_voxel_bwd_{_sfx(dt)}")
        fn(*[_p(a) for a in args], ctypes.c_int64(flatten_ids.size), _p(_c(v_volume, dt)),
           ctypes.c_uint32(dim2), ctypes.c_uint32(dim1), ctypes.c_uint32(dim0),
           ctypes.c_uint32(tile_size), ctypes.c_uint32(n2), ctypes.c_uint32(n1),
           ctypes.c_uint32(n0), _p(v_m), _p(v_c), _p(v_o))
    return v_m, v_c, v_o
