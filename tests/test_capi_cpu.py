"""The C ABI library on the CPU: it loads, exports every declared symbol,
and rejects invalid arguments before touching any device."""

import ctypes
import os
import re

import pytest

from r2splat.cuda import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                      "r2splat_hip.h")


def _declared():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    return sorted(set(re.findall(r"\b(r2s_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(_lib.LIB_PATH), "build the library first (python bt-3dgs_amd/build.py)"
    return _lib.load()


def test_exports_every_declared_symbol(lib):
    declared = _declared()
    assert len(declared) >= 40
    for name in declared:
        assert hasattr(lib, name), f"{name} missing from {_lib.LIB_PATH}"
    assert sorted(_lib.SYMBOLS) == declared, "ctypes table and header disagree"
    assert lib.r2s_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_are_rejected_without_a_device(lib):
    rc = lib.r2s_parameter_transform_fwd_f32(None, None, 5e-4, 1.0, None, None, -1, None)
    assert rc == 1001
    assert b"negative" in lib.r2s_last_error()
    # Empty inputs are a no-op that succeeds.
    assert lib.r2s_parameter_transform_fwd_f32(None, None, 5e-4, 1.0, None, None, 0, None) == 0
    assert lib.r2s_last_error() == b""
    rc = lib.r2s_world_to_image_projection_fwd_f32(None, None, None, None, 16, 16, 1e-8, 0.0,
                                                   None, None, None, 1, 4, None)
    assert rc == 1001 and b"radius_clip must be positive" in lib.r2s_last_error()
    rc = lib.r2s_rasterize_fwd_f32(None, None, None, None, None, None, 0, 1, 1, 64, 64, 40, 2, 2,
                                   None, None, 0, None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()
    rc = lib.r2s_isect_emit_sort_2d_f32(None, None, 1, 1, 10, 16, 4, 4, None, 1 << 31, 5, None,
                                        None, None, None, None, None, 0, None)
    assert rc == 1002  # beyond the int32 offset range
    rc = lib.r2s_isect_emit_sort_2d_f32(None, None, 1, 1, 10, 16, 4, 4, None, 100, 3, None, None,
                                        None, None, None, None, 0, None)
    assert rc == 1001 and b"end_bit" in lib.r2s_last_error()
    rc = lib.r2s_voxelize_fwd_f32(None, None, None, None, None, 0, 1, 8, 8, 8, 11, 1, 1, 1, None,
                                  None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()


def test_fused_projection_pack_checks_its_arguments(lib):
    args = [None] * 5 + [16, 16, 1e-8, 3.0] + [None] * 6
    # No payload (or conics): the fused entry needs both.
    rc = lib.r2s_project_pack_fwd_f32(*args, None, None, None, None, None, None, 1, 4, None)
    assert rc == 1001 and b"null conics or payload" in lib.r2s_last_error()
    conics = ctypes.c_void_p(64)  # never dereferenced: the checks come first
    args[12] = conics
    misaligned = ctypes.c_void_p(64 + 4)
    rc = lib.r2s_project_pack_fwd_f32(*args, misaligned, None, None, None, None, None, 0, 4,
                                      None)
    assert rc == 1001 and b"16-byte aligned" in lib.r2s_last_error()
    aligned = ctypes.c_void_p(128)
    rc = lib.r2s_project_pack_fwd_f32(*args, aligned, None, aligned, None, None, None, 0, 4, None)
    assert rc == 1001 and b"zero targets need" in lib.r2s_last_error()
    rc = lib.r2s_project_pack_fwd_f32(*args, aligned, None, None, None, None, None, 0, 4, None)
    assert rc == 0  # C * N == 0: nothing to do


def test_tile_sizes_whose_products_wrap_are_rejected(lib):
    # 65536^2 and 2048^3 wrap to 0 in 32 bits; both must fail the tile-size
    # check before any launch (the backward would otherwise pick a kernel for
    # the first 32 rows only and report success).
    rc = lib.r2s_rasterize_fwd_f32(None, None, None, None, None, None, 0, 1, 1, 64, 64, 65536, 1,
                                   1, None, None, 0, None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()
    rc = lib.r2s_rasterize_bwd_f32(None, None, None, None, None, None, None, 5, None, 1, 1, 64,
                                   64, 65536, 1, 1, None, None, None, None, None, None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()
    rc = lib.r2s_rasterize_bwd_emit_f32(None, None, None, None, None, None, None, None, None, 5,
                                        None, 1, 1, 64, 64, 65536, 1, 1, None, None, None, None,
                                        None, None, 0, None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()
    rc = lib.r2s_voxelize_fwd_f32(None, None, None, None, None, 0, 1, 8, 8, 8, 2048, 1, 1, 1,
                                  None, None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()
    rc = lib.r2s_voxelize_bwd_f32(None, None, None, None, None, None, 5, None, 1, 8, 8, 8, 2048,
                                  1, 1, 1, None, None, None, None)
    assert rc == 1001 and b"tile_size" in lib.r2s_last_error()


def test_reach_mask_entries_check_their_arguments(lib):
    # Reach masks exist for tile size 8 only; the backward needs them given.
    buf = ctypes.create_string_buffer(64)
    rc = lib.r2s_voxelize_fwd_reach_f32(None, None, None, None, None, 0, 1, 8, 8, 8, 4, 2, 2, 2,
                                        buf, buf, None)
    assert rc == 1001 and b"reach masks need tile_size 8" in lib.r2s_last_error()
    rc = lib.r2s_voxelize_bwd_emit_reach_f32(None, None, None, None, None, None, None, None, 5,
                                             None, 1, 8, 8, 8, 8, 1, 1, 1, None, None, None,
                                             None, None, 0, None)
    assert rc == 1001 and b"null reach masks" in lib.r2s_last_error()
    rc = lib.r2s_voxelize_bwd_emit_reach_f32(None, None, None, None, None, None, None, None, 5,
                                             None, 1, 8, 8, 8, 4, 2, 2, 2, buf, None, None, None,
                                             None, 0, None)
    assert rc == 1001 and b"reach masks need tile_size 8" in lib.r2s_last_error()


def test_workspace_queries(lib):
    assert lib.r2s_isect_workspace_bytes(0, 0, 11) == 0
    small = lib.r2s_isect_workspace_bytes(0, 1000, 11)
    big = lib.r2s_isect_workspace_bytes(0, 10_000_000, 11)
    # Keys up to 11 bits sort in one pass: keys + ids (8 B per record) plus
    # two 2048-digit tables per 4096 records.
    assert 8 * 1000 <= small < big and big >= 10 * 10_000_000
    # Wider keys take two or more passes and ping-pong (key, id, emission index).
    assert lib.r2s_isect_workspace_bytes(0, 10_000_000, 15) >= 24 * 10_000_000
    assert lib.r2s_isect_workspace_bytes(500_000, 0, 0) > 0
    assert lib.r2s_mask_workspace_bytes(1_000_000) > 0
    buf = ctypes.create_string_buffer(16)
    rc = lib.r2s_isect_emit_sort_2d_f32(None, None, 1, 1, 10, 16, 4, 4, None, 100, 5, buf, buf,
                                        None, None, None, buf, 16, None)
    assert rc in (1001, 1004)


def test_row_workspaces_hold_the_slots_the_tests_read(lib):
    # One row per record at its emission index: the GPU tests index the
    # workspace with these slot counts.
    from helpers import RASTER_ROW_SLOTS, VOXEL_ROW_SLOTS
    n = 1000
    assert lib.r2s_voxelize_bwd_workspace_bytes(n, 4) == n * VOXEL_ROW_SLOTS * 4
    assert lib.r2s_voxelize_bwd_workspace_bytes(n, 8) == n * VOXEL_ROW_SLOTS * 8
    for b in (4, 8):  # rows, then the packed payload of 8 values per (view, Gaussian)
        assert lib.r2s_rasterize_bwd_workspace_bytes(n, 7, b) == (n * RASTER_ROW_SLOTS + 7 * 8) * b


def test_noalloc_forward_rejects_partial_tiles_beyond_its_array(lib):
    # 64x64 tiles of 16 with 8192 records each split 8 ways: 4096 * 8 * 256
    # pixels, 32 MiB in float32 (fits) and 64 MiB in float64 (does not).  The
    # size check comes before any pointer is read or any HIP call is made.
    n_keys, n = 64 * 64, 64 * 64 * 8192
    assert lib.r2s_rasterize_workspace_bytes(n_keys, n, 16, 4) == 32 << 20
    rc = lib.r2s_rasterize_fwd_noalloc_f64(None, None, None, None, None, None, n, 1, 1, 1024, 1024,
                                           16, 64, 64, None, None)
    assert rc == 1002 and b"static scratch holds 33554432" in lib.r2s_last_error()
    rc = lib.r2s_rasterize_fwd_noalloc_f32(None, None, None, None, None, None, 2 * n, 2, 1, 1024,
                                           1024, 16, 64, 64, None, None)
    assert rc == 1002
    # Argument checks still come first.
    rc = lib.r2s_rasterize_fwd_noalloc_f32(None, None, None, None, None, None, n, 1, 1, 1024, 1024,
                                           0, 64, 64, None, None)
    assert rc == 1001


def test_densify_arguments_are_checked_without_a_device(lib):
    C = _lib.Column
    cols = (C * 1)()
    cols[0] = C(None, None, None, 0, 0, _lib.COL_COPY)
    assert lib.r2s_densify_remove(None, 0, cols, 1, None) == 1001
    assert b"width 0" in lib.r2s_last_error()
    assert lib.r2s_densify_remove(None, 5, cols, 1, None) == 1001
    assert b"null keep" in lib.r2s_last_error()
    cols[0] = C(None, None, None, 0, 1, _lib.COL_HISTORY)
    assert lib.r2s_densify_remove(None, 0, cols, 1, None) == 1001
    assert b"history" in lib.r2s_last_error()
    cols[0] = C(None, None, None, 3, 1, _lib.COL_COPY)
    assert lib.r2s_densify_remove(None, 0, cols, 1, None) == 1001
    assert b"3 rows, the operation writes 0" in lib.r2s_last_error()
    cols[0] = C(None, None, None, 0, 3, _lib.COL_PARENT)
    assert lib.r2s_densify_split(None, 0, None, 0, 0, None, cols, 1, None) == 1001
    assert b"width 1" in lib.r2s_last_error()
    cols[0] = C(None, None, None, 0, 3, _lib.COL_MEANS)
    assert lib.r2s_densify_split(None, 0, None, 0, 0, None, cols, 1, None) == 1001
    assert b"geometry" in lib.r2s_last_error()
    fake = ctypes.c_void_p(256)  # never dereferenced: the size check fails first
    assert lib.r2s_densify_split(fake, 2, None, 0, (1 << 31) - 2, None, None, 0, None) == 1002
    assert lib.r2s_densify_duplicate(None, 4, None, 0, 0, None, 0, None) == 1001  # null mask
    # Nothing to write is a successful no-op.
    assert lib.r2s_densify_remove(None, 0, None, 0, None) == 0
    assert lib.r2s_densify_split(None, 0, None, 0, 0, None, None, 0, None) == 0


def test_loss_and_optimizer_arguments_are_checked_without_a_device(lib):
    out = ctypes.c_void_p(256)  # never dereferenced: the checks fail first
    # Even windows are rejected (metric.py's padding would change the map size).
    assert lib.r2s_projection_loss_fwd_f32(out, out, None, None, 1, 8, 8, 10, out, None, 0,
                                           None) == 1001
    assert b"window_size must be odd" in lib.r2s_last_error()
    assert lib.r2s_projection_loss_fwd_f32(out, out, out, None, 1, 8, 8, 11, out, None, 0,
                                           None) == 1001
    assert b"go together" in lib.r2s_last_error()
    assert lib.r2s_projection_loss_fwd_f32(out, out, None, None, 1, 8, 8, 11, out, None, 0,
                                           None) == 1004
    assert lib.r2s_projection_loss_workspace_bytes(2, 64, 64) >= 3 * 2 * 64 * 64 * 4
    assert lib.r2s_tv_fwd_f32(None, 4, 4, 4, 1, out, None, 0, None) == 1001
    assert lib.r2s_tv_workspace_bytes() > 0
    assert lib.r2s_hierarchy_loss_fwd_f32(None, None, 5, None, None, None, 0, 1.0, out, None, 0,
                                          None) == 1001
    assert b"null child arrays" in lib.r2s_last_error()
    A = _lib.AdamTensor
    table = (A * 1)()
    table[0] = A(None, None, None, None, 10, 0.1, 0.999, 0.001, 0.0, 1.0, 1e-8, -1e-3)
    assert lib.r2s_adam_step_f32(ctypes.cast(table, ctypes.c_void_p), 1, None) == 1001
    assert b"null pointer" in lib.r2s_last_error()
    table[0] = A(None, None, None, None, 0, 0.1, 0.999, 0.001, 0.0, 1.0, 1e-8, -1e-3)
    assert lib.r2s_adam_step_f32(ctypes.cast(table, ctypes.c_void_p), 1, None) == 0
