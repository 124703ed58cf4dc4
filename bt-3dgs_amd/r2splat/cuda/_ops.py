"""Tensor-level operators over the HIP C ABI.

Each function keeps the name, argument order, return tuple and input checks
of the reference pybind operator it replaces (``r2splat/cuda/include/Ops.h``
and the ``*.cpp`` tensor wrappers in ``r2splat/cuda/csrc``).  Outputs and
scratch space are allocated with torch's caching allocator on the input's
device; work is enqueued on torch's current stream of that device.  There is
no CPU fallback: without the library every call raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import math
import threading
import warnings
from typing import NamedTuple, Optional, Tuple

import torch

from . import _backend

Tensor = torch.Tensor


# ---------------------------------------------------------------- plumbing --

def _lib():
    return _backend.library()


def _check_input(t: Tensor, name: str) -> None:
    # common.h:25-30 R2SPLAT_CHECK_INPUT
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _check(cond: bool, *msg) -> None:
    if not cond:
        raise RuntimeError("".join(str(m) for m in msg))


def _suffix(t: Tensor, op: str) -> str:
    # AT_DISPATCH_FLOATING_TYPES: float32 and float64 only.
    if t.dtype == torch.float32:
        return "f32"
    if t.dtype == torch.float64:
        return "f64"
    raise RuntimeError(f'"{op}" not implemented for \'{t.dtype}\'')


def _ptr(t: Optional[Tensor]):
    return None if t is None else t.data_ptr()


# The current stream's handle without building a torch Stream object per call
# (torch's raw accessor where this build has it).
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device):
    if _RAW_STREAM is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _RAW_STREAM(idx)
    return torch.cuda.current_stream(device).cuda_stream


_FUNCS = {}  # entry point name -> (library, its ctypes function)


def _call(name: str, *args) -> None:
    lib = _lib()
    hit = _FUNCS.get(name)
    if hit is None or hit[0] is not lib:
        hit = _FUNCS[name] = (lib, getattr(lib, name))
    rc = hit[1](*args)
    if rc != 0:
        msg = lib.r2s_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def _workspace(nbytes: int, device: torch.device) -> Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def _check_record_count(n_isects: int, op: str) -> None:
    # The tile offsets are int32, as in the reference (IsectTiles.cpp:191); the
    # sort would otherwise need tens of GB before the library rejects the size.
    if n_isects > 2 ** 31 - 1:
        raise RuntimeError(f"{op}: {n_isects} tile records exceed the int32 offset range "
                           f"(2**31 - 1)")


def _end_bit(n_keys: int) -> int:
    # IsectTiles.cpp:146-147
    return int(math.ceil(math.log2(float(n_keys + 1))))


# Record counts of recent binning calls, per (device, kind, items, keys).
# The next call with the same sizes allocates its outputs for the largest
# of them plus a margin and launches the emit + sort before reading its own
# count back (the kernels read the count on the device and write nothing if
# it exceeds the capacity), so the device does not sit idle while the host
# waits for the count, allocates and launches.  The outputs are then the
# leading n records of the larger buffers.  A short guess costs one exact
# relaunch.
_COUNT_HISTORY = {}
_COUNT_HISTORY_LEN = 8
_PINNED_COUNT = threading.local()  # per host thread: a count read back by one call at a time


def _note_count(key, n: int) -> None:
    hist = _COUNT_HISTORY.setdefault(key, [])
    hist.append(n)
    del hist[:-_COUNT_HISTORY_LEN]


TOO_MANY = object()  # _emit_and_sort: the count exceeds max_records


def _emit_and_sort(launch, offsets: Tensor, n_items: int, n_keys: int, op: str,
                   dev: torch.device, kind: str, max_records: Optional[int] = None,
                   keep_ids: bool = True):
    """The emit + sort half of a binning op (IsectTiles.cpp:100-169): returns
    (isect_ids, flatten_ids, emit_ids, isect_src), or None without records,
    or TOO_MANY when there are more than max_records records (nothing
    allocated for them).  launch(capacity, end_bit, outputs, workspace)
    enqueues the library call.  keep_ids=False: isect_ids is None and the
    sort writes no keys (the caller's launch passes the tile offsets)."""
    lib = _lib()
    end_bit = _end_bit(n_keys)
    key = (dev.index, kind, n_items, n_keys)

    def alloc(cap):
        outs = (torch.empty((cap,), dtype=torch.int64, device=dev) if keep_ids else None,
                torch.empty((cap,), dtype=torch.int32, device=dev),
                torch.empty((cap,), dtype=torch.int32, device=dev),
                torch.empty((cap,), dtype=torch.int32, device=dev))
        return outs, _workspace(lib.r2s_isect_workspace_bytes(0, cap, end_bit), dev)

    recent = _COUNT_HISTORY.get(key)
    if recent:
        guess = max(recent)
        cap = min(guess + guess // 8 + 4096, 2 ** 31 - 1)
        if max_records is not None:
            # A list that fits the speculative capacity must also fit the
            # caller's limit; a longer one falls through to the check below.
            cap = min(cap, max_records)
        outs, ws = alloc(cap)
        pinned = getattr(_PINNED_COUNT, "by_device", None)
        if pinned is None:
            pinned = _PINNED_COUNT.by_device = {}
        host = pinned.get(dev.index)
        if host is None:
            host = pinned[dev.index] = torch.empty(1, dtype=torch.int64, pin_memory=True)
        host.copy_(offsets[n_items:n_items + 1], non_blocking=True)
        ready = torch.cuda.Event()
        ready.record()
        launch(cap, end_bit, outs, ws)
        ready.synchronize()
        n = int(host[0])
        _note_count(key, n)
        if n <= cap:
            return None if n == 0 else tuple(None if t is None else t[:n] for t in outs)
    else:
        n = int(offsets[n_items].item())  # the one host read-back (IsectTiles.cpp:100)
        _note_count(key, n)
    if max_records is not None and n > max_records:
        return TOO_MANY
    if n == 0:
        return None
    _check_record_count(n, op)
    outs, ws = alloc(n)
    launch(n, end_bit, outs, ws)
    return outs


# Binned records.  Besides the reference's sorted lists, the binning kernels
# describe the records in emission order (Gaussian-major, before the sort by
# tile): emit_ids[e] is the id of emitted record e and isect_src[r] the
# emission index of sorted record r.  With them the backward ops run the
# two-pass kernels, which store each record's partials at its emission index
# and then sum them per Gaussian, instead of one device-scope atomic per
# record and partial (about 3x slower at the headline shape).


class TileLists(NamedTuple):
    """Output of :func:`bin_tiles_2d` / :func:`bin_tiles_3d`."""

    tiles_per_gauss: Tensor
    # int64 tile keys, sorted; None for a list binned with keep_ids=False
    # (read isect_ids, which then recovers them from tile_offsets).
    keys: Optional[Tensor]
    flatten_ids: Tensor  # int32 ids in (key, emission) order
    emit_ids: Optional[Tensor]   # None when there are no records
    isect_src: Optional[Tensor]
    # Each key's first index in the sorted list, as isect_offset_encode /
    # isect_offset_encode_3d return it (written by the sort); None when
    # there are no records.
    tile_offsets: Optional[Tensor] = None

    @property
    def emission(self) -> Optional[Tuple[Tensor, Tensor]]:
        return None if self.emit_ids is None else (self.emit_ids, self.isect_src)

    @property
    def isect_ids(self) -> Tensor:
        """The sorted int64 tile keys (IsectTiles.cpp:113-169's isect_ids):
        the stored array, or, for a list binned without it, a new array
        recovered from tile_offsets (one launch per access)."""
        if self.keys is not None:
            return self.keys
        return keys_from_offsets(self.tile_offsets, self.flatten_ids.numel())


# The reference's operator signatures (isect_tiles -> rasterize_to_pixels_bwd*)
# pass only flatten_ids between the ops.  So that those callers still get the
# two-pass backward, isect_tiles / isect_tiles_3d also attach the emission
# arrays to the flatten_ids tensor they return (attribute _EMIT_ATTR, with
# the tensor's version counter).  A flatten_ids that is not the returned
# tensor itself, unmodified -- a clone, slice, .to() copy, or a list built
# elsewhere -- is not in the table; the backward then runs the one-pass
# kernels, counts the call in PATH_COUNTS["one_pass"] and warns once per
# process.  r2splat.ops passes the arrays explicitly and never relies on it.
_EMIT_ATTR = "_r2s_emission_order"
PATH_COUNTS = {"two_pass": 0, "one_pass": 0}
_WARNED_ONE_PASS = False


class OnePassBackwardWarning(UserWarning):
    """A backward op ran the one-pass atomic kernels for lack of emission order."""


def _remember_emission(lists: TileLists, n_keys: int) -> None:
    if lists.emit_ids is not None:
        fl = lists.flatten_ids
        setattr(fl, _EMIT_ATTR, (lists.emit_ids, lists.isect_src, fl._version, int(n_keys)))


def emission_order(flatten_ids: Tensor, n_keys: int) -> Optional[Tuple[Tensor, Tensor]]:
    """(emit_ids, isect_src) that isect_tiles* returned with this very
    flatten_ids tensor for n_keys tile keys, if it is unmodified; else None."""
    rec = getattr(flatten_ids, _EMIT_ATTR, None)
    if rec is None:
        return None
    ids, src, version, nk = rec
    if version != flatten_ids._version or nk != int(n_keys) or ids.numel() != flatten_ids.numel():
        return None
    return ids, src


def _note_path(two_pass: bool, op: str) -> None:
    global _WARNED_ONE_PASS
    PATH_COUNTS["two_pass" if two_pass else "one_pass"] += 1
    if not two_pass and not _WARNED_ONE_PASS:
        _WARNED_ONE_PASS = True
        warnings.warn(
            f"{op}: flatten_ids carries no emission order (not the tensor isect_tiles* "
            "returned, or modified since), so the one-pass atomic backward runs; pass the "
            "emission arrays explicitly (r2splat.cuda._ops.TileLists) to keep the two-pass "
            "form", OnePassBackwardWarning, stacklevel=4)


# ------------------------------------------------------ parameter transform --

def parameter_transform_fwd(quats: Tensor, scale_ori: Tensor, scale_min: float,
                            scale_max: float) -> Tuple[Tensor, Tensor]:
    """ParameterTransform.cpp:34-84 -> (covars [N,6], max_scales [N])."""
    _check_input(quats, "quats")
    _check_input(scale_ori, "scale_ori")
    _check(quats.dim() == 2 and quats.size(1) == 4,
           "quats must be 2D [N, 4], got shape ", list(quats.shape))
    _check(scale_ori.dim() == 2 and scale_ori.size(1) == 3,
           "scale_ori must be 2D [N, 3], got shape ", list(scale_ori.shape))
    N = quats.size(0)
    _check(scale_ori.size(0) == N, "scale_ori batch dim (", scale_ori.size(0),
           ") doesn't match quats N=", N)
    covars = torch.empty((N, 6), dtype=quats.dtype, device=quats.device)
    max_scales = torch.empty((N,), dtype=quats.dtype, device=quats.device)
    if N == 0:
        return covars, max_scales
    _check(scale_ori.dtype == quats.dtype, "quats and scale_ori must share a dtype")
    sfx = _suffix(quats, "parameter_transform_fwd")
    with torch.cuda.device(quats.device):
        _call(f"r2s_parameter_transform_fwd_{sfx}", _ptr(quats), _ptr(scale_ori),
              float(scale_min), float(scale_max), _ptr(covars), _ptr(max_scales), N,
              _stream(quats.device))
    return covars, max_scales


def parameter_transform_bwd(quats: Tensor, scale_ori: Tensor, scale_min: float,
                            scale_max: float, v_covars: Tensor) -> Tuple[Tensor, Tensor]:
    """ParameterTransform.cpp:90-144 -> (v_quats [N,4], v_scale_ori [N,3])."""
    for t, n in ((quats, "quats"), (scale_ori, "scale_ori"), (v_covars, "v_covars")):
        _check_input(t, n)
    _check(quats.dim() == 2 and quats.size(1) == 4, "quats must be 2D [N, 4]")
    _check(scale_ori.dim() == 2 and scale_ori.size(1) == 3, "scale_ori must be 2D [N, 3]")
    _check(v_covars.dim() == 2 and v_covars.size(1) == 6, "v_covars must be 2D [N, 6]")
    N = quats.size(0)
    _check(scale_ori.size(0) == N and v_covars.size(0) == N, "Batch dimension mismatch")
    v_quats = torch.empty((N, 4), dtype=quats.dtype, device=quats.device)
    v_scale = torch.empty((N, 3), dtype=quats.dtype, device=quats.device)
    if N == 0:
        return v_quats, v_scale
    _check(scale_ori.dtype == quats.dtype and v_covars.dtype == quats.dtype,
           "quats, scale_ori and v_covars must share a dtype")
    sfx = _suffix(quats, "parameter_transform_bwd")
    with torch.cuda.device(quats.device):
        _call(f"r2s_parameter_transform_bwd_{sfx}", _ptr(quats), _ptr(scale_ori),
              float(scale_min), float(scale_max), _ptr(v_covars), _ptr(v_quats), _ptr(v_scale),
              N, _stream(quats.device))
    return v_quats, v_scale


def prepare_gaussians(quats: Tensor, raw_scales: Tensor, raw_opacities: Tensor,
                      scale_min: float, scale_max: float) -> Tuple[Tensor, Tensor, Tensor]:
    """Fused parameter_transform_fwd + softplus (r2splat/ops/direct.py:85-91)."""
    for t, n in ((quats, "quats"), (raw_scales, "scale_ori"), (raw_opacities, "raw_opacities")):
        _check_input(t, n)
    _check(quats.dim() == 2 and quats.size(1) == 4,
           "quats must be 2D [N, 4], got shape ", list(quats.shape))
    _check(raw_scales.dim() == 2 and raw_scales.size(1) == 3,
           "scale_ori must be 2D [N, 3], got shape ", list(raw_scales.shape))
    N = quats.size(0)
    _check(raw_scales.size(0) == N, "scale_ori batch dim (", raw_scales.size(0),
           ") doesn't match quats N=", N)
    _check(raw_opacities.dim() == 1 and raw_opacities.size(0) == N,
           "raw_opacities must be 1D [N]")
    _check(raw_scales.dtype == quats.dtype and raw_opacities.dtype == quats.dtype,
           "quats, scale_ori and raw_opacities must share a dtype")
    dev, dt = quats.device, quats.dtype
    covars = torch.empty((N, 6), dtype=dt, device=dev)
    max_scales = torch.empty((N,), dtype=dt, device=dev)
    opac = torch.empty((N,), dtype=dt, device=dev)
    if N == 0:
        return covars, max_scales, opac
    sfx = _suffix(quats, "prepare_gaussians")
    with torch.cuda.device(dev):
        _call(f"r2s_prepare_gaussians_{sfx}", _ptr(quats), _ptr(raw_scales), _ptr(raw_opacities),
              float(scale_min), float(scale_max), _ptr(covars), _ptr(max_scales), _ptr(opac), N,
              _stream(dev))
    return covars, max_scales, opac


def opacity_bwd(raw_opacities: Tensor, v_opacity_cn: Optional[Tensor],
                v_opacity_3d: Optional[Tensor]) -> Tensor:
    """v_raw = (sum_c v_opacity_cn[c] + v_opacity_3d) * sigmoid(raw) (explicit.py:319,370,379)."""
    _check_input(raw_opacities, "raw_opacities")
    N = raw_opacities.size(0)
    C = 0
    if v_opacity_cn is not None:
        _check_input(v_opacity_cn, "v_opacity")
        _check(v_opacity_cn.dim() == 2 and v_opacity_cn.size(1) == N, "v_opacity must be [C, N]")
        C = v_opacity_cn.size(0)
    if v_opacity_3d is not None:
        _check_input(v_opacity_3d, "v_opacity_3d")
        _check(v_opacity_3d.shape == (N,), "v_opacity_3d must be [N]")
    out = torch.empty_like(raw_opacities)
    if N == 0:
        return out
    sfx = _suffix(raw_opacities, "opacity_bwd")
    with torch.cuda.device(raw_opacities.device):
        _call(f"r2s_opacity_bwd_{sfx}", _ptr(raw_opacities), _ptr(v_opacity_cn),
              _ptr(v_opacity_3d), _ptr(out), C, N, _stream(raw_opacities.device))
    return out


# ------------------------------------------------------------- projection --

def _check_cameras(means, covars, viewmats, Ks):
    _check(means.dim() == 2 and means.size(1) == 3,
           "means must be 2D [N, 3], got shape ", list(means.shape))
    _check(covars.dim() == 2 and covars.size(1) == 6,
           "covars must be 2D [N, 6], got shape ", list(covars.shape))
    _check(viewmats.dim() == 3 and viewmats.size(1) == 4 and viewmats.size(2) == 4,
           "viewmats must be 3D [C, 4, 4], got shape ", list(viewmats.shape))
    _check(Ks.dim() == 3 and Ks.size(1) == 3 and Ks.size(2) == 3,
           "Ks must be 3D [C, 3, 3], got shape ", list(Ks.shape))
    N, C = means.size(0), viewmats.size(0)
    _check(covars.size(0) == N, "covars dim 0 (", covars.size(0), ") doesn't match N=", N)
    _check(Ks.size(0) == C, "Ks batch dim (", Ks.size(0), ") doesn't match C=", C)
    return C, N


def world_to_image_projection_fwd(means: Tensor, covars: Tensor, viewmats: Tensor, Ks: Tensor,
                                  dim1: int, dim0: int, eps_blur: float,
                                  radius_clip: float) -> Tuple[Tensor, Tensor, Tensor]:
    """WorldToImageProjection.cpp:38-119 -> (means2d [C,N,2], cov2d [C,N,6], radii [C,N,2])."""
    for t, n in ((means, "means"), (covars, "covars"), (viewmats, "viewmats"), (Ks, "Ks")):
        _check_input(t, n)
    C, N = _check_cameras(means, covars, viewmats, Ks)
    _check(float(radius_clip) > 0.0, "radius_clip must be positive, got ", float(radius_clip))
    dev, dt = means.device, means.dtype
    means2d = torch.empty((C, N, 2), dtype=dt, device=dev)
    cov2d = torch.empty((C, N, 6), dtype=dt, device=dev)
    radii = torch.zeros((C, N, 2), dtype=torch.int32, device=dev)
    if C * N == 0:
        return means2d, cov2d, radii
    sfx = _suffix(means, "world_to_image_projection_fwd")
    with torch.cuda.device(dev):
        _call(f"r2s_world_to_image_projection_fwd_{sfx}", _ptr(means), _ptr(covars),
              _ptr(viewmats), _ptr(Ks), int(dim1), int(dim0), float(eps_blur),
              float(radius_clip), _ptr(means2d), _ptr(cov2d), _ptr(radii), C, N, _stream(dev))
    return means2d, cov2d, radii


def world_to_image_projection_bwd(means: Tensor, covars: Tensor, viewmats: Tensor, Ks: Tensor,
                                  dim1: int, dim0: int, v_means2d: Tensor,
                                  v_cov2d_3x3: Tensor) -> Tuple[Tensor, Tensor]:
    """WorldToImageProjection.cpp:127-206 -> (v_means [N,3], v_covars [N,6])."""
    for t, n in ((means, "means"), (covars, "covars"), (viewmats, "viewmats"), (Ks, "Ks"),
                 (v_means2d, "v_means2d"), (v_cov2d_3x3, "v_cov2d_3x3")):
        _check_input(t, n)
    _check(means.dim() == 2 and means.size(1) == 3, "means must be 2D [N, 3]")
    _check(covars.dim() == 2 and covars.size(1) == 6, "covars must be 2D [N, 6]")
    _check(viewmats.dim() == 3 and viewmats.size(1) == 4 and viewmats.size(2) == 4,
           "viewmats must be 3D [C, 4, 4]")
    _check(Ks.dim() == 3 and Ks.size(1) == 3 and Ks.size(2) == 3, "Ks must be 3D [C, 3, 3]")
    _check(v_means2d.dim() == 3 and v_means2d.size(2) == 2, "v_means2d must be 3D [C, N, 2]")
    _check(v_cov2d_3x3.dim() == 3 and v_cov2d_3x3.size(2) == 6,
           "v_cov2d_3x3 must be 3D [C, N, 6]")
    N, C = means.size(0), viewmats.size(0)
    _check(covars.size(0) == N, "covars dim 0 mismatch")
    _check(v_means2d.size(0) == C and v_means2d.size(1) == N, "v_means2d shape mismatch")
    _check(v_cov2d_3x3.size(0) == C and v_cov2d_3x3.size(1) == N, "v_cov2d_3x3 shape mismatch")
    dev, dt = means.device, means.dtype
    v_means = torch.empty((N, 3), dtype=dt, device=dev)
    v_covars = torch.empty((N, 6), dtype=dt, device=dev)
    if C * N == 0:
        # The reference returns uninitialised tensors here; zeros are the sum
        # over an empty camera set.
        return v_means.zero_(), v_covars.zero_()
    sfx = _suffix(means, "world_to_image_projection_bwd")
    with torch.cuda.device(dev):
        _call(f"r2s_world_to_image_projection_bwd_{sfx}", _ptr(means), _ptr(covars),
              _ptr(viewmats), _ptr(Ks), int(dim1), int(dim0), _ptr(v_means2d),
              _ptr(v_cov2d_3x3), _ptr(v_means), _ptr(v_covars), C, N, _stream(dev))
    return v_means, v_covars


def conics_mu_fwd(cov2d_3x3: Tensor, eps: float) -> Tuple[Tensor, Tensor]:
    """ConicsMu.cpp:35-80 -> (conics [C,N,3], mus [C,N])."""
    _check_input(cov2d_3x3, "cov2d_3x3")
    _check(cov2d_3x3.dim() == 3, "cov2d_3x3 must be 3D [C, N, 6], got dim=", cov2d_3x3.dim())
    _check(cov2d_3x3.size(2) == 6, "cov2d_3x3 last dim must be 6, got ", cov2d_3x3.size(2))
    C, N = cov2d_3x3.size(0), cov2d_3x3.size(1)
    dev, dt = cov2d_3x3.device, cov2d_3x3.dtype
    conics = torch.empty((C, N, 3), dtype=dt, device=dev)
    mus = torch.empty((C, N), dtype=dt, device=dev)
    if C * N == 0:
        return conics, mus
    sfx = _suffix(cov2d_3x3, "conics_mu_fwd")
    with torch.cuda.device(dev):
        _call(f"r2s_conics_mu_fwd_{sfx}", _ptr(cov2d_3x3), float(eps), _ptr(conics), _ptr(mus),
              C * N, _stream(dev))
    return conics, mus


def conics_mu_bwd(cov2d_3x3: Tensor, eps: float, conics: Tensor, mus: Tensor, v_conics: Tensor,
                  v_mus: Tensor) -> Tensor:
    """ConicsMu.cpp:87-159 -> v_cov2d_3x3 [C,N,6]."""
    for t, n in ((cov2d_3x3, "cov2d_3x3"), (conics, "conics"), (mus, "mus"),
                 (v_conics, "v_conics"), (v_mus, "v_mus")):
        _check_input(t, n)
    _check(cov2d_3x3.dim() == 3, "cov2d_3x3 must be 3D [C, N, 6]")
    _check(conics.dim() == 3, "conics must be 3D [C, N, 3]")
    _check(mus.dim() == 2, "mus must be 2D [C, N]")
    _check(v_conics.dim() == 3, "v_conics must be 3D [C, N, 3]")
    _check(v_mus.dim() == 2, "v_mus must be 2D [C, N]")
    C, N = cov2d_3x3.size(0), cov2d_3x3.size(1)
    _check(cov2d_3x3.size(2) == 6, "cov2d_3x3 last dim must be 6")
    _check(tuple(conics.shape) == (C, N, 3), "conics shape must be [C, N, 3]")
    _check(tuple(mus.shape) == (C, N), "mus shape must be [C, N]")
    _check(tuple(v_conics.shape) == (C, N, 3), "v_conics shape must be [C, N, 3]")
    _check(tuple(v_mus.shape) == (C, N), "v_mus shape must be [C, N]")
    out = torch.empty((C, N, 6), dtype=cov2d_3x3.dtype, device=cov2d_3x3.device)
    if C * N == 0:
        return out
    sfx = _suffix(cov2d_3x3, "conics_mu_bwd")
    with torch.cuda.device(cov2d_3x3.device):
        _call(f"r2s_conics_mu_bwd_{sfx}", _ptr(cov2d_3x3), float(eps), _ptr(conics), _ptr(mus),
              _ptr(v_conics), _ptr(v_mus), _ptr(out), C * N, _stream(cov2d_3x3.device))
    return out


def project_gaussians_fwd(means: Tensor, covars: Tensor, opacities: Tensor, viewmats: Tensor,
                          Ks: Tensor, img_w: int, img_h: int, eps2d: float, radius_clip: float):
    """Fused world_to_image_projection_fwd + conics_mu_fwd + opacity broadcast
    (r2splat/ops/direct.py:149-161) -> (means2d, cov2d, radii, conics, mus, opacity[C,N])."""
    for t, n in ((means, "means"), (covars, "covars"), (opacities, "opacities"),
                 (viewmats, "viewmats"), (Ks, "Ks")):
        _check_input(t, n)
    C, N = _check_cameras(means, covars, viewmats, Ks)
    _check(opacities.dim() == 1 and opacities.size(0) == N, "opacities must be 1D [N]")
    _check(float(radius_clip) > 0.0, "radius_clip must be positive, got ", float(radius_clip))
    dev, dt = means.device, means.dtype
    means2d = torch.empty((C, N, 2), dtype=dt, device=dev)
    cov2d = torch.empty((C, N, 6), dtype=dt, device=dev)
    radii = torch.empty((C, N, 2), dtype=torch.int32, device=dev)
    conics = torch.empty((C, N, 3), dtype=dt, device=dev)
    mus = torch.empty((C, N), dtype=dt, device=dev)
    opac = torch.empty((C, N), dtype=dt, device=dev)
    if C * N == 0:
        return means2d, cov2d, radii, conics, mus, opac
    sfx = _suffix(means, "project_gaussians_fwd")
    with torch.cuda.device(dev):
        _call(f"r2s_project_gaussians_fwd_{sfx}", _ptr(means), _ptr(covars), _ptr(opacities),
              _ptr(viewmats), _ptr(Ks), int(img_w), int(img_h), float(eps2d),
              float(radius_clip), _ptr(means2d), _ptr(cov2d), _ptr(radii), _ptr(conics),
              _ptr(mus), _ptr(opac), C, N, _stream(dev))
    return means2d, cov2d, radii, conics, mus, opac


def project_pack_fwd(means: Tensor, covars: Tensor, opacities: Tensor, viewmats: Tensor,
                     Ks: Tensor, img_w: int, img_h: int, eps2d: float, radius_clip: float,
                     zero_outputs: bool = False, absgrad: bool = False):
    """:func:`project_gaussians_fwd` and :func:`raster_pack` on its outputs in
    one launch -> (means2d, cov2d, radii, conics, mus, opacity[C,N], payload,
    outputs), each bit for bit what the two calls return."""
    for t, n in ((means, "means"), (covars, "covars"), (opacities, "opacities"),
                 (viewmats, "viewmats"), (Ks, "Ks")):
        _check_input(t, n)
    C, N = _check_cameras(means, covars, viewmats, Ks)
    _check(opacities.dim() == 1 and opacities.size(0) == N, "opacities must be 1D [N]")
    _check(float(radius_clip) > 0.0, "radius_clip must be positive, got ", float(radius_clip))
    dev, dt = means.device, means.dtype
    means2d = torch.empty((C, N, 2), dtype=dt, device=dev)
    cov2d = torch.empty((C, N, 6), dtype=dt, device=dev)
    radii = torch.empty((C, N, 2), dtype=torch.int32, device=dev)
    conics = torch.empty((C, N, 3), dtype=dt, device=dev)
    mus = torch.empty((C, N), dtype=dt, device=dev)
    opac = torch.empty((C, N), dtype=dt, device=dev)
    payload = torch.empty((C * N * 8,), dtype=dt, device=dev)
    outs = None
    if zero_outputs:
        outs = (torch.empty_like(means2d) if absgrad else None, torch.empty_like(means2d),
                torch.empty_like(conics), torch.empty_like(opac), torch.empty_like(mus))
    if C * N == 0:
        return means2d, cov2d, radii, conics, mus, opac, payload, outs
    sfx = _suffix(means, "project_pack_fwd")
    z = (None,) * 5 if outs is None else outs
    with torch.cuda.device(dev):
        _call(f"r2s_project_pack_fwd_{sfx}", _ptr(means), _ptr(covars), _ptr(opacities),
              _ptr(viewmats), _ptr(Ks), int(img_w), int(img_h), float(eps2d),
              float(radius_clip), _ptr(means2d), _ptr(cov2d), _ptr(radii), _ptr(conics),
              _ptr(mus), _ptr(opac), _ptr(payload), *[_ptr(t) for t in z], C, N, _stream(dev))
    return means2d, cov2d, radii, conics, mus, opac, payload, outs


def project_gaussians_bwd(means: Tensor, covars: Tensor, viewmats: Tensor, Ks: Tensor,
                          img_w: int, img_h: int, eps2d: float, cov2d: Tensor, conics: Tensor,
                          mus: Tensor, v_means2d: Tensor, v_conics: Tensor,
                          v_mus: Tensor) -> Tuple[Tensor, Tensor]:
    """Fused conics_mu_bwd + world_to_image_projection_bwd (explicit.py:299-316)."""
    for t, n in ((means, "means"), (covars, "covars"), (viewmats, "viewmats"), (Ks, "Ks"),
                 (cov2d, "cov2d_3x3"), (conics, "conics"), (mus, "mus"),
                 (v_means2d, "v_means2d"), (v_conics, "v_conics"), (v_mus, "v_mus")):
        _check_input(t, n)
    C, N = _check_cameras(means, covars, viewmats, Ks)
    for t, shape, n in ((cov2d, (C, N, 6), "cov2d_3x3"), (conics, (C, N, 3), "conics"),
                        (mus, (C, N), "mus"), (v_means2d, (C, N, 2), "v_means2d"),
                        (v_conics, (C, N, 3), "v_conics"), (v_mus, (C, N), "v_mus")):
        _check(tuple(t.shape) == shape, f"{n} shape must be {list(shape)}")
    dev, dt = means.device, means.dtype
    v_means = torch.empty((N, 3), dtype=dt, device=dev)
    v_covars = torch.empty((N, 6), dtype=dt, device=dev)
    if N == 0:
        return v_means, v_covars
    sfx = _suffix(means, "project_gaussians_bwd")
    with torch.cuda.device(dev):
        _call(f"r2s_project_gaussians_bwd_{sfx}", _ptr(means), _ptr(covars), _ptr(viewmats),
              _ptr(Ks), int(img_w), int(img_h), float(eps2d), _ptr(cov2d), _ptr(conics),
              _ptr(mus), _ptr(v_means2d), _ptr(v_conics), _ptr(v_mus), _ptr(v_means),
              _ptr(v_covars), C, N, _stream(dev))
    return v_means, v_covars


def explicit_backward_tail(means: Tensor, covars: Tensor, viewmats: Tensor, Ks: Tensor,
                           img_w: int, img_h: int, eps2d: float, cov2d: Tensor, conics: Tensor,
                           mus: Tensor, v_means2d: Tensor, v_conics: Tensor, v_mus: Tensor,
                           add_means: Optional[Tensor], add_covars: Optional[Tensor],
                           quats: Tensor, raw_scales: Tensor, scale_min: float,
                           scale_max: float, raw_opacities: Tensor, v_opacity_cn: Tensor,
                           v_opacity_3d: Optional[Tensor]
                           ) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    """project_gaussians_bwd (plus add_means / add_covars), parameter_transform_bwd
    of the summed covariance gradient and opacity_bwd in one pass:
    (v_means [N,3], v_quats [N,4], v_raw_scales [N,3], v_raw_opacities [N]),
    bit-identical to the three ops in turn (explicit.py:299-316,
    ParameterTransformBwd.cu:66-245)."""
    for t, n in ((means, "means"), (covars, "covars"), (viewmats, "viewmats"), (Ks, "Ks"),
                 (cov2d, "cov2d_3x3"), (conics, "conics"), (mus, "mus"),
                 (v_means2d, "v_means2d"), (v_conics, "v_conics"), (v_mus, "v_mus"),
                 (quats, "quats"), (raw_scales, "raw_scales"),
                 (raw_opacities, "raw_opacities"), (v_opacity_cn, "v_opacity_cn")):
        _check_input(t, n)
    C, N = _check_cameras(means, covars, viewmats, Ks)
    _check(C >= 1, "explicit_backward_tail needs at least one view")
    for t, shape, n in ((cov2d, (C, N, 6), "cov2d_3x3"), (conics, (C, N, 3), "conics"),
                        (mus, (C, N), "mus"), (v_means2d, (C, N, 2), "v_means2d"),
                        (v_conics, (C, N, 3), "v_conics"), (v_mus, (C, N), "v_mus"),
                        (quats, (N, 4), "quats"), (raw_scales, (N, 3), "raw_scales"),
                        (raw_opacities, (N,), "raw_opacities"),
                        (v_opacity_cn, (C, N), "v_opacity_cn")):
        _check(tuple(t.shape) == shape, f"{n} shape must be {list(shape)}")
    _check((add_means is None) == (add_covars is None),
           "add_means and add_covars must be given together")
    for t, shape, n in ((add_means, (N, 3), "add_means"), (add_covars, (N, 6), "add_covars"),
                        (v_opacity_3d, (N,), "v_opacity_3d")):
        if t is not None:
            _check_input(t, n)
            _check(tuple(t.shape) == shape, f"{n} shape must be {list(shape)}")
    dev, dt = means.device, means.dtype
    for t in (covars, viewmats, Ks, cov2d, conics, mus, v_means2d, v_conics, v_mus, add_means,
              add_covars, quats, raw_scales, raw_opacities, v_opacity_cn, v_opacity_3d):
        _check(t is None or (t.dtype == dt and t.device == dev),
               "explicit_backward_tail inputs must share one dtype and device")
    v_means = torch.empty((N, 3), dtype=dt, device=dev)
    v_quats = torch.empty((N, 4), dtype=dt, device=dev)
    v_raw_scales = torch.empty((N, 3), dtype=dt, device=dev)
    v_raw_opac = torch.empty((N,), dtype=dt, device=dev)
    if N == 0:
        return v_means, v_quats, v_raw_scales, v_raw_opac
    sfx = _suffix(means, "explicit_backward_tail")
    with torch.cuda.device(dev):
        _call(f"r2s_explicit_backward_tail_{sfx}", _ptr(means), _ptr(covars), _ptr(viewmats),
              _ptr(Ks), int(img_w), int(img_h), float(eps2d), _ptr(cov2d), _ptr(conics),
              _ptr(mus), _ptr(v_means2d), _ptr(v_conics), _ptr(v_mus), _ptr(add_means),
              _ptr(add_covars), _ptr(quats), _ptr(raw_scales), float(scale_min),
              float(scale_max), _ptr(raw_opacities), _ptr(v_opacity_cn), _ptr(v_opacity_3d),
              _ptr(v_means), _ptr(v_quats), _ptr(v_raw_scales), _ptr(v_raw_opac), C, N,
              _stream(dev))
    return v_means, v_quats, v_raw_scales, v_raw_opac


# ---------------------------------------------------------------- binning --

def bin_tiles_2d(means2d: Tensor, radii: Tensor, tile_size: int, n_tiles_dim1: int,
                 n_tiles_dim0: int, keep_ids: bool = True) -> TileLists:
    """IsectTiles.cpp:31-170: the records of every (view, Gaussian, tile) overlap,
    sorted by (tile key, emission index), with their emission order.
    keep_ids=False: the int64 keys are not stored (lists.keys is None; the
    backward ops find each record's key from tile_offsets)."""
    _check_input(means2d, "means2d")
    _check_input(radii, "radii")
    _check(means2d.dim() == 3, "means2d must be 3D [C, N, 2]")
    _check(radii.dim() == 2 or (radii.dim() == 3 and radii.size(2) == 2),
           "radii must be 2D [C, N] or 3D [C, N, 2]")
    _check(means2d.size(2) == 2, "means2d last dim must be 2")
    _check(means2d.size(0) == radii.size(0), "C dimension must match")
    _check(means2d.size(1) == radii.size(1), "N dimension must match")
    _check(radii.dtype == torch.int32, "radii must be int32")
    C, N = means2d.size(0), means2d.size(1)
    dev = means2d.device
    tw, th, ts = int(n_tiles_dim1), int(n_tiles_dim0), int(tile_size)
    tiles_per_gauss = torch.empty((C, N), dtype=torch.int32, device=dev)
    empty = TileLists(tiles_per_gauss, torch.empty((0,), dtype=torch.int64, device=dev),
                      torch.empty((0,), dtype=torch.int32, device=dev), None, None)
    if C * N == 0:
        return empty
    lib = _lib()
    sfx = _suffix(means2d, "isect_tiles")
    rect = 1 if radii.dim() == 3 else 0
    with torch.cuda.device(dev):
        st = _stream(dev)
        offsets = torch.empty((C * N + 1,), dtype=torch.int64, device=dev)
        ws = _workspace(lib.r2s_isect_workspace_bytes(C * N, 0, 0), dev)
        _call(f"r2s_isect_count_2d_{sfx}", _ptr(means2d), _ptr(radii), rect, C, N, ts, tw, th,
              _ptr(tiles_per_gauss), _ptr(offsets), _ptr(ws), ws.numel(), st)

        tile_offsets = torch.empty((C, th, tw), dtype=torch.int32, device=dev)

        def launch(cap, end_bit, outs, ws):
            _call(f"r2s_isect_emit_sort_2d_{sfx}", _ptr(means2d), _ptr(radii), rect, C, N, ts,
                  tw, th, _ptr(offsets), cap, end_bit, *[_ptr(t) for t in outs],
                  _ptr(tile_offsets), _ptr(ws), ws.numel(), st)

        res = _emit_and_sort(launch, offsets, C * N, C * tw * th, "isect_tiles", dev, "2d",
                             keep_ids=keep_ids)
    if res is None:
        return empty
    return TileLists(tiles_per_gauss, *res, tile_offsets)


def isect_tiles(means2d: Tensor, radii: Tensor, tile_size: int, n_tiles_dim1: int,
                n_tiles_dim0: int) -> Tuple[Tensor, Tensor, Tensor]:
    """IsectTiles.cpp:31-170 -> (tiles_per_gauss [C,N], isect_ids i64, flatten_ids i32)."""
    lists = bin_tiles_2d(means2d, radii, tile_size, n_tiles_dim1, n_tiles_dim0)
    _remember_emission(lists, means2d.size(0) * int(n_tiles_dim1) * int(n_tiles_dim0))
    return lists.tiles_per_gauss, lists.isect_ids, lists.flatten_ids


def keys_from_offsets(tile_offsets: Tensor, n_isects: int) -> Tensor:
    """The sorted int64 keys of a list of n_isects records from its
    tile_offsets (each key's first index): the inverse of
    isect_offset_encode / isect_offset_encode_3d."""
    _check_input(tile_offsets, "tile_offsets")
    _check(tile_offsets.dtype == torch.int32, "tile_offsets must be int32")
    dev = tile_offsets.device
    keys = torch.empty((int(n_isects),), dtype=torch.int64, device=dev)
    if keys.numel() > 0:
        with torch.cuda.device(dev):
            _call("r2s_isect_keys_from_offsets", _ptr(tile_offsets), tile_offsets.numel(),
                  keys.numel(), _ptr(keys), _stream(dev))
    return keys


def isect_offset_encode(isect_ids: Tensor, C: int, n_tiles_dim1: int,
                        n_tiles_dim0: int) -> Tensor:
    """IsectTiles.cpp:176-215 -> tile_offsets [C, n_tiles_dim0, n_tiles_dim1] int32."""
    _check_input(isect_ids, "isect_ids")
    _check(isect_ids.dtype == torch.int64, "isect_ids must be int64")
    dev = isect_ids.device
    C, tw, th = int(C), int(n_tiles_dim1), int(n_tiles_dim0)
    offsets = torch.empty((C, th, tw), dtype=torch.int32, device=dev)
    if offsets.numel() == 0:
        return offsets
    with torch.cuda.device(dev):
        _call("r2s_isect_offset_encode", _ptr(isect_ids), isect_ids.numel(), C * tw * th,
              _ptr(offsets), _stream(dev))
    return offsets


def bin_tiles_3d(means3d: Tensor, radii: Tensor, tile_size: int, n_tiles_dim2: int,
                 n_tiles_dim1: int, n_tiles_dim0: int,
                 max_records: Optional[int] = None, keep_ids: bool = True) -> Optional[TileLists]:
    """IsectTiles3D.cpp:31-162: the (Gaussian, brick) records, sorted by
    (brick key, emission index), with their emission order.  With
    ``max_records``, None when there would be more records than that (the
    caller then bins the volume in z-slabs, bin_tiles_3d_slab).  keep_ids as
    for bin_tiles_2d."""
    _check_input(means3d, "means3d")
    _check_input(radii, "radii")
    _check(means3d.dim() == 2, "means3d must be 2D [N, 3]")
    _check(radii.dim() == 2, "radii must be 2D [N, 3]")
    _check(means3d.size(1) == 3, "means3d last dim must be 3")
    _check(radii.size(1) == 3, "radii last dim must be 3")
    _check(means3d.size(0) == radii.size(0), "N dimension must match")
    _check(radii.dtype == torch.int32, "radii must be int32")
    N = means3d.size(0)
    dev = means3d.device
    n2, n1, n0, ts = int(n_tiles_dim2), int(n_tiles_dim1), int(n_tiles_dim0), int(tile_size)
    tiles_per_gauss = torch.empty((N,), dtype=torch.int32, device=dev)
    empty = TileLists(tiles_per_gauss, torch.empty((0,), dtype=torch.int64, device=dev),
                      torch.empty((0,), dtype=torch.int32, device=dev), None, None)
    if N == 0:
        return empty
    lib = _lib()
    sfx = _suffix(means3d, "isect_tiles_3d")
    with torch.cuda.device(dev):
        st = _stream(dev)
        offsets = torch.empty((N + 1,), dtype=torch.int64, device=dev)
        ws = _workspace(lib.r2s_isect_workspace_bytes(N, 0, 0), dev)
        _call(f"r2s_isect_count_3d_{sfx}", _ptr(means3d), _ptr(radii), N, ts, n2, n1, n0,
              _ptr(tiles_per_gauss), _ptr(offsets), _ptr(ws), ws.numel(), st)

        tile_offsets = torch.empty((n0, n1, n2), dtype=torch.int32, device=dev)

        def launch(cap, end_bit, outs, ws):
            _call(f"r2s_isect_emit_sort_3d_{sfx}", _ptr(means3d), _ptr(radii), N, ts, n2, n1,
                  n0, _ptr(offsets), cap, end_bit, *[_ptr(t) for t in outs],
                  _ptr(tile_offsets), _ptr(ws), ws.numel(), st)

        # IsectTiles3D.cpp:96 reads the count back here.
        res = _emit_and_sort(launch, offsets, N, n2 * n1 * n0, "isect_tiles_3d", dev, "3d",
                             max_records, keep_ids=keep_ids)
    if res is TOO_MANY:
        return None
    if res is None:
        return empty
    return TileLists(tiles_per_gauss, *res, tile_offsets)


def isect_tiles_3d(means3d: Tensor, radii: Tensor, tile_size: int, n_tiles_dim2: int,
                   n_tiles_dim1: int, n_tiles_dim0: int) -> Tuple[Tensor, Tensor, Tensor]:
    """IsectTiles3D.cpp:31-162 -> (tiles_per_gauss [N], isect_ids i64, flatten_ids i32)."""
    lists = bin_tiles_3d(means3d, radii, tile_size, n_tiles_dim2, n_tiles_dim1, n_tiles_dim0)
    _remember_emission(lists, int(n_tiles_dim2) * int(n_tiles_dim1) * int(n_tiles_dim0))
    return lists.tiles_per_gauss, lists.isect_ids, lists.flatten_ids


def isect_offset_encode_3d(isect_ids: Tensor, n_tiles_dim2: int, n_tiles_dim1: int,
                           n_tiles_dim0: int) -> Tensor:
    """IsectTiles3D.cpp:168-204 -> tile_offsets [n0, n1, n2] int32."""
    _check_input(isect_ids, "isect_ids")
    _check(isect_ids.dtype == torch.int64, "isect_ids must be int64")
    dev = isect_ids.device
    n2, n1, n0 = int(n_tiles_dim2), int(n_tiles_dim1), int(n_tiles_dim0)
    offsets = torch.empty((n0, n1, n2), dtype=torch.int32, device=dev)
    if offsets.numel() == 0:
        return offsets
    with torch.cuda.device(dev):
        _call("r2s_isect_offset_encode", _ptr(isect_ids), isect_ids.numel(), n0 * n1 * n2,
              _ptr(offsets), _stream(dev))
    return offsets


# Z-slabs.  A volume whose brick list would exceed SLAB_RECORDS records (or
# the int32 offsets of the reference's list, 2**31 - 1) is binned, voxelized
# and back-propagated one slab of brick layers (dim0) at a time.  A slab's
# list is the segment of the whole list whose bricks lie in its layers (keys
# relative to its first layer), so the forward is the same per voxel and the
# backward's per-Gaussian sums are added slab by slab.  SLAB_RECORDS bounds
# the memory of one slab: about 70 bytes per record for the lists, the sort
# and the backward rows, 19 GB at 2**28 records.
SLAB_RECORDS = 1 << 28


def layer_counts_3d(means3d: Tensor, radii: Tensor, tile_size: int, n_tiles_dim2: int,
                    n_tiles_dim1: int, n_tiles_dim0: int) -> list:
    """Records of each brick layer (dim0) of the volume's list, on the host."""
    _check_input(means3d, "means3d")
    _check_input(radii, "radii")
    N, n0 = means3d.size(0), int(n_tiles_dim0)
    dev = means3d.device
    counts = torch.empty((max(n0, 1),), dtype=torch.int64, device=dev)
    ws = _workspace(8 * (n0 + 1), dev)
    with torch.cuda.device(dev):
        _call(f"r2s_isect_layer_counts_3d_{_suffix(means3d, 'isect_tiles_3d')}", _ptr(means3d),
              _ptr(radii), N, int(tile_size), int(n_tiles_dim2), int(n_tiles_dim1), n0,
              _ptr(counts), _ptr(ws), ws.numel(), _stream(dev))
    return counts[:n0].tolist()


def plan_slabs(layer_counts, limit: Optional[int] = None) -> list:
    """Consecutive brick-layer ranges [z0, z1) of at most ``limit`` records
    each (default: SLAB_RECORDS as it is at the call; a layer above the limit
    on its own; one above the int32 offset range raises RuntimeError)."""
    if limit is None:
        limit = SLAB_RECORDS
    slabs, z0, run = [], 0, 0
    for z, c in enumerate(layer_counts):
        _check_record_count(int(c), "isect_tiles_3d (one brick layer)")
        if z > z0 and run + c > limit:
            slabs.append((z0, z))
            z0, run = z, 0
        run += int(c)
    if len(layer_counts) > z0:
        slabs.append((z0, len(layer_counts)))
    return slabs


def bin_tiles_3d_slab(means3d: Tensor, radii: Tensor, tile_size: int, n_tiles_dim2: int,
                      n_tiles_dim1: int, n_tiles_dim0: int, z0: int, z1: int,
                      keep_ids: bool = True) -> Tuple[TileLists, Tensor]:
    """(lists, tile_offsets [z1 - z0, n1, n2]) of the brick layers [z0, z1):
    the records of the whole volume's list (bin_tiles_3d) whose brick lies in
    those layers, in the same order, with keys relative to layer z0.
    keep_ids as for bin_tiles_2d."""
    _check_input(means3d, "means3d")
    _check_input(radii, "radii")
    _check(means3d.dim() == 2 and means3d.size(1) == 3, "means3d must be 2D [N, 3]")
    _check(radii.dim() == 2 and radii.size(1) == 3 and radii.dtype == torch.int32,
           "radii must be int32 [N, 3]")
    N = means3d.size(0)
    dev = means3d.device
    n2, n1, n0, ts = int(n_tiles_dim2), int(n_tiles_dim1), int(n_tiles_dim0), int(tile_size)
    z0, z1 = int(z0), int(z1)
    _check(0 <= z0 <= z1 <= n0, f"brick layers [{z0}, {z1}) outside [0, {n0})")
    n_keys = (z1 - z0) * n1 * n2
    lib = _lib()
    sfx = _suffix(means3d, "isect_tiles_3d")
    tpg = torch.empty((N,), dtype=torch.int32, device=dev)
    offs = torch.empty((z1 - z0, n1, n2), dtype=torch.int32, device=dev)
    empty = TileLists(tpg, torch.empty((0,), dtype=torch.int64, device=dev),
                      torch.empty((0,), dtype=torch.int32, device=dev), None, None)
    with torch.cuda.device(dev):
        st = _stream(dev)
        offsets = torch.empty((N + 1,), dtype=torch.int64, device=dev)
        ws = _workspace(lib.r2s_isect_workspace_bytes(N, 0, 0), dev)
        _call(f"r2s_isect_count_3d_slab_{sfx}", _ptr(means3d), _ptr(radii), N, ts, n2, n1, n0,
              z0, z1, _ptr(tpg), _ptr(offsets), _ptr(ws), ws.numel(), st)
        n = int(offsets[N].item())
        _check_record_count(n, "isect_tiles_3d (z-slab)")
        if n == 0 or n_keys == 0:
            offs.zero_()
            return empty, offs
        end_bit = _end_bit(n_keys)
        outs = (torch.empty((n,), dtype=torch.int64, device=dev) if keep_ids else None,
                torch.empty((n,), dtype=torch.int32, device=dev),
                torch.empty((n,), dtype=torch.int32, device=dev),
                torch.empty((n,), dtype=torch.int32, device=dev))
        ws = _workspace(lib.r2s_isect_workspace_bytes(0, n, end_bit), dev)
        _call(f"r2s_isect_emit_sort_3d_slab_{sfx}", _ptr(means3d), _ptr(radii), N, ts, n2, n1, n0,
              z0, z1, _ptr(offsets), n, end_bit, *[_ptr(t) for t in outs], _ptr(offs), _ptr(ws),
              ws.numel(), st)
    return TileLists(tpg, *outs, offs), offs


def voxelize_slab(means3d: Tensor, conics: Tensor, opacities: Tensor, tile_offsets: Tensor,
                  lists: TileLists, volume: Tensor, tile_size: int, z0: int) -> None:
    """Writes the voxel slices of the brick layers [z0, z0 + nz) of ``volume``
    [dim0, dim1, dim2] from their slab's lists (VoxelizeToVoxelsFwd.cu:69-221)."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (volume, "volume")):
        _check_input(t, n)
    N = _check_voxel(means3d, conics, opacities, tile_offsets, lists.flatten_ids)
    d0, d1, d2 = volume.shape
    nz, n1, n2 = tile_offsets.shape
    dev = means3d.device
    with torch.cuda.device(dev):
        _call(f"r2s_voxelize_fwd_slab_{_suffix(means3d, 'voxelize_to_voxels_fwd')}",
              _ptr(means3d), _ptr(conics), _ptr(opacities), _ptr(tile_offsets),
              _ptr(lists.flatten_ids) if lists.flatten_ids.numel() else None,
              lists.flatten_ids.numel(), N, d2, d1, d0, int(tile_size), n2, n1, int(z0), nz,
              _ptr(volume), _stream(dev))


def voxel_backward_slab(means3d: Tensor, conics: Tensor, opacities: Tensor,
                        tile_offsets: Tensor, lists: TileLists, v_volume: Tensor,
                        tile_size: int, z0: int):
    """The voxelizer's VJP over one slab's lists (VoxelizeToVoxelsBwd.cu:71-441,
    two-pass): (v_means3d, v_conics, v_opacities) of that slab's records,
    zero for Gaussians without records in it."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (v_volume, "v_render_output")):
        _check_input(t, n)
    N = _check_voxel(means3d, conics, opacities, tile_offsets, lists.flatten_ids)
    d0, d1, d2 = v_volume.shape
    nz, n1, n2 = tile_offsets.shape
    n = lists.flatten_ids.numel()
    v_m, v_c, v_o = (torch.empty_like(t) for t in (means3d, conics, opacities))
    dev = means3d.device
    with torch.cuda.device(dev):
        if n == 0:
            for t in (v_m, v_c, v_o):
                t.zero_()
            return v_m, v_c, v_o
        ws = _workspace(_lib().r2s_voxelize_bwd_workspace_bytes(n, means3d.element_size()), dev)
        _call(f"r2s_voxelize_bwd_emit_slab_{_suffix(means3d, 'voxelize_to_voxels_bwd')}",
              _ptr(means3d), _ptr(conics), _ptr(opacities), _ptr(tile_offsets),
              _ptr(lists.keys), _ptr(lists.flatten_ids), _ptr(lists.emit_ids),
              _ptr(lists.isect_src), n, _ptr(v_volume), N, d2, d1, d0, int(tile_size), n2, n1,
              int(z0), nz, _ptr(v_m), _ptr(v_c), _ptr(v_o), _ptr(ws), ws.numel(), _stream(dev))
    return v_m, v_c, v_o


# -------------------------------------------------------------- rasterizer --

def _check_raster(means2d, conics, opacities, mus, tile_offsets, flatten_ids):
    _check(means2d.dim() == 3, "means2d must be 3D [C, N, 2]")
    _check(conics.dim() == 3, "conics must be 3D [C, N, 3]")
    _check(opacities.dim() == 2, "opacities must be 2D [C, N]")
    _check(mus.dim() == 2, "mus must be 2D [C, N]")
    _check(tile_offsets.dim() == 3, "tile_offsets must be 3D [C, n_tiles_dim0, n_tiles_dim1]")
    _check(flatten_ids.dim() == 1, "flatten_ids must be 1D [n_isects]")
    _check(means2d.size(2) == 2, "means2d last dim must be 2")
    _check(conics.size(2) == 3, "conics last dim must be 3")
    C, N = means2d.size(0), means2d.size(1)
    _check(conics.size(0) == C and conics.size(1) == N, "conics shape must match means2d [C, N, 3]")
    _check(opacities.size(0) == C and opacities.size(1) == N, "opacities shape must match [C, N]")
    _check(mus.size(0) == C and mus.size(1) == N, "mus shape must match [C, N]")
    _check(tile_offsets.size(0) == C, "tile_offsets C dimension must match")
    _check(tile_offsets.dtype == torch.int32 and flatten_ids.dtype == torch.int32,
           "tile_offsets and flatten_ids must be int32")
    for t in (conics, opacities, mus):
        _check(t.dtype == means2d.dtype, "means2d, conics, opacities and mus must share a dtype")
    return C, N


def rasterize_to_pixels_fwd(means2d: Tensor, conics: Tensor, opacities: Tensor, mus: Tensor,
                            tile_offsets: Tensor, flatten_ids: Tensor, dim1: int, dim0: int,
                            tile_size: int) -> Tensor:
    """RasterizeToPixels.cpp:25-114 -> image [C, dim0, dim1]."""
    for t, n in ((means2d, "means2d"), (conics, "conics"), (opacities, "opacities"),
                 (mus, "mus"), (tile_offsets, "tile_offsets"), (flatten_ids, "flatten_ids")):
        _check_input(t, n)
    C, N = _check_raster(means2d, conics, opacities, mus, tile_offsets, flatten_ids)
    W, H, ts = int(dim1), int(dim0), int(tile_size)
    th, tw = tile_offsets.size(1), tile_offsets.size(2)
    dev = means2d.device
    out = torch.empty((C, H, W), dtype=means2d.dtype, device=dev)
    n_isects = flatten_ids.numel()
    if C == 0 or N == 0 or n_isects == 0:
        return out.zero_()
    sfx = _suffix(means2d, "rasterize_to_pixels_fwd")
    lib = _lib()
    with torch.cuda.device(dev):
        nbytes = lib.r2s_rasterize_workspace_bytes(C * tw * th, n_isects, ts,
                                                   means2d.element_size())
        ws = _workspace(nbytes, dev) if nbytes > 0 else None
        _call(f"r2s_rasterize_fwd_{sfx}", _ptr(means2d), _ptr(conics), _ptr(opacities),
              _ptr(mus), _ptr(tile_offsets), _ptr(flatten_ids), n_isects, C, N, W, H, ts, tw, th,
              _ptr(out), _ptr(ws), 0 if ws is None else ws.numel(), _stream(dev))
    return out


_LOOKUP = object()  # emission order: look it up on flatten_ids (the wrapper path)


def _resolve_emission(emission, flatten_ids: Tensor, n_keys: int, op: str):
    if emission is _LOOKUP:
        emit = emission_order(flatten_ids, n_keys)
    else:
        emit = emission
        if emit is not None:
            _check(emit[0].numel() == flatten_ids.numel() and
                   emit[1].numel() == flatten_ids.numel(),
                   f"{op}: emission arrays must have one entry per record")
    _note_path(emit is not None, op)
    return emit


def _raster_bwd(means2d, conics, opacities, mus, tile_offsets, isect_ids, flatten_ids,
                v_render, dim1, dim0, tile_size, absgrad, op, emission=_LOOKUP):
    C, N = _check_raster(means2d, conics, opacities, mus, tile_offsets, flatten_ids)
    _check(v_render.dim() == 3, "v_render_output must be 3D [C, dim0, dim1]")
    W, H, ts = int(dim1), int(dim0), int(tile_size)
    _check(v_render.size(0) == C and v_render.size(1) == H and v_render.size(2) == W,
           "v_render_output shape must be [C, dim0, dim1]")
    th, tw = tile_offsets.size(1), tile_offsets.size(2)
    n_isects = flatten_ids.numel()
    empty = C == 0 or N == 0 or n_isects == 0
    emit = None if empty else _resolve_emission(emission, flatten_ids, C * tw * th, op)
    # The two-pass form stores every output (zero for Gaussians without
    # records); the one-pass form accumulates into zeros.
    alloc = torch.empty_like if emit is not None else torch.zeros_like
    v_means2d = alloc(means2d)
    v_abs = alloc(means2d) if absgrad else None
    v_conics = alloc(conics)
    v_opac = alloc(opacities)
    v_mus = alloc(mus)
    if empty:
        return v_abs, v_means2d, v_conics, v_opac, v_mus
    sfx = _suffix(means2d, op)
    dev = means2d.device
    with torch.cuda.device(dev):
        if emit is not None:
            ws = _workspace(_lib().r2s_rasterize_bwd_workspace_bytes(
                n_isects, C * N, means2d.element_size()), dev)
            _call(f"r2s_rasterize_bwd_emit_{sfx}", _ptr(means2d), _ptr(conics), _ptr(opacities),
                  _ptr(mus), _ptr(tile_offsets), _ptr(isect_ids), _ptr(flatten_ids),
                  _ptr(emit[0]), _ptr(emit[1]), n_isects, _ptr(v_render), C, N, W, H, ts, tw,
                  th, _ptr(v_abs), _ptr(v_means2d), _ptr(v_conics), _ptr(v_opac), _ptr(v_mus),
                  _ptr(ws), ws.numel(), _stream(dev))
        else:
            _call(f"r2s_rasterize_bwd_{sfx}", _ptr(means2d), _ptr(conics), _ptr(opacities),
                  _ptr(mus), _ptr(tile_offsets), _ptr(isect_ids), _ptr(flatten_ids), n_isects,
                  _ptr(v_render), C, N, W, H, ts, tw, th, _ptr(v_abs), _ptr(v_means2d),
                  _ptr(v_conics), _ptr(v_opac), _ptr(v_mus), _stream(dev))
    return v_abs, v_means2d, v_conics, v_opac, v_mus


def rasterize_to_pixels_bwd(means2d: Tensor, conics: Tensor, opacities: Tensor, mus: Tensor,
                            tile_offsets: Tensor, flatten_ids: Tensor, v_render_output: Tensor,
                            dim1: int, dim0: int, tile_size: int, absgrad: bool):
    """RasterizeToPixels.cpp:122-222 (pixel mode) ->
    (v_means2d_abs or None, v_means2d, v_conics, v_opacities, v_mus)."""
    for t, n in ((means2d, "means2d"), (conics, "conics"), (opacities, "opacities"),
                 (mus, "mus"), (tile_offsets, "tile_offsets"), (flatten_ids, "flatten_ids"),
                 (v_render_output, "v_render_output")):
        _check_input(t, n)
    return _raster_bwd(means2d, conics, opacities, mus, tile_offsets, None, flatten_ids,
                       v_render_output, dim1, dim0, tile_size, bool(absgrad),
                       "rasterize_to_pixels_bwd")


def rasterize_to_pixels_bwd_per_gaussian(means2d: Tensor, conics: Tensor, opacities: Tensor,
                                         mus: Tensor, tile_offsets: Tensor, isect_ids: Tensor,
                                         flatten_ids: Tensor, v_render_output: Tensor, dim1: int,
                                         dim0: int, tile_size: int, absgrad: bool):
    """RasterizeToPixels.cpp:226-317 (primitive mode, the default)."""
    for t, n in ((means2d, "means2d"), (conics, "conics"), (opacities, "opacities"),
                 (mus, "mus"), (tile_offsets, "tile_offsets"), (isect_ids, "isect_ids"),
                 (flatten_ids, "flatten_ids"), (v_render_output, "v_render_output")):
        _check_input(t, n)
    _check(isect_ids.dim() == 1, "isect_ids must be 1D [n_isects]")
    _check(isect_ids.dtype == torch.int64, "isect_ids must be int64")
    _check(isect_ids.size(0) == flatten_ids.size(0),
           "isect_ids and flatten_ids must have the same length")
    return _raster_bwd(means2d, conics, opacities, mus, tile_offsets, isect_ids, flatten_ids,
                       v_render_output, dim1, dim0, tile_size, bool(absgrad),
                       "rasterize_to_pixels_bwd_per_gaussian")


def raster_backward(means2d: Tensor, conics: Tensor, opacities: Tensor, mus: Tensor,
                    tile_offsets: Tensor, lists: TileLists, v_image: Tensor, img_w: int,
                    img_h: int, tile_size: int, absgrad: bool):
    """The rasterizer's VJP over lists returned by :func:`bin_tiles_2d`, with
    their emission order passed explicitly (both reference modes compute the
    same sums; RasterizeToPixels.cpp:122-317) ->
    (v_means2d_abs or None, v_means2d, v_conics, v_opacities, v_mus)."""
    for t, n in ((means2d, "means2d"), (conics, "conics"), (opacities, "opacities"),
                 (mus, "mus"), (tile_offsets, "tile_offsets"), (lists.flatten_ids, "flatten_ids"),
                 (v_image, "v_render_output")):
        _check_input(t, n)
    return _raster_bwd(means2d, conics, opacities, mus, tile_offsets, lists.keys,
                       lists.flatten_ids, v_image, img_w, img_h, tile_size, bool(absgrad),
                       "raster_backward", emission=lists.emission)


# The packed passes of r2splat.ops: the mean, conic, o mu and the alpha
# test's limit of every (view, Gaussian) pair packed once per call into 32
# bytes (float32), read by the forward and the two-pass backward as one load
# per record instead of four arrays' lines.

PACKED_TILE_SIZES = (8, 16, 32)


def raster_pack(means2d: Tensor, conics: Tensor, opacities: Tensor, mus: Tensor,
                zero_outputs: bool = False, absgrad: bool = False):
    """-> (payload [C*N*8] of the inputs' dtype, outputs): with
    ``zero_outputs`` the raster backward's five outputs (v_means2d_abs only
    with ``absgrad``), zeroed by the same launch, else None."""
    for t, n in ((means2d, "means2d"), (conics, "conics"), (opacities, "opacities"),
                 (mus, "mus")):
        _check_input(t, n)
    _check(means2d.dim() == 3 and means2d.size(2) == 2, "means2d must be [C, N, 2]")
    C, N = means2d.size(0), means2d.size(1)
    _check(conics.shape == (C, N, 3) and opacities.shape == (C, N) and mus.shape == (C, N),
           "conics [C,N,3], opacities and mus [C,N] must match means2d")
    _check(conics.dtype == means2d.dtype and opacities.dtype == means2d.dtype
           and mus.dtype == means2d.dtype, "means2d, conics, opacities and mus must share a dtype")
    dev = means2d.device
    payload = torch.empty((C * N * 8,), dtype=means2d.dtype, device=dev)
    outs = None
    if zero_outputs:
        outs = (torch.empty_like(means2d) if absgrad else None, torch.empty_like(means2d),
                torch.empty_like(conics), torch.empty_like(opacities), torch.empty_like(mus))
    if C * N == 0:
        return payload, outs
    sfx = _suffix(means2d, "rasterize_pack")
    z = (None,) * 5 if outs is None else outs
    with torch.cuda.device(dev):
        _call(f"r2s_rasterize_pack_{sfx}", _ptr(means2d), _ptr(conics), _ptr(opacities),
              _ptr(mus), C, N, _ptr(payload), *[_ptr(t) for t in z], _stream(dev))
    return payload, outs


def rasterize_packed(payload: Tensor, tile_offsets: Tensor, flatten_ids: Tensor, C: int, N: int,
                     img_w: int, img_h: int, tile_size: int) -> Tensor:
    """The rasterizer forward over a payload of :func:`raster_pack` (tile
    sizes 8, 16 and 32) -> image [C, img_h, img_w], the same as
    rasterize_to_pixels_fwd's bit for bit."""
    for t, n in ((payload, "payload"), (tile_offsets, "tile_offsets"),
                 (flatten_ids, "flatten_ids")):
        _check_input(t, n)
    C, N, W, H, ts = int(C), int(N), int(img_w), int(img_h), int(tile_size)
    _check(ts in PACKED_TILE_SIZES, "the packed rasterizer takes tile sizes 8, 16 and 32")
    _check(payload.numel() == C * N * 8, "payload must hold 8 values per (view, Gaussian)")
    _check(tile_offsets.dim() == 3 and tile_offsets.size(0) == C, "tile_offsets must be [C,th,tw]")
    th, tw = tile_offsets.size(1), tile_offsets.size(2)
    dev = payload.device
    out = torch.empty((C, H, W), dtype=payload.dtype, device=dev)
    n_isects = flatten_ids.numel()
    if C == 0 or N == 0 or n_isects == 0:
        return out.zero_()
    sfx = _suffix(payload, "rasterize_packed")
    lib = _lib()
    with torch.cuda.device(dev):
        nbytes = lib.r2s_rasterize_workspace_bytes(C * tw * th, n_isects, ts,
                                                   payload.element_size())
        ws = _workspace(nbytes, dev) if nbytes > 0 else None
        _call(f"r2s_rasterize_fwd_packed_{sfx}", _ptr(payload), _ptr(tile_offsets),
              _ptr(flatten_ids), n_isects, C, N, W, H, ts, tw, th, _ptr(out), _ptr(ws),
              0 if ws is None else ws.numel(), _stream(dev))
    return out


def raster_backward_packed(payload: Tensor, opacities: Tensor, mus: Tensor,
                           tile_offsets: Tensor, lists: TileLists, v_image: Tensor, img_w: int,
                           img_h: int, tile_size: int, absgrad: bool, zeroed_outputs=None):
    """:func:`raster_backward` over a payload of :func:`raster_pack` (the
    two-pass kernels without their own pack launch) -> (v_means2d_abs or None,
    v_means2d, v_conics, v_opacities, v_mus).  ``zeroed_outputs``: the
    outputs raster_pack zeroed (written in place and returned), else new."""
    for t, n in ((payload, "payload"), (opacities, "opacities"), (mus, "mus"),
                 (tile_offsets, "tile_offsets"), (lists.flatten_ids, "flatten_ids"),
                 (v_image, "v_render_output")):
        _check_input(t, n)
    _check(opacities.dim() == 2, "opacities must be [C, N]")
    C, N = opacities.size(0), opacities.size(1)
    W, H, ts = int(img_w), int(img_h), int(tile_size)
    _check(payload.numel() == C * N * 8, "payload must hold 8 values per (view, Gaussian)")
    _check(v_image.shape == (C, H, W), "v_render_output shape must be [C, dim0, dim1]")
    dev, dt = payload.device, payload.dtype
    zeroed = zeroed_outputs is not None and (zeroed_outputs[0] is not None or not absgrad)
    if zeroed:
        outs = (zeroed_outputs[0] if absgrad else None,) + tuple(zeroed_outputs[1:])
    else:
        outs = (torch.empty((C, N, 2), dtype=dt, device=dev) if absgrad else None,
                torch.empty((C, N, 2), dtype=dt, device=dev),
                torch.empty((C, N, 3), dtype=dt, device=dev),
                torch.empty((C, N), dtype=dt, device=dev),
                torch.empty((C, N), dtype=dt, device=dev))
    if C * N == 0:
        return outs
    n_isects = lists.flatten_ids.numel()
    th, tw = tile_offsets.size(1), tile_offsets.size(2)
    if n_isects > 0:
        _check(lists.emission is not None, "raster_backward_packed needs the emission order")
        _note_path(True, "raster_backward_packed")
    emit, src = lists.emission if n_isects > 0 else (None, None)
    sfx = _suffix(payload, "raster_backward_packed")
    with torch.cuda.device(dev):
        nbytes = _lib().r2s_rasterize_bwd_workspace_bytes(n_isects, 0, payload.element_size())
        ws = _workspace(nbytes, dev) if nbytes > 0 else None
        _call(f"r2s_rasterize_bwd_packed_{sfx}", _ptr(payload), _ptr(opacities), _ptr(mus),
              _ptr(tile_offsets), _ptr(lists.keys), _ptr(lists.flatten_ids), _ptr(emit),
              _ptr(src), n_isects, _ptr(v_image), C, N, W, H, ts, tw, th,
              *[_ptr(t) for t in outs], 1 if zeroed else 0, _ptr(ws),
              0 if ws is None else ws.numel(), _stream(dev))
    return outs


# ------------------------------------------------------------ voxelization --

def world_to_volume_mapping_fwd(means: Tensor, covars: Tensor, max_scales: Tensor,
                                ranges: Tensor, centers: Tensor, dim2: int, dim1: int,
                                dim0: int, eps3d: float,
                                radius_clip: float) -> Tuple[Tensor, Tensor, Tensor]:
    """WorldToVolumeMapping.cpp:37-112 -> (means3d [N,3], conics [N,6], radii [N,3])."""
    for t, n in ((means, "means"), (covars, "covars"), (max_scales, "max_scales"),
                 (ranges, "ranges"), (centers, "centers")):
        _check_input(t, n)
    _check(means.dim() == 2 and means.size(1) == 3,
           "means must be 2D [N, 3], got shape ", list(means.shape))
    _check(covars.dim() == 2 and covars.size(1) == 6,
           "covars must be 2D [N, 6], got shape ", list(covars.shape))
    _check(max_scales.dim() == 1, "max_scales must be 1D [N], got dim ", max_scales.dim())
    _check(ranges.dim() == 1 and ranges.size(0) == 3,
           "ranges must be 1D [3], got shape ", list(ranges.shape))
    _check(centers.dim() == 1 and centers.size(0) == 3,
           "centers must be 1D [3], got shape ", list(centers.shape))
    N = means.size(0)
    _check(covars.size(0) == N, "covars batch dim (", covars.size(0), ") doesn't match N=", N)
    _check(max_scales.size(0) == N, "max_scales batch dim (", max_scales.size(0),
           ") doesn't match N=", N)
    dev, dt = means.device, means.dtype
    means3d = torch.empty((N, 3), dtype=dt, device=dev)
    conics = torch.empty((N, 6), dtype=dt, device=dev)
    radii = torch.empty((N, 3), dtype=torch.int32, device=dev)
    if N == 0:
        return means3d, conics, radii
    _check(covars.dtype == dt and ranges.dtype == dt and centers.dtype == dt,
           "means, covars, ranges and centers must share a dtype")
    sfx = _suffix(means, "world_to_volume_mapping_fwd")
    with torch.cuda.device(dev):
        _call(f"r2s_world_to_volume_mapping_fwd_{sfx}", _ptr(means), _ptr(covars),
              _ptr(ranges), _ptr(centers), int(dim2), int(dim1), int(dim0),
              float(eps3d), float(radius_clip), _ptr(means3d), _ptr(conics), _ptr(radii), N,
              _stream(dev))
    return means3d, conics, radii


def world_to_volume_mapping_bwd(means: Tensor, covars: Tensor, ranges: Tensor, centers: Tensor,
                                dim2: int, dim1: int, dim0: int, eps3d: float,
                                v_means3d_v: Tensor, v_conics: Tensor) -> Tuple[Tensor, Tensor]:
    """WorldToVolumeMapping.cpp:119-192 -> (v_means [N,3], v_covars [N,6])."""
    for t, n in ((means, "means"), (covars, "covars"), (ranges, "ranges"), (centers, "centers"),
                 (v_means3d_v, "v_means3d_v"), (v_conics, "v_conics")):
        _check_input(t, n)
    _check(means.dim() == 2 and means.size(1) == 3, "means must be 2D [N, 3]")
    _check(covars.dim() == 2 and covars.size(1) == 6, "covars must be 2D [N, 6]")
    _check(ranges.dim() == 1 and ranges.size(0) == 3, "ranges must be 1D [3]")
    _check(centers.dim() == 1 and centers.size(0) == 3, "centers must be 1D [3]")
    _check(v_means3d_v.dim() == 2 and v_means3d_v.size(1) == 3, "v_means3d_v must be 2D [N, 3]")
    _check(v_conics.dim() == 2 and v_conics.size(1) == 6, "v_conics must be 2D [N, 6]")
    N = means.size(0)
    _check(covars.size(0) == N, "covars shape mismatch")
    _check(v_means3d_v.size(0) == N, "v_means3d_v shape mismatch")
    _check(v_conics.size(0) == N, "v_conics shape mismatch")
    dev, dt = means.device, means.dtype
    v_means = torch.empty((N, 3), dtype=dt, device=dev)
    v_covars = torch.empty((N, 6), dtype=dt, device=dev)
    if N == 0:
        return v_means, v_covars
    _check(all(t.dtype == dt for t in (covars, ranges, centers, v_means3d_v, v_conics)),
           "world_to_volume_mapping_bwd inputs must share a dtype")
    sfx = _suffix(means, "world_to_volume_mapping_bwd")
    with torch.cuda.device(dev):
        _call(f"r2s_world_to_volume_mapping_bwd_{sfx}", _ptr(means), _ptr(covars),
              _ptr(ranges), _ptr(centers), int(dim2), int(dim1), int(dim0),
              float(eps3d), _ptr(v_means3d_v), _ptr(v_conics), _ptr(v_means), _ptr(v_covars), N,
              _stream(dev))
    return v_means, v_covars


def _check_voxel(means3d, conics, opacities, tile_offsets, flatten_ids):
    _check(means3d.dim() == 2, "means3d must be 2D [N, 3]")
    _check(conics.dim() == 2, "conics must be 2D [N, 6]")
    _check(opacities.dim() == 1, "opacities must be 1D [N]")
    _check(tile_offsets.dim() == 3,
           "tile_offsets must be 3D [n_tiles_dim0, n_tiles_dim1, n_tiles_dim2]")
    _check(flatten_ids.dim() == 1, "flatten_ids must be 1D [n_isects]")
    _check(means3d.size(1) == 3, "means3d last dim must be 3")
    _check(conics.size(1) == 6, "conics last dim must be 6")
    N = means3d.size(0)
    _check(conics.size(0) == N, "conics first dim must match N")
    _check(opacities.size(0) == N, "opacities first dim must match N")
    _check(tile_offsets.dtype == torch.int32 and flatten_ids.dtype == torch.int32,
           "tile_offsets and flatten_ids must be int32")
    for t in (conics, opacities):
        _check(t.dtype == means3d.dtype, "means3d, conics and opacities must share a dtype")
    return N


def voxelize_to_voxels_fwd(means3d: Tensor, conics: Tensor, opacities: Tensor,
                           tile_offsets: Tensor, flatten_ids: Tensor, dim2: int, dim1: int,
                           dim0: int, tile_size: int) -> Tensor:
    """VoxelizeToVoxels.cpp:31-108 -> volume [dim0, dim1, dim2]."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (flatten_ids, "flatten_ids")):
        _check_input(t, n)
    N = _check_voxel(means3d, conics, opacities, tile_offsets, flatten_ids)
    d2, d1, d0, ts = int(dim2), int(dim1), int(dim0), int(tile_size)
    n0, n1, n2 = tile_offsets.size(0), tile_offsets.size(1), tile_offsets.size(2)
    dev = means3d.device
    n_isects = flatten_ids.numel()
    if N == 0 or n_isects == 0:
        return torch.zeros((d0, d1, d2), dtype=means3d.dtype, device=dev)
    out = torch.empty((d0, d1, d2), dtype=means3d.dtype, device=dev)
    sfx = _suffix(means3d, "voxelize_to_voxels_fwd")
    with torch.cuda.device(dev):
        _call(f"r2s_voxelize_fwd_{sfx}", _ptr(means3d), _ptr(conics), _ptr(opacities),
              _ptr(tile_offsets), _ptr(flatten_ids), n_isects, N, d2, d1, d0, ts, n2, n1, n0,
              _ptr(out), _stream(dev))
    return out


def voxelize_with_reach(means3d: Tensor, conics: Tensor, opacities: Tensor,
                        tile_offsets: Tensor, flatten_ids: Tensor, dim2: int, dim1: int,
                        dim0: int) -> Tuple[Tensor, Optional[Tensor]]:
    """:func:`voxelize_to_voxels_fwd` at tile size 8 that also returns each
    record's reach mask (the brick rows its alpha-test ellipsoid reaches, one
    int64 per record at its list position) for :func:`voxel_backward` over the
    same inputs and lists (None when there are no records)."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (flatten_ids, "flatten_ids")):
        _check_input(t, n)
    N = _check_voxel(means3d, conics, opacities, tile_offsets, flatten_ids)
    d2, d1, d0 = int(dim2), int(dim1), int(dim0)
    n0, n1, n2 = tile_offsets.size(0), tile_offsets.size(1), tile_offsets.size(2)
    dev = means3d.device
    n_isects = flatten_ids.numel()
    if N == 0 or n_isects == 0:
        return torch.zeros((d0, d1, d2), dtype=means3d.dtype, device=dev), None
    out = torch.empty((d0, d1, d2), dtype=means3d.dtype, device=dev)
    reach = torch.empty(n_isects, dtype=torch.int64, device=dev)
    sfx = _suffix(means3d, "voxelize_to_voxels_fwd")
    with torch.cuda.device(dev):
        _call(f"r2s_voxelize_fwd_reach_{sfx}", _ptr(means3d), _ptr(conics), _ptr(opacities),
              _ptr(tile_offsets), _ptr(flatten_ids), n_isects, N, d2, d1, d0, 8, n2, n1, n0,
              _ptr(out), _ptr(reach), _stream(dev))
    return out, reach


def _voxel_bwd(means3d, conics, opacities, tile_offsets, isect_ids, flatten_ids, v_render,
               dim2, dim1, dim0, tile_size, op, emission=_LOOKUP, reach=None):
    N = _check_voxel(means3d, conics, opacities, tile_offsets, flatten_ids)
    _check(v_render.dim() == 3, "v_render_output must be 3D [dim0, dim1, dim2]")
    d2, d1, d0, ts = int(dim2), int(dim1), int(dim0), int(tile_size)
    n0, n1, n2 = tile_offsets.size(0), tile_offsets.size(1), tile_offsets.size(2)
    n_isects = flatten_ids.numel()
    empty = N == 0 or n_isects == 0
    emit = None if empty else _resolve_emission(emission, flatten_ids, n2 * n1 * n0, op)
    # As in _raster_bwd: the two-pass form stores every output.
    alloc = torch.empty_like if emit is not None else torch.zeros_like
    v_means3d = alloc(means3d)
    v_conics = alloc(conics)
    v_opac = alloc(opacities)
    if empty:
        return v_means3d, v_conics, v_opac
    _check(tuple(v_render.shape) == (d0, d1, d2), "v_render_output shape must be [dim0, dim1, dim2]")
    sfx = _suffix(means3d, op)
    dev = means3d.device
    with torch.cuda.device(dev):
        if emit is not None and reach is not None:
            _check(ts == 8 and reach.dtype == torch.int64 and reach.numel() == n_isects
                   and reach.is_contiguous() and reach.device == dev,
                   "reach masks must come from voxelize_with_reach over these lists")
            ws = _workspace(_lib().r2s_voxelize_bwd_workspace_bytes(n_isects,
                                                                    means3d.element_size()), dev)
            _call(f"r2s_voxelize_bwd_emit_reach_{sfx}", _ptr(means3d), _ptr(conics),
                  _ptr(opacities), _ptr(tile_offsets), _ptr(isect_ids), _ptr(flatten_ids),
                  _ptr(emit[0]), _ptr(emit[1]), n_isects, _ptr(v_render), N, d2, d1, d0, ts,
                  n2, n1, n0, _ptr(reach), _ptr(v_means3d), _ptr(v_conics), _ptr(v_opac),
                  _ptr(ws), ws.numel(), _stream(dev))
        elif emit is not None:
            ws = _workspace(_lib().r2s_voxelize_bwd_workspace_bytes(n_isects,
                                                                    means3d.element_size()), dev)
            _call(f"r2s_voxelize_bwd_emit_{sfx}", _ptr(means3d), _ptr(conics), _ptr(opacities),
                  _ptr(tile_offsets), _ptr(isect_ids), _ptr(flatten_ids), _ptr(emit[0]),
                  _ptr(emit[1]), n_isects, _ptr(v_render), N, d2, d1, d0, ts, n2, n1, n0,
                  _ptr(v_means3d), _ptr(v_conics), _ptr(v_opac), _ptr(ws), ws.numel(),
                  _stream(dev))
        else:
            _call(f"r2s_voxelize_bwd_{sfx}", _ptr(means3d), _ptr(conics), _ptr(opacities),
                  _ptr(tile_offsets), _ptr(isect_ids), _ptr(flatten_ids), n_isects,
                  _ptr(v_render), N, d2, d1, d0, ts, n2, n1, n0, _ptr(v_means3d),
                  _ptr(v_conics), _ptr(v_opac), _stream(dev))
    return v_means3d, v_conics, v_opac


def voxelize_to_voxels_bwd(means3d: Tensor, conics: Tensor, opacities: Tensor,
                           tile_offsets: Tensor, flatten_ids: Tensor, v_render_output: Tensor,
                           dim2: int, dim1: int, dim0: int, tile_size: int):
    """VoxelizeToVoxels.cpp:115-192 (pixel mode) -> (v_means3d, v_conics, v_opacities)."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (flatten_ids, "flatten_ids"),
                 (v_render_output, "v_render_output")):
        _check_input(t, n)
    return _voxel_bwd(means3d, conics, opacities, tile_offsets, None, flatten_ids,
                      v_render_output, dim2, dim1, dim0, tile_size, "voxelize_to_voxels_bwd")


def voxelize_to_voxels_bwd_per_gaussian(means3d: Tensor, conics: Tensor, opacities: Tensor,
                                        tile_offsets: Tensor, isect_ids: Tensor,
                                        flatten_ids: Tensor, v_render_output: Tensor, dim2: int,
                                        dim1: int, dim0: int, tile_size: int):
    """VoxelizeToVoxels.cpp:195-278 (primitive mode, the default)."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (isect_ids, "isect_ids"),
                 (flatten_ids, "flatten_ids"), (v_render_output, "v_render_output")):
        _check_input(t, n)
    _check(isect_ids.dim() == 1, "isect_ids must be 1D")
    _check(isect_ids.dtype == torch.int64, "isect_ids must be int64")
    _check(isect_ids.size(0) == flatten_ids.size(0),
           "isect_ids and flatten_ids must have the same length")
    return _voxel_bwd(means3d, conics, opacities, tile_offsets, isect_ids, flatten_ids,
                      v_render_output, dim2, dim1, dim0, tile_size,
                      "voxelize_to_voxels_bwd_per_gaussian")


def voxel_backward(means3d: Tensor, conics: Tensor, opacities: Tensor, tile_offsets: Tensor,
                   lists: TileLists, v_volume: Tensor, dim2: int, dim1: int, dim0: int,
                   tile_size: int, reach: Optional[Tensor] = None):
    """The voxelizer's VJP over lists returned by :func:`bin_tiles_3d`, with
    their emission order passed explicitly (VoxelizeToVoxels.cpp:115-278) ->
    (v_means3d, v_conics, v_opacities).  ``reach``: the masks
    :func:`voxelize_with_reach` returned for the same inputs and lists (the
    backward then skips the culling setup)."""
    for t, n in ((means3d, "means3d"), (conics, "conics"), (opacities, "opacities"),
                 (tile_offsets, "tile_offsets"), (lists.flatten_ids, "flatten_ids"),
                 (v_volume, "v_render_output")):
        _check_input(t, n)
    return _voxel_bwd(means3d, conics, opacities, tile_offsets, lists.keys,
                      lists.flatten_ids, v_volume, dim2, dim1, dim0, tile_size,
                      "voxel_backward", emission=lists.emission, reach=reach)


# -------------------------------------------------------------- compaction --

def mask_split(mask: Tensor) -> Tuple[Tensor, int]:
    """(indices, n_true): ascending indices of true entries, then of false entries.

    ``indices[:n_true]`` equals ``torch.where(mask)[0]`` and
    ``indices[n_true:]`` equals ``torch.where(~mask)[0]``
    (src/strategies/binary_tree.py:68,101-102,158).
    """
    _check(isinstance(mask, torch.Tensor) and mask.is_cuda, "mask must be a CUDA tensor")
    m = mask.reshape(-1)
    if m.dtype != torch.bool and m.dtype != torch.uint8:
        m = m != 0
    m = m.contiguous().view(torch.uint8)
    n = m.numel()
    dev = m.device
    out = torch.empty((n,), dtype=torch.int64, device=dev)
    count = torch.empty((1,), dtype=torch.int64, device=dev)
    lib = _lib()
    with torch.cuda.device(dev):
        ws = _workspace(lib.r2s_mask_workspace_bytes(n), dev)
        _call("r2s_mask_split", _ptr(m) if n else None, n, _ptr(out) if n else None,
              _ptr(count), _ptr(ws), ws.numel(), _stream(dev))
        n_true = int(count.item())
    return out, n_true


# ------------------------------------------------------------- densify --
#
# One launch rebuilds every column of the Gaussian table (parameters, Adam
# moments, tree buffers, strategy statistics, history archive) for the
# binary-tree strategy's split / duplicate / remove
# (src/strategies/binary_tree.py:17-171, src/utils/ops.py:61-103).
# A column is given as (src, role, extra): `role` is one of the _lib.COL_*
# values; `extra` is the live column appended to a history archive
# (role COL_HISTORY) and None otherwise.

def _densify_table(columns, n_rows: int, main_rows: int, hist_rows: int, n_sel: int, what: str):
    from . import _lib as L

    table = (L.Column * max(len(columns), 1))()
    outs, used = [], 0
    for i, col in enumerate(columns):
        src, role, extra = col
        _check_input(src, f"{what}: column {i}")
        _check(src.dtype in (torch.float32, torch.int32),
               f"{what}: column {i} must be float32 or int32, got {src.dtype}")
        _check(src.dim() >= 1, f"{what}: column {i} must have a row dimension")
        width = int(math.prod(src.shape[1:]))
        _check(1 <= width <= L.DENSIFY_MAX_WIDTH,
               f"{what}: column {i} has {width} values per row (1..{L.DENSIFY_MAX_WIDTH})")
        if role in (L.COL_MEANS, L.COL_RAW_SCALES, L.COL_RAW_OPACITIES):
            _check(src.dtype == torch.float32, f"{what}: column {i} (role {role}) must be float32")
        if role in (L.COL_PARENT, L.COL_LEVEL):
            _check(src.dtype == torch.int32 and width == 1,
                   f"{what}: column {i} (parent / level) must be int32 [N]")
        if role == L.COL_HISTORY:
            _check(extra is not None, f"{what}: history column {i} needs its live column")
            _check_input(extra, f"{what}: live column of history column {i}")
            _check(extra.dtype == src.dtype and tuple(extra.shape[1:]) == tuple(src.shape[1:]),
                   f"{what}: history column {i} and its live column differ in dtype or shape")
            _check(extra.size(0) == n_rows,
                   f"{what}: live column of history column {i} has {extra.size(0)} rows, "
                   f"expected {n_rows}")
            _check(src.size(0) == hist_rows,
                   f"{what}: history column {i} has {src.size(0)} rows, expected {hist_rows}")
            if n_sel == 0:
                outs.append(src)  # nothing to archive: the archive is returned as is
                continue
            rows = hist_rows + n_sel
        else:
            _check(extra is None, f"{what}: column {i}: only history columns take a live column")
            _check(src.size(0) == n_rows,
                   f"{what}: column {i} has {src.size(0)} rows, expected {n_rows}")
            rows = main_rows
        dst = torch.empty((rows,) + tuple(src.shape[1:]), dtype=src.dtype, device=src.device)
        table[used] = L.Column(src.data_ptr() if src.numel() else None,
                               dst.data_ptr() if dst.numel() else None,
                               extra.data_ptr() if extra is not None and extra.numel() else None,
                               rows, width, role)
        used += 1
        outs.append(dst)
    return table, used, outs


def _densify_mask(mask: Tensor, n_rows: int, what: str):
    _check(isinstance(mask, torch.Tensor) and mask.is_cuda, f"{what}: mask must be a CUDA tensor")
    _check(mask.dim() == 1 and mask.size(0) == n_rows,
           f"{what}: mask must be 1-D with {n_rows} entries")
    m = mask if mask.dtype in (torch.bool, torch.uint8) else mask != 0
    return m.contiguous().view(torch.uint8)


def densify_split(mask: Tensor, columns, history_rows: int = 0, geometry=None):
    """Split the rows where ``mask`` is true (binary_tree.py:93-148).

    Each non-history column becomes ``cat(src[rest], child_plus, child_minus)``
    (children of the selected rows, in ascending order); history columns
    become ``cat(src, extra[sel])``.  ``geometry`` is ``(quats, raw_scales,
    scale_min[3], scale_max[3], scale_eps, sigmoid_scales)`` of the live
    table, required by the MEANS / RAW_SCALES roles.  Returns
    ``(outputs, n_sel)`` with outputs in column order.
    """
    from . import _lib as L

    n = int(mask.shape[0]) if isinstance(mask, torch.Tensor) and mask.dim() == 1 else -1
    m = _densify_mask(mask, n, "densify_split")
    idx, n_sel = mask_split(m)
    n_rest = n - n_sel
    dev = m.device
    table, used, outs = _densify_table(columns, n, n_rest + 2 * n_sel, history_rows, n_sel,
                                       "densify_split")
    geo = None
    if geometry is not None:
        quats, raw_scales, smin, smax, eps, sigmoid = geometry
        for t, name in ((quats, "quats"), (raw_scales, "raw_scales")):
            _check_input(t, name)
            _check(t.dtype == torch.float32, f"densify_split: {name} must be float32")
        _check(tuple(quats.shape) == (n, 4) and tuple(raw_scales.shape) == (n, 3),
               "densify_split: geometry must be quats [N,4] and raw_scales [N,3]")
        smin = [float(v) for v in smin]
        smax = [float(v) for v in smax]
        _check(len(smin) == 3 and len(smax) == 3, "densify_split: three scale bounds per side")
        geo = L.SplitGeometry(quats.data_ptr() if n else None, raw_scales.data_ptr() if n else None,
                              (ctypes.c_float * 3)(*smin), (ctypes.c_float * 3)(*smax),
                              float(eps), int(bool(sigmoid)))
    with torch.cuda.device(dev):
        _call("r2s_densify_split", idx.data_ptr() if n_sel else None, n_sel,
              idx[n_sel:].data_ptr() if n_rest else None, n_rest, int(history_rows),
              ctypes.byref(geo) if geo is not None else None, table, used, _stream(dev))
    return outs, n_sel


def densify_duplicate(mask: Tensor, columns, history_rows: int = 0):
    """Duplicate the rows where ``mask`` is true (binary_tree.py:60-90).

    Each non-history column becomes ``cat(src', src'[sel])`` where ``src'``
    is ``src`` with the selected rows' parent / level updated (roles PARENT,
    LEVEL) and the copies' Adam moments zero (role ZERO_NEW).  Returns
    ``(outputs, n_sel)``.
    """
    n = int(mask.shape[0]) if isinstance(mask, torch.Tensor) and mask.dim() == 1 else -1
    m = _densify_mask(mask, n, "densify_duplicate")
    idx, n_sel = mask_split(m)
    dev = m.device
    table, used, outs = _densify_table(columns, n, n + n_sel, history_rows, n_sel,
                                       "densify_duplicate")
    with torch.cuda.device(dev):
        _call("r2s_densify_duplicate", m.data_ptr() if n else None, n,
              idx.data_ptr() if n_sel else None, n_sel, int(history_rows), table, used,
              _stream(dev))
    return outs, n_sel


def densify_remove(mask: Tensor, columns):
    """Keep the rows where ``mask`` is false (binary_tree.py:151-171).
    Returns ``(outputs, n_removed)``."""
    n = int(mask.shape[0]) if isinstance(mask, torch.Tensor) and mask.dim() == 1 else -1
    m = _densify_mask(mask, n, "densify_remove")
    idx, n_sel = mask_split(m)
    n_keep = n - n_sel
    dev = m.device
    table, used, outs = _densify_table(columns, n, n_keep, 0, 0, "densify_remove")
    with torch.cuda.device(dev):
        _call("r2s_densify_remove", idx[n_sel:].data_ptr() if n_keep else None, n_keep, table,
              used, _stream(dev))
    return outs, n_sel


# ---------------------------------------------------------- projection loss --

def _loss_images(t: Tensor, name: str) -> Tensor:
    _check(isinstance(t, torch.Tensor) and t.is_cuda, f"{name} must be a CUDA tensor")
    _check(t.dtype == torch.float32, f"{name} must be float32, got {t.dtype}")
    return t.contiguous()


def projection_loss_fwd(render: Tensor, target: Tensor, edge_target: Optional[Tensor],
                        edge_mask: Optional[Tensor], window_size: int = 11):
    """Losses [3] = (mean |r - t|, 1 - mean SSIM(r, t), mean m |r - e|) over
    images [n, H, W] (loss.py:135-172, metric.py:36-54), and the workspace the
    backward needs."""
    r = _loss_images(render, "render")
    _check(r.dim() == 3, "render must be [n, H, W]")
    t = _loss_images(target, "target")
    _check(t.shape == r.shape, "target must have the render's shape")
    if (edge_target is None) != (edge_mask is None):
        raise RuntimeError("edge_target and edge_mask go together")
    e = m = None
    if edge_target is not None:
        e = _loss_images(edge_target, "edge_target")
        m = _loss_images(edge_mask, "edge_mask")
        _check(e.shape == r.shape and m.shape == r.shape,
               "edge_target and edge_mask must have the render's shape")
    n, H, W = r.shape
    dev = r.device
    lib = _lib()
    losses = torch.empty(3, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        ws = _workspace(lib.r2s_projection_loss_workspace_bytes(n, H, W), dev)
        _call("r2s_projection_loss_fwd_f32", _ptr(r), _ptr(t), _ptr(e), _ptr(m), n, H, W,
              int(window_size), _ptr(losses), _ptr(ws), ws.numel(), _stream(dev))
    return losses, ws


def projection_loss_bwd(render: Tensor, target: Tensor, edge_target: Optional[Tensor],
                        edge_mask: Optional[Tensor], grad_losses: Tensor, workspace: Tensor,
                        window_size: int = 11) -> Tensor:
    """v_render [n, H, W] for upstream gradients grad_losses [3] of the three losses."""
    r = _loss_images(render, "render")
    t = _loss_images(target, "target")
    e = None if edge_target is None else _loss_images(edge_target, "edge_target")
    m = None if edge_mask is None else _loss_images(edge_mask, "edge_mask")
    g = _loss_images(grad_losses, "grad_losses")
    _check(g.numel() == 3, "grad_losses must hold three values")
    n, H, W = r.shape
    dev = r.device
    out = torch.empty_like(r)
    with torch.cuda.device(dev):
        _call("r2s_projection_loss_bwd_f32", _ptr(r), _ptr(t), _ptr(e), _ptr(m), n, H, W,
              int(window_size), _ptr(g), _ptr(workspace), workspace.numel(), _ptr(out),
              _stream(dev))
    return out


# ---------------------------------------------------------------------- TV --

def _tv_volume(vol: Tensor) -> Tensor:
    v = _loss_images(vol, "volume")
    _check(v.dim() == 3, "tv_3d_loss expects 3D volume")
    _check(v.numel() < 2 ** 31 * 256, "volume too large")
    return v


def tv_fwd(volume: Tensor, mean: bool = True) -> Tensor:
    """loss.py:10-21 compute_tv_loss of a [D0, D1, D2] volume (0-dim result)."""
    v = _tv_volume(volume)
    dev = v.device
    lib = _lib()
    out = torch.empty((), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        ws = _workspace(lib.r2s_tv_workspace_bytes(), dev)
        _call("r2s_tv_fwd_f32", _ptr(v), *v.shape, int(bool(mean)), _ptr(out), _ptr(ws),
              ws.numel(), _stream(dev))
    return out


def tv_bwd(volume: Tensor, grad_out: Tensor, mean: bool = True) -> Tensor:
    """d tv / d volume scaled by the upstream gradient grad_out (0-dim)."""
    v = _tv_volume(volume)
    g = _loss_images(grad_out, "grad_out")
    _check(g.numel() == 1, "grad_out must be a scalar")
    dev = v.device
    out = torch.empty_like(v)
    with torch.cuda.device(dev):
        _call("r2s_tv_bwd_f32", _ptr(v), *v.shape, int(bool(mean)), _ptr(g), _ptr(out),
              _stream(dev))
    return out


# --------------------------------------------------------- hierarchy loss --

def hierarchy_loss_fwd(child_means: Tensor, parent: Tensor, history_means: Tensor,
                       parent_scales: Tensor, history_quats: Tensor, history_count: int,
                       max_parent_distance_factor: float = 1.0):
    """loss.py:27-71 compute_hierarchy_loss with the archived scales already
    activated: (out [2] = (loss, count), workspace for the backward)."""
    c = _loss_images(child_means, "child_means")
    _check(c.dim() == 2 and c.size(1) == 3, "child_means must be [N, 3]")
    _check(isinstance(parent, torch.Tensor) and parent.is_cuda, "parent must be a CUDA tensor")
    par = parent.to(torch.int32).contiguous()
    _check(par.numel() == c.size(0), "parent must have one entry per child")
    hm = _loss_images(history_means, "history_means")
    hs = _loss_images(parent_scales, "parent_scales")
    hq = _loss_images(history_quats, "history_quats")
    _check(hm.size(0) >= history_count and hs.size(0) >= history_count and
           hq.size(0) >= history_count, "history shorter than history_count")
    n = c.size(0)
    dev = c.device
    lib = _lib()
    out = torch.empty(2, dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        ws = _workspace(lib.r2s_hierarchy_workspace_bytes(n), dev)
        _call("r2s_hierarchy_loss_fwd_f32", _ptr(c), _ptr(par), n, _ptr(hm), _ptr(hs), _ptr(hq),
              int(history_count), float(max_parent_distance_factor), _ptr(out), _ptr(ws),
              ws.numel(), _stream(dev))
    return out, ws


def hierarchy_loss_bwd(n: int, grad_out: Tensor, out: Tensor, workspace: Tensor) -> Tensor:
    """d loss / d child_means [N, 3] times the upstream gradient grad_out."""
    g = _loss_images(grad_out, "grad_out")
    dev = out.device
    v = torch.empty((n, 3), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        _call("r2s_hierarchy_loss_bwd_f32", n, _ptr(g), _ptr(out), _ptr(workspace),
              workspace.numel(), _ptr(v), _stream(dev))
    return v
