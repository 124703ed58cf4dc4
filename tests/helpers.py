"""Shared helpers of the test suite."""

from __future__ import annotations

import math

import numpy as np
import torch

from r2splat import geometry, scenes

# Parity bar for floating-point outputs (float32): rel 1e-4 / abs 1e-5.
RTOL = 1e-4
ATOL = 1e-5


def make_scene(n, seed, n_det=64, n_views=1, log_mu=-4.0, log_sigma=0.5, extent=1.0):
    """Seeded Gaussians + cone-beam views (DSO 1.0, DSD 1.5, sDetector 3.0)."""
    g = torch.Generator().manual_seed(seed)
    raw = scenes.random_gaussians(n, g, log_mu, log_sigma, extent)
    angles = (torch.rand(n_views, generator=g) * 2 * math.pi).tolist()
    viewmats, Ks = geometry.cone_beam_views(angles, n_det)
    return raw, viewmats, Ks, g


def np32(t):
    return t.detach().cpu().numpy()


def assert_close(actual, expected, name, rtol=RTOL, atol=ATOL):
    """Elementwise |a - e| <= atol + rtol |e|, NaN patterns equal."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    if a.size == 0:
        return
    assert np.array_equal(np.isnan(a), np.isnan(e)), f"{name}: NaN pattern differs"
    finite = ~np.isnan(e)
    err = np.abs(a - e)
    bad = (err > atol + rtol * np.abs(e)) & finite
    nbad = int(bad.sum())
    if nbad:
        worst = np.unravel_index(np.argmax(np.where(bad, err, -1)), a.shape)
        raise AssertionError(f"{name}: {nbad}/{a.size} outside rtol={rtol} atol={atol}; worst "
                             f"at {worst}: actual={a[worst]!r} expected={e[worst]!r}")


# ---------------------------------------------------------------- parity --
#
# Floating-point outputs of the rasterizer and voxelizer are checked against
# the oracle one precision up (the "anchor": float64 for float32 kernels, the
# 80-bit long double for float64 kernels) on the kernel's own inputs:
#
#   |a - anchor| <= max(atol + rtol |anchor|, 2 |lowp - anchor|,
#                       KAPPA u |terms|) + band
#
# * atol + rtol |anchor|: the north-star bar (rel 1e-4 / abs 1e-5 in float32;
#   rel 1e-9 / abs 1e-12 in float64);
# * 2 |lowp - anchor|: twice the error of the reference's own summation order
#   in the kernel's precision (the oracle run in float32 / float64), for sums
#   that cancel below the bar's reach;
# * KAPPA u |terms|: the sum of the absolute values of the terms that make
#   the output (oracle/c/r2s_oracle.c `mag`: |term| (1 + S) with S the sum
#   of |sigma's terms|) times the kernel precision's unit roundoff u and
#   KAPPA = 2: what any evaluation order may differ by when the terms cancel.
#   A single realisation of the reference order's error is no bound for
#   another order: at config 2 a v_conic sum of 1.99 over 38,400 pixel terms
#   has u |terms| = 0.088; the kernel's result was 2.9e-3 off, the reference
#   order's 1.1e-3.  Elements that need this clause are the "conditioning"
#   class; the report gives the largest err / (u |terms|) among them
#   (`kappa_max`), so a widening shows as a number, not only as a count;
# * band: the summed |contribution| of the terms whose alpha test lies within
#   the flip bracket (oracle/c/r2s_oracle.c), non-zero only for outputs that
#   contain a term at an alpha cut-off.  An element that needs it is an alpha
#   flip; flips are counted and reported, never absorbed in a budget.
#
# The bracket is eta (S + |sigma*| + 1) on the exponent (S: the sum of
# |sigma's terms|, sigma*: the exponent at the cut-off).  The float32
# kernels' exponent sigma log2(e) = (h_a dx + h_b dy) dx + h_c dy^2 differs
# from the float64 one by at most 2.6 u (S + |sigma*| + 1) and their limit
# log2(|w| / thr) by 1.5 u (u = 2^-24, measured over 2e6 terms on the cut-off
# contour with conic anisotropy up to e^6); eta = 8 u covers both twice.

U32 = 2.0 ** -24
U64 = 2.0 ** -53
KAPPA = 2
UNIT = {np.dtype(np.float32): U32, np.dtype(np.float64): U64}
ETA = {np.dtype(np.float32): 8 * U32, np.dtype(np.float64): 8 * U64}
BAR = {np.dtype(np.float32): (1e-4, 1e-5), np.dtype(np.float64): (1e-9, 1e-12)}
ANCHOR = {np.dtype(np.float32): np.float64, np.dtype(np.float64): np.longdouble}


class ParityReport(dict):
    """Counts of one check: elements, those inside the bar, those that needed
    the reference-order term, those that needed the conditioning term, and
    alpha flips (those that needed the band); kappa_max is the largest
    err / (u |terms|) of the conditioning class."""

    def __str__(self):
        return ", ".join(f"{k}={v}" for k, v in self.items())


# Default cap on the elements of one output that need the conditioning term
# or the flip band, as a fraction of the output's elements (check_raster,
# check_voxel and the sampled checks; a test may pass a measured cap of its
# own, e.g. for needle-like stress footprints).  At most MIN_CAPPED such
# elements are always allowed, so small outputs are not failed by one flip.
MAX_FRAC = 1e-3
MIN_CAPPED = 4


def assert_parity(actual, anchor, lowp, band, name, rtol=None, atol=None, max_flips=None,
                  mag=None, max_frac=None):
    """Every element within the bar described above, else AssertionError.

    ``max_flips``: most alpha flips allowed; ``max_frac``: most elements of
    the conditioning and flip classes together, as a fraction of the
    elements (at least MIN_CAPPED).  Returns the ParityReport."""
    a = np.asarray(actual)
    kdt = np.dtype(a.dtype)
    r0, a0 = BAR.get(kdt, BAR[np.dtype(np.float32)])
    rtol = r0 if rtol is None else rtol
    atol = a0 if atol is None else atol
    A = np.asarray(anchor, dtype=np.longdouble)
    L = np.asarray(lowp, dtype=np.longdouble)
    X = a.astype(np.longdouble)
    assert X.shape == A.shape == L.shape, f"{name}: shapes {X.shape} {A.shape} {L.shape}"
    rep = ParityReport(n=int(X.size), within_bar=0, reference_order=0, conditioning=0,
                       alpha_flips=0)
    if X.size == 0:
        return rep
    assert np.array_equal(np.isnan(X), np.isnan(A)), f"{name}: NaN pattern differs"
    fin = np.isfinite(A)
    assert np.array_equal(X[~fin & ~np.isnan(A)], A[~fin & ~np.isnan(A)]), \
        f"{name}: infinities differ"
    B = np.zeros_like(A) if band is None else np.asarray(band, dtype=np.longdouble)
    err = np.where(fin, np.abs(X - A), 0)
    bar = atol + rtol * np.abs(A)
    order = 2 * np.abs(L - A)
    cond = order
    if mag is not None:
        uM = UNIT.get(kdt, U32) * np.asarray(mag, dtype=np.longdouble)
        cond = np.maximum(order, KAPPA * uM)
    ok_bar = err <= bar
    ok_order = err <= np.maximum(bar, order)
    ok_cond = err <= np.maximum(bar, cond)
    ok_flip = err <= np.maximum(bar, cond) + B
    rep["within_bar"] = int(ok_bar.sum())
    rep["reference_order"] = int((ok_order & ~ok_bar).sum())
    rep["conditioning"] = int((ok_cond & ~ok_order).sum())
    rep["alpha_flips"] = int((ok_flip & ~ok_cond).sum())
    if rep["conditioning"]:
        need = ok_cond & ~ok_order
        rep["kappa_max"] = round(float((err[need] / uM[need]).max()), 4)
    bad = ~ok_flip & fin
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - np.maximum(bar, cond) - B, -1)),
                             X.shape)
        raise AssertionError(
            f"{name}: {int(bad.sum())}/{X.size} outside the parity bar (rtol={rtol}, "
            f"atol={atol}); worst at {i}: actual={float(X[i])!r} anchor={float(A[i])!r} "
            f"reference-order={float(L[i])!r} band={float(B[i])!r}"
            + ("" if mag is None else f" |terms|={float(np.asarray(mag)[i])!r}"))
    if max_flips is not None:
        assert rep["alpha_flips"] <= max_flips, f"{name}: {rep}"
    if max_frac is not None:
        cap = max(int(round(max_frac * X.size)), MIN_CAPPED)
        assert rep["conditioning"] + rep["alpha_flips"] <= cap, \
            f"{name}: conditioning + alpha flips above {cap} ({max_frac:g} of {X.size}): {rep}"
    return rep


def _oracle_inputs(arrays, dt):
    return [np.asarray(x).astype(dt) for x in arrays]


def raster_references(m2, con, op, mu, off, fl, W, H, ts, v_image=None, absgrad=True):
    """Oracle references for a rasterizer kernel run on these (numpy) inputs,
    in the inputs' dtype: dict(fwd=(anchor, lowp, band, mag), bwd=[(anchor,
    lowp, band, mag) per output of the 5-tuple]); bwd only when v_image is
    given."""
    from oracle import native

    kdt = np.dtype(np.asarray(m2).dtype)
    hi, eta = ANCHOR[kdt], ETA[kdt]
    lo_in = _oracle_inputs((m2, con, op, mu), kdt)
    hi_in = _oracle_inputs((m2, con, op, mu), hi)
    out = {}
    lo = native.raster_fwd(*lo_in, off, fl, W, H, ts)
    an, bd, mg = native.raster_fwd(*hi_in, off, fl, W, H, ts, eta=eta, band=True, mag=True)
    out["fwd"] = (an, lo, bd, mg)
    if v_image is not None:
        v = np.asarray(v_image)
        lo_g = native.raster_bwd(*lo_in, off, fl, v.astype(kdt), W, H, ts, absgrad)
        an_g, bd_g, mg_g = native.raster_bwd(*hi_in, off, fl, v.astype(hi), W, H, ts, absgrad,
                                             eta=eta, band=True, mag=True)
        out["bwd"] = list(zip(an_g, lo_g, bd_g, mg_g))
    return out


def voxel_references(m3, con, op, off, fl, d2, d1, d0, ts, v_volume=None):
    """As raster_references for the voxelizer: fwd and the 3-tuple bwd."""
    from oracle import native

    kdt = np.dtype(np.asarray(m3).dtype)
    hi, eta = ANCHOR[kdt], ETA[kdt]
    lo_in = _oracle_inputs((m3, con, op), kdt)
    hi_in = _oracle_inputs((m3, con, op), hi)
    out = {}
    lo = native.voxel_fwd(*lo_in, off, fl, d2, d1, d0, ts)
    an, bd, mg = native.voxel_fwd(*hi_in, off, fl, d2, d1, d0, ts, eta=eta, band=True, mag=True)
    out["fwd"] = (an, lo, bd, mg)
    if v_volume is not None:
        v = np.asarray(v_volume)
        lo_g = native.voxel_bwd(*lo_in, off, fl, v.astype(kdt), d2, d1, d0, ts)
        an_g, bd_g, mg_g = native.voxel_bwd(*hi_in, off, fl, v.astype(hi), d2, d1, d0, ts,
                                            eta=eta, band=True, mag=True)
        out["bwd"] = list(zip(an_g, lo_g, bd_g, mg_g))
    return out


RASTER_GRAD_NAMES = ("v_means2d_abs", "v_means2d", "v_conics", "v_opacities", "v_mus")
VOXEL_GRAD_NAMES = ("v_means3d", "v_conics", "v_opacities")


def check_raster(refs, image=None, grads=None, tag="", max_flips=None, max_frac=MAX_FRAC):
    """assert_parity over a rasterizer's image and / or 5-tuple of gradients,
    each output's conditioning + flip classes capped at max_frac of its
    elements; returns {name: ParityReport}."""
    reps = {}
    if image is not None:
        an, lo, bd, mg = refs["fwd"]
        reps["image"] = assert_parity(image, an, lo, bd, f"{tag}image", max_flips=max_flips,
                                      mag=mg, max_frac=max_frac)
    if grads is not None:
        for g, (an, lo, bd, mg), n in zip(grads, refs["bwd"], RASTER_GRAD_NAMES):
            if an is None:
                assert g is None, f"{tag}{n}: expected None"
                continue
            reps[n] = assert_parity(g, an, lo, bd, f"{tag}{n}", max_flips=max_flips, mag=mg,
                                    max_frac=max_frac)
    return reps


def check_voxel(refs, volume=None, grads=None, tag="", max_flips=None, max_frac=MAX_FRAC):
    """As check_raster for the voxelizer: volume and / or the 3-tuple."""
    reps = {}
    if volume is not None:
        an, lo, bd, mg = refs["fwd"]
        reps["volume"] = assert_parity(volume, an, lo, bd, f"{tag}volume", max_flips=max_flips,
                                       mag=mg, max_frac=max_frac)
    if grads is not None:
        for g, (an, lo, bd, mg), n in zip(grads, refs["bwd"], VOXEL_GRAD_NAMES):
            reps[n] = assert_parity(g, an, lo, bd, f"{tag}{n}", max_flips=max_flips, mag=mg,
                                    max_frac=max_frac)
    return reps


def assert_equal(actual, expected, name):
    a, e = np.asarray(actual), np.asarray(expected)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    diff = a != e
    if a.dtype.kind == "f":
        diff &= ~(np.isnan(a) & np.isnan(e))
    n = int(diff.sum())
    if n:
        idx = np.argwhere(diff)[0]
        raise AssertionError(f"{name}: {n}/{a.size} entries differ; first at {tuple(idx)}: "
                             f"{a[tuple(idx)]!r} vs {e[tuple(idx)]!r}")


PARAM_GRADS = ("means", "quats", "raw_scales", "raw_opacities")


def check_parameter_gradients(got, args, raster_grads, voxel_grads=None, min_plain=0.999):
    """Composed parameter gradients of explicit_backward against the oracle.

    ``got``: {name: array} for PARAM_GRADS from the kernels; ``args``: the
    positional arguments of oracle.compose.explicit_backward for the float32
    forward (the kernels' own geometry and tile lists); ``raster_grads`` /
    ``voxel_grads``: the kernels' raster / voxel VJP outputs, which the caller
    checks against the oracle with assert_parity.

    The chain after those VJPs (conics/mu and projection VJPs, the mapping
    VJP, the parameter transform and the opacity chain) is linear in them and
    is checked on the kernels' own raster / voxel gradients: every element of
    ``got`` meets assert_parity against the chain evaluated in float64 on
    them, with the float32 chain on them as the reference order.  Together
    with the raster / voxel check this covers every composed gradient.  The
    composition from scratch (float64 vs float32, the reference order end to
    end) differs by what the raster / voxel sums differ, carried through the
    chain: at least ``min_plain`` of each parameter gradient's elements must
    be within the plain bar of it (all but MIN_CAPPED in small outputs).  Returns ({name: ParityReport} of the chain
    check, {name: fraction within the plain bar end to end})."""
    from oracle import compose

    chain = dict(raster_grads=raster_grads, voxel_grads=voxel_grads)
    chain_lo = compose.explicit_backward(*args, **chain)
    chain_hi = compose.explicit_backward(*args, dtype=np.float64, **chain)
    reports = {}
    for name in PARAM_GRADS:
        reports[name] = assert_parity(np.asarray(got[name]), chain_hi[name], chain_lo[name], None,
                                      f"grad {name} (chain on the kernels' raster / voxel VJPs)",
                                      max_frac=MAX_FRAC)
    hi64 = compose.explicit_backward(*args, dtype=np.float64)
    plain = {}
    for name in PARAM_GRADS:
        g = np.asarray(got[name], np.float64)
        a = np.asarray(hi64[name], np.float64)
        inside = np.abs(g - a) <= 1e-5 + 1e-4 * np.abs(a)
        plain[name] = float(inside.mean())
        cap = max(int(round((1 - min_plain) * inside.size)), MIN_CAPPED)
        assert int((~inside).sum()) <= cap, (
            f"grad {name}: {int((~inside).sum())} of {inside.size} elements outside the plain "
            f"bar of the float64 composition end to end (at most {cap}: {min_plain} within)")
    return reports, plain


# ------------------------------------------------------- sampled checks --
#
# Lists too long for the whole oracle (config 5) are checked on a sample of
# tiles: the forward's pixels of those tiles, and the per-record partials of
# their records as the two-pass backward kernels store them (one row per
# record at its emission index), against oracle/native.py's *_records.

# Oracle value index of row slot k.  The oracle's raster record values are
# (abs x, abs y, v_xy x, v_xy y, conic 0..2, opacity, mu); the kernels' raster
# row is (v_xy x, v_xy y, conic 0..2, T0, abs x, abs y) in 8 slots, the
# opacity and mu partials being mu T0 and o T0.  Voxel rows: 10 slots, the
# oracle's 10 values in order (test_capi_cpu checks both slot counts against
# the library's workspace sizes).
RASTER_ROW = (2, 3, 4, 5, 6, None, 0, 1)
RASTER_ROW_SLOTS = 8
VOXEL_ROW = tuple(range(10))
VOXEL_ROW_SLOTS = 10


def sample_keys(tile_offsets, n_isects, n_sample, seed=0):
    """The most loaded tile / brick plus n_sample - 1 random non-empty ones."""
    off = np.asarray(tile_offsets).reshape(-1).astype(np.int64)
    cnt = np.diff(np.append(off, n_isects))
    live = np.flatnonzero(cnt > 0)
    rng = np.random.default_rng(seed)
    pick = rng.choice(live, size=min(n_sample - 1, live.size), replace=False)
    return np.unique(np.append(pick, int(np.argmax(cnt))))


def _row_values(rows_f32, src, rec, order, slots, n_values):
    r = np.asarray(rows_f32).reshape(-1, slots)[np.asarray(src)[rec]]
    out = np.zeros((rec.size, n_values), np.float64)
    for slot, j in enumerate(order):
        if j is not None:
            out[:, j] = r[:, slot]
    return out, r


def check_raster_sampled(m2, con, op, mu, off, fl, v_image, W, H, ts, keys, image=None,
                         rows=None, isect_src=None, tag="", max_frac=MAX_FRAC):
    """assert_parity over the sampled tiles' pixels of ``image`` and over
    their records' rows (``rows`` [n_isects * 8] float32 at emission index
    ``isect_src``; the opacity and mu partials formed as mu T0 and o T0 from
    the row's T0), all numpy float32."""
    from oracle import native

    eta = ETA[np.dtype(np.float32)]
    lo = [np.asarray(a, np.float32) for a in (m2, con, op, mu)]
    hi = [a.astype(np.float64) for a in lo]
    reps = {}
    if image is not None:
        an, bd, mg = native.raster_fwd(*hi, off, fl, W, H, ts, eta=eta, band=True, mag=True,
                                       keys=keys)
        lw = native.raster_fwd(*lo, off, fl, W, H, ts, keys=keys)
        tw = np.asarray(off).shape[2]
        mask = np.zeros(an.shape, bool)
        n_t = tw * np.asarray(off).shape[1]
        for k in np.asarray(keys):
            c, t = divmod(int(k), n_t)
            ty, tx = divmod(t, tw)
            mask[c, ty * ts:(ty + 1) * ts, tx * ts:(tx + 1) * ts] = True
        reps["image"] = assert_parity(np.asarray(image)[mask], an[mask], lw[mask], bd[mask],
                                      f"{tag}image (sampled tiles)", mag=mg[mask],
                                      max_frac=max_frac)
    if rows is not None:
        rec, val, bd, mg = native.raster_records(*hi, off, fl, np.asarray(v_image, np.float64),
                                                 W, H, ts, keys, eta=eta)
        _, lv, _, _ = native.raster_records(*lo, off, fl, np.asarray(v_image, np.float32), W, H,
                                            ts, keys)
        got, r = _row_values(rows, isect_src, rec, RASTER_ROW, RASTER_ROW_SLOTS, 9)
        # Opacity and mu partials from the row's T0 (products in float64).
        g = np.asarray(fl).reshape(-1)[rec].astype(np.int64)
        got[:, 7] = hi[3].reshape(-1)[g] * r[:, 5]
        got[:, 8] = hi[2].reshape(-1)[g] * r[:, 5]
        reps["records"] = assert_parity(got.astype(np.float32), val, lv, bd,
                                        f"{tag}record partials (sampled)", mag=mg,
                                        max_frac=max_frac)
        reps["records"]["records"] = int(rec.size)
    return reps


def check_voxel_sampled(m3, con, op, off, fl, v_volume, d2, d1, d0, ts, keys, volume=None,
                        rows=None, isect_src=None, tag="", key_offset=0, max_frac=MAX_FRAC):
    """As check_raster_sampled for the voxelizer (rows of 10 values).  With
    ``key_offset`` the lists are one z-slab's (keys relative to the slab's
    first brick layer) and ``volume`` is the whole volume."""
    from oracle import native

    eta = ETA[np.dtype(np.float32)]
    lo = [np.asarray(a, np.float32) for a in (m3, con, op)]
    hi = [a.astype(np.float64) for a in lo]
    reps = {}
    n0, n1, n2 = np.asarray(off).shape
    if volume is not None:
        an, bd, mg = native.voxel_fwd(*hi, off, fl, d2, d1, d0, ts, eta=eta, band=True, mag=True,
                                      keys=keys, key_offset=key_offset)
        lw = native.voxel_fwd(*lo, off, fl, d2, d1, d0, ts, keys=keys, key_offset=key_offset)
        mask = np.zeros(an.shape, bool)
        for k in np.asarray(keys):
            b0, rem = divmod(int(k) + key_offset, n1 * n2)
            b1, b2 = divmod(rem, n2)
            mask[b0 * ts:(b0 + 1) * ts, b1 * ts:(b1 + 1) * ts, b2 * ts:(b2 + 1) * ts] = True
        reps["volume"] = assert_parity(np.asarray(volume)[mask], an[mask], lw[mask], bd[mask],
                                       f"{tag}volume (sampled bricks)", mag=mg[mask],
                                       max_frac=max_frac)
    if rows is not None:
        rec, val, bd, mg = native.voxel_records(*hi, off, fl, np.asarray(v_volume, np.float64),
                                                d2, d1, d0, ts, keys, eta=eta,
                                                key_offset=key_offset)
        _, lv, _, _ = native.voxel_records(*lo, off, fl, np.asarray(v_volume, np.float32), d2, d1,
                                           d0, ts, keys, key_offset=key_offset)
        got, _ = _row_values(rows, isect_src, rec, VOXEL_ROW, VOXEL_ROW_SLOTS, 10)
        reps["records"] = assert_parity(got.astype(np.float32), val, lv, bd,
                                        f"{tag}record partials (sampled)", mag=mg,
                                        max_frac=max_frac)
        reps["records"]["records"] = int(rec.size)
    return reps
