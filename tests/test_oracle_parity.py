"""Pins the parity machinery of tests/helpers.py on the CPU.

* The 80-bit oracle (the anchor of the float64 kernels) agrees with the
  float64 one and with the masked dense autograd reference.
* The flip band covers every element whose value moves when the alpha
  cut-off moves within the bracket, by at least the amount it moves.
* A float32 evaluation in another order (dense numpy, pairwise sums) passes
  the bar, with its alpha flips counted; planted mistakes in the oracle's
  own inputs or outputs (a dropped record, a transposed conic term, a
  swapped axis, a scaled gradient) fail it.
"""

import numpy as np
import pytest

from helpers import (ETA, assert_parity, check_raster, check_voxel, raster_references,
                     voxel_references)
from oracle import binning, native


def _raster_scene(seed=3, N=400, W=48, H=40, ts=16):
    r = np.random.default_rng(seed)
    means2d = r.uniform(-5, W + 5, size=(1, N, 2))
    A = r.normal(size=(N, 2, 2)) * 2
    cov = A @ A.transpose(0, 2, 1) + np.eye(2)
    inv = np.linalg.inv(cov)
    conics = np.stack([inv[:, 0, 0], inv[:, 0, 1], inv[:, 1, 1]], -1)[None]
    radii = np.ceil(3 * np.sqrt(np.stack([cov[:, 0, 0], cov[:, 1, 1]], -1))).astype(np.int32)[None]
    opac = r.uniform(0.05, 1, size=(1, N))
    mus = r.uniform(0.5, 2, size=(1, N))
    tw, th = -(-W // ts), -(-H // ts)
    m32 = means2d.astype(np.float32)
    _, keys, ids = binning.isect_tiles(m32, radii, ts, tw, th)
    off = binning.isect_offset_encode(keys, 1, tw, th)
    f = lambda a: a.astype(np.float32)  # noqa: E731
    return dict(m2=m32, con=f(conics), op=f(opac), mu=f(mus), off=off, fl=ids, W=W, H=H, ts=ts,
                v=f(r.normal(size=(1, H, W))))


def _voxel_scene(seed=4, N=120, dims=(20, 17, 22), ts=8):
    r = np.random.default_rng(seed)
    d2, d1, d0 = dims
    m3 = r.uniform(-2, 24, size=(N, 3))
    A = r.normal(size=(N, 3, 3)) * 1.2
    cov = A @ A.transpose(0, 2, 1) + 0.8 * np.eye(3)
    P = np.linalg.inv(cov)
    conics = P[:, [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]]
    rad = np.ceil(3 * np.sqrt(np.diagonal(cov, axis1=1, axis2=2))).astype(np.int32)
    opac = r.uniform(0.01, 1, size=N)
    n2, n1, n0 = (-(-d // ts) for d in dims)
    m32 = m3.astype(np.float32)
    _, keys, ids = binning.isect_tiles_3d(m32, rad, ts, n2, n1, n0)
    off = binning.isect_offset_encode_3d(keys, n2, n1, n0)
    f = lambda a: a.astype(np.float32)  # noqa: E731
    return dict(m3=m32, con=f(conics), op=f(opac), off=off, fl=ids, dims=dims, ts=ts,
                v=f(r.normal(size=(d0, d1, d2))))


def test_long_double_anchor_agrees_with_float64():
    s = _raster_scene()
    args = (s["off"], s["fl"], s["W"], s["H"], s["ts"])
    hi = [np.asarray(s[k], np.longdouble) for k in ("m2", "con", "op", "mu")]
    lo = [np.asarray(s[k], np.float64) for k in ("m2", "con", "op", "mu")]
    img80 = native.raster_fwd(*hi, *args)
    img64 = native.raster_fwd(*lo, *args)
    assert img80.dtype == np.longdouble and float(np.abs(img80).max()) > 0.1
    np.testing.assert_allclose(img64, img80.astype(np.float64), rtol=1e-13, atol=1e-16)
    off, fl, W, H, ts = args
    g80 = native.raster_bwd(*hi, off, fl, s["v"].astype(np.longdouble), W, H, ts)
    g64 = native.raster_bwd(*lo, off, fl, s["v"].astype(np.float64), W, H, ts)
    for a, b in zip(g64, g80):
        np.testing.assert_allclose(a, b.astype(np.float64), rtol=1e-10, atol=1e-13)
    v = _voxel_scene()
    vargs = (v["off"], v["fl"], *v["dims"], v["ts"])
    vol80 = native.voxel_fwd(*[np.asarray(v[k], np.longdouble) for k in ("m3", "con", "op")],
                             *vargs)
    vol64 = native.voxel_fwd(*[np.asarray(v[k], np.float64) for k in ("m3", "con", "op")], *vargs)
    np.testing.assert_allclose(vol64, vol80.astype(np.float64), rtol=1e-13, atol=1e-16)


def _cutoff_scene():
    """Gaussians whose alpha at one pixel centre is thr (1 + k 1e-7), k in
    -20..20: the cut-off decides those terms within the bracket."""
    n = 41
    W = H = 16
    means2d = np.zeros((1, n, 2))
    means2d[0, :, 0] = 7.5 + 0.013 * np.arange(n)
    means2d[0, :, 1] = 8.0
    conics = np.tile(np.array([0.9, 0.05, 0.7]), (1, n, 1))
    dx, dy = 0.5 - means2d[0, :, 0], 0.5 - means2d[0, :, 1]  # pixel (0, 0)
    sigma = 0.5 * (0.9 * dx * dx + 0.7 * dy * dy) + 0.05 * dx * dy
    target = 1e-5 * (1 + 1e-7 * (np.arange(n) - 20))
    opac = (target * np.exp(sigma))[None]
    mus = np.ones((1, n))
    radii = np.full((1, n, 2), 16, np.int32)
    _, keys, ids = binning.isect_tiles(means2d.astype(np.float32), radii, 16, 1, 1)
    off = binning.isect_offset_encode(keys, 1, 1, 1)
    return means2d, conics, opac, mus, off, ids, W, H


def test_band_covers_every_cutoff_move():
    m2, con, op, mu, off, fl, W, H = _cutoff_scene()
    eta = ETA[np.dtype(np.float32)]
    img, band = native.raster_fwd(m2, con, op, mu, off, fl, W, H, 16, eta=eta, band=True)
    assert band[0, 0, 0] > 0 and band[0, 0, 0] <= 41 * 1.01e-5
    v = np.random.default_rng(0).normal(size=(1, H, W))
    g, gb = native.raster_bwd(m2, con, op, mu, off, fl, v, W, H, 16, eta=eta, band=True)
    moved = 0
    for rel in (-3e-6, -1e-6, 1e-6, 3e-6):  # cut-off moves inside the bracket
        img2 = native.raster_fwd(m2, con, op, mu, off, fl, W, H, 16, thr=1e-5 * (1 + rel))
        d = np.abs(img2 - img)
        assert (d <= band + 1e-12 * np.abs(img) + 1e-18).all()  # + the sums' rounding
        moved += int((d > 0).sum())
        g2 = native.raster_bwd(m2, con, op, mu, off, fl, v, W, H, 16, thr=1e-5 * (1 + rel))
        for a, b, bb in zip(g, g2, gb):
            assert (np.abs(a - b) <= bb + 1e-12 * np.abs(a) + 1e-18).all()
    assert moved > 0
    # Pixels whose terms are far from every cut-off have no band (near the
    # means every alpha is ~1e-5 e^sigma(corner) >> 1e-5).
    assert (band[0, 6:11, 6:11] == 0).all()
    assert (band > 0).sum() < 20


def test_band_covers_voxel_cutoff_moves():
    v = _voxel_scene(N=300)
    args = (v["off"], v["fl"], *v["dims"], v["ts"])
    hi = [np.asarray(v[k], np.float64) for k in ("m3", "con", "op")]
    eta = 1e-4  # a wide bracket, so that this scene has terms inside it
    vol, band = native.voxel_fwd(*hi, *args, eta=eta, band=True)
    g, gb = native.voxel_bwd(*hi, *args[:2], v["v"].astype(np.float64), *args[2:], eta=eta,
                             band=True)
    assert (band > 0).sum() > 10
    for rel in (-5e-5, 5e-5):
        vol2 = native.voxel_fwd(*hi, *args, thr=1e-6 * (1 + rel))
        d = np.abs(vol2 - vol)
        assert (d > 0).sum() > 0 and (d <= band + 1e-12 * np.abs(vol) + 1e-18).all()
        g2 = native.voxel_bwd(*hi, *args[:2], v["v"].astype(np.float64), *args[2:],
                              thr=1e-6 * (1 + rel))
        for a, b, bb in zip(g, g2, gb):
            assert (np.abs(a - b) <= bb + 1e-12 * np.abs(a) + 1e-18).all()


def _dense_f32_image(s):
    """The rasterizer's forward in another float32 order: dense over each
    tile's pixels with numpy's pairwise sums over the tile's records."""
    W, H, ts = s["W"], s["H"], s["ts"]
    tw = -(-W // ts)
    off, fl = s["off"].reshape(-1), s["fl"]
    img = np.zeros((H, W), np.float32)
    f = np.float32
    for t in range(off.size):
        a, b = off[t], (off[t + 1] if t + 1 < off.size else fl.size)
        if a == b:
            continue
        g = fl[a:b]
        ty, tx = divmod(t, tw)
        ys = np.arange(ty * ts, min(H, ty * ts + ts))
        xs = np.arange(tx * ts, min(W, tx * ts + ts))
        py, px = np.meshgrid(ys.astype(f) + f(0.5), xs.astype(f) + f(0.5), indexing="ij")
        m = s["m2"][0, g]
        c = s["con"][0, g]
        dx = px[None] - m[:, 0, None, None]
        dy = py[None] - m[:, 1, None, None]
        sig = (f(0.5) * (c[:, 0, None, None] * dx * dx + c[:, 2, None, None] * dy * dy)
               + c[:, 1, None, None] * dx * dy)
        al = (s["op"][0, g] * s["mu"][0, g])[:, None, None] * np.exp(-sig)
        keep = (sig >= 0) & (np.abs(al) >= f(1e-5))
        img[ys[0]:ys[-1] + 1, xs[0]:xs[-1] + 1] = np.where(keep, al, f(0)).sum(0)
    return img[None]


def test_other_float32_order_passes_and_planted_mistakes_fail():
    s = _raster_scene()
    refs = raster_references(s["m2"], s["con"], s["op"], s["mu"], s["off"], s["fl"], s["W"],
                             s["H"], s["ts"], v_image=s["v"])
    rep = check_raster(refs, image=_dense_f32_image(s))
    assert rep["image"]["n"] == s["W"] * s["H"]
    lo32 = native.raster_bwd(s["m2"], s["con"], s["op"], s["mu"], s["off"], s["fl"], s["v"],
                             s["W"], s["H"], s["ts"])
    check_raster(refs, grads=lo32)

    def fails(image=None, grads=None):
        with pytest.raises(AssertionError, match="outside the parity bar"):
            check_raster(refs, image=image, grads=grads)

    base = (s["m2"], s["con"], s["op"], s["mu"], s["off"])
    # A dropped record (the list's last one replaced by its predecessor's id).
    fl_bad = s["fl"].copy()
    fl_bad[-1] = fl_bad[-2]
    fails(image=native.raster_fwd(*base, fl_bad, s["W"], s["H"], s["ts"]))
    # The conic's off-diagonal term with the wrong sign.
    con_bad = s["con"].copy()
    con_bad[..., 1] *= -1
    fails(image=native.raster_fwd(s["m2"], con_bad, *base[2:], s["fl"], s["W"], s["H"], s["ts"]))
    # x and y of the mean swapped.
    fails(image=native.raster_fwd(np.ascontiguousarray(s["m2"][..., ::-1]), *base[1:], s["fl"],
                                  s["W"], s["H"], s["ts"]))
    # A gradient 1e-3 too large for one Gaussian.
    g_bad = [None if x is None else x.copy() for x in lo32]
    i = int(np.argmax(np.abs(g_bad[1][0, :, 0])))
    g_bad[1][0, i, 0] *= 1.001
    fails(grads=g_bad)
    # The absolute gradient from the signed one.
    g_bad = list(lo32)
    g_bad[0] = np.abs(lo32[1])
    fails(grads=g_bad)


def test_voxel_float32_oracle_passes_and_planted_mistakes_fail():
    v = _voxel_scene()
    d2, d1, d0 = v["dims"]
    refs = voxel_references(v["m3"], v["con"], v["op"], v["off"], v["fl"], d2, d1, d0, v["ts"],
                            v_volume=v["v"])
    lo = native.voxel_fwd(v["m3"], v["con"], v["op"], v["off"], v["fl"], d2, d1, d0, v["ts"])
    check_voxel(refs, volume=lo)
    g = native.voxel_bwd(v["m3"], v["con"], v["op"], v["off"], v["fl"], v["v"], d2, d1, d0,
                         v["ts"])
    check_voxel(refs, grads=g)
    # The z axis (dim0) of the volume reversed.
    with pytest.raises(AssertionError, match="outside the parity bar"):
        check_voxel(refs, volume=lo[::-1].copy())
    con_bad = v["con"].copy()
    con_bad[:, [2, 4]] = con_bad[:, [4, 2]]  # xz and yz terms transposed
    bad = native.voxel_bwd(v["m3"], con_bad, v["op"], v["off"], v["fl"], v["v"], d2, d1, d0,
                           v["ts"])
    with pytest.raises(AssertionError, match="outside the parity bar"):
        check_voxel(refs, grads=bad)


def test_assert_parity_reports_categories():
    anchor = np.array([1.0, 0.0, 5.0, 0.0], np.float64)
    lowp = np.array([1.0, 3e-5, 5.0, 0.0], np.float64)
    band = np.array([0.0, 0.0, 0.0, 1e-3], np.float64)
    act = np.array([1.00005, 5e-5, 5.0004, 4e-4], np.float32)
    rep = assert_parity(act, anchor, lowp, band, "t")
    assert rep == dict(n=4, within_bar=2, reference_order=1, conditioning=0, alpha_flips=1)
    with pytest.raises(AssertionError):
        assert_parity(act, anchor, lowp, band, "t", max_flips=0)
    # |terms| = 4000 allows 2 u 4000 = 4.8e-4 of cancellation error: the
    # element that needed its band now passes on its conditioning, which
    # needed err / (u |terms|) = 1.68.
    mag = np.array([1.0, 0.0, 5.0, 4000.0])
    rep = assert_parity(act, anchor, lowp, band, "t", mag=mag)
    assert (rep["conditioning"], rep["alpha_flips"]) == (1, 0)
    assert rep["kappa_max"] == pytest.approx(4e-4 / (2.0 ** -24 * 4000), rel=1e-3)
    with pytest.raises(AssertionError, match="outside the parity bar"):
        assert_parity(act, anchor, lowp, None, "t", mag=mag / 10)
    # The cap on the conditioning and flip classes: of 10,000 elements, 5
    # that need their band pass a cap of 1e-3 (10 elements), not one of 1e-4
    # (the floor of 4 elements).
    big = np.zeros(10_000)
    act5 = np.zeros(10_000, np.float32)
    act5[:5] = 4e-4
    band5 = np.where(np.arange(10_000) < 5, 1e-3, 0.0)
    assert assert_parity(act5, big, big, band5, "c", max_frac=1e-3)["alpha_flips"] == 5
    with pytest.raises(AssertionError, match="conditioning \\+ alpha flips above 4"):
        assert_parity(act5, big, big, band5, "c", max_frac=1e-4)
    with pytest.raises(AssertionError, match="NaN pattern"):
        assert_parity(np.array([np.nan], np.float32), np.zeros(1), np.zeros(1), None, "n")


def test_sampled_tiles_and_records_reproduce_the_whole_oracle():
    s = _raster_scene(N=600)
    args = (s["m2"], s["con"], s["op"], s["mu"], s["off"], s["fl"])
    full = native.raster_fwd(*args, s["W"], s["H"], s["ts"])
    keys = np.array([0, 4, 7, 8])
    part = native.raster_fwd(*args, s["W"], s["H"], s["ts"], keys=keys)
    tw = -(-s["W"] // s["ts"])
    for k in keys:
        ty, tx = divmod(int(k), tw)
        sl = np.s_[0, ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16]
        assert np.array_equal(part[sl], full[sl])
    assert part.sum() < full.sum()
    # Per-record partials of every tile, summed per Gaussian in record order,
    # are the backward outputs; the listed-tile subset picks their rows.
    all_keys = np.arange(s["off"].size)
    rec, val, _, mg = native.raster_records(*args, s["v"], s["W"], s["H"], s["ts"], all_keys)
    assert np.array_equal(rec, np.arange(s["fl"].size))
    grads = native.raster_bwd(*args, s["v"], s["W"], s["H"], s["ts"])
    N = s["m2"].shape[1]
    sums = np.zeros((N, 9), np.float32)
    for r in range(rec.size):
        sums[s["fl"][r]] += val[r]
    want = np.concatenate([grads[0][0], grads[1][0], grads[2][0], grads[3][0][:, None],
                           grads[4][0][:, None]], 1)
    assert np.array_equal(sums, want)
    assert (mg >= np.abs(val) * (1 - 1e-6)).all()
    rec2, val2, _, _ = native.raster_records(*args, s["v"], s["W"], s["H"], s["ts"], keys)
    assert np.array_equal(val2, val[rec2])
    v = _voxel_scene()
    d2, d1, d0 = v["dims"]
    vargs = (v["m3"], v["con"], v["op"], v["off"], v["fl"])
    vfull = native.voxel_fwd(*vargs, d2, d1, d0, v["ts"])
    vpart = native.voxel_fwd(*vargs, d2, d1, d0, v["ts"], keys=[3, 5])
    assert np.array_equal(vpart[0:8, 0:8, 24:], vfull[0:8, 0:8, 24:])  # brick 5: (0, 1, 2)
    vrec, vval, _, _ = native.voxel_records(*vargs, v["v"], d2, d1, d0, v["ts"],
                                            np.arange(v["off"].size))
    vg = native.voxel_bwd(*vargs, v["v"], d2, d1, d0, v["ts"])
    vs = np.zeros((v["m3"].shape[0], 10), np.float32)
    for r in range(vrec.size):
        vs[v["fl"][r]] += vval[r]
    assert np.array_equal(vs, np.concatenate([vg[0], vg[1], vg[2][:, None]], 1))


def test_voxel_oracle_on_slab_segments_with_a_key_offset():
    v = _voxel_scene(N=300)
    d2, d1, d0 = v["dims"]
    n0, n1, n2 = v["off"].shape
    # The whole list's segment of brick layers [1, 3) as a slab: keys
    # relative to layer 1, offsets of its 2 layers.
    keys_full = np.repeat(np.arange(v["off"].size), np.diff(np.append(v["off"].reshape(-1),
                                                                      v["fl"].size)))
    plane = n1 * n2
    seg = (keys_full >= plane) & (keys_full < 3 * plane)
    rel = keys_full[seg] - plane
    off = np.searchsorted(rel, np.arange(2 * plane), "left").astype(np.int32).reshape(2, n1, n2)
    fl_seg = v["fl"][seg]
    vargs = (v["m3"], v["con"], v["op"])
    full = native.voxel_fwd(*vargs, v["off"], v["fl"], d2, d1, d0, v["ts"])
    slab = native.voxel_fwd(*vargs, off, fl_seg, d2, d1, d0, v["ts"], key_offset=plane)
    assert np.array_equal(slab[8:24], full[8:24]) and not slab[:8].any()
    rec_f, val_f, _, _ = native.voxel_records(*vargs, v["off"], v["fl"], v["v"], d2, d1, d0,
                                              v["ts"], np.arange(plane, 3 * plane))
    rec_s, val_s, _, _ = native.voxel_records(*vargs, off, fl_seg, v["v"], d2, d1, d0, v["ts"],
                                              np.arange(2 * plane), key_offset=plane)
    assert np.array_equal(val_s, val_f) and rec_s.size == seg.sum()
