"""Pins oracle/loss.py (projection L1 + SSIM + edge terms and their gradient)."""

import numpy as np
import pytest
import torch
from scipy.signal import correlate2d
from scipy.signal.windows import gaussian

from oracle import loss as L


@pytest.mark.parametrize("ws", [1, 7, 11, 15])
def test_window_is_the_normalised_gaussian(ws):
    g1, g2 = L.gaussian_window(ws)
    ref = gaussian(ws, 1.5)
    ref = ref / ref.sum()
    np.testing.assert_allclose(g1, ref, rtol=1e-6)
    np.testing.assert_allclose(g2, np.outer(ref, ref), rtol=2e-6)
    assert g2.dtype == np.float32 and abs(float(g2.sum()) - 1.0) < 1e-6


def test_filter_is_zero_padded_same_correlation():
    rng = np.random.default_rng(0)
    img = rng.normal(size=(23, 31))
    _, win = L.gaussian_window(11)
    np.testing.assert_allclose(L.filter2d(img, win),
                               correlate2d(img, win.astype(np.float64), mode="same",
                                           boundary="fill"), rtol=1e-12, atol=1e-12)


def test_ssim_of_an_image_with_itself_is_one():
    x = np.random.default_rng(1).uniform(size=(2, 40, 37))
    l1, ssim_loss, edge = L.projection_losses(x, x)
    assert l1 == 0 and abs(ssim_loss) < 1e-12 and edge == 0


def test_constant_images_closed_form_in_the_interior():
    a, b = 0.7, 0.2
    x, y = np.full((30, 30), a), np.full((30, 30), b)
    S = L.ssim_terms(x, y)[0]
    inner = S[5:-5, 5:-5]  # the whole window inside the image
    # The float32 window sums to W = 1 + O(1e-7): mu = aW, var = a^2 W (1 - W), cov = ab W (1 - W).
    W = float(L.gaussian_window(11)[1].astype(np.float64).sum())
    mx, my = a * W, b * W
    vx, vy, cxy = a * a * W * (1 - W), b * b * W * (1 - W), a * b * W * (1 - W)
    expect = ((2 * mx * my + L.C1) * (2 * cxy + L.C2)) / ((mx ** 2 + my ** 2 + L.C1) *
                                                          (vx + vy + L.C2))
    np.testing.assert_allclose(inner, expect, rtol=1e-12)
    # Border pixels see the zero padding: their means are smaller.
    assert S[0, 0] != inner[0, 0]


def _torch_total(x, y, e, m, scales, ws):
    _, win = L.gaussian_window(ws)
    w = torch.tensor(win, dtype=torch.float64)[None, None]
    xs = x[:, None]
    ys = y[:, None]
    conv = lambda t: torch.nn.functional.conv2d(t, w, padding=ws // 2)  # noqa: E731
    mu1, mu2 = conv(xs), conv(ys)
    s11 = conv(xs * xs) - mu1 ** 2
    s22 = conv(ys * ys) - mu2 ** 2
    s12 = conv(xs * ys) - mu1 * mu2
    S = ((2 * mu1 * mu2 + L.C1) * (2 * s12 + L.C2)) / ((mu1 ** 2 + mu2 ** 2 + L.C1) *
                                                        (s11 + s22 + L.C2))
    l1 = (x - y).abs().mean()
    edge = (m * (x - e).abs()).mean()
    return scales[0] * l1 + scales[1] * (1 - S.mean()) + scales[2] * edge


@pytest.mark.parametrize("ws", [11, 5])
def test_gradient_matches_autograd(ws):
    rng = np.random.default_rng(2)
    x = rng.uniform(size=(2, 21, 26))
    y = np.clip(x + rng.normal(0, 0.2, size=x.shape), 0, 1)
    e = rng.uniform(size=x.shape)
    m = (rng.uniform(size=x.shape) < 0.3).astype(np.float64)
    scales = (1.0, 0.25, 0.7)
    g = L.projection_loss_grad(x, y, e, m, scales, ws)
    xt = torch.tensor(x, requires_grad=True)
    total = _torch_total(xt, torch.tensor(y), torch.tensor(e), torch.tensor(m), scales, ws)
    total.backward()
    np.testing.assert_allclose(g, xt.grad.numpy(), rtol=1e-9, atol=1e-14)
    # The oracle's forward values equal the autograd restatement's too.
    l1, sl, ed = L.projection_losses(x, y, e, m, ws)
    np.testing.assert_allclose(scales[0] * l1 + scales[1] * sl + scales[2] * ed, total.item(),
                               rtol=1e-12)


def test_gradient_matches_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.uniform(0.2, 0.8, size=(1, 12, 13))
    y = rng.uniform(0.2, 0.8, size=x.shape)
    g = L.projection_loss_grad(x, y, scales=(0.0, 1.0, 0.0))
    h = 1e-6
    for idx in [(0, 0, 0), (0, 5, 6), (0, 11, 12), (0, 3, 9)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd = (L.projection_losses(xp, y)[1] - L.projection_losses(xm, y)[1]) / (2 * h)
        assert abs(fd - g[idx]) < 1e-7 * max(1.0, abs(fd)), (idx, fd, g[idx])


def test_tv_of_a_ramp_and_its_gradient():
    d0, d1, d2 = 4, 5, 6
    a, b, c = np.meshgrid(np.arange(d0), np.arange(d1), np.arange(d2), indexing="ij")
    vol = 0.5 * a - 2.0 * b + 0.25 * c
    terms = (d0 - 1) * d1 * d2 + d0 * (d1 - 1) * d2 + d0 * d1 * (d2 - 1)
    expect = (0.5 * (d0 - 1) * d1 * d2 + 2.0 * d0 * (d1 - 1) * d2 + 0.25 * d0 * d1 * (d2 - 1))
    assert abs(L.tv(vol, "sum") - expect) < 1e-12
    assert abs(L.tv(vol) - expect / terms) < 1e-12
    rng = np.random.default_rng(4)
    v = rng.normal(size=(3, 4, 5))
    vt = torch.tensor(v, requires_grad=True)
    dx = (vt[1:] - vt[:-1]).abs()
    dy = (vt[:, 1:] - vt[:, :-1]).abs()
    dz = (vt[:, :, 1:] - vt[:, :, :-1]).abs()
    ((dx.sum() + dy.sum() + dz.sum()) / (dx.numel() + dy.numel() + dz.numel()) * 2.5).backward()
    np.testing.assert_allclose(L.tv_grad(v, 2.5), vt.grad.numpy(), rtol=1e-12, atol=1e-15)


def test_hierarchy_loss_closed_form_and_autograd():
    # A child on the parent's second principal axis at 2.5 scales, factor 1.5:
    # excess (2.5 - 1.5) / 1.5, squared.
    q = np.array([[0.8, 0.2, -0.4, 0.4]])
    qn = q / np.linalg.norm(q)
    from scipy.spatial.transform import Rotation
    R = Rotation.from_quat(qn[:, [1, 2, 3, 0]]).as_matrix()[0]
    s = np.array([[0.3, 0.2, 0.5]])
    p = np.array([[0.1, -0.2, 0.3]])
    child = p + 2.5 * s[0, 1] * R[:, 1]
    loss, _ = L.hierarchy_loss(child, np.array([0]), p, s, q, 1, 1.5)
    assert abs(loss - ((2.5 - 1.5) / 1.5) ** 2) < 1e-12
    # Random children: the gradient against autograd of a direct restatement.
    rng = np.random.default_rng(5)
    h, n = 20, 60
    hm, hs, hq = rng.normal(size=(h, 3)), rng.uniform(0.05, 0.5, (h, 3)), rng.normal(size=(h, 4))
    par = rng.integers(-2, h + 3, n)
    cm = hm[np.clip(par, 0, h - 1)] + rng.normal(0, 0.4, (n, 3))
    loss, grad = L.hierarchy_loss(cm, par, hm, hs, hq, h, 0.8)
    ct = torch.tensor(cm, requires_grad=True)
    valid = torch.tensor((par >= 0) & (par < h))
    ids = torch.tensor(par)[valid]
    qt = torch.nn.functional.normalize(torch.tensor(hq)[ids], dim=-1)
    Rt = torch.tensor(Rotation.from_quat(qt.numpy()[:, [1, 2, 3, 0]]).as_matrix())
    local = torch.einsum("nji,nj->ni", Rt, ct[valid] - torch.tensor(hm)[ids])
    r = torch.linalg.norm(local / torch.tensor(hs)[ids].clamp_min(1e-6), dim=-1)
    ref = (torch.relu(r - 0.8) / 0.8).square().mean()
    ref.backward()
    assert abs(loss - ref.item()) < 1e-12
    np.testing.assert_allclose(grad, ct.grad.numpy(), rtol=1e-9, atol=1e-14)


@pytest.mark.parametrize("ws", [1, 11])
def test_gradient_magnitude_bounds_the_gradient(ws):
    rng = np.random.default_rng(3)
    x = rng.uniform(size=(2, 19, 23))
    y = np.clip(x + rng.normal(0, 0.2, size=x.shape), 0, 1)
    e = rng.uniform(size=x.shape)
    m = (rng.uniform(size=x.shape) < 0.3).astype(np.float64)
    scales = (1.0, 0.25, 0.7)
    g = L.projection_loss_grad(x, y, e, m, scales, ws)
    mag = L.projection_loss_grad_magnitude(x, y, e, m, scales, ws)
    assert (mag >= np.abs(g) * (1 - 1e-12)).all()
    if ws == 1:  # the cancelling terms are ~1e3 times the gradient
        assert np.median(mag / np.maximum(np.abs(g), 1e-300)) > 10


def test_hierarchy_magnitude_bounds_the_gradient():
    rng = np.random.default_rng(4)
    h, n = 50, 400
    hm = rng.normal(size=(h, 3))
    hs = np.exp(rng.normal(-1.5, 0.5, size=(h, 3)))
    hq = rng.normal(size=(h, 4))
    par = rng.integers(-2, h + 2, n)
    cm = hm[np.clip(par, 0, h - 1)] + rng.normal(0, 0.3, (n, 3))
    _, g = L.hierarchy_loss(cm, par, hm, hs, hq, h, 0.9)
    mag = L.hierarchy_grad_magnitude(cm, par, hm, hs, hq, h, 0.9)
    assert (mag >= np.abs(g) * (1 - 1e-12)).all()
    assert (mag[np.abs(g) > 0] > 2 * np.abs(g[np.abs(g) > 0])).all()
