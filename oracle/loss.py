"""Projection loss (L1 + SSIM + masked edge L1) and volume TV restated in numpy -- TEST INFRASTRUCTURE ONLY.

Restates ``ssim2d`` / ``_gaussian`` / ``_create_window`` of
``src/utils/metric.py:13-54`` and the projection terms of
``BinaryTreeLossComputer.__call__`` (``src/utils/loss.py:135-172``):

    l1   = mean |x - y|
    ssim = 1 - mean S,   S = (2 mu_x mu_y + c1)(2 s_xy + c2) /
                             ((mu_x^2 + mu_y^2 + c1)(s_xx + s_yy + c2))
    edge = mean m |x - e|

with mu, s from the 2-D Gaussian window (float32 values, as the reference
builds them) applied with zero padding.  Arithmetic is float64 on the
float32 inputs, so the oracle is the exact value the float32 kernels
approximate.  The gradient is the adjoint of the window filter:
d(sum S)/dx = G*A + 2 x G*B + y G*C with A = dS/dmu_x, B = dS/dE[x^2],
C = dS/dE[xy] (G symmetric, zero padding).

``tv`` / ``tv_grad`` restate compute_tv_loss (``src/utils/loss.py:10-21``)
and its gradient.

Pinned in tests/test_oracle_loss.py: the window against scipy's Gaussian
window, the filter against scipy.signal.correlate2d, SSIM(x, x) = 1 and the
constant-image closed form, the gradient against torch autograd in float64
and central finite differences; TV against a linear ramp's closed form and
its gradient against torch autograd.
"""

from __future__ import annotations

import math

import numpy as np

C1 = float(np.float32(0.01 ** 2))
C2 = float(np.float32(0.03 ** 2))


def gaussian_window(window_size=11, sigma=1.5):
    """metric.py:13-34: float32 1-D taps normalised by their float32 sum; the
    2-D window is their float32 outer product."""
    e = np.array([math.exp(-((x - window_size // 2) ** 2) / float(2 * sigma ** 2))
                  for x in range(window_size)], dtype=np.float32)
    g = (e / np.float32(e.sum(dtype=np.float32))).astype(np.float32)
    return g, np.outer(g, g).astype(np.float32)


def filter2d(img, window):
    """Zero-padded 'same' correlation of [H, W] with an odd square window, float64."""
    img = np.asarray(img, np.float64)
    k = window.shape[0]
    r = k // 2
    h, w = img.shape
    pad = np.zeros((h + 2 * r, w + 2 * r))
    pad[r:r + h, r:r + w] = img
    out = np.zeros((h, w))
    win = window.astype(np.float64)
    for i in range(k):
        for j in range(k):
            out += win[i, j] * pad[i:i + h, j:j + w]
    return out


def ssim_terms(x, y, window_size=11):
    """SSIM map S and its partials A = dS/dmu_x, B = dS/dE[x^2], C = dS/dE[xy]."""
    _, win = gaussian_window(window_size)
    x = np.asarray(x, np.float64)
    y = np.asarray(y, np.float64)
    mu1, mu2 = filter2d(x, win), filter2d(y, win)
    m11, m22, m12 = filter2d(x * x, win), filter2d(y * y, win), filter2d(x * y, win)
    s11, s22, s12 = m11 - mu1 ** 2, m22 - mu2 ** 2, m12 - mu1 * mu2
    n1, n2 = 2 * mu1 * mu2 + C1, 2 * s12 + C2
    d1, d2 = mu1 ** 2 + mu2 ** 2 + C1, s11 + s22 + C2
    S = n1 * n2 / (d1 * d2)
    A = 2 * mu2 * (n2 - n1) / (d1 * d2) - 2 * mu1 * S * (1 / d1 - 1 / d2)
    B = -S / d2
    C = 2 * n1 / (d1 * d2)
    return S, A, B, C


def projection_losses(x, y, e=None, m=None, window_size=11):
    """(l1, 1 - mean SSIM, mean m |x - e|) over images [n, H, W]."""
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    s = sum(ssim_terms(x[i], y[i], window_size)[0].sum() for i in range(x.shape[0]))
    n = x.size
    l1 = np.abs(x - y).sum() / n
    edge = 0.0 if e is None else (np.asarray(m, np.float64) * np.abs(x - e)).sum() / n
    return l1, 1.0 - s / n, edge


def projection_loss_grad(x, y, e=None, m=None, scales=(1.0, 1.0, 1.0), window_size=11):
    """d(scales . losses)/dx over images [n, H, W] (sign(0) = 0, as torch)."""
    _, win = gaussian_window(window_size)
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    n = x.size
    g = scales[0] * np.sign(x - y) / n
    for i in range(x.shape[0]):
        _, A, B, C = ssim_terms(x[i], y[i], window_size)
        d = filter2d(A, win) + 2 * x[i] * filter2d(B, win) + y[i] * filter2d(C, win)
        g[i] -= scales[1] * d / n
    if e is not None:
        g += scales[2] * np.asarray(m, np.float64) * np.sign(x - np.asarray(e, np.float64)) / n
    return g


def projection_loss_grad_magnitude(x, y, e=None, m=None, scales=(1.0, 1.0, 1.0),
                                   window_size=11):
    """Sum of the absolute values of the terms of projection_loss_grad, per
    pixel: sign terms |s| / n, and s_ssim (G*|A| + 2|x| G*|B| + |y| G*|C|) / n
    with |A| the sum of the absolute values of A's four terms.  Where the
    window's variances vanish (window size 1, flat regions), 2 x G*B and the
    -2 mu_x S / d2 term of G*A are of size 2 x S / c2 ~ 1e3 and cancel: any
    float32 evaluation then differs from the exact gradient by about u times
    this magnitude, not u times the gradient."""
    _, win = gaussian_window(window_size)
    x, y = np.asarray(x, np.float64), np.asarray(y, np.float64)
    n = x.size
    g = np.full(x.shape, abs(scales[0]) / n)
    for i in range(x.shape[0]):
        mu1, mu2 = filter2d(x[i], win), filter2d(y[i], win)
        m11, m22, m12 = filter2d(x[i] * x[i], win), filter2d(y[i] * y[i], win), filter2d(
            x[i] * y[i], win)
        s11, s22, s12 = m11 - mu1 ** 2, m22 - mu2 ** 2, m12 - mu1 * mu2
        n1, n2 = 2 * mu1 * mu2 + C1, 2 * s12 + C2
        d1, d2 = mu1 ** 2 + mu2 ** 2 + C1, s11 + s22 + C2
        S = n1 * n2 / (d1 * d2)
        a_abs = (np.abs(2 * mu2 * n2 / (d1 * d2)) + np.abs(2 * mu2 * n1 / (d1 * d2))
                 + np.abs(2 * mu1 * S / d1) + np.abs(2 * mu1 * S / d2))
        B, C = -S / d2, 2 * n1 / (d1 * d2)
        t = (filter2d(a_abs, win) + 2 * np.abs(x[i]) * filter2d(np.abs(B), win)
             + np.abs(y[i]) * filter2d(np.abs(C), win))
        g[i] += abs(scales[1]) * t / n
    if e is not None:
        g += abs(scales[2]) * np.abs(np.asarray(m, np.float64)) / n
    return g


def tv(vol, reduction="mean"):
    """loss.py:10-21 compute_tv_loss in float64."""
    v = np.asarray(vol, np.float64)
    terms = [np.abs(np.diff(v, axis=a)) for a in range(3)]
    total = sum(t.sum() for t in terms)
    if reduction == "mean":
        total = total / max(1, sum(t.size for t in terms))
    return total


def tv_grad(vol, grad_out=1.0, reduction="mean"):
    """d tv / d vol * grad_out: per axis sgn(v - v_prev) - sgn(v_next - v)."""
    v = np.asarray(vol, np.float64)
    g = np.zeros_like(v)
    count = 0
    for a in range(3):
        s = np.sign(np.diff(v, axis=a))
        count += s.size
        lo = [slice(None)] * 3
        hi = [slice(None)] * 3
        lo[a] = slice(0, -1)
        hi[a] = slice(1, None)
        g[tuple(lo)] -= s
        g[tuple(hi)] += s
    scale = grad_out / max(1, count) if reduction == "mean" else grad_out
    return g * scale


def hierarchy_loss(child_means, parent, hist_means, parent_scales, hist_quats, history_count,
                   factor=1.0):
    """loss.py:27-71 compute_hierarchy_loss (archived scales already activated),
    float64: returns (loss, d loss / d child_means)."""
    c = np.asarray(child_means, np.float64)
    par = np.asarray(parent).astype(np.int64)
    valid = (par >= 0) & (par < history_count)
    grad = np.zeros_like(c)
    if not valid.any():
        return 0.0, grad
    ids = par[valid]
    q = np.asarray(hist_quats, np.float64)[ids]
    q = q / np.maximum(np.linalg.norm(q, axis=1), 1e-12)[:, None]
    w, x, y, z = q.T
    R = np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
                  2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
                  2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
                 -1).reshape(-1, 3, 3)
    s = np.maximum(np.asarray(parent_scales, np.float64)[ids], 1e-6)
    d = c[valid] - np.asarray(hist_means, np.float64)[ids]
    u = np.einsum("nji,nj->ni", R, d) / s
    r = np.linalg.norm(u, axis=1)
    a = max(float(factor), 1e-6)
    e = np.maximum(r - a, 0.0) / a
    n = int(valid.sum())
    k = np.where(e > 0, 2 * e / (a * np.where(r > 0, r, 1.0) * n), 0.0)
    grad[valid] = np.einsum("nij,nj->ni", R, (k[:, None] * u / s))
    return float((e * e).mean()), grad


def hierarchy_grad_magnitude(child_means, parent, hist_means, parent_scales, hist_quats,
                             history_count, factor=1.0):
    """Per child and component, a first-order bound (in units of the unit
    roundoff) on the error of evaluating d loss / d child_means in another
    order: the gradient is R v with v = k u / s, so component i sums
    |R_ij v_j| (which cancel when the child lies along a principal axis),
    each carrying the relative error of v: the difference d = c - p cancels
    when the child is near the parent (|c| + |p|) / |d|, and the excess
    r - a when it is near the parent's ellipsoid (r + a) / |r - a|."""
    c = np.asarray(child_means, np.float64)
    par = np.asarray(parent).astype(np.int64)
    valid = (par >= 0) & (par < history_count)
    out = np.zeros_like(c)
    if not valid.any():
        return out
    ids = par[valid]
    q = np.asarray(hist_quats, np.float64)[ids]
    q = q / np.maximum(np.linalg.norm(q, axis=1), 1e-12)[:, None]
    w, x, y, z = q.T
    R = np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
                  2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
                  2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
                 -1).reshape(-1, 3, 3)
    s = np.maximum(np.asarray(parent_scales, np.float64)[ids], 1e-6)
    pm = np.asarray(hist_means, np.float64)[ids]
    d = c[valid] - pm
    u = np.einsum("nji,nj->ni", R, d) / s
    r = np.linalg.norm(u, axis=1)
    a = max(float(factor), 1e-6)
    e = np.maximum(r - a, 0.0) / a
    n = int(valid.sum())
    k = np.where(e > 0, 2 * e / (a * np.where(r > 0, r, 1.0) * n), 0.0)
    v = k[:, None] * u / s
    excess = (r + a) / np.maximum(np.abs(r - a), 1e-300)
    near = (np.abs(c[valid]).sum(1) + np.abs(pm).sum(1)) / np.maximum(
        np.linalg.norm(d, axis=1), 1e-300)
    rel = 1 + excess + near * (1 + r / np.maximum(np.abs(r - a), 1e-300))
    out[valid] = np.einsum("nij,nj->ni", np.abs(R), np.abs(v)) * rel[:, None]
    return out
