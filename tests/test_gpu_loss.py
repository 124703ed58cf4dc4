"""Fused projection loss (L1 + SSIM + edge), volume TV and hierarchy loss
against the oracle.

The oracle is float64 on the float32 inputs.  Losses agree within 1e-5
absolute.  Gradients meet helpers.assert_parity (rel 1e-4 / abs 1e-5, or
within twice the error of the reference's own float32 formulation -- the
torch restatement of src/utils/loss.py / metric.py below -- against the
float64 oracle, or within 8 u times the sum of |terms| of the gradient's
formula where it cancels: oracle/loss.py *_magnitude), compared as gradients
of the summed loss, i.e. scaled by the mean's element count, so that the
absolute term means the same at every image size.
"""

import numpy as np
import pytest
import torch

from helpers import assert_parity, np32
from oracle import loss as L
from r2splat.ops import loss as LO

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _images(n, h, w, seed, edge=True):
    rng = np.random.default_rng(seed)
    x = rng.uniform(0, 1, (n, h, w)).astype(np.float32)
    y = np.clip(x + rng.normal(0, 0.15, x.shape), 0, 1).astype(np.float32)
    e = np.clip(x + rng.normal(0, 0.3, x.shape), 0, 1).astype(np.float32) if edge else None
    m = (rng.uniform(size=x.shape) < 0.2).astype(np.float32) if edge else None
    return x, y, e, m


def _t(a):
    return None if a is None else torch.from_numpy(a)[..., None].to(DEV)  # [n, H, W, 1]


CASES = [(1, 64, 64, 11), (3, 50, 70, 11), (1, 512, 512, 11), (2, 33, 47, 7), (1, 40, 40, 1),
         (1, 45, 38, 15)]


@pytest.mark.parametrize("n,h,w,ws", CASES)
@pytest.mark.parametrize("edge", [True, False])
def test_projection_losses_and_gradient(n, h, w, ws, edge):
    x, y, e, m = _images(n, h, w, 100 + h + ws, edge)
    scales = (1.0, 0.25, 0.8)
    r = _t(x).requires_grad_(True)
    l1, sl, ed = LO.projection_losses(r, _t(y), _t(m), _t(e), ssim_window=ws)
    el1, esl, eed = L.projection_losses(x, y, e, m, ws)
    assert abs(l1.item() - el1) < 1e-6 * max(1, el1) + 1e-7
    assert abs(sl.item() - esl) < 1e-5
    assert abs(ed.item() - eed) < 1e-6 * max(1, eed) + 1e-7
    (scales[0] * l1 + scales[1] * sl + scales[2] * ed).backward()
    n_el = x.size
    g = np32(r.grad)[..., 0].astype(np.float64) * n_el
    expect = L.projection_loss_grad(x, y, e, m, scales, ws) * n_el
    lowp = _torch_f32_grad(x, y, e, m, scales, ws).astype(np.float64) * n_el
    mag = L.projection_loss_grad_magnitude(x, y, e, m, scales, ws) * n_el
    print(assert_parity(g.astype(np.float32), expect, lowp, None, "n * d loss / d render",
                        mag=mag))


def _torch_f32_grad(x, y, e, m, scales, ws):
    """d(scales . losses)/dx of the reference's float32 formulation
    (src/utils/metric.py:36-54 ssim with a conv2d of the float32 window,
    src/utils/loss.py:135-172 l1 / edge means), by torch autograd on the CPU."""
    _, win = L.gaussian_window(ws)
    w = torch.tensor(win, dtype=torch.float32)[None, None]
    xt = torch.tensor(x, requires_grad=True)
    yt = torch.tensor(y)
    conv = lambda t: torch.nn.functional.conv2d(t[:, None], w, padding=ws // 2)  # noqa: E731
    mu1, mu2 = conv(xt), conv(yt)
    s11 = conv(xt * xt) - mu1 * mu1
    s22 = conv(yt * yt) - mu2 * mu2
    s12 = conv(xt * yt) - mu1 * mu2
    S = ((2 * mu1 * mu2 + L.C1) * (2 * s12 + L.C2)) / ((mu1 * mu1 + mu2 * mu2 + L.C1) *
                                                        (s11 + s22 + L.C2))
    total = scales[0] * (xt - yt).abs().mean() + scales[1] * (1 - S.mean())
    if e is not None:
        total = total + scales[2] * (torch.tensor(m) * (xt - torch.tensor(e)).abs()).mean()
    total.backward()
    return xt.grad.numpy()


def test_projection_loss_is_deterministic():
    x, y, e, m = _images(2, 96, 80, 7)
    outs = []
    for _ in range(2):
        r = _t(x).requires_grad_(True)
        l1, sl, ed = LO.projection_losses(r, _t(y), _t(m), _t(e))
        (l1 + sl + ed).backward()
        outs.append((l1.item(), sl.item(), ed.item(), r.grad.clone()))
    assert outs[0][:3] == outs[1][:3]
    assert torch.equal(outs[0][3], outs[1][3])


def test_binary_tree_loss_computer_matches_the_oracle_total():
    x, y, e, m = _images(1, 128, 96, 8)
    rng = np.random.default_rng(9)
    vol = rng.normal(size=(32, 32, 32)).astype(np.float32)
    comp = LO.BinaryTreeLossComputer(w_l1=1.0, w_ssim=0.25, w_tv=0.05, w_edge=0.5,
                                     w_hierarchy=0.05, ssim_window=11)
    r = _t(x).requires_grad_(True)
    v = torch.from_numpy(vol)[None].to(DEV).requires_grad_(True)
    hier = torch.tensor(0.3, device=DEV, requires_grad=True)
    out = comp(r, _t(y), _t(m), v, hierarchy_loss=hier, edge_targets=_t(e),
               edge_weight_override=0.7)
    assert set(out) == {"proj_l1", "proj_ssim", "vol_tv", "edge", "hierarchy", "edge_weight",
                        "total"}
    el1, esl, eed = L.projection_losses(x, y, e, m)
    etv = L.tv(vol)
    expect = 1.0 * el1 + 0.25 * esl + 0.05 * etv + 0.7 * eed + 0.05 * 0.3
    assert abs(out["total"].item() - expect) < 2e-5
    out["total"].backward()
    gx = L.projection_loss_grad(x, y, e, m, (1.0, 0.25, 0.7))
    assert np.abs(np32(r.grad)[..., 0] - gx).max() < 2e-3 * np.abs(gx).max()
    np.testing.assert_allclose(np32(v.grad)[0], L.tv_grad(vol, 0.05), rtol=1e-6, atol=1e-12)
    assert abs(hier.grad.item() - 0.05) < 1e-8
    assert out["edge_weight"].item() == np.float32(0.7)
    # Each term stays differentiable on its own (the SSIM term alone here).
    r2 = _t(x).requires_grad_(True)
    comp(r2, _t(y), _t(m), None, edge_targets=_t(e))["proj_ssim"].backward()
    gs = L.projection_loss_grad(x, y, e, m, (0.0, 1.0, 0.0))
    assert np.abs(np32(r2.grad)[..., 0] - gs).max() < 2e-3 * np.abs(gs).max()
    # A plain-number hierarchy term, as the reference's arithmetic accepts.
    num = comp(_t(x), _t(y), _t(m), None, hierarchy_loss=0.3, edge_targets=_t(e))
    assert abs(num["total"].item() - (el1 + 0.25 * esl + 0.5 * eed + 0.05 * 0.3)) < 2e-5
    plain = LO.LossComputer(w_l1=1.0, w_ssim=0.25, w_tv=0.0)(_t(x), _t(y))
    assert set(plain) == {"proj_l1", "proj_ssim", "vol_tv", "total"}
    assert plain["vol_tv"].item() == 0.0


def test_ssim2d_metric():
    x, y, _, _ = _images(2, 70, 60, 10, edge=False)
    a = torch.from_numpy(x)[:, None].to(DEV)
    b = torch.from_numpy(y)[:, None].to(DEV)
    assert abs(LO.ssim2d(a, b).item() - (1 - L.projection_losses(x, y)[1])) < 1e-5
    assert abs(LO.ssim2d(a, a).item() - 1.0) < 1e-6


@pytest.mark.parametrize("shape", [(32, 32, 32), (1, 40, 33, 17), (128, 128, 128), (1, 1, 5),
                                   (1, 1, 1)])
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_tv_loss_and_gradient(shape, reduction):
    rng = np.random.default_rng(sum(shape))
    vol = rng.normal(size=shape).astype(np.float32)
    vol[..., :2] = 0.0  # exact zero differences: sign(0) = 0
    v = torch.from_numpy(vol).to(DEV).requires_grad_(True)
    tv = LO.compute_tv_loss(v, reduction)
    base = vol[0] if vol.ndim == 4 else vol
    expect = L.tv(base, reduction)
    assert abs(tv.item() - expect) <= 1e-6 * abs(expect) + 1e-7
    (tv * 3.0).backward()
    g = np32(v.grad)
    g = g[0] if g.ndim == 4 else g
    np.testing.assert_allclose(g, L.tv_grad(base, 3.0, reduction), rtol=1e-6, atol=1e-12)


def _sigmoid_scales(raw):
    return 5e-4 + (1.0 - 5e-4) * torch.sigmoid(raw)


@pytest.mark.parametrize("n,h", [(5000, 3000), (20, 0), (64, 5)])
def test_hierarchy_loss_and_gradient(n, h):
    rng = np.random.default_rng(n + h)
    hm = rng.normal(size=(max(h, 1), 3)).astype(np.float32)[:h]
    hs = rng.normal(-1.5, 0.5, size=(h, 3)).astype(np.float32)
    hq = rng.normal(size=(h, 4)).astype(np.float32)
    par = rng.integers(-3, h + 3, n).astype(np.int32) if h else np.full(n, -1, np.int32)
    base = hm[np.clip(par, 0, max(h - 1, 0))] if h else np.zeros((n, 3), np.float32)
    cm = (base + rng.normal(0, 0.3, (n, 3))).astype(np.float32)
    c = torch.from_numpy(cm).to(DEV).requires_grad_(True)
    loss = LO.compute_hierarchy_loss(c, torch.from_numpy(par).to(DEV), torch.from_numpy(hm).to(DEV),
                                     torch.from_numpy(hs).to(DEV), torch.from_numpy(hq).to(DEV),
                                     _sigmoid_scales, 0.9)
    if h == 0:
        assert loss.item() == 0.0 and not loss.requires_grad
        return
    act = np32(_sigmoid_scales(torch.from_numpy(hs)))
    exp_loss, exp_grad = L.hierarchy_loss(cm, par, hm, act, hq, h, 0.9)
    assert abs(loss.item() - exp_loss) <= 1e-5 * max(1.0, exp_loss)
    (loss * 2.0).backward()
    k = int(((par >= 0) & (par < h)).sum())  # the mean's count
    g = np32(c.grad).astype(np.float64) * k
    lowp = _torch_f32_hierarchy_grad(cm, par, hm, act, hq, h, 0.9) * 2.0 * k
    mag = L.hierarchy_grad_magnitude(cm, par, hm, act, hq, h, 0.9) * 2.0 * k
    print(assert_parity(g.astype(np.float32), 2.0 * exp_grad * k, lowp, None,
                        "count * d loss / d child_means", mag=mag))


def _torch_f32_hierarchy_grad(cm, par, hm, act, hq, h, factor):
    """src/utils/loss.py:27-71 in float32 torch on the CPU (autograd)."""
    c = torch.tensor(cm, requires_grad=True)
    p = torch.tensor(par).long()
    valid = (p >= 0) & (p < h)
    ids = p[valid]
    q = torch.nn.functional.normalize(torch.tensor(hq)[ids], dim=-1)
    w, x, y, z = q.unbind(-1)
    R = torch.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
                     2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
                     2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
                    -1).reshape(-1, 3, 3)
    s = torch.tensor(act)[ids].clamp_min(1e-6)
    d = c[valid] - torch.tensor(hm)[ids]
    u = (R.transpose(1, 2) @ d[..., None])[..., 0] / s
    a = max(float(factor), 1e-6)
    e = torch.relu(u.norm(dim=-1) - a) / a
    (e * e).mean().backward()
    return c.grad.numpy().astype(np.float64)
