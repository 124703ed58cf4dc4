"""Pins the oracle's element-wise operators (oracle/ops.py) on the CPU.

Each check uses a formulation independent of the oracle's hand-expanded
expressions: dense matrix products and torch.linalg in float64, torch
autograd for the VJPs, closed-form special cases and the literal known-answer
inputs of the reference's tests/test_cuda_gaussian_ops.py.
"""

import math

import numpy as np
import pytest
import torch

from oracle import ops



@pytest.fixture(autouse=True)
def _float64_default():
    # Dense references in this module are float64; restore the global default.
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)
SMIN, SMAX = 5e-4, 1.0


def _rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------ parameter transform --

def _covars_closed_form(quats, scales):
    # tests/test_cuda_gaussian_ops.py:32-50 (the reference test's own formula)
    rot = torch.nn.functional.normalize(quats, dim=-1)
    w, x, y, z = rot.unbind(-1)
    m = torch.stack((1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
                     2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
                     2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)),
                    -1).reshape(-1, 3, 3)
    full = m @ torch.diag_embed(scales.square()) @ m.transpose(-1, -2)
    return full[:, (0, 0, 0, 1, 1, 2), (0, 1, 2, 1, 2, 2)]


def test_parameter_transform_matches_closed_form_and_autograd():
    r = _rng(0)
    q = r.normal(size=(500, 4)) * 0.7
    s = r.normal(size=(500, 3))
    cov, ms = ops.parameter_transform_fwd(q, s, SMIN, SMAX)
    qt, st = torch.tensor(q, requires_grad=True), torch.tensor(s, requires_grad=True)
    scales = SMIN + (SMAX - SMIN) * torch.sigmoid(st)
    ref = _covars_closed_form(qt, scales)
    np.testing.assert_allclose(cov, ref.detach().numpy(), rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(ms, scales.detach().amax(-1).numpy(), rtol=1e-14)
    v = r.normal(size=(500, 6))
    vq, vs = ops.parameter_transform_bwd(q, s, SMIN, SMAX, v)
    gq, gs = torch.autograd.grad((ref * torch.tensor(v)).sum(), (qt, st))
    np.testing.assert_allclose(vq, gq.numpy(), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(vs, gs.numpy(), rtol=1e-9, atol=1e-12)
    # float32 restatement stays within the parity tolerance of float64.
    cov32, _ = ops.parameter_transform_fwd(q.astype(np.float32), s.astype(np.float32), SMIN, SMAX)
    assert cov32.dtype == np.float32
    np.testing.assert_allclose(cov32, cov, rtol=1e-4, atol=1e-6)


def test_parameter_transform_invariants():
    r = _rng(1)
    s = r.normal(size=(64, 3))
    sc = SMIN + (SMAX - SMIN) / (1 + np.exp(-s))
    ident = np.tile([1.0, 0, 0, 0], (64, 1))
    cov, ms = ops.parameter_transform_fwd(ident, s, SMIN, SMAX)
    np.testing.assert_allclose(cov[:, [0, 3, 5]], sc ** 2, rtol=1e-14)
    np.testing.assert_array_equal(cov[:, [1, 2, 4]], 0.0)
    np.testing.assert_allclose(ms, sc.max(-1), rtol=1e-15)
    q = r.normal(size=(64, 4))
    c1, _ = ops.parameter_transform_fwd(q, s, SMIN, SMAX)
    c3, _ = ops.parameter_transform_fwd(3.0 * q, s, SMIN, SMAX)  # scale invariance
    np.testing.assert_allclose(c1, c3, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(c1[:, 0] + c1[:, 3] + c1[:, 5], (sc ** 2).sum(-1), rtol=1e-12)
    full = c1[:, [0, 1, 2, 1, 3, 4, 2, 4, 5]].reshape(-1, 3, 3)
    assert (np.linalg.eigvalsh(full) > 0).all()


def test_softplus_matches_torch():
    x = np.linspace(-30, 30, 1001)
    np.testing.assert_allclose(ops.softplus(x), torch.nn.functional.softplus(torch.tensor(x)),
                               rtol=1e-15, atol=1e-300)


# -------------------------------------------------------------- projection --

def _scene(n, seed, width=64, height=48):
    r = _rng(seed)
    means = r.uniform(-1, 1, size=(n, 3))
    q = r.normal(size=(n, 4))
    s = r.normal(-3.0, 0.6, size=(n, 3))
    covars, _ = ops.parameter_transform_fwd(q, s, SMIN, SMAX)
    ang = r.uniform(0, 2 * math.pi)
    # Cone-beam pose: source on a circle of radius 1.2 looking at the origin
    # (inside the cube's corner region, so some Gaussians fall behind it).
    cam = np.array([1.2 * math.cos(ang), 1.2 * math.sin(ang), 0.1])
    fwd = -cam / np.linalg.norm(cam)
    right = np.cross(fwd, [0, 0, 1.0])
    right /= np.linalg.norm(right)
    down = np.cross(fwd, right)
    R = np.stack([right, down, fwd])
    vm = np.eye(4)
    vm[:3, :3] = R
    vm[:3, 3] = -R @ cam
    K = np.array([[70.0, 0, width / 2 + 1.5], [0, 66.0, height / 2 - 2.0], [0, 0, 1]])
    return means, covars, vm[None], K[None]


def _torch_projection(means, covars, vm, K, width, height):
    """Matrix formulation: p_c = R p + t, J with the FOV clamp, cov = J Sc J^T."""
    R, t = vm[:3, :3], vm[:3, 3]
    fx, fy, cx, cy = K[0, 0], K[1, 1], K[0, 2], K[1, 2]
    pc = means @ R.T + t
    x, y, z = pc.unbind(-1)
    m2 = torch.stack([fx * x / z + cx, fy * y / z + cy], -1)
    tfx, tfy = 0.5 * width / fx, 0.5 * height / fy
    tx = z * torch.clamp(x / z, -(cx / fx + 0.3 * tfx), (width - cx) / fx + 0.3 * tfx)
    ty = z * torch.clamp(y / z, -(cy / fy + 0.3 * tfy), (height - cy) / fy + 0.3 * tfy)
    ln = torch.sqrt(tx * tx + ty * ty + z * z)
    zero = torch.zeros_like(z)
    J = torch.stack([torch.stack([fx / z, zero, -fx * tx / z ** 2], -1),
                     torch.stack([zero, fy / z, -fy * ty / z ** 2], -1),
                     torch.stack([tx / ln, ty / ln, z / ln], -1)], -2)
    S = covars[:, [0, 1, 2, 1, 3, 4, 2, 4, 5]].reshape(-1, 3, 3)
    Sc = R @ S @ R.T
    cov = J @ Sc @ J.transpose(-1, -2)
    return m2, cov[:, (0, 0, 0, 1, 1, 2), (0, 1, 2, 1, 2, 2)], z


def test_projection_forward_matches_matrix_formulation():
    W_, H_ = 64, 48
    means, covars, vm, K = _scene(3000, 2, W_, H_)
    m2, c2, radii = ops.world_to_image_projection_fwd(means, covars, vm, K, W_, H_, 1e-8, 3.0)
    tm2, tc2, z = _torch_projection(torch.tensor(means), torch.tensor(covars),
                                    torch.tensor(vm[0]), torch.tensor(K[0]), W_, H_)
    keep = (z > 0.01).numpy()
    assert keep.sum() > 2000 and (~keep).sum() > 10
    np.testing.assert_allclose(m2[0][keep], tm2.numpy()[keep], rtol=1e-12, atol=1e-10)
    np.testing.assert_allclose(c2[0][keep], tc2.numpy()[keep], rtol=1e-10, atol=1e-12)
    assert (m2[0][~keep] == 0).all() and (c2[0][~keep] == 0).all() and (radii[0][~keep] == 0).all()
    # Radii: ceil(3 sqrt(var + eps)) per axis where the blurred 2x2 is PD and on screen.
    a, d = tc2[:, 0].numpy() + 1e-8, tc2[:, 3].numpy() + 1e-8
    rx, ry = np.ceil(3 * np.sqrt(a)), np.ceil(3 * np.sqrt(d))
    mx, my = tm2[:, 0].numpy(), tm2[:, 1].numpy()
    on = keep & (a * d - tc2[:, 1].numpy() ** 2 > 0) & ~((mx + rx <= 0) | (mx - rx >= W_)
                                                         | (my + ry <= 0) | (my - ry >= H_))
    assert on.sum() > 100 and (~on & keep).sum() > 10
    np.testing.assert_array_equal(radii[0][on], np.stack([rx, ry], -1)[on])
    assert (radii[0][~on] == 0).all()


def test_projection_special_cases():
    # A Gaussian on the optical axis projects to the principal point exactly.
    vm = np.eye(4)[None]
    K = np.array([[[100.0, 0, 31.5], [0, 90.0, 20.25], [0, 0, 1]]])
    means = np.array([[0.0, 0.0, 2.0], [0.0, 0.0, 0.005], [0.0, 0.0, -1.0]])
    covars = np.tile([0.01, 0, 0, 0.01, 0, 0.01], (3, 1))
    m2, c2, r = ops.world_to_image_projection_fwd(means, covars, vm, K, 64, 40, 1e-8, 3.0)
    np.testing.assert_array_equal(m2[0, 0], [31.5, 20.25])
    # Isotropic on-axis: a = fx^2 s^2 / z^2, f = s^2 (ray row is the unit z axis).
    np.testing.assert_allclose(c2[0, 0], [100 ** 2 * 0.01 / 4, 0, 0, 90 ** 2 * 0.01 / 4, 0, 0.01],
                               rtol=1e-14, atol=1e-16)
    assert (m2[0, 1:] == 0).all() and (c2[0, 1:] == 0).all() and (r[0, 1:] == 0).all()


def test_projection_backward_matches_autograd():
    W_, H_ = 64, 48
    means, covars, vm, K = _scene(2000, 3, W_, H_)
    r = _rng(4)
    v_m2 = r.normal(size=(1, 2000, 2))
    v_c2 = r.normal(size=(1, 2000, 6))
    vm_o, vc_o = ops.world_to_image_projection_bwd(means, covars, vm, K, W_, H_, v_m2, v_c2)
    mt = torch.tensor(means, requires_grad=True)
    ct = torch.tensor(covars, requires_grad=True)
    tm2, tc2, z = _torch_projection(mt, ct, torch.tensor(vm[0]), torch.tensor(K[0]), W_, H_)
    keep = (z > 0.01).detach()
    loss = ((tm2 * torch.tensor(v_m2[0])).sum(-1) + (tc2 * torch.tensor(v_c2[0])).sum(-1))
    gm, gc = torch.autograd.grad(loss[keep].sum(), (mt, ct))
    np.testing.assert_allclose(vm_o, gm.numpy(), rtol=1e-8, atol=1e-9)
    np.testing.assert_allclose(vc_o, gc.numpy(), rtol=1e-8, atol=1e-9)
    # Two cameras sum their VJPs.
    vm2 = np.concatenate([vm, vm])
    K2 = np.concatenate([K, K])
    v2m, v2c = ops.world_to_image_projection_bwd(means, covars, vm2, K2, W_, H_,
                                                 np.concatenate([v_m2, v_m2]),
                                                 np.concatenate([v_c2, v_c2]))
    np.testing.assert_allclose(v2m, 2 * vm_o, rtol=1e-14, atol=1e-14)


def test_projection_backward_finite_differences():
    W_, H_ = 64, 48
    means, covars, vm, K = _scene(40, 5, W_, H_)
    r = _rng(6)
    v_m2, v_c2 = r.normal(size=(1, 40, 2)), r.normal(size=(1, 40, 6))
    vm_o, vc_o = ops.world_to_image_projection_bwd(means, covars, vm, K, W_, H_, v_m2, v_c2)

    def loss(m, c):
        a, b, _ = ops.world_to_image_projection_fwd(m, c, vm, K, W_, H_, 1e-8, 3.0)
        return float((a * v_m2).sum() + (b * v_c2).sum())

    h = 1e-6
    for g in range(0, 40, 7):
        for k in range(3):
            mp, mn = means.copy(), means.copy()
            mp[g, k] += h
            mn[g, k] -= h
            fd = (loss(mp, covars) - loss(mn, covars)) / (2 * h)
            assert abs(fd - vm_o[g, k]) <= 1e-5 * (1 + abs(fd)), (g, k, fd, vm_o[g, k])


# ---------------------------------------------------------------- conics/mu --

def _unpack(c, eps):
    return c[..., [0, 1, 2, 1, 3, 4, 2, 4, 5]].reshape(c.shape[:-1] + (3, 3)) + eps * torch.eye(3)


@pytest.mark.parametrize("eps", [0.0, 1e-8])
def test_conics_mu_reference_kats(eps):
    # Literal inputs of tests/test_cuda_gaussian_ops.py:102-115.
    cov = np.array([[[1e-2, 0.0, 0.0, 1e-2, 0.0, f] for f in (1e-6, 9e-6, 11e-6, 1e-4)],
                    [[1e-2, 2e-3, 1e-5, 2e-2, -2e-5, f] for f in (1e-6, 4e-6, 6e-6, 1e-4)]])
    conics, mus = ops.conics_mu_fwd(cov, eps)
    ref = torch.tensor(cov, requires_grad=True)
    full = _unpack(ref, eps)
    d2, d3 = torch.linalg.det(full[..., :2, :2]), torch.linalg.det(full)
    con_ref = torch.linalg.inv(full[..., :2, :2])[..., (0, 0, 1), (0, 1, 1)]
    mu_ref = (2 * math.pi * d3 / d2).sqrt()
    np.testing.assert_allclose(conics, con_ref.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(mus, mu_ref.detach().numpy(), rtol=1e-12)
    v_con = np.linspace(-0.2, 0.3, conics.size).reshape(conics.shape)
    v_mu = np.linspace(0.5, 1.2, mus.size).reshape(mus.shape)
    got = ops.conics_mu_bwd(cov, eps, conics, mus, v_con, v_mu)
    gate = (d3 > 1e-9).detach()  # ConicsMuBwd.cu:139-140
    assert gate.any() and (~gate).any()
    exp = torch.autograd.grad((con_ref * torch.tensor(v_con)).sum()
                              + (mu_ref * torch.tensor(v_mu) * gate).sum(), ref)[0]
    np.testing.assert_allclose(got, exp.numpy(), rtol=1e-9, atol=1e-12)


def test_conics_mu_degenerate_cases():
    # tests/test_cuda_gaussian_ops.py:155-197 inputs.
    for last in (0.0, -1e-6):
        cov = np.array([[[1e-2, 2e-3, 0.0, 2e-2, 0.0, last]]])
        con, mu = ops.conics_mu_fwd(cov, 0.0)
        assert mu[0, 0] == 0.0
        ref = torch.tensor(cov, requires_grad=True)
        inv2 = torch.linalg.inv(_unpack(ref, 0.0)[..., :2, :2])[..., (0, 0, 1), (0, 1, 1)]
        np.testing.assert_allclose(con, inv2.detach().numpy(), rtol=1e-12)
        g = ops.conics_mu_bwd(cov, 0.0, con, mu, np.ones_like(con), np.ones_like(mu))
        exp = torch.autograd.grad(inv2.sum(), ref)[0]
        np.testing.assert_allclose(g, exp.numpy(), rtol=1e-10, atol=1e-12)
    cov = np.array([[[1e-6, 0.0, 0.0, 1e-6, 0.0, 1.0]]])
    con, mu = ops.conics_mu_fwd(cov, 1e-8)
    assert (con == 0).all() and (mu == 0).all()
    assert (ops.conics_mu_bwd(cov, 1e-8, con, mu, np.ones_like(con), np.ones_like(mu)) == 0).all()


def test_conics_mu_random_pd_matches_autograd():
    r = _rng(7)
    A = r.normal(size=(400, 3, 3))
    S = A @ A.transpose(0, 2, 1) + 0.1 * np.eye(3)
    cov = S[:, [0, 0, 0, 1, 1, 2], [0, 1, 2, 1, 2, 2]][None]
    con, mu = ops.conics_mu_fwd(cov, 1e-8)
    ref = torch.tensor(cov, requires_grad=True)
    full = _unpack(ref, 1e-8)
    con_ref = torch.linalg.inv(full[..., :2, :2])[..., (0, 0, 1), (0, 1, 1)]
    mu_ref = (2 * math.pi * torch.linalg.det(full) / torch.linalg.det(full[..., :2, :2])).sqrt()
    np.testing.assert_allclose(con, con_ref.detach().numpy(), rtol=1e-10)
    np.testing.assert_allclose(mu, mu_ref.detach().numpy(), rtol=1e-12)
    vc, vm = r.normal(size=con.shape), r.normal(size=mu.shape)
    g = ops.conics_mu_bwd(cov, 1e-8, con, mu, vc, vm)
    e = torch.autograd.grad((con_ref * torch.tensor(vc)).sum() + (mu_ref * torch.tensor(vm)).sum(),
                            ref)[0]
    np.testing.assert_allclose(g, e.numpy(), rtol=1e-8, atol=1e-10)


# ----------------------------------------------------------- volume mapping --

def test_volume_mapping_matches_linalg_and_autograd():
    r = _rng(8)
    n = 600
    means = r.uniform(-1, 1, size=(n, 3))
    covars, _ = ops.parameter_transform_fwd(r.normal(size=(n, 4)), r.normal(-3, 0.5, (n, 3)),
                                            SMIN, SMAX)
    ranges, centers = np.array([2.0, 1.6, 2.4]), np.array([0.1, -0.05, 0.2])
    dims = (48, 40, 56)
    m3, con, rad = ops.world_to_volume_mapping_fwd(means, covars, ranges, centers, *dims, 1e-8, 3.0)
    scale = np.array(dims) / ranges
    np.testing.assert_allclose(m3, (means - centers) * scale + np.array(dims) / 2, rtol=1e-14)
    ct = torch.tensor(covars, requires_grad=True)
    mt = torch.tensor(means, requires_grad=True)
    D = torch.diag(torch.tensor(scale))
    Sv = D @ ct[:, [0, 1, 2, 1, 3, 4, 2, 4, 5]].reshape(-1, 3, 3) @ D + 1e-8 * torch.eye(3)
    P = torch.linalg.inv(Sv)[:, (0, 0, 0, 1, 1, 2), (0, 1, 2, 1, 2, 2)]
    np.testing.assert_allclose(con, P.detach().numpy(), rtol=1e-9)
    sv = torch.diagonal(Sv.detach(), dim1=-2, dim2=-1).numpy()
    np.testing.assert_array_equal(rad, np.ceil(3 * np.sqrt(sv)).astype(np.int32))
    m3t = (mt - torch.tensor(centers)) * torch.tensor(scale) + torch.tensor(dims) / 2
    vm3, vc3 = r.normal(size=(n, 3)), r.normal(size=(n, 6))
    gm, gc = torch.autograd.grad((m3t * torch.tensor(vm3)).sum() + (P * torch.tensor(vc3)).sum(),
                                 (mt, ct))
    vm, vc = ops.world_to_volume_mapping_bwd(means, covars, ranges, centers, *dims, 1e-8, vm3, vc3)
    np.testing.assert_allclose(vm, gm.numpy(), rtol=1e-14)
    np.testing.assert_allclose(vc, gc.numpy(), rtol=1e-8, atol=1e-12)


def test_volume_mapping_isotropic_kat_and_singular():
    s2, eps = 0.04, 1e-6
    cov = np.array([[s2, 0, 0, s2, 0, s2], [0, 0, 0, 0, 0, 0]])
    means = np.zeros((2, 3))
    m3, con, rad = ops.world_to_volume_mapping_fwd(means, cov, np.array([2.0, 2, 2]), np.zeros(3),
                                                   32, 32, 32, eps, 3.0)
    rr = 16.0  # voxels per world unit
    np.testing.assert_allclose(con[0], [1 / (rr * rr * s2 + eps), 0, 0, 1 / (rr * rr * s2 + eps),
                                        0, 1 / (rr * rr * s2 + eps)], rtol=1e-14)
    np.testing.assert_array_equal(m3[0], [16, 16, 16])
    # Singular (det 1e-18 < 1e-12): zero conic and radii (WorldToVolumeMappingFwd.cu:157-163).
    assert (con[1] == 0).all() and (rad[1] == 0).all()
