"""Element-wise operators restated in numpy (test infrastructure only).

Every function mirrors the expression order of the reference CUDA kernel it
cites, in the dtype of its inputs (float32 or float64), with no fused
multiply-add.  numpy float arithmetic, division and sqrt are IEEE correctly
rounded, so for kernels without transcendental functions the float32 results
are bit-reproducible by a device build that uses the same order and
``-ffp-contract=off``.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "parameter_transform_fwd",
    "parameter_transform_bwd",
    "softplus",
    "world_to_image_projection_fwd",
    "world_to_image_projection_bwd",
    "conics_mu_fwd",
    "conics_mu_bwd",
    "world_to_volume_mapping_fwd",
    "world_to_volume_mapping_bwd",
]


def _k(dtype):
    """Scalar constructor of the array dtype (keeps numpy in that precision)."""
    return np.dtype(dtype).type


def _quat_rotation(quats, k):
    # ParameterTransformFwd.cu:210-221 and 236-252 (normalise, then R rows)
    rw, rx, ry, rz = quats[:, 0], quats[:, 1], quats[:, 2], quats[:, 3]
    qnorm = np.sqrt(rw * rw + rx * rx + ry * ry + rz * rz)
    qdenom = np.maximum(qnorm, k(1e-12))
    inv_qnorm = k(1) / qdenom
    w, x, y, z = rw * inv_qnorm, rx * inv_qnorm, ry * inv_qnorm, rz * inv_qnorm
    x2, y2, z2 = x * x, y * y, z * z
    xy, xz, yz = x * y, x * z, y * z
    wx, wy, wz = w * x, w * y, w * z
    one, two = k(1), k(2)
    R = (
        (one - two * (y2 + z2), two * (xy - wz), two * (xz + wy)),
        (two * (xy + wz), one - two * (x2 + z2), two * (yz - wx)),
        (two * (xz - wy), two * (yz + wx), one - two * (x2 + y2)),
    )
    return (w, x, y, z), R, qnorm, inv_qnorm


def _activate_scales(raw_scales, scale_min, scale_max, k):
    # ParameterTransformFwd.cu:223-230: s = sigmoid(raw) * (max - min) + min
    smin, smax = k(scale_min), k(scale_max)
    rng = smax - smin
    sig = k(1) / (k(1) + np.exp(-raw_scales))
    return sig, sig * rng + smin, rng


def parameter_transform_fwd(quats, raw_scales, scale_min, scale_max):
    """ParameterTransformFwd.cu:53-129 -> (covars [N,6], max_scales [N])."""
    k = _k(quats.dtype)
    with np.errstate(all="ignore"):
        _, R, _, _ = _quat_rotation(quats, k)
        _, s, _ = _activate_scales(raw_scales, scale_min, scale_max, k)
        max_scales = np.maximum(s[:, 0], np.maximum(s[:, 1], s[:, 2]))
        sq = (s[:, 0] * s[:, 0], s[:, 1] * s[:, 1], s[:, 2] * s[:, 2])

        def c(i, j):
            # ParameterTransformFwd.cu:259-264: sum_k R_ik R_jk s_k^2
            return (R[i][0] * R[j][0] * sq[0] + R[i][1] * R[j][1] * sq[1]
                    + R[i][2] * R[j][2] * sq[2])

        covars = np.stack([c(0, 0), c(0, 1), c(0, 2), c(1, 1), c(1, 2), c(2, 2)], -1)
    return covars.astype(quats.dtype), max_scales.astype(quats.dtype)


def parameter_transform_bwd(quats, raw_scales, scale_min, scale_max, v_covars):
    """ParameterTransformBwd.cu:66-245 -> (v_quats [N,4], v_raw_scales [N,3])."""
    k = _k(quats.dtype)
    with np.errstate(all="ignore"):
        (w, x, y, z), R, qnorm, inv_qnorm = _quat_rotation(quats, k)
        sig, s, rng = _activate_scales(raw_scales, scale_min, scale_max, k)
        half, two = k(0.5), k(2)
        v0 = v_covars[:, 0]
        v1 = v_covars[:, 1] * half
        v2 = v_covars[:, 2] * half
        v3 = v_covars[:, 3]
        v4 = v_covars[:, 4] * half
        v5 = v_covars[:, 5]
        vc = ((v0, v1, v2), (v1, v3, v4), (v2, v4, v5))
        # ParameterTransformBwd.cu:140-152 and 162-171
        vM = [[None] * 3 for _ in range(3)]
        vR = [[None] * 3 for _ in range(3)]
        for i in range(3):
            for j in range(3):
                inner = vc[i][0] * R[0][j] + vc[i][1] * R[1][j] + vc[i][2] * R[2][j]
                vM[i][j] = two * inner * s[:, j]
                vR[i][j] = two * inner * s[:, j] * s[:, j]
        # ParameterTransformBwd.cu:188-210
        vw = two * (x * (vR[2][1] - vR[1][2]) + y * (vR[0][2] - vR[2][0])
                    + z * (vR[1][0] - vR[0][1]))
        vx = two * (k(-2) * x * (vR[1][1] + vR[2][2]) + y * (vR[0][1] + vR[1][0])
                    + z * (vR[0][2] + vR[2][0]) + w * (vR[2][1] - vR[1][2]))
        vy = two * (x * (vR[0][1] + vR[1][0]) + k(-2) * y * (vR[0][0] + vR[2][2])
                    + z * (vR[1][2] + vR[2][1]) + w * (vR[0][2] - vR[2][0]))
        vz = two * (x * (vR[0][2] + vR[2][0]) + y * (vR[1][2] + vR[2][1])
                    + k(-2) * z * (vR[0][0] + vR[1][1]) + w * (vR[1][0] - vR[0][1]))
        # ParameterTransformBwd.cu:219-229
        vs = [R[0][j] * vM[0][j] + R[1][j] * vM[1][j] + R[2][j] * vM[2][j] for j in range(3)]
        v_raw = np.stack([vs[j] * sig[:, j] * (k(1) - sig[:, j]) * rng for j in range(3)], -1)
        # ParameterTransformBwd.cu:232-244
        dot = w * vw + x * vx + y * vy + z * vz
        proj = np.stack([(vw - w * dot) * inv_qnorm, (vx - x * dot) * inv_qnorm,
                         (vy - y * dot) * inv_qnorm, (vz - z * dot) * inv_qnorm], -1)
        raw = np.stack([vw * inv_qnorm, vx * inv_qnorm, vy * inv_qnorm, vz * inv_qnorm], -1)
        v_quats = np.where((qnorm > k(1e-12))[:, None], proj, raw)
    return v_quats.astype(quats.dtype), v_raw.astype(quats.dtype)


def softplus(x):
    """torch.nn.functional.softplus (beta 1, threshold 20), r2splat/ops/direct.py:91."""
    k = _k(x.dtype)
    with np.errstate(over="ignore"):
        return np.where(x > k(20), x, np.log1p(np.exp(x))).astype(x.dtype)


def _camera(viewmat, K):
    R = ((viewmat[0, 0], viewmat[0, 1], viewmat[0, 2]),
         (viewmat[1, 0], viewmat[1, 1], viewmat[1, 2]),
         (viewmat[2, 0], viewmat[2, 1], viewmat[2, 2]))
    t = (viewmat[0, 3], viewmat[1, 3], viewmat[2, 3])
    return R, t, K[0, 0], K[1, 1], K[0, 2], K[1, 2]


def _fov_limits(width, height, fx, fy, cx, cy, k):
    # WorldToImageProjectionFwd.cu:149-156
    W, H = k(width), k(height)
    tan_fovx = k(0.5) * W / fx
    tan_fovy = k(0.5) * H / fy
    lim_x_pos = (W - cx) / fx + k(0.3) * tan_fovx
    lim_x_neg = cx / fx + k(0.3) * tan_fovx
    lim_y_pos = (H - cy) / fy + k(0.3) * tan_fovy
    lim_y_neg = cy / fy + k(0.3) * tan_fovy
    return lim_x_pos, lim_x_neg, lim_y_pos, lim_y_neg


def _camera_cov(covars, R):
    # WorldToImageProjectionFwd.cu:184-207: Sigma_c = R Sigma R^T via M = Sigma R^T
    s00, s01, s02, s11, s12, s22 = (covars[:, i] for i in range(6))
    S = ((s00, s01, s02), (s01, s11, s12), (s02, s12, s22))
    M = [[S[i][0] * R[j][0] + S[i][1] * R[j][1] + S[i][2] * R[j][2] for j in range(3)]
         for i in range(3)]
    Sc = {}
    for i, j in ((0, 0), (0, 1), (0, 2), (1, 1), (1, 2), (2, 2)):
        Sc[i, j] = R[i][0] * M[0][j] + R[i][1] * M[1][j] + R[i][2] * M[2][j]
    return Sc


def world_to_image_projection_fwd(means, covars, viewmats, Ks, width, height,
                                  eps2d, radius_clip):
    """WorldToImageProjectionFwd.cu:74-283 -> (means2d [C,N,2], cov2d [C,N,6], radii [C,N,2]).

    ``eps2d`` and ``radius_clip`` are float in the reference signature
    (WorldToImageProjection.cpp:45-46) and are rounded to float32 first.
    """
    dt = means.dtype
    k = _k(dt)
    eps = k(np.float32(eps2d))
    clip = k(np.float32(radius_clip))
    C, N = viewmats.shape[0], means.shape[0]
    means2d = np.zeros((C, N, 2), dt)
    cov2d = np.zeros((C, N, 6), dt)
    radii = np.zeros((C, N, 2), np.int32)
    px, py, pz = means[:, 0], means[:, 1], means[:, 2]
    with np.errstate(all="ignore"):
        for c in range(C):
            R, t, fx, fy, cx, cy = _camera(viewmats[c], Ks[c])
            # WorldToImageProjectionFwd.cu:124-126
            x = R[0][0] * px + R[0][1] * py + R[0][2] * pz + t[0]
            y = R[1][0] * px + R[1][1] * py + R[1][2] * pz + t[1]
            z = R[2][0] * px + R[2][1] * py + R[2][2] * pz + t[2]
            keep = ~(z <= k(0.01))                       # cu:129-136
            rz = k(1) / z
            rz2 = rz * rz
            mx = fx * x * rz + cx                        # cu:143-144
            my = fy * y * rz + cy
            lxp, lxn, lyp, lyn = _fov_limits(width, height, fx, fy, cx, cy, k)
            tx = z * np.fmin(lxp, np.fmax(-lxn, x * rz))  # cu:158-159
            ty = z * np.fmin(lyp, np.fmax(-lyn, y * rz))
            l = np.sqrt(tx * tx + ty * ty + z * z)        # cu:164-177
            rl = k(1) / l
            J00 = fx * rz
            J02 = -fx * tx * rz2
            J11 = fy * rz
            J12 = -fy * ty * rz2
            J20, J21, J22 = tx * rl, ty * rl, z * rl
            Sc = _camera_cov(covars, R)
            Sc00, Sc01, Sc02 = Sc[0, 0], Sc[0, 1], Sc[0, 2]
            Sc11, Sc12, Sc22 = Sc[1, 1], Sc[1, 2], Sc[2, 2]
            # cu:215-231 (N = Sigma_c J^T, C2 = J N; J01 = J10 = 0)
            N00 = Sc00 * J00 + Sc02 * J02
            N01 = Sc01 * J11 + Sc02 * J12
            N02 = Sc00 * J20 + Sc01 * J21 + Sc02 * J22
            N11 = Sc11 * J11 + Sc12 * J12
            N12 = Sc01 * J20 + Sc11 * J21 + Sc12 * J22
            N20 = Sc02 * J00 + Sc22 * J02
            N21 = Sc12 * J11 + Sc22 * J12
            N22 = Sc02 * J20 + Sc12 * J21 + Sc22 * J22
            C00 = J00 * N00 + J02 * N20
            C01 = J00 * N01 + J02 * N21
            C02 = J00 * N02 + J02 * N22
            C11 = J11 * N11 + J12 * N21
            C12 = J11 * N12 + J12 * N22
            C22 = J20 * N02 + J21 * N12 + J22 * N22
            cov = np.stack([C00, C01, C02, C11, C12, C22], -1)
            # cu:250-282 radii
            a_blur = C00 + eps
            d_blur = C11 + eps
            det_blur = a_blur * d_blur - C01 * C01
            rad_x = np.ceil(clip * np.sqrt(np.fmax(k(0), a_blur)))
            rad_y = np.ceil(clip * np.sqrt(np.fmax(k(0), d_blur)))
            ok = ~(det_blur <= k(0))
            ok &= np.isfinite(rad_x) & np.isfinite(rad_y) & (rad_x > 0) & (rad_y > 0)
            ok &= ~((mx + rad_x <= k(0)) | (mx - rad_x >= k(width))
                    | (my + rad_y <= k(0)) | (my - rad_y >= k(height)))
            ok &= keep
            means2d[c, :, 0] = np.where(keep, mx, k(0))
            means2d[c, :, 1] = np.where(keep, my, k(0))
            cov2d[c] = np.where(keep[:, None], cov, k(0))
            radii[c, :, 0] = np.where(ok, np.where(ok, rad_x, 0), 0).astype(np.int32)
            radii[c, :, 1] = np.where(ok, np.where(ok, rad_y, 0), 0).astype(np.int32)
    return means2d, cov2d, radii


def world_to_image_projection_bwd(means, covars, viewmats, Ks, width, height,
                                  v_means2d, v_cov2d):
    """WorldToImageProjectionBwd.cu:68-554 -> (v_means [N,3], v_covars [N,6]), summed over C."""
    dt = means.dtype
    k = _k(dt)
    C, N = viewmats.shape[0], means.shape[0]
    v_means = np.zeros((N, 3), dt)
    v_covars = np.zeros((N, 6), dt)
    px, py, pz = means[:, 0], means[:, 1], means[:, 2]
    two = k(2)
    with np.errstate(all="ignore"):
        for c in range(C):
            R, t, fx, fy, cx, cy = _camera(viewmats[c], Ks[c])
            x = R[0][0] * px + R[0][1] * py + R[0][2] * pz + t[0]
            y = R[1][0] * px + R[1][1] * py + R[1][2] * pz + t[1]
            z = R[2][0] * px + R[2][1] * py + R[2][2] * pz + t[2]
            keep = ~(z <= k(0.01))                               # cu:125-128
            rz = k(1) / z
            rz2 = rz * rz
            rz3 = rz2 * rz
            lxp, lxn, lyp, lyn = _fov_limits(width, height, fx, fy, cx, cy, k)
            xrz, yrz = x * rz, y * rz
            tx = z * np.fmin(lxp, np.fmax(-lxn, xrz))
            ty = z * np.fmin(lyp, np.fmax(-lyn, yrz))
            x_cl = (xrz > lxp) | (xrz < -lxn)                   # cu:149-150
            y_cl = (yrz > lyp) | (yrz < -lyn)
            l = np.sqrt(tx * tx + ty * ty + z * z)
            rl = k(1) / l
            rl2 = rl * rl
            J00 = fx * rz
            J02 = -fx * tx * rz2
            J11 = fy * rz
            J12 = -fy * ty * rz2
            J20, J21, J22 = tx * rl, ty * rl, z * rl
            Sc = _camera_cov(covars, R)
            Sc00, Sc01, Sc02 = Sc[0, 0], Sc[0, 1], Sc[0, 2]
            Sc11, Sc12, Sc22 = Sc[1, 1], Sc[1, 2], Sc[2, 2]
            vm2x, vm2y = v_means2d[c, :, 0], v_means2d[c, :, 1]
            va, vb, vcv, vd, ve, vf = (v_cov2d[c, :, i] for i in range(6))
            # cu:220-222 part A
            v_pc_x = fx * rz * vm2x
            v_pc_y = fy * rz * vm2y
            v_pc_z = -(fx * x * rz2 * vm2x + fy * y * rz2 * vm2y)
            # cu:234-254 part B: v_Sigma_c = J^T G_upper J
            T00 = va * J00 + vcv * J20
            T01 = vb * J11 + vcv * J21
            T02 = va * J02 + vb * J12 + vcv * J22
            T10 = ve * J20
            T11 = vd * J11 + ve * J21
            T12 = vd * J12 + ve * J22
            T20 = vf * J20
            T21 = vf * J21
            T22 = vf * J22
            vSc = (
                (J00 * T00 + J20 * T20, J00 * T01 + J20 * T21, J00 * T02 + J20 * T22),
                (J11 * T10 + J21 * T20, J11 * T11 + J21 * T21, J11 * T12 + J21 * T22),
                (J02 * T00 + J12 * T10 + J22 * T20, J02 * T01 + J12 * T11 + J22 * T21,
                 J02 * T02 + J12 * T12 + J22 * T22),
            )
            # cu:268-298: v_Sigma = R^T v_Sigma_c R, symmetric-parameter gather
            Q = [[vSc[i][0] * R[0][j] + vSc[i][1] * R[1][j] + vSc[i][2] * R[2][j]
                  for j in range(3)] for i in range(3)]
            vS = [[R[0][i] * Q[0][j] + R[1][i] * Q[1][j] + R[2][i] * Q[2][j]
                   for j in range(3)] for i in range(3)]
            vs6 = np.stack([vS[0][0], vS[0][1] + vS[1][0], vS[0][2] + vS[2][0],
                            vS[1][1], vS[1][2] + vS[2][1], vS[2][2]], -1)
            # cu:386-416 part C: v_J = (G + G^T) J Sigma_c
            G = ((two * va, vb, vcv), (vb, two * vd, ve), (vcv, ve, two * vf))
            U = (
                (J00 * Sc00 + J02 * Sc02, J00 * Sc01 + J02 * Sc12, J00 * Sc02 + J02 * Sc22),
                (J11 * Sc01 + J12 * Sc02, J11 * Sc11 + J12 * Sc12, J11 * Sc12 + J12 * Sc22),
                (J20 * Sc00 + J21 * Sc01 + J22 * Sc02, J20 * Sc01 + J21 * Sc11 + J22 * Sc12,
                 J20 * Sc02 + J21 * Sc12 + J22 * Sc22),
            )
            vJ = [[G[i][0] * U[0][j] + G[i][1] * U[1][j] + G[i][2] * U[2][j]
                   for j in range(3)] for i in range(3)]
            # cu:443-537 propagate v_J to p_c (clipped branches)
            v_pc_z = v_pc_z + -fx * rz2 * vJ[0][0]
            v_pc_z = v_pc_z + -fy * rz2 * vJ[1][1]
            v_pc_z = v_pc_z + rl * vJ[2][2]
            v_pc_x = np.where(x_cl, v_pc_x, v_pc_x + -fx * rz2 * vJ[0][2])
            v_pc_z = v_pc_z + two * fx * tx * rz3 * vJ[0][2]
            v_pc_y = np.where(y_cl, v_pc_y, v_pc_y + -fy * rz2 * vJ[1][2])
            v_pc_z = v_pc_z + two * fy * ty * rz3 * vJ[1][2]
            v_pc_x = np.where(x_cl, v_pc_x, v_pc_x + rl * vJ[2][0])
            v_pc_y = np.where(y_cl, v_pc_y, v_pc_y + rl * vJ[2][1])
            v_l = -tx * rl2 * vJ[2][0] - ty * rl2 * vJ[2][1] - z * rl2 * vJ[2][2]
            v_pc_x = np.where(x_cl, v_pc_x, v_pc_x + v_l * tx * rl)
            v_pc_y = np.where(y_cl, v_pc_y, v_pc_y + v_l * ty * rl)
            v_pc_z = v_pc_z + v_l * z * rl
            zx = v_pc_z + v_l * tx * rl * (tx / z)
            zx = zx + (tx / z) * rl * vJ[2][0]
            v_pc_z = np.where(x_cl, zx, v_pc_z)
            zy = v_pc_z + v_l * ty * rl * (ty / z)
            zy = zy + (ty / z) * rl * vJ[2][1]
            v_pc_z = np.where(y_cl, zy, v_pc_z)
            v_pc_z = np.where(x_cl, v_pc_z + -fx * (tx / z) * rz2 * vJ[0][2], v_pc_z)
            v_pc_z = np.where(y_cl, v_pc_z + -fy * (ty / z) * rz2 * vJ[1][2], v_pc_z)
            # cu:543-545
            vp = np.stack([R[0][0] * v_pc_x + R[1][0] * v_pc_y + R[2][0] * v_pc_z,
                           R[0][1] * v_pc_x + R[1][1] * v_pc_y + R[2][1] * v_pc_z,
                           R[0][2] * v_pc_x + R[1][2] * v_pc_y + R[2][2] * v_pc_z], -1)
            v_means += np.where(keep[:, None], vp, k(0))
            v_covars += np.where(keep[:, None], vs6, k(0))
    return v_means.astype(dt), v_covars.astype(dt)


def conics_mu_fwd(cov2d, eps):
    """ConicsMuFwd.cu:36-100 -> (conics [...,3], mus [...])."""
    k = _k(cov2d.dtype)
    e = k(eps)
    a, b, c, d, ee, f = (cov2d[..., i] for i in range(6))
    with np.errstate(all="ignore"):
        ab, db, fb = a + e, d + e, f + e
        D2b = ab * db - b * b
        D3b = ab * db * fb - ab * ee * ee - b * b * fb + k(2) * b * c * ee - c * c * db
        valid = ~(D2b <= k(1e-9))
        inv = k(1) / D2b
        conics = np.stack([db * inv, -b * inv, ab * inv], -1)
        ratio = D3b * inv
        mus = np.where(ratio > k(0), np.sqrt(k(2.0 * np.pi) * ratio), k(0))
        conics = np.where(valid[..., None], conics, k(0))
        mus = np.where(valid, mus, k(0))
    return conics.astype(cov2d.dtype), mus.astype(cov2d.dtype)


def conics_mu_bwd(cov2d, eps, conics, mus, v_conics, v_mus):
    """ConicsMuBwd.cu:50-170 -> v_cov2d [...,6].

    Keeps the kernel's gate: the mu gradient is zero unless mu > 0 and
    D3b > 1e-9 (ConicsMuBwd.cu:126-140).
    """
    dt = cov2d.dtype
    k = _k(dt)
    e = k(eps)
    u11, u12, u22 = conics[..., 0], conics[..., 1], conics[..., 2]
    vu11, vu12, vu22 = v_conics[..., 0], v_conics[..., 1], v_conics[..., 2]
    two = k(2)
    with np.errstate(all="ignore"):
        ga = -(vu11 * u11 * u11 + vu12 * u11 * u12 + vu22 * u12 * u12)
        gb = -(vu11 * two * u11 * u12 + vu12 * (u11 * u22 + u12 * u12)
               + vu22 * two * u12 * u22)
        gd = -(vu11 * u12 * u12 + vu12 * u12 * u22 + vu22 * u22 * u22)
        zero = np.zeros_like(ga)
        ab = cov2d[..., 0] + e
        b = cov2d[..., 1]
        c = cov2d[..., 2]
        db = cov2d[..., 3] + e
        ee = cov2d[..., 4]
        fb = cov2d[..., 5] + e
        D3b = ab * db * fb - ab * ee * ee - b * b * fb + two * b * c * ee - c * c * db
        inv = k(1) / D3b
        q00 = (db * fb - ee * ee) * inv
        q01 = (c * ee - b * fb) * inv
        q02 = (b * ee - c * db) * inv
        q11 = (ab * fb - c * c) * inv
        q12 = (b * c - ab * ee) * inv
        q22 = (ab * db - b * b) * inv
        h = k(0.5) * mus * v_mus
        gate = (mus > k(0)) & (D3b > k(1e-9))
        ga = np.where(gate, ga + h * (q00 - u11), ga)
        gb = np.where(gate, gb + h * (two * q01 - two * u12), gb)
        gc = np.where(gate, zero + h * (two * q02), zero)
        gd = np.where(gate, gd + h * (q11 - u22), gd)
        ge = np.where(gate, zero + h * (two * q12), zero)
        gf = np.where(gate, zero + h * q22, zero)
        out = np.stack([ga, gb, gc, gd, ge, gf], -1)
        degenerate = (u11 == 0) & (u12 == 0) & (u22 == 0)       # cu:79-87
        out = np.where(degenerate[..., None], k(0), out)
    return out.astype(dt)


def _volume_scale(ranges, dims, k):
    # WorldToVolumeMappingFwd.cu:110-120: r = (dim2/rx, dim1/ry, dim0/rz)
    dim2, dim1, dim0 = dims
    return k(dim2) / ranges[0], k(dim1) / ranges[1], k(dim0) / ranges[2]


def _invert_sym3x3(a00, a01, a02, a11, a12, a22, k):
    # WorldToVolumeMappingFwd.cu:55-83 (cofactors, |det| < 1e-12 -> zeros)
    c00 = a11 * a22 - a12 * a12
    c01 = a02 * a12 - a01 * a22
    c02 = a01 * a12 - a02 * a11
    c11 = a00 * a22 - a02 * a02
    c12 = a01 * a02 - a00 * a12
    c22 = a00 * a11 - a01 * a01
    det = a00 * c00 + a01 * c01 + a02 * c02
    ok = ~(np.abs(det) < k(1e-12))
    inv = k(1) / det
    out = [c00 * inv, c01 * inv, c02 * inv, c11 * inv, c12 * inv, c22 * inv]
    out = [np.where(ok, v, k(0)) for v in out]
    return ok, out


def world_to_volume_mapping_fwd(means, covars, ranges, centers, dim2, dim1, dim0,
                                eps3d, radius_clip):
    """WorldToVolumeMappingFwd.cu:90-189 -> (means3d [N,3], conics [N,6], radii [N,3])."""
    dt = means.dtype
    k = _k(dt)
    eps, clip = k(eps3d), k(radius_clip)
    with np.errstate(all="ignore"):
        r0, r1, r2 = _volume_scale(ranges, (dim2, dim1, dim0), k)
        half = k(0.5)
        m3 = np.stack([(means[:, 0] - centers[0]) * r0 + k(dim2) * half,
                       (means[:, 1] - centers[1]) * r1 + k(dim1) * half,
                       (means[:, 2] - centers[2]) * r2 + k(dim0) * half], -1)
        s00, s01, s02, s11, s12, s22 = (covars[:, i] for i in range(6))
        Sv00 = r0 * r0 * s00 + eps
        Sv01 = r0 * r1 * s01
        Sv02 = r0 * r2 * s02
        Sv11 = r1 * r1 * s11 + eps
        Sv12 = r1 * r2 * s12
        Sv22 = r2 * r2 * s22 + eps
        ok, inv = _invert_sym3x3(Sv00, Sv01, Sv02, Sv11, Sv12, Sv22, k)
        conics = np.stack(inv, -1)
        rad = [np.ceil(clip * np.sqrt(np.fmax(k(0), v))) for v in (Sv00, Sv11, Sv22)]
        good = ok.copy()
        for v in rad:
            good &= np.isfinite(v) & (v > 0)
        radii = np.stack([np.where(good, v, 0) for v in rad], -1).astype(np.int32)
    return m3.astype(dt), conics.astype(dt), radii


def world_to_volume_mapping_bwd(means, covars, ranges, centers, dim2, dim1, dim0,
                                eps3d, v_means3d, v_conics):
    """WorldToVolumeMappingBwd.cu:83-198 -> (v_means [N,3], v_covars [N,6])."""
    dt = means.dtype
    k = _k(dt)
    eps = k(eps3d)
    with np.errstate(all="ignore"):
        r0, r1, r2 = _volume_scale(ranges, (dim2, dim1, dim0), k)
        v_means = np.stack([v_means3d[:, 0] * r0, v_means3d[:, 1] * r1,
                            v_means3d[:, 2] * r2], -1)
        s00, s01, s02, s11, s12, s22 = (covars[:, i] for i in range(6))
        Sv = (r0 * r0 * s00 + eps, r0 * r1 * s01, r0 * r2 * s02,
              r1 * r1 * s11 + eps, r1 * r2 * s12, r2 * r2 * s22 + eps)
        ok, (P00, P01, P02, P11, P12, P22) = _invert_sym3x3(*Sv, k)
        vc00, vc01, vc02, vc11, vc12, vc22 = (v_conics[:, i] for i in range(6))
        # cu:166-188: v_Sv = -P V_upper P
        T00 = vc00 * P00 + vc01 * P01 + vc02 * P02
        T01 = vc00 * P01 + vc01 * P11 + vc02 * P12
        T02 = vc00 * P02 + vc01 * P12 + vc02 * P22
        T10 = vc11 * P01 + vc12 * P02
        T11 = vc11 * P11 + vc12 * P12
        T12 = vc11 * P12 + vc12 * P22
        T20 = vc22 * P02
        T21 = vc22 * P12
        T22 = vc22 * P22
        vS00 = -(P00 * T00 + P01 * T10 + P02 * T20)
        vS01 = -(P00 * T01 + P01 * T11 + P02 * T21)
        vS02 = -(P00 * T02 + P01 * T12 + P02 * T22)
        vS10 = -(P01 * T00 + P11 * T10 + P12 * T20)
        vS11 = -(P01 * T01 + P11 * T11 + P12 * T21)
        vS12 = -(P01 * T02 + P11 * T12 + P12 * T22)
        vS20 = -(P02 * T00 + P12 * T10 + P22 * T20)
        vS21 = -(P02 * T01 + P12 * T11 + P22 * T21)
        vS22 = -(P02 * T02 + P12 * T12 + P22 * T22)
        vc = np.stack([vS00 * r0 * r0, (vS01 + vS10) * r0 * r1, (vS02 + vS20) * r0 * r2,
                       vS11 * r1 * r1, (vS12 + vS21) * r1 * r2, vS22 * r2 * r2], -1)
        vc = np.where(ok[:, None], vc, k(0))
    return v_means.astype(dt), vc.astype(dt)
