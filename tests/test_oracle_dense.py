"""The dense torch formulation (oracle/dense.py, the CPU baseline's workload)
against the numpy / C oracle, in float64.

The two are written independently: the dense form evaluates every Gaussian
at every pixel (voxel) as broadcast torch expressions and takes its backward
from torch autograd, while the oracle follows the reference kernels' tiled
loops and hand-written VJPs.  Values agree to float64 rounding; the composed
parameter gradients of one config-1-style call (a view and a volume from
the same Gaussians) agree to 1e-9 relative.
"""

import numpy as np
import torch

from helpers import make_scene
from oracle import compose, dense

SMIN, SMAX, EPS, CLIP = 5e-4, 1.0, 1e-8, 3.0


def _scene():
    raw, vm, Ks, g = make_scene(400, 11, n_det=64, log_mu=-3.0, log_sigma=0.4, extent=0.6)
    f = lambda t: t.double().numpy()  # noqa: E731
    return raw, f(vm), f(Ks), g, [f(t) for t in (raw.means, raw.quats, raw.raw_scales,
                                               raw.raw_opacities)]


def _close(a, b, name, rtol=1e-11, atol=1e-13):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    scale = atol * max(1.0, float(np.abs(b).max()))
    err = np.abs(a - b) - rtol * np.abs(b)
    assert float(err.max()) <= scale, f"{name}: max excess {float(err.max()):.3e}"


def test_dense_preprocessing_and_sums_equal_the_oracle():
    _, vm, Ks, _, (means, quats, scales, opac) = _scene()
    T = torch.from_numpy
    cov_o, ms_o, op_o = compose.prepare(quats, scales, opac, SMIN, SMAX)
    cov_d, ms_d, op_d = dense.activate(T(quats), T(scales), T(opac), SMIN, SMAX)
    _close(cov_d, cov_o, "covars")
    _close(ms_d, ms_o, "max_scales")
    _close(op_d, op_o, "opacities")

    proj = compose.rasterize_forward(means, cov_o, op_o, vm, Ks, 64, 64, 16, EPS, CLIP)
    m2, c2, r2 = dense.project(T(means), T(cov_o), T(vm[0]), T(Ks[0]), 64, 64, EPS, CLIP)
    _close(m2, proj["means2d"][0], "means2d")
    _close(c2, proj["cov2d"][0], "cov2d", atol=1e-12)
    assert np.array_equal(r2.numpy(), proj["radii"][0])
    assert int((r2 > 0).all(-1).sum()) > 300
    con, mu = dense.conics_mu(T(proj["cov2d"][0]), EPS)
    _close(con, proj["conics"][0], "conics")
    _close(mu, proj["mus"][0], "mus")
    image = dense.raster(T(proj["means2d"][0]), T(proj["conics"][0]),
                         T(proj["opacity"][0] * proj["mus"][0]),
                         dense.cover_2d(T(proj["means2d"][0]), T(proj["radii"][0]), 16, 64, 64))
    assert float(image.abs().sum()) > 1.0
    _close(image, proj["output"][0], "image", atol=1e-12)

    rng, ctr = np.full(3, 2.0), np.zeros(3)
    vox = compose.voxelize_forward(means, cov_o, op_o, rng, ctr, 40, 32, 24, 8, EPS, CLIP)
    m3, c3, r3 = dense.volume_mapping(T(means), T(cov_o), T(rng), T(ctr), 40, 32, 24, EPS, CLIP)
    _close(m3, vox["means3d"], "means3d")
    _close(c3, vox["conics"], "conics3d", rtol=1e-9)
    assert np.array_equal(r3.numpy(), vox["radii"])
    volume = dense.voxel(T(vox["means3d"]), T(vox["conics"]), T(op_o),
                         dense.cover_3d(T(vox["means3d"]), T(vox["radii"]), 8, 40, 32, 24))
    assert tuple(volume.shape) == (24, 32, 40) and float(volume.abs().sum()) > 1.0
    _close(volume, vox["output"], "volume", atol=1e-12)


def test_dense_call_gradients_equal_the_oracle_chain():
    _, vm, Ks, g, (means, quats, scales, opac) = _scene()
    v_image = torch.randn(64, 64, generator=g, dtype=torch.float64)
    v_volume = torch.randn(24, 32, 40, generator=g, dtype=torch.float64)
    params = [torch.from_numpy(a.copy()).requires_grad_(True)
              for a in (means, quats, scales, opac)]
    image, volume = dense.config1_call(params, torch.from_numpy(vm[0]), torch.from_numpy(Ks[0]),
                                       64, 64, v_image, (40, 32, 24), v_volume, scale_min=SMIN,
                                       scale_max=SMAX, eps=EPS, radius_clip=CLIP, chunk=96)
    cov_o, _, op_o = compose.prepare(quats, scales, opac, SMIN, SMAX)
    proj = compose.rasterize_forward(means, cov_o, op_o, vm, Ks, 64, 64, 16, EPS, CLIP)
    vox = compose.voxelize_forward(means, cov_o, op_o, np.full(3, 2.0), np.zeros(3), 40, 32, 24,
                                   8, EPS, CLIP)
    _close(image, proj["output"][0], "image", atol=1e-12)
    _close(volume, vox["output"], "volume", atol=1e-12)
    want = compose.explicit_backward(cov_o, proj, vox, means, quats, scales, opac, SMIN, SMAX,
                                     v_image.numpy()[None], v_volume.numpy())
    for p, name in zip(params, ("means", "quats", "raw_scales", "raw_opacities")):
        assert float(np.abs(want[name]).max()) > 0
        _close(p.grad, want[name], name, rtol=1e-9, atol=1e-10)
