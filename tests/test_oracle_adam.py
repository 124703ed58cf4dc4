"""Pins oracle/adam.py against torch.optim.Adam on the CPU."""

import numpy as np
import pytest
import torch

from oracle import adam as A


@pytest.mark.parametrize("wd", [0.0, 0.01])
@pytest.mark.parametrize("betas", [(0.9, 0.999), (0.6, 0.95)])
def test_oracle_matches_torch_adam_on_cpu(wd, betas):
    rng = np.random.default_rng(0)
    p0 = rng.normal(size=(257, 3)).astype(np.float32)
    grads = [rng.normal(size=p0.shape).astype(np.float32) * 10 ** rng.uniform(-3, 1)
             for _ in range(6)]
    tp = torch.nn.Parameter(torch.from_numpy(p0.copy()))
    opt = torch.optim.Adam([tp], lr=3e-3, betas=betas, eps=1e-15, weight_decay=wd,
                           foreach=False)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for t, g in enumerate(grads, start=1):
        tp.grad = torch.from_numpy(g)
        opt.step()
        p, m, v = A.adam_step(p, g, m, v, t, 3e-3, betas[0], betas[1], 1e-15, wd)
        st = opt.state[tp]
        # torch's CPU kernels may contract to FMAs: an ulp or two of each
        # operation, relative to the operands (lerp cancels).
        np.testing.assert_allclose(st["exp_avg"].numpy(), m, rtol=1e-6,
                                   atol=1e-6 * np.abs(m).max())
        np.testing.assert_allclose(st["exp_avg_sq"].numpy(), v, rtol=1e-6,
                                   atol=1e-6 * np.abs(v).max())
        np.testing.assert_allclose(tp.detach().numpy(), p, rtol=1e-6, atol=1e-9)
