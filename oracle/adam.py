"""Adam step restated in numpy float32 -- TEST INFRASTRUCTURE ONLY.

Restates torch.optim.Adam's update (torch/optim/adam.py, the algorithm the
trainer's per-group optimizers run: src/models/gaussian_model.py:514-530)
for one tensor, one float32 rounding per operation:

    g = grad (+ wd * p);  m = lerp(m, g, 1 - beta1)
    v = v * beta2 + (1 - beta2) * g * g
    p = p - lr / (1 - beta1^t) * m / (sqrt(v) / sqrt(1 - beta2^t) + eps)

The step scalars are computed in double and rounded to float32, as torch
passes Python floats to its float32 kernels.  Pinned against
torch.optim.Adam on the CPU in tests/test_oracle_adam.py.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def lerp(a, b, w):
    """ATen's lerp: from the start for |w| < 0.5, else from the end."""
    w = F32(w)
    if abs(w) < 0.5:
        return (a + w * (b - a)).astype(F32)
    return (b - (b - a) * (F32(1) - w)).astype(F32)


def adam_step(p, g, m, v, step, lr, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0):
    """One step with step count `step` (after the increment); returns new (p, m, v)."""
    p, g, m, v = (np.asarray(a, F32) for a in (p, g, m, v))
    if weight_decay != 0:
        g = (g + F32(weight_decay) * p).astype(F32)
    m = lerp(m, g, 1 - beta1)
    v = (v * F32(beta2)).astype(F32)
    v = (v + F32(1 - beta2) * (g * g)).astype(F32)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    step_size = F32((lr / bc1) * -1)
    den = (np.sqrt(v) / F32(bc2 ** 0.5) + F32(eps)).astype(F32)
    p = (p + step_size * (m / den)).astype(F32)
    return p, m, v
