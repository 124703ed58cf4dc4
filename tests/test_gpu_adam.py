"""Fused Adam step (r2splat.optim) against torch.optim.Adam on the GPU and
against the numpy oracle."""

import numpy as np
import pytest
import torch

from helpers import np32
from oracle import adam as A
from r2splat import optim

pytestmark = pytest.mark.gpu

DEV = "cuda"
SHAPES = {"means": (5003, 3), "scales": (5003, 3), "quats": (5003, 4), "opacities": (5003,)}
LRS = {"means": 1.6e-4, "scales": 5e-3, "quats": 1e-3, "opacities": 5e-2}


def _params(seed):
    g = torch.Generator().manual_seed(seed)
    return {k: torch.randn(s, generator=g).to(DEV) for k, s in SHAPES.items()}


def _grads(seed, steps):
    g = torch.Generator().manual_seed(seed)
    return [{k: (torch.randn(s, generator=g) * 10 ** (torch.rand(1, generator=g) * 4 - 3)).to(DEV)
             for k, s in SHAPES.items()} for _ in range(steps)]


def _build(init, cls, **kw):
    params = {k: torch.nn.Parameter(v.clone()) for k, v in init.items()}
    opts = {k: cls([{"params": p, "name": k}], lr=LRS[k], eps=1e-15, **kw)
            for k, p in params.items()}
    return params, opts


def _ulps(a, b):
    a, b = np32(a).view(np.int32).astype(np.int64), np32(b).view(np.int32).astype(np.int64)
    return int(np.abs(a - b).max()) if a.size else 0


@pytest.mark.parametrize("wd", [0.0, 1e-2])
def test_fused_step_equals_torch_adam(wd):
    init, grads = _params(0), _grads(1, 7)
    ref_p, ref_o = _build(init, torch.optim.Adam, weight_decay=wd, foreach=True)
    our_p, our_o = _build(init, optim.Adam, weight_decay=wd)
    for step, gr in enumerate(grads):
        for k in SHAPES:
            ref_p[k].grad = gr[k].clone()
            our_p[k].grad = gr[k].clone()
        for o in ref_o.values():
            o.step()
        if step % 2:
            optim.step_all(our_o)
        else:
            for o in our_o.values():
                o.step()
        for k in SHAPES:
            rs, os_ = ref_o[k].state[ref_p[k]], our_o[k].state[our_p[k]]
            assert torch.equal(rs["step"], os_["step"])
            # The same float32 operations and FMAs as torch's kernels: at most
            # an ulp apart, and in practice equal.
            u = (_ulps(rs["exp_avg"], os_["exp_avg"]), _ulps(rs["exp_avg_sq"], os_["exp_avg_sq"]),
                 _ulps(ref_p[k].detach(), our_p[k].detach()))
            assert u[0] <= 1 and u[1] <= 1 and u[2] <= 2, (k, step, u)


def test_misaligned_parameters_take_the_element_path():
    # Parameters viewing their storage one element in: the kernel's 16-byte
    # loads do not apply, so every element goes through the element loop,
    # which must give the same values as torch's Adam (and as the aligned
    # path, which test_fused_step_equals_torch_adam checks).
    init, grads = _params(6), _grads(7, 3)
    ref_p, ref_o = _build(init, torch.optim.Adam, foreach=True)
    our_p = {}
    for k, v in init.items():
        flat = torch.empty(v.numel() + 1, device=DEV)
        view = flat[1:].view(v.shape)
        view.copy_(v)
        our_p[k] = torch.nn.Parameter(view)
        assert our_p[k].data_ptr() % 16 != 0
    our_o = {k: optim.Adam([{"params": p, "name": k}], lr=LRS[k], eps=1e-15)
             for k, p in our_p.items()}
    for gr in grads:
        for k in SHAPES:
            ref_p[k].grad = gr[k].clone()
            our_p[k].grad = gr[k].clone()
        for o in ref_o.values():
            o.step()
        optim.step_all(our_o)
        for k in SHAPES:
            rs, os_ = ref_o[k].state[ref_p[k]], our_o[k].state[our_p[k]]
            u = (_ulps(rs["exp_avg"], os_["exp_avg"]), _ulps(rs["exp_avg_sq"], os_["exp_avg_sq"]),
                 _ulps(ref_p[k].detach(), our_p[k].detach()))
            assert u[0] <= 1 and u[1] <= 1 and u[2] <= 2, (k, u)


def test_fused_step_matches_the_oracle():
    init, grads = _params(2), _grads(3, 5)
    our_p, our_o = _build(init, optim.Adam, betas=(0.8, 0.99))
    ref = {k: (np32(v), np.zeros(v.shape, np.float32), np.zeros(v.shape, np.float32))
           for k, v in init.items()}
    for t, gr in enumerate(grads, start=1):
        for k in SHAPES:
            our_p[k].grad = gr[k]
        optim.step_all(our_o.values())
        for k in SHAPES:
            p, m, v = A.adam_step(ref[k][0], np32(gr[k]), ref[k][1], ref[k][2], t, LRS[k],
                                  0.8, 0.99, 1e-15)
            ref[k] = (p, m, v)
            st = our_o[k].state[our_p[k]]
            np.testing.assert_allclose(np32(st["exp_avg"]), m, rtol=1e-6,
                                       atol=1e-6 * np.abs(m).max())
            np.testing.assert_allclose(np32(st["exp_avg_sq"]), v, rtol=1e-6,
                                       atol=1e-6 * np.abs(v).max())
            # The device rounds p + step * (m / d) once (FMA), numpy twice: an ulp of
            # the update, whose size is about lr.
            np.testing.assert_allclose(np32(our_p[k].detach()), p, rtol=1e-6,
                                       atol=1e-6 * LRS[k])


def test_parameters_without_gradients_are_skipped_and_state_dict_round_trips():
    init, grads = _params(4), _grads(5, 2)
    our_p, our_o = _build(init, optim.Adam)
    our_p["means"].grad = grads[0]["means"]
    optim.step_all(our_o)
    assert len(our_o["quats"].state) == 0
    assert torch.equal(our_p["quats"].detach(), init["quats"])
    sd = our_o["means"].state_dict()
    twin = torch.optim.Adam([our_p["means"]], lr=LRS["means"], eps=1e-15)
    twin.load_state_dict(sd)
    assert torch.equal(twin.state[our_p["means"]]["exp_avg"],
                       our_o["means"].state[our_p["means"]]["exp_avg"])


def test_unsupported_options_raise():
    p = torch.nn.Parameter(torch.zeros(3, device=DEV))
    with pytest.raises(NotImplementedError):
        optim.Adam([p], amsgrad=True)
    with pytest.raises(NotImplementedError):
        optim.Adam([p], maximize=True)
