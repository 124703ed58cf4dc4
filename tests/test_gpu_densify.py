"""Fused densify / prune (r2splat.ops.densify) against the numpy oracle.

The model object carries the attributes of the reference's
BinaryTreeGaussianModel (parameters, tree and history buffers, the scale
activation) and real torch.optim.Adam optimizers, as built by
gaussian_model.py:514-530.  Copies, zeros, tree links and the archive are
compared bit-exactly; split children within float32 tolerances (they pass
through exp / log / sqrt, which the device and numpy round differently by
an ulp).
"""

import numpy as np
import pytest
import torch

from helpers import np32
from oracle import densify as D
from r2splat.ops import densify

pytestmark = pytest.mark.gpu

DEV = "cuda"


class TreeModel(torch.nn.Module):
    def __init__(self, t, act, trainable=D.PARAMS):
        super().__init__()
        for name in D.PARAMS:
            p = torch.nn.Parameter(torch.from_numpy(t[name].copy()).to(DEV),
                                   requires_grad=name in trainable)
            setattr(self, name, p)
        self.register_buffer("parent", torch.from_numpy(t["parent"].copy()).to(DEV))
        self.register_buffer("level", torch.from_numpy(t["level"].copy()).to(DEV))
        for x in D.HISTORY:
            self.register_buffer("history_" + x, torch.from_numpy(t["history_" + x].copy()).to(DEV))
        self._use_sigmoid_scale = act["sigmoid"]
        lo, hi = act["lo"], act["hi"]
        self._scale_min = torch.tensor(lo[0] if np.all(lo == lo[0]) else lo)
        self._scale_max = torch.tensor(hi[0] if np.all(hi == hi[0]) else hi)
        self._scale_eps = act["eps"]
        self.trainable_param_keys = list(trainable)


def _build(t, act, trainable=D.PARAMS):
    model = TreeModel(t, act, trainable)
    opts = {}
    for name in trainable:
        p = getattr(model, name)
        opt = torch.optim.Adam([{"params": p, "name": name}], lr=1e-3, eps=1e-15)
        p.grad = torch.ones_like(p)
        opt.step()
        p.grad = None
        st = opt.state[p]
        st["exp_avg"].copy_(torch.from_numpy(t["moments"][name]["exp_avg"]))
        st["exp_avg_sq"].copy_(torch.from_numpy(t["moments"][name]["exp_avg_sq"]))
        opts[name] = opt
    with torch.no_grad():  # the optimizer step moved the parameters; restore them
        for name in trainable:
            getattr(model, name).copy_(torch.from_numpy(t[name]))
    state = {k: torch.from_numpy(v.copy()).to(DEV) for k, v in t["state"].items()}
    state["scene_scale"] = 1.0
    return model, opts, state


def _oracle_table(t, trainable):
    out = dict(t)
    out["moments"] = {k: v for k, v in t["moments"].items() if k in trainable}
    return out


def _check(model, opts, state, exp, trainable, n_rest, n_sel, op, steps):
    for x in D.HISTORY:
        assert torch.equal(getattr(model, "history_" + x).cpu(),
                           torch.from_numpy(exp["history_" + x])), x
    assert torch.equal(model.parent.cpu(), torch.from_numpy(exp["parent"]))
    assert torch.equal(model.level.cpu(), torch.from_numpy(exp["level"]))
    for name in D.PARAMS:
        got, want = np32(getattr(model, name).detach()), exp[name]
        assert got.shape == want.shape, name
        if name not in trainable:
            continue
        assert getattr(model, name).requires_grad
        if op != "split":
            assert np.array_equal(got, want), name
            continue
        assert np.array_equal(got[:n_rest], want[:n_rest]), name
        kids, wk = got[n_rest:], want[n_rest:]
        if name == "means":
            np.testing.assert_allclose(kids, wk, rtol=1e-5, atol=1e-6, err_msg=name)
        elif name == "scales":
            act = model_act(model)
            np.testing.assert_allclose(D.activate_scale(kids, act).astype(np.float64),
                                       D.activate_scale(wk, act), rtol=2e-6, atol=1e-9)
            ok = np.abs(wk) < 8  # away from saturation the raw values agree too
            np.testing.assert_allclose(kids[ok], wk[ok], rtol=1e-4, atol=1e-5)
        elif name == "opacities":
            np.testing.assert_allclose(kids, wk, rtol=1e-4, atol=1e-5)
        else:
            assert np.array_equal(kids, wk), name
    for name in trainable:
        p = getattr(model, name)
        opt = opts[name]
        assert opt.param_groups[0]["params"][0] is p
        st = opt.state[p]
        assert torch.equal(st["step"].cpu(), torch.tensor(float(steps)))
        for key in ("exp_avg", "exp_avg_sq"):
            assert torch.equal(st[key].cpu(), torch.from_numpy(exp["moments"][name][key])), key
    for k, v in exp["state"].items():
        assert torch.equal(state[k].cpu(), torch.from_numpy(v)), k


def model_act(model):
    lo = model._scale_min.reshape(-1).expand(3).numpy() if model._use_sigmoid_scale else 0
    hi = model._scale_max.reshape(-1).expand(3).numpy() if model._use_sigmoid_scale else 0
    return D.scale_activation(model._use_sigmoid_scale, lo, hi, model._scale_eps)


ACTS = {
    "sigmoid": D.scale_activation(True, 5e-4, 1.0, 1e-5),
    "per_axis": D.scale_activation(True, [1e-4, 5e-4, 1e-3], [0.5, 1.0, 2.0], 1e-5),
    "exp": D.scale_activation(False),
}


def _table(n, seed, act, h=17):
    t = D.random_table(n, np.random.default_rng(seed), n_history=h)
    if not act["sigmoid"]:
        t["scales"] = np.log(D.activate_scale(t["scales"], ACTS["sigmoid"])).astype(np.float32)
    return t


@pytest.mark.parametrize("act_name", list(ACTS))
@pytest.mark.parametrize("revised", [False, True])
@pytest.mark.parametrize("frac", [0.0, 0.3, 1.0])
def test_split_matches_the_oracle(act_name, revised, frac):
    act = ACTS[act_name]
    n = 5000
    t = _table(n, 11, act)
    mask = np.random.default_rng(12).uniform(size=n) < frac
    model, opts, state = _build(t, act)
    hist_before = model.history_means
    densify.split(model, opts, state, torch.from_numpy(mask).to(DEV), model.trainable_param_keys,
                  revised_opacity=revised)
    exp = D.split(t, mask, act, revised_opacity=revised)
    ns = int(mask.sum())
    _check(model, opts, state, exp, D.PARAMS, n - ns, ns, "split", 1)
    if ns == 0:
        assert model.history_means is hist_before


@pytest.mark.parametrize("frac", [0.0, 0.25, 1.0])
def test_duplicate_matches_the_oracle(frac):
    act = ACTS["sigmoid"]
    n = 4099
    t = _table(n, 21, act)
    mask = np.random.default_rng(22).uniform(size=n) < frac
    model, opts, state = _build(t, act)
    densify.duplicate(model, opts, state, torch.from_numpy(mask).to(DEV),
                      model.trainable_param_keys)
    _check(model, opts, state, D.duplicate(t, mask), D.PARAMS, n, int(mask.sum()), "duplicate", 1)


@pytest.mark.parametrize("frac", [0.0, 0.4, 1.0])
def test_remove_matches_the_oracle(frac):
    act = ACTS["sigmoid"]
    n = 3000
    t = _table(n, 31, act)
    mask = np.random.default_rng(32).uniform(size=n) < frac
    model, opts, state = _build(t, act)
    densify.remove(model, opts, state, torch.from_numpy(mask).to(DEV), model.trainable_param_keys)
    _check(model, opts, state, D.remove(t, mask), D.PARAMS, n - int(mask.sum()),
           int(mask.sum()), "remove", 1)


def test_untrained_parameters_are_left_alone_as_in_the_reference():
    """Only trainable_param_keys are rewritten (utils/ops.py:85-89)."""
    act = ACTS["sigmoid"]
    n = 777
    trainable = ("means", "opacities")
    t = _table(n, 41, act)
    mask = np.random.default_rng(42).uniform(size=n) < 0.5
    model, opts, state = _build(t, act, trainable)
    densify.split(model, opts, state, torch.from_numpy(mask).to(DEV), list(trainable))
    exp = D.split(_oracle_table(t, trainable), mask, act, trainable=trainable)
    ns = int(mask.sum())
    _check(model, opts, state, exp, trainable, n - ns, ns, "split", 1)
    assert model.quats.shape[0] == n and not model.quats.requires_grad


def test_a_training_step_runs_on_the_rewritten_table():
    act = ACTS["sigmoid"]
    n = 2048
    t = _table(n, 51, act)
    model, opts, state = _build(t, act)
    rng = np.random.default_rng(52)
    densify.duplicate(model, opts, state, torch.from_numpy(rng.uniform(size=n) < 0.1).to(DEV),
                      model.trainable_param_keys)
    n1 = model.means.shape[0]
    densify.split(model, opts, state, torch.from_numpy(rng.uniform(size=n1) < 0.1).to(DEV),
                  model.trainable_param_keys, revised_opacity=True)
    n2 = model.means.shape[0]
    densify.remove(model, opts, state, torch.from_numpy(rng.uniform(size=n2) < 0.1).to(DEV),
                   model.trainable_param_keys)
    for name in D.PARAMS:
        p = getattr(model, name)
        assert p.shape[0] == model.parent.shape[0] == state["grad2d"].shape[0]
        p.grad = torch.ones_like(p)
        before = p.detach().clone()
        opts[name].step()
        assert not torch.equal(before, p.detach())
        assert torch.equal(opts[name].state[p]["step"].cpu(), torch.tensor(2.0))


def test_config4_sized_split_and_prune():
    """N = 500k (config 4): 1 % split then 1 % prune; copies bit-exact."""
    act = ACTS["sigmoid"]
    n = 500_000
    t = _table(n, 61, act, h=300_000)
    rng = np.random.default_rng(62)
    mask = rng.uniform(size=n) < 0.01
    model, opts, state = _build(t, act)
    densify.split(model, opts, state, torch.from_numpy(mask).to(DEV), model.trainable_param_keys)
    exp = D.split(t, mask, act)
    ns = int(mask.sum())
    _check(model, opts, state, exp, D.PARAMS, n - ns, ns, "split", 1)
    n1 = n + ns
    prune = rng.uniform(size=n1) < 0.01
    densify.remove(model, opts, state, torch.from_numpy(prune).to(DEV), model.trainable_param_keys)
    exp2 = D.remove(exp, prune)
    for name in ("quats", "parent", "level"):
        assert np.array_equal(np32(getattr(model, name).detach()), exp2[name]), name
    assert torch.equal(state["count"].cpu(), torch.from_numpy(exp2["state"]["count"]))
