"""Densify / prune of the binary-tree Gaussian model, one HIP launch per call.

Drop-in for ``duplicate``, ``split`` and ``remove`` of
``src/strategies/binary_tree.py`` (lines 60-90, 93-148, 151-171), with the
same signatures and the same effect on the model, its optimizers and the
strategy state:

* the history archive (``history_means`` ... ``history_level``) gains the
  selected rows (``_append_history``, lines 17-57);
* ``parent`` / ``level`` are rebuilt (children point at their archived
  parent, one level deeper);
* every trainable parameter is replaced by a new ``nn.Parameter`` and its
  Adam state re-keyed (``src/utils/ops.py:61-103``): moments gathered, and
  zero for new rows;
* every tensor in ``state`` is gathered like the parameters.

The reference does this with one ``torch.where`` (a host sync) per call plus
an index_select / repeat / cat chain per array: about 30 small kernels.
Here the index lists come from one compaction pass (one host read of the
selected count) and every array of the table is written by a single launch
(``r2s_densify_*``).  The model is used through the attributes the
reference's ``BinaryTreeGaussianModel`` has: the parameters, the tree
buffers, the history buffers and the scale activation
(``_use_sigmoid_scale``, ``_scale_min``, ``_scale_max``, ``_scale_eps``).
"""

from __future__ import annotations

from typing import Any, Dict, List

import torch
from torch import Tensor

from ..cuda import _lib as L
from ..cuda import _wrapper

__all__ = ["duplicate", "split", "remove"]

# (history buffer, live attribute) pairs archived by _append_history (binary_tree.py:30-56).
_HISTORY = (("history_means", "means"), ("history_scales", "scales"),
            ("history_quats", "quats"), ("history_opacities", "opacities"),
            ("history_parent", "parent"), ("history_level", "level"))


def _history_columns(model) -> list:
    return [(getattr(model, h), L.COL_HISTORY, getattr(model, live).detach())
            for h, live in _HISTORY]


def _tensor_states(state: Dict[str, Any]) -> List[str]:
    return [k for k, v in state.items() if isinstance(v, torch.Tensor)]


def _moment_keys(optimizers, name: str, param: Tensor) -> List[str]:
    if name not in optimizers:
        return []
    st = optimizers[name].state.get(param, {})
    return [k for k in st if k != "step"]


def _plan(model, optimizers, state, trainable_param_keys, param_role, moment_role):
    """Column list plus the bookkeeping to put the outputs back."""
    cols, slots = [], []
    for name in trainable_param_keys:
        p = getattr(model, name)
        cols.append((p.detach(), param_role(name), None))
        slots.append(("param", name, None))
        for key in _moment_keys(optimizers, name, p):
            cols.append((optimizers[name].state[p][key], moment_role, None))
            slots.append(("moment", name, key))
    for k in _tensor_states(state):
        cols.append((state[k], L.COL_COPY, None))
        slots.append(("state", k, None))
    return cols, slots


def _install(model, optimizers, state, trainable_param_keys, slots, outs) -> None:
    """Put the rewritten arrays in place.

    Each trainable parameter becomes a new ``nn.Parameter`` over its rewritten
    rows.  Its optimizer state dict moves, as one object, from the old
    parameter to the new one, with every tensor moment (each key but "step")
    swapped for its rewritten array, and the optimizer's groups point at the
    new parameter.  That is the effect of utils/ops.py:85-103 for optimizers
    of one parameter group each, which is how the model builds them.  A
    parameter without an optimizer must be frozen; the assertion message is
    the reference's.
    """
    written = dict(zip(slots, outs))
    for name in trainable_param_keys:
        old = getattr(model, name)
        new = torch.nn.Parameter(written[("param", name, None)], requires_grad=old.requires_grad)
        setattr(model, name, new)
        opt = optimizers.get(name)
        if opt is None:
            assert not old.requires_grad, (
                f"Optimizer for {name} is not found, but parameter is trainable "
                f"(requires_grad={old.requires_grad})."
            )
            continue
        moved = opt.state.pop(old, {})
        moved.update({k: written[("moment", name, k)] for k in moved if k != "step"})
        for group in opt.param_groups:
            group["params"] = [new]
        opt.state[new] = moved
    state.update({name: t for (kind, name, _), t in written.items() if kind == "state"})


def _history_rows(model) -> int:
    return int(model.history_parent.shape[0])


def _install_history(model, outs) -> None:
    for (h, _), t in zip(_HISTORY, outs):
        setattr(model, h, t)


@torch.no_grad()
def duplicate(model: torch.nn.Module, optimizers: Dict[str, torch.optim.Optimizer],
              state: Dict[str, Any], mask: Tensor, trainable_param_keys: List[str]):
    """binary_tree.py:60-90: append copies of the masked Gaussians."""
    cols, slots = _plan(model, optimizers, state, trainable_param_keys,
                        lambda name: L.COL_COPY, L.COL_ZERO_NEW)
    n_hist = len(_HISTORY)
    tree = [(model.parent, L.COL_PARENT, None), (model.level, L.COL_LEVEL, None)]
    all_cols = _history_columns(model) + tree + cols
    outs, n_sel = _wrapper.densify_duplicate(mask, all_cols, _history_rows(model))
    if n_sel > 0:
        _install_history(model, outs[:n_hist])
    model.parent, model.level = outs[n_hist], outs[n_hist + 1]
    _install(model, optimizers, state, trainable_param_keys, slots, outs[n_hist + 2:])


@torch.no_grad()
def split(model: torch.nn.Module, optimizers: Dict[str, torch.optim.Optimizer],
          state: Dict[str, Any], mask: Tensor, trainable_param_keys: List[str],
          revised_opacity: bool = False):
    """binary_tree.py:93-148: replace each masked Gaussian by two children
    offset by +/- its longest axis, that axis shortened by 1.6."""

    def role(name: str) -> int:
        if name == "means":
            return L.COL_MEANS
        if name == "scales":
            return L.COL_RAW_SCALES
        if name == "opacities" and revised_opacity:
            return L.COL_RAW_OPACITIES
        return L.COL_COPY

    cols, slots = _plan(model, optimizers, state, trainable_param_keys, role, L.COL_ZERO_NEW)
    n_hist = len(_HISTORY)
    tree = [(model.parent, L.COL_PARENT, None), (model.level, L.COL_LEVEL, None)]
    all_cols = _history_columns(model) + tree + cols
    outs, n_sel = _wrapper.densify_split(mask, all_cols, _history_rows(model),
                                         _geometry(model))
    if n_sel > 0:
        _install_history(model, outs[:n_hist])
    model.parent, model.level = outs[n_hist], outs[n_hist + 1]
    _install(model, optimizers, state, trainable_param_keys, slots, outs[n_hist + 2:])


@torch.no_grad()
def remove(model: torch.nn.Module, optimizers: Dict[str, torch.optim.Optimizer],
           state: Dict[str, Tensor], mask: Tensor, trainable_param_keys: List[str]):
    """binary_tree.py:151-171: drop the masked Gaussians."""
    cols, slots = _plan(model, optimizers, state, trainable_param_keys,
                        lambda name: L.COL_COPY, L.COL_COPY)
    tree = [(model.parent, L.COL_COPY, None), (model.level, L.COL_COPY, None)]
    outs, _ = _wrapper.densify_remove(mask, tree + cols)
    model.parent, model.level = outs[0], outs[1]
    _install(model, optimizers, state, trainable_param_keys, slots, outs[2:])


def _bounds(v) -> List[float]:
    t = torch.as_tensor(v, dtype=torch.float32).reshape(-1).cpu()
    if t.numel() == 1:
        return [float(t[0])] * 3
    if t.numel() == 3:
        return [float(x) for x in t]
    raise ValueError("scale bounds must be a scalar or one value per axis")


def _geometry(model):
    """Live quats / raw scales and the scale activation of gaussian_model.py:258-274."""
    if model._use_sigmoid_scale:
        lo, hi, eps = _bounds(model._scale_min), _bounds(model._scale_max), model._scale_eps
    else:
        lo, hi, eps = [0.0] * 3, [0.0] * 3, 0.0
    return (model.quats.detach(), model.scales.detach(), lo, hi, float(eps),
            bool(model._use_sigmoid_scale))
