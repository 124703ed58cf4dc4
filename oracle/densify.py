"""Densify / prune of the binary-tree model table, restated in numpy -- TEST INFRASTRUCTURE ONLY.

Restates ``duplicate`` / ``split`` / ``remove`` and ``_append_history`` of
``src/strategies/binary_tree.py`` (lines 17-171) and the optimizer-state
rewrite of ``src/utils/ops.py:61-103`` on a plain table:

    table = {"means" [N,3], "scales" [N,3] (raw), "quats" [N,4], "opacities" [N] (raw),
             "parent" [N] i32, "level" [N] i32,
             "history_<x>" for x in means, scales, quats, opacities, parent, level,
             "moments": {param name: {state key: array [N, ...]}},
             "state": {key: array [N, ...]}}

Float arithmetic is float32, one rounding per torch elementwise op, in the
reference's order.  Two choices follow torch's CUDA kernels, which the
reference runs on: the division by the host scalar 1.6 is a multiplication
by the float32 reciprocal, and the transcendental functions are numpy's
float32 ones (equal to the device's up to an ulp).

How this restatement is pinned (tests/test_oracle_densify.py): an
independent rotation routine (scipy) for the child offsets, the forward
activations for the inverted scales and the revised opacity's closed form,
brute-force loops for the row order and the tree links, and the reference's
own consequence that a split tree's archive reproduces every leaf's
ancestry.
"""

from __future__ import annotations

import copy

import numpy as np

F32 = np.float32
HISTORY = ("means", "scales", "quats", "opacities", "parent", "level")
PARAMS = ("means", "scales", "quats", "opacities")


def scale_activation(sigmoid=True, lo=5e-4, hi=1.0, eps=1e-5):
    """gaussian_model.py:686-715 bounds: per-axis float32 lo / hi and eps."""
    return dict(sigmoid=bool(sigmoid), lo=np.broadcast_to(np.asarray(lo, F32), (3,)).copy(),
                hi=np.broadcast_to(np.asarray(hi, F32), (3,)).copy(), eps=float(eps))


def activate_scale(raw, act):
    """gaussian_model.py:258-264."""
    raw = np.asarray(raw, F32)
    if not act["sigmoid"]:
        return np.exp(raw)
    sig = F32(1) / (F32(1) + np.exp(-raw))
    return act["lo"] + (act["hi"] - act["lo"]) * sig


def inverse_activate_scale(scales, act):
    """gaussian_model.py:266-274: clamp by eps inside the bounds, then logit."""
    scales = np.asarray(scales, F32)
    if not act["sigmoid"]:
        return np.log(np.maximum(scales, F32(1e-12)))
    lo, hi = act["lo"], act["hi"]
    clamped = np.minimum(np.maximum(scales, lo + F32(act["eps"])), hi - F32(act["eps"]))
    sig = (clamped - lo) / (hi - lo)
    sig = np.minimum(np.maximum(sig, F32(1e-6)), F32(1.0 - 1e-6))
    return np.log(sig / (F32(1) - sig))


def softplus(x):
    """torch.nn.functional.softplus (beta 1, threshold 20)."""
    x = np.asarray(x, F32)
    with np.errstate(over="ignore"):
        return np.where(x > F32(20), x, np.log1p(np.exp(x))).astype(F32)


def normalized_quat_to_rotmat(q):
    """src/utils/math.py:35-53 (rows of the matrix, wxyz quaternions)."""
    w, x, y, z = (q[:, i] for i in range(4))
    one, two = F32(1), F32(2)
    m = np.stack([one - two * (y * y + z * z), two * (x * y - w * z), two * (x * z + w * y),
                  two * (x * y + w * z), one - two * (x * x + z * z), two * (y * z - w * x),
                  two * (x * z - w * y), two * (y * z + w * x), one - two * (x * x + y * y)], -1)
    return m.reshape(-1, 3, 3)


def where_split(mask):
    """torch.where(mask)[0], torch.where(~mask)[0] (binary_tree.py:101-102)."""
    mask = np.asarray(mask, bool)
    return np.nonzero(mask)[0], np.nonzero(~mask)[0]


def _children(t, sel, act, revised_opacity):
    """binary_tree.py:99-112, 122-135: per selected row, the children's
    means (+ block, - block), raw scales and raw opacities."""
    scales = activate_scale(t["scales"][sel], act)
    q = t["quats"][sel].astype(F32)
    nrm = np.sqrt(((q[:, 0] * q[:, 0] + q[:, 1] * q[:, 1]) + q[:, 2] * q[:, 2]) + q[:, 3] * q[:, 3])
    q = q / np.maximum(nrm, F32(1e-12))[:, None]
    rot = normalized_quat_to_rotmat(q)
    longest = np.argmax(scales, axis=-1)
    rows = np.arange(sel.size)
    s_long = scales[rows, longest]
    offset = rot[rows, :, longest] * s_long[:, None]        # einsum with one nonzero term
    means = t["means"][sel].astype(F32)
    plus, minus = means + offset, means + (-offset)
    target = scales.copy()
    inv = F32(1) / F32(1.6)
    target[rows, longest] = np.maximum(s_long * inv, F32(1e-12))
    raw_scales = inverse_activate_scale(target, act)
    if revised_opacity:
        base = np.minimum(softplus(t["opacities"][sel]), F32(0.9999))
        fresh = F32(1) - np.sqrt(F32(1) - base)
        raw_opac = np.log(np.expm1(fresh)).astype(F32)
    else:
        raw_opac = t["opacities"][sel]
    return plus, minus, raw_scales, raw_opac


def _append_history(t, sel):
    """binary_tree.py:17-57: archive the selected rows; returns their new indices."""
    start = t["history_parent"].shape[0]
    if sel.size == 0:
        return np.zeros(0, np.int32)
    for x in HISTORY:
        t["history_" + x] = np.concatenate([t["history_" + x], t[x][sel]], axis=0)
    return np.arange(start, start + sel.size, dtype=np.int32)


def split(table, mask, act, trainable=PARAMS, revised_opacity=False):
    """binary_tree.py:93-148 on a copy of ``table``."""
    t = copy.deepcopy(table)
    sel, rest = where_split(mask)
    plus, minus, raw_scales, raw_opac = _children(table, sel, act, revised_opacity)
    hist = _append_history(t, sel)
    split_level = table["level"][sel] + np.int32(1)
    t["parent"] = np.concatenate([table["parent"][rest], hist, hist]).astype(np.int32)
    t["level"] = np.concatenate([table["level"][rest], split_level, split_level]).astype(np.int32)
    for name in trainable:
        p = table[name]
        if name == "means":
            new = np.concatenate([plus, minus])
        elif name == "scales":
            new = np.concatenate([raw_scales, raw_scales])
        elif name == "opacities" and revised_opacity:
            new = np.concatenate([raw_opac, raw_opac])
        else:
            new = np.concatenate([p[sel], p[sel]])
        t[name] = np.concatenate([p[rest], new]).astype(p.dtype)
        for key, v in table["moments"].get(name, {}).items():
            zeros = np.zeros((2 * sel.size,) + v.shape[1:], v.dtype)
            t["moments"][name][key] = np.concatenate([v[rest], zeros])
    for key, v in table["state"].items():
        t["state"][key] = np.concatenate([v[rest], v[sel], v[sel]])
    return t


def duplicate(table, mask, trainable=PARAMS):
    """binary_tree.py:60-90 on a copy of ``table``."""
    t = copy.deepcopy(table)
    sel, _ = where_split(mask)
    hist = _append_history(t, sel)
    parent = table["parent"].copy()
    parent[sel] = hist
    t["parent"] = np.concatenate([parent, hist]).astype(np.int32)
    level = table["level"].copy()
    level[sel] = level[sel] + np.int32(1)
    t["level"] = np.concatenate([level, level[sel]]).astype(np.int32)
    for name in trainable:
        p = table[name]
        t[name] = np.concatenate([p, p[sel]])
        for key, v in table["moments"].get(name, {}).items():
            zeros = np.zeros((sel.size,) + v.shape[1:], v.dtype)
            t["moments"][name][key] = np.concatenate([v, zeros])
    for key, v in table["state"].items():
        t["state"][key] = np.concatenate([v, v[sel]])
    return t


def remove(table, mask, trainable=PARAMS):
    """binary_tree.py:151-171 on a copy of ``table``."""
    t = copy.deepcopy(table)
    _, keep = where_split(mask)
    t["parent"] = table["parent"][keep]
    t["level"] = table["level"][keep]
    for name in trainable:
        t[name] = table[name][keep]
        for key, v in table["moments"].get(name, {}).items():
            t["moments"][name][key] = v[keep]
    for key, v in table["state"].items():
        t["state"][key] = v[keep]
    return t


def random_table(n, rng, n_history=0, act=None, with_moments=True, radii=True):
    """A seeded table in the model's parameterisation (for tests)."""
    act = act or scale_activation()
    log_scales = rng.normal(-3.0, 1.0, (n, 3))
    scales = np.exp(log_scales).astype(F32)
    t = {
        "means": rng.uniform(-1, 1, (n, 3)).astype(F32),
        "scales": inverse_activate_scale(scales, act).astype(F32),
        "quats": rng.normal(0, 1, (n, 4)).astype(F32),
        "opacities": np.log(np.expm1(rng.uniform(1e-3, 1.0, n))).astype(F32),
        "parent": rng.integers(-1, max(n_history, 1), n).astype(np.int32),
        "level": rng.integers(0, 20, n).astype(np.int32),
    }
    for x in HISTORY:
        ref = t[x]
        t["history_" + x] = (rng.normal(0, 1, (n_history,) + ref.shape[1:]).astype(F32)
                             if ref.dtype == F32 else
                             rng.integers(-1, 100, (n_history,) + ref.shape[1:]).astype(np.int32))
    t["moments"] = {}
    if with_moments:
        for name in PARAMS:
            shape = t[name].shape
            t["moments"][name] = {"exp_avg": rng.normal(0, 1e-3, shape).astype(F32),
                                  "exp_avg_sq": rng.uniform(0, 1e-6, shape).astype(F32)}
    t["state"] = {"grad2d": rng.uniform(0, 1, n).astype(F32),
                  "count": rng.integers(0, 100, n).astype(F32)}
    if radii:
        t["state"]["radii"] = rng.uniform(0, 0.5, n).astype(F32)
    return t
