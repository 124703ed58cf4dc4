"""Pins oracle/densify.py (split / duplicate / remove of the binary-tree table).

Each check is independent of the restated formula:
* child offsets against scipy's quaternion rotation in float64;
* inverted child scales through the forward activation in float64;
* the revised opacity through its closed form 1 - (1 - o_child)^2 = o_parent;
* row order, tree links, Adam zeros and state repeats against brute-force loops;
* the archive of a grown tree reproduces every leaf's ancestry.
"""

import numpy as np
import pytest
from scipy.spatial.transform import Rotation

from oracle import densify as D

ACT = D.scale_activation(True, 5e-4, 1.0, 1e-5)


def _act64(raw, act):
    raw = np.asarray(raw, np.float64)
    if not act["sigmoid"]:
        return np.exp(raw)
    lo, hi = act["lo"].astype(np.float64), act["hi"].astype(np.float64)
    return lo + (hi - lo) / (1.0 + np.exp(-raw))


def _softplus64(x):
    return np.log1p(np.exp(np.asarray(x, np.float64)))


@pytest.fixture(scope="module")
def table():
    return D.random_table(300, np.random.default_rng(0), n_history=40)


@pytest.fixture(scope="module")
def mask():
    return np.random.default_rng(1).uniform(size=300) < 0.3


@pytest.mark.parametrize("act", [ACT, D.scale_activation(False)], ids=["sigmoid", "exp"])
def test_children_straddle_the_parent_along_its_rotated_longest_axis(table, mask, act):
    t = dict(table)
    if not act["sigmoid"]:
        t["scales"] = np.log(_act64(table["scales"], ACT)).astype(np.float32)
    out = D.split(t, mask, act)
    sel, rest = D.where_split(mask)
    ns, nr = sel.size, rest.size
    plus, minus = out["means"][nr:nr + ns].astype(np.float64), out["means"][nr + ns:].astype(np.float64)
    s = _act64(t["scales"][sel], act)
    axis = np.argmax(s, axis=1)
    q = t["quats"][sel].astype(np.float64)
    rot = Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix()  # scipy is scalar-last
    expect = rot[np.arange(ns), :, axis] * s[np.arange(ns), axis][:, None]
    np.testing.assert_allclose((plus - minus) / 2, expect, rtol=2e-5, atol=1e-7)
    np.testing.assert_allclose((plus + minus) / 2, t["means"][sel], rtol=1e-6, atol=1e-6)
    assert np.array_equal(out["means"][:nr], t["means"][rest])


def test_child_scales_are_the_parent_scales_with_the_longest_axis_over_1_6(table, mask):
    out = D.split(table, mask, ACT)
    sel, rest = D.where_split(mask)
    ns, nr = sel.size, rest.size
    s = _act64(table["scales"][sel], ACT)
    axis = np.argmax(s, axis=1)
    target = s.copy()
    target[np.arange(ns), axis] /= 1.6
    lo, hi, eps = 5e-4, 1.0, 1e-5
    target = np.clip(target, lo + eps, hi - eps)
    for blk in (out["scales"][nr:nr + ns], out["scales"][nr + ns:]):
        np.testing.assert_allclose(_act64(blk, ACT), target, rtol=1e-5)
    assert np.array_equal(out["scales"][nr:nr + ns], out["scales"][nr + ns:])


def test_revised_opacity_composes_back_to_the_parent(table, mask):
    out = D.split(table, mask, ACT, revised_opacity=True)
    sel, rest = D.where_split(mask)
    ns, nr = sel.size, rest.size
    child = _softplus64(out["opacities"][nr:nr + ns])
    parent = np.minimum(_softplus64(table["opacities"][sel]), 0.9999)
    np.testing.assert_allclose(1 - (1 - child) ** 2, parent, rtol=1e-4, atol=1e-6)
    plain = D.split(table, mask, ACT, revised_opacity=False)
    assert np.array_equal(plain["opacities"][nr:nr + ns], table["opacities"][sel])


def test_split_rows_links_moments_and_state_by_brute_force(table, mask):
    out = D.split(table, mask, ACT)
    n, h = mask.size, table["history_parent"].size
    kept = [i for i in range(n) if not mask[i]]
    chosen = [i for i in range(n) if mask[i]]
    ns = len(chosen)
    assert out["means"].shape[0] == len(kept) + 2 * ns
    for name in ("quats", "opacities"):
        exp = [table[name][i] for i in kept] + [table[name][i] for i in chosen] * 2
        assert np.array_equal(out[name], np.array(exp))
    exp_parent = [table["parent"][i] for i in kept] + [h + j for j in range(ns)] * 2
    exp_level = [table["level"][i] for i in kept] + [table["level"][i] + 1 for i in chosen] * 2
    assert np.array_equal(out["parent"], np.array(exp_parent, np.int32))
    assert np.array_equal(out["level"], np.array(exp_level, np.int32))
    for x in D.HISTORY:
        exp = list(table["history_" + x]) + [table[x][i] for i in chosen]
        assert np.array_equal(out["history_" + x], np.array(exp).reshape(out["history_" + x].shape))
    for name, mom in table["moments"].items():
        for key, v in mom.items():
            got = out["moments"][name][key]
            assert np.array_equal(got[:len(kept)], v[kept])
            assert not got[len(kept):].any()
    for key, v in table["state"].items():
        exp = [v[i] for i in kept] + [v[i] for i in chosen] * 2
        assert np.array_equal(out["state"][key], np.array(exp))


def test_duplicate_by_brute_force(table, mask):
    out = D.duplicate(table, mask)
    n, h = mask.size, table["history_parent"].size
    chosen = [i for i in range(n) if mask[i]]
    rank = {i: j for j, i in enumerate(chosen)}
    exp_parent = [h + rank[i] if mask[i] else table["parent"][i] for i in range(n)]
    exp_parent += [h + j for j in range(len(chosen))]
    exp_level = [table["level"][i] + (1 if mask[i] else 0) for i in range(n)]
    exp_level += [table["level"][i] + 1 for i in chosen]
    assert np.array_equal(out["parent"], np.array(exp_parent, np.int32))
    assert np.array_equal(out["level"], np.array(exp_level, np.int32))
    for name in D.PARAMS:
        exp = list(table[name]) + [table[name][i] for i in chosen]
        assert np.array_equal(out[name], np.array(exp))
        for key, v in table["moments"][name].items():
            got = out["moments"][name][key]
            assert np.array_equal(got[:n], v) and not got[n:].any()
    # The archive holds the pre-duplication parent / level of the chosen rows.
    assert np.array_equal(out["history_parent"][h:], table["parent"][chosen])
    assert np.array_equal(out["history_level"][h:], table["level"][chosen])


def test_remove_by_brute_force(table, mask):
    out = D.remove(table, mask)
    kept = [i for i in range(mask.size) if not mask[i]]
    for name in D.PARAMS + ("parent", "level"):
        assert np.array_equal(out[name], table[name][kept])
    for key, v in table["state"].items():
        assert np.array_equal(out["state"][key], v[kept])
    for x in D.HISTORY:
        assert np.array_equal(out["history_" + x], table["history_" + x])


def test_grown_tree_archive_reproduces_every_leaf_ancestry():
    """Grow a tree from one root by splits; every leaf's parent chain through
    the archive has its level as length, and each archived node sits midway
    between its two children while they are both leaves."""
    act = ACT
    raw = D.inverse_activate_scale(np.full((1, 3), 0.3, np.float32), act)
    root = {"means": np.zeros((1, 3), np.float32), "scales": raw.astype(np.float32),
            "quats": np.array([[0.9, 0.1, -0.3, 0.2]], np.float32),
            "opacities": np.zeros(1, np.float32), "parent": np.full(1, -1, np.int32),
            "level": np.zeros(1, np.int32), "moments": {}, "state": {}}
    for x in D.HISTORY:
        root["history_" + x] = np.zeros((0,) + root[x].shape[1:], root[x].dtype)
    t = root
    rng = np.random.default_rng(3)
    for _ in range(6):
        t = D.split(t, rng.uniform(size=t["parent"].size) < 0.7, act)
    hp, hl = t["history_parent"], t["history_level"]
    for i in range(t["parent"].size):
        depth, p = 0, int(t["parent"][i])
        while p >= 0:
            assert hl[p] == t["level"][i] - depth - 1
            depth, p = depth + 1, int(hp[p])
        assert depth == t["level"][i]
    # Sibling leaves: the same parent index, present twice.
    par, counts = np.unique(t["parent"], return_counts=True)
    for p in par[(counts == 2) & (par >= 0)]:
        a, b = np.nonzero(t["parent"] == p)[0]
        np.testing.assert_allclose((t["means"][a] + t["means"][b]) / 2, t["history_means"][p],
                                   atol=2e-6)
