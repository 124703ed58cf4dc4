"""The CPU oracle reproduces the committed golden fixtures exactly.

The fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py)
pin the oracle's outputs: any change to an oracle function that alters a
result on these seeded cases fails here, bit for bit.
"""

import os

import numpy as np
import pytest

from golden import make_golden as mg

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return dict(np.load(os.path.join(HERE, name)))


def _inputs(f):
    keys = ("means", "quats", "raw_scales", "raw_opacities", "viewmats", "Ks", "v_image",
            "ranges", "centers", "v_volume", "mask")
    return {k: f[k] for k in keys}


@pytest.mark.parametrize("name,fn", [("projection_small.npz", mg.projection),
                                     ("voxel_small.npz", mg.voxel)])
def test_oracle_reproduces_fixture(name, fn):
    f = _load(name)
    out = fn(_inputs(f))
    assert out, "no outputs"
    for k, v in out.items():
        assert v.dtype == f[k].dtype, k
        assert np.array_equal(v, f[k], equal_nan=True), f"{name}: {k} differs"


def test_compaction_fixture():
    f = _load("compaction.npz")
    sel, rest = np.nonzero(f["mask"])[0], np.nonzero(~f["mask"])[0]
    assert np.array_equal(sel, f["sel"]) and np.array_equal(rest, f["rest"])
    assert np.array_equal(mg.compaction(dict(mask=f["mask"]))["sel"], f["sel"])
