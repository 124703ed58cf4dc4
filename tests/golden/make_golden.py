"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

The fixtures are small seeded cases (inputs and the oracle's outputs) of the
projection path, the voxel path and the compaction.  tests/test_golden_oracle.py
checks that the oracle still reproduces them exactly; tests/test_gpu_golden.py
checks the HIP operators against them.  Inputs are generated here with numpy /
torch CPU generators; nothing from the reference tree is read or run.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for p in (ROOT, os.path.join(ROOT, "bt-3dgs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

SCALE_MIN, SCALE_MAX = 5e-4, 1.0
EPS = 1e-8
CLIP = 3.0


def inputs(seed: int = 7, n: int = 200):
    import torch

    from r2splat import geometry, scenes

    g = torch.Generator().manual_seed(seed)
    raw = scenes.random_gaussians(n, g, -3.4, 0.5)
    viewmats, Ks = geometry.cone_beam_views([1.1], 48)
    rng = np.random.default_rng(seed)
    return dict(
        means=raw.means.numpy(), quats=raw.quats.numpy(), raw_scales=raw.raw_scales.numpy(),
        raw_opacities=raw.raw_opacities.numpy(), viewmats=viewmats.numpy(), Ks=Ks.numpy(),
        v_image=rng.standard_normal((1, 48, 48)).astype(np.float32),
        ranges=np.full(3, 2.0, np.float32), centers=np.zeros(3, np.float32),
        v_volume=rng.standard_normal((20, 12, 16)).astype(np.float32),
        mask=rng.random(1000) < 0.35)


def projection(d):
    from oracle import compose

    covars, _, opac = compose.prepare(d["quats"], d["raw_scales"], d["raw_opacities"], SCALE_MIN,
                                      SCALE_MAX)
    proj = compose.rasterize_forward(d["means"], covars, opac, d["viewmats"], d["Ks"], 48, 48, 16,
                                     EPS, CLIP)
    grads = compose.explicit_backward(covars, proj, None, d["means"], d["quats"],
                                      d["raw_scales"], d["raw_opacities"], SCALE_MIN, SCALE_MAX,
                                      d["v_image"], None, absgrad=True)
    out = dict(covars=covars, opacities=opac, means2d=proj["means2d"], cov2d=proj["cov2d"],
               conics=proj["conics"], mus=proj["mus"], radii=proj["radii"],
               isect_ids=proj["isect_ids"], flatten_ids=proj["flatten_ids"],
               tile_offsets=proj["tile_offsets"], image=proj["output"])
    out.update({f"grad_{k}": v for k, v in grads.items()})
    return out


def voxel(d):
    from oracle import compose, native, ops

    covars, _, opac = compose.prepare(d["quats"], d["raw_scales"], d["raw_opacities"], SCALE_MIN,
                                      SCALE_MAX)
    vox = compose.voxelize_forward(d["means"], covars, opac, d["ranges"], d["centers"], 16, 12,
                                   20, 8, EPS, CLIP)
    vm3, vc3, vo3 = native.voxel_bwd(vox["means3d"], vox["conics"], vox["opacity"],
                                     vox["tile_offsets"], vox["flatten_ids"], d["v_volume"], 16,
                                     12, 20, 8)
    vm, vc = ops.world_to_volume_mapping_bwd(d["means"], covars, d["ranges"], d["centers"], 16,
                                             12, 20, EPS, vm3, vc3)
    return dict(covars=covars, opacities=opac, vox_means3d=vox["means3d"],
                vox_conics=vox["conics"], vox_radii=vox["radii"],
                vox_isect_ids=vox["isect_ids"], vox_flatten_ids=vox["flatten_ids"],
                vox_tile_offsets=vox["tile_offsets"], volume=vox["output"],
                vox_v_means3d=vm3, vox_v_conics=vc3, vox_v_opacities=vo3, vox_v_means=vm,
                vox_v_covars=vc)


def compaction(d):
    from oracle import binning

    sel, rest = binning.where_split(d["mask"])
    return dict(sel=sel, rest=rest)


def main() -> None:
    from oracle import native

    native.build()
    d = inputs()
    np.savez_compressed(os.path.join(HERE, "projection_small.npz"), **d, **projection(d))
    np.savez_compressed(os.path.join(HERE, "voxel_small.npz"), **d, **voxel(d))
    np.savez_compressed(os.path.join(HERE, "compaction.npz"), mask=d["mask"], **compaction(d))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
