"""Z-slab voxelization: volumes whose brick list exceeds r2splat.cuda._ops
SLAB_RECORDS records are binned, voxelized and back-propagated one slab of
brick layers at a time.

* Per-layer record counts equal the oracle's box cover.
* A slab's list is the segment of the whole volume's list whose bricks lie in
  its layers, keys shifted to the slab's first layer -- bit for bit.
* The slabbed forward equals the one-list forward bit for bit; the slabbed
  backward meets the parity bar against the oracle.
* Config 5's 512^3 volume with 5 % needles (7.5e9 brick records, beyond the
  int32 offsets of one list) runs through r2splat.ops; sampled bricks of two
  slabs are checked against the oracle (voxels and per-record partials).
"""

import numpy as np
import pytest
import torch

import pipeline_check
from helpers import (VOXEL_ROW_SLOTS, check_voxel, check_voxel_sampled, np32, sample_keys,
                     voxel_references)
from oracle import binning
from r2splat import scenes
from r2splat.cuda import _backend, _ops
from r2splat.cuda import _wrapper as W
from r2splat.ops import _passes

pytestmark = pytest.mark.gpu
DEV = "cuda"
SMIN, SMAX = 5e-4, 1.0

# Config 5's 5 % needles cross the middle bricks of the 512^3 volume by the
# hundred; each voxel there sums many needle terms whose float32 sigma errs
# by about u S (S up to ~1e4), beyond the bar's 1e-4 relative.  Measured:
# 2.7 % and 3.6 % of the sampled voxels of the two slabs checked need the
# conditioning term (err / (u |terms|) at most 1.2), 0.07 % of their records'
# partials.  The cap is about twice the largest.
SLAB_NEEDLE_FRAC = 0.08


def _scene(n, seed, dims, log_mu=-3.2, needle_fraction=None):
    g = torch.Generator().manual_seed(seed)
    if needle_fraction is None:
        raw = scenes.random_gaussians(n, g, log_mu, 0.5)
    else:
        raw = scenes.stress_gaussians(n, g, needle_fraction=needle_fraction)
    cov, ms, op = W.prepare_gaussians(raw.quats.to(DEV), raw.raw_scales.to(DEV),
                                      raw.raw_opacities.to(DEV), SMIN, SMAX)
    d2, d1, d0 = dims
    m3, con, r3 = W.world_to_volume_mapping_fwd(raw.means.to(DEV), cov, ms,
                                                torch.full((3,), 2.0, device=DEV),
                                                torch.zeros(3, device=DEV), d2, d1, d0, 1e-8, 3.0)
    return dict(raw=raw, cov=cov, ms=ms, op=op, m3=m3, con=con, r3=r3, g=g)


def test_slab_lists_are_segments_of_the_whole_list():
    dims = (64, 48, 72)
    s = _scene(6000, 31, dims)
    n2, n1, n0 = 8, 6, 9
    whole = _ops.bin_tiles_3d(s["m3"], s["r3"], 8, n2, n1, n0)
    ids, fl = np32(whole.isect_ids), np32(whole.flatten_ids)
    assert ids.size > 10_000
    layers = _ops.layer_counts_3d(s["m3"], s["r3"], 8, n2, n1, n0)
    lo, hi, count = binning.tile_boxes_3d(np32(s["m3"]), np32(s["r3"]), 8, n2, n1, n0)
    area = (hi[0] - lo[0]) * (hi[1] - lo[1])
    want = [int(area[(count > 0) & (lo[2] <= z) & (z < hi[2])].sum()) for z in range(n0)]
    assert layers == want and sum(layers) == ids.size
    plan = _ops.plan_slabs(layers, limit=ids.size // 3)
    assert len(plan) >= 3 and plan[0][0] == 0 and plan[-1][1] == n0
    assert all(a[1] == b[0] for a, b in zip(plan, plan[1:]))
    plane = n1 * n2
    for z0, z1 in plan:
        sl, off = _ops.bin_tiles_3d_slab(s["m3"], s["r3"], 8, n2, n1, n0, z0, z1)
        seg = (ids >= z0 * plane) & (ids < z1 * plane)
        assert np.array_equal(np32(sl.isect_ids), ids[seg] - z0 * plane)
        assert np.array_equal(np32(sl.flatten_ids), fl[seg])
        assert np.array_equal(np32(off).reshape(-1),
                              np.searchsorted(ids[seg] - z0 * plane,
                                              np.arange((z1 - z0) * plane), "left"))
        src = np32(sl.isect_src).astype(np.int64)
        assert np.array_equal(np.sort(src), np.arange(src.size))
        assert np.array_equal(np32(sl.emit_ids)[src], fl[seg])


def test_slabbed_volume_pass_matches_one_list(monkeypatch):
    dims = (48, 40, 56)
    s = _scene(5000, 32, dims)
    d2, d1, d0 = dims
    rng, ctr = torch.full((3,), 2.0, device=DEV), torch.zeros(3, device=DEV)
    means = s["raw"].means.to(DEV)
    kw = dict(dim2=d2, dim1=d1, dim0=d0, tile_size=8, eps3d=1e-8, radius_clip=3.0)
    one = _passes.VolumePass.run(means, s["cov"], s["ms"], s["op"], rng, ctr, **kw)
    assert not one.slabs
    n_rec = one.lists.isect_ids.numel()
    monkeypatch.setattr(_ops, "SLAB_RECORDS", n_rec // 4)
    sl = _passes.VolumePass.run(means, s["cov"], s["ms"], s["op"], rng, ctr, **kw)
    assert len(sl.slabs) >= 4 and sl.lists is None
    assert torch.equal(sl.volume, one.volume)  # same records, same order per voxel
    v = torch.randn(one.volume.shape, generator=s["g"])
    refs = voxel_references(np32(one.means3d), np32(one.conics), np32(one.weights),
                            np32(one.tile_offsets), np32(one.lists.flatten_ids), d2, d1, d0, 8,
                            v_volume=v.numpy())
    for name, p in (("one list", one), ("slabs", sl)):
        ops = _backend._C
        if p.slabs:
            parts = None
            n2, n1, n0 = -(-d2 // 8), -(-d1 // 8), -(-d0 // 8)
            for z0, z1 in p.slabs:
                lists, off = ops.bin_tiles_3d_slab(p.means3d, p.radii, 8, n2, n1, n0, z0, z1)
                part = ops.voxel_backward_slab(p.means3d, p.conics, p.weights, off, lists,
                                               v.to(DEV), 8, z0)
                parts = list(part) if parts is None else [a + b for a, b in zip(parts, part)]
            got = parts
        else:
            got = ops.voxel_backward(p.means3d, p.conics, p.weights, p.tile_offsets, p.lists,
                                     v.to(DEV), d2, d1, d0, 8)
        for k, r in check_voxel(refs, grads=[np32(t) for t in got], tag=f"{name} ").items():
            print(name, k, r)
    # Through the public API: the slabbed explicit step gives the same volume,
    # and every output and parameter gradient meets the bar against the
    # oracle composition (the slabs' lists concatenated equal the oracle's
    # whole list).
    from r2splat import geometry

    vm, Ks = geometry.cone_beam_views([0.3], 32)
    out = pipeline_check.run(s["raw"], vm, Ks, 32, 32, volume_shape=dims, v_volume=v)
    assert out["state"].voxel.slabs and torch.equal(out["vox"].volume.detach(), one.volume)
    reports = pipeline_check.check_against_oracle(out, s["raw"], vm, Ks, 32, 32,
                                                  volume_shape=dims)
    assert "voxel v_conics" in reports and "means (chain)" in reports


def _rows_slab(p, lists, off, v, z0):
    lib, P = _backend.library(), _ops._ptr
    n, N = lists.flatten_ids.numel(), p["m3"].shape[0]
    rows = torch.empty(lib.r2s_voxelize_bwd_workspace_bytes(n, 4), dtype=torch.uint8,
                       device=DEV)
    nz, n1, n2 = off.shape
    rc = lib.r2s_voxelize_bwd_rows_slab_f32(P(p["m3"]), P(p["con"]), P(p["op"]), P(off),
                                            P(lists.isect_ids), P(lists.flatten_ids),
                                            P(lists.isect_src), n, P(v), N, 512, 512, 512, 8, n2,
                                            n1, z0, nz, P(rows), rows.numel(),
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.r2s_last_error()
    return rows.view(torch.float32)


def test_config5_512_volume_with_needles_in_slabs():
    s = _scene(2_000_000, 5, (512, 512, 512), needle_fraction=0.05)
    nb = 64
    layers = _ops.layer_counts_3d(s["m3"], s["r3"], 8, nb, nb, nb)
    total = sum(layers)
    print(f"config 5 (5 % needles): {total} brick records", flush=True)
    assert total > 2 ** 31  # one list would overflow the int32 offsets
    plan = _ops.plan_slabs(layers)
    print(f"{len(plan)} slabs", flush=True)
    assert plan[-1][1] == nb and len(plan) > 8
    rng, ctr = torch.full((3,), 2.0, device=DEV), torch.zeros(3, device=DEV)
    kw = dict(dim2=512, dim1=512, dim0=512, tile_size=8, eps3d=1e-8, radius_clip=3.0)
    means = s["raw"].means.to(DEV)
    p = _passes.VolumePass.run(means, s["cov"], s["ms"], s["op"], rng, ctr, **kw)
    assert tuple(p.slabs) == tuple(plan)
    torch.cuda.synchronize()
    print("forward done", flush=True)
    vol = p.volume
    v = torch.randn((512, 512, 512), generator=s["g"]).to(DEV)
    # Two slabs (the most loaded and a middle one), sampled bricks.
    loads = [sum(layers[a:b]) for a, b in plan]
    picks = sorted({int(np.argmax(loads)), len(plan) // 2})
    for i in picks:
        z0, z1 = plan[i]
        lists, off = _ops.bin_tiles_3d_slab(s["m3"], s["r3"], 8, nb, nb, nb, z0, z1)
        n = lists.flatten_ids.numel()
        keys = sample_keys(np32(off), n, 12, seed=i)
        rows = _rows_slab(s, lists, off, v, z0)
        o = np32(off).reshape(-1).astype(np.int64)
        pos = np.concatenate([np.arange(o[k], o[k + 1] if k + 1 < o.size else n) for k in keys])
        src = lists.isect_src[torch.from_numpy(pos).to(DEV)].long()
        sub = rows.view(-1, VOXEL_ROW_SLOTS)[src].cpu().numpy()
        del rows
        lookup = np.full(n, -1, np.int64)
        lookup[pos] = np.arange(pos.size)
        reps = check_voxel_sampled(np32(s["m3"]), np32(s["con"]), np32(s["op"]), np32(off),
                                   np32(lists.flatten_ids), np32(v), 512, 512, 512, 8, keys,
                                   volume=np32(vol), rows=sub.reshape(-1), isect_src=lookup,
                                   tag=f"slab {z0}-{z1} ", key_offset=z0 * nb * nb,
                                   max_frac=SLAB_NEEDLE_FRAC)
        for k, r in reps.items():
            print(f"slab [{z0}, {z1})", k, r, flush=True)
        del lists, off
    g = p.vjp(v, means, s["cov"])
    again = p.vjp(v, means, s["cov"])
    for a, b in zip(g, again):
        assert bool(torch.isfinite(a).all()) and torch.equal(a, b)
