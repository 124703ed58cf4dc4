"""Benchmark of the r2splat HIP backend on one MI355X.

Headline (``value``): projection forward + backward calls per second at the
BASELINE config-4 shape -- 500,000 Gaussians grown as a binary tree from one
root, 512x512 cone-beam detector, one view per call (call i projects view
(18 i) mod 360 degrees, so 20 consecutive calls cover the orbit once),
upstream image gradient N(0,1).  One call = prepare_explicit_gaussians ->
explicit_rasterize -> explicit_backward, the reference's training path.

Also reported: the voxelizer at config 3 (200k Gaussians, 256^3, fwd + bwd,
Mvox/s and % of HBM peak), the training-step shape of config 4 (projection +
128^3 voxelization fwd/bwd + compaction every 100 steps), the fused
densify / prune rewrite of the config-4 model table, the config-5 stress
shapes (the 512^3 volume with 5 % needles in z-slabs), per-kernel event
timings over the orbit views, the rooflines of the dominant raster and voxel
kernels, the CPU baseline (the reference's dense torch formulation of
config 1 on the host's threads) and the CPU oracle on the headline workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                       [--no-voxel] [--no-train] [--no-densify] [--no-losses]
                       [--no-stress] [--kernel-reps R] [--copy-bytes B]
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "bt-3dgs_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402
import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, AMD public spec
# MI355X fp32 vector peak, 157.3 TFLOP/s (AMD public spec), expressed as
# wave64 FMA instructions: 157.3e12 / (2 flop x 64 lanes) = 1228.9 G/s.
VALU_PEAK_TFLOPS = 157.3
VALU_PEAK_G_WAVE_INSTR = VALU_PEAK_TFLOPS * 1e3 / 128
SMIN, SMAX = 5e-4, 1.0
EPS = 1e-8
DET = 512
N_PROJ = 500_000
N_VOX, VOX_DIM = 200_000, 256


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# The headline's call i projects view (18 i) mod 360 degrees: any 20
# consecutive calls cover the orbit once, 18 degrees apart.
ORBIT_STRIDE = 18
ORBIT_VIEWS = 360 // ORBIT_STRIDE


def orbit_view(i):
    return (i * ORBIT_STRIDE) % 360


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


class Projection:
    """Config-4 projection workload resident on the device."""

    def __init__(self, dev, n=N_PROJ, det=DET, seed=0, stress=False):
        from r2splat import geometry, scenes

        g = torch.Generator().manual_seed(seed)
        if stress:  # config 5: log-scales N(-5, 1), 5 % needles
            raw = scenes.stress_gaussians(n, g)
        else:
            raw = scenes.binary_tree_gaussians(n, g, opacity="uniform")
        self.raw = raw
        self.params = [torch.nn.Parameter(t.clone().to(dev)) for t in
                       (raw.means, raw.quats, raw.raw_scales, raw.raw_opacities)]
        angles = [math.radians(k) for k in range(360)]
        vm, Ks = geometry.cone_beam_views(angles, det)
        self.viewmats = vm.to(dev)
        self.Ks = Ks.to(dev)
        self.v_images = torch.randn(4, 1, det, det, generator=g).to(dev)
        self.det = det
        self.step_i = 0

    def step(self):
        from r2splat.ops import explicit

        means, quats, scales, opac = self.params
        for p in self.params:
            p.grad = None
        i = self.step_i
        k = orbit_view(i)
        self.step_i += 1
        state = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN,
                                                    scale_max=SMAX)
        res = explicit.explicit_rasterize(state, means, self.viewmats[k:k + 1],
                                          self.Ks[k:k + 1], img_w=self.det, img_h=self.det,
                                          tile_size=16, eps2d=EPS, radius_clip=3.0, absgrad=True)
        res.image.grad = self.v_images[i % 4]
        explicit.explicit_backward(state, means, quats, scales, opac)
        return state


# configs/optim/binary_tree.yaml initial learning rates.
LRS = {"means": 6.0e-4, "scales": 4.0e-3, "quats": 3.0e-4, "opacities": 1.0e-2}


class BenchTreeModel:
    """The attributes of the reference's BinaryTreeGaussianModel that the
    training step touches: the four parameters (cloned from the config-4
    tree), parent / level, the archive of the N - 1 split ancestors and the
    bounded-sigmoid scale activation."""

    def __init__(self, proj: Projection):
        dev = proj.viewmats.device
        means, quats, scales, opac = (t.detach().clone() for t in proj.params)
        self.means = torch.nn.Parameter(means)
        self.quats = torch.nn.Parameter(quats)
        self.scales = torch.nn.Parameter(scales)
        self.opacities = torch.nn.Parameter(opac)
        n = means.shape[0]
        h = n - 1
        # A stand-in archive of N - 1 ancestors: leaf i's parent is entry
        # min(i, h - 1), holding that leaf's own parameters.
        self.parent = torch.clamp(torch.arange(n, device=dev), max=h - 1).to(torch.int32)
        self.level = torch.full((n,), 19, dtype=torch.int32, device=dev)
        self.history_means = means[:h].clone()
        self.history_scales = scales[:h].clone()
        self.history_quats = quats[:h].clone()
        self.history_opacities = opac[:h].clone()
        self.history_parent = torch.clamp(torch.arange(h, device=dev) // 2 - 1, min=-1).to(
            torch.int32)
        self.history_level = torch.full((h,), 18, dtype=torch.int32, device=dev)
        self._use_sigmoid_scale = True
        self._scale_min = torch.tensor(SMIN)
        self._scale_max = torch.tensor(SMAX)
        self._scale_eps = 1e-5
        self.trainable_param_keys = ["means", "scales", "quats", "opacities"]

    def param_dict(self):
        return {k: getattr(self, k) for k in self.trainable_param_keys}

    @staticmethod
    def activate_scale(raw):
        return SMIN + (SMAX - SMIN) * torch.sigmoid(raw)


class TrainStep:
    """Config-4 training step: projection of one view and a 128^3
    voxelization over [-1, 1]^3 sharing the prepared state; the trainer's
    loss (configs/trainer/binary_tree.yaml weights: L1 1.0, SSIM 0.25 with an
    11x11 window, TV 0.05, edge 1.0, hierarchy 0.05) against a synthetic
    target and edge mask and its backward into v_image / v_volume / means;
    the explicit backward; the
    Adam step of the four parameter groups (configs/optim/binary_tree.yaml
    learning rates); and, every 100th step, a 1 % split and a 1 % prune of the
    whole model table (parameters, Adam moments, tree buffers, statistics,
    archive).  The model is a copy: the headline workload is not changed."""

    def __init__(self, proj: Projection, dim=128, seed=2):
        from r2splat import optim
        from r2splat.ops import loss

        g = torch.Generator().manual_seed(seed)
        dev = proj.viewmats.device
        self.proj = proj
        self.model = BenchTreeModel(proj)
        self.opts = {k: optim.Adam([{"params": p, "name": k}], lr=LRS[k], eps=1e-15)
                     for k, p in self.model.param_dict().items()}
        n = self.model.means.shape[0]
        self.state = {"grad2d": torch.zeros(n, device=dev), "count": torch.zeros(n, device=dev),
                      "radii": torch.zeros(n, device=dev), "scene_scale": 1.0}
        self.dim = dim
        self.ranges = torch.full((3,), 2.0, device=dev)
        self.centers = torch.zeros(3, device=dev)
        det = proj.det
        self.targets = torch.rand(1, det, det, 1, generator=g).to(dev)
        self.edge_mask = (torch.rand(1, det, det, 1, generator=g) < 0.1).float().to(dev)
        self.loss = loss.BinaryTreeLossComputer(w_l1=1.0, w_ssim=0.25, w_tv=0.05, w_edge=1.0,
                                                w_hierarchy=0.05, ssim_window=11)
        self.mask_gen = torch.Generator(device=dev).manual_seed(seed)
        self.step_i = 0
        self.refines = 0

    def step(self):
        from r2splat import optim
        from r2splat.ops import densify, explicit, loss

        p, m = self.proj, self.model
        k = self.step_i % 360
        state = explicit.prepare_explicit_gaussians(m.quats, m.scales, m.opacities,
                                                    scale_min=SMIN, scale_max=SMAX)
        res = explicit.explicit_rasterize(state, m.means, p.viewmats[k:k + 1], p.Ks[k:k + 1],
                                          img_w=p.det, img_h=p.det, tile_size=16, eps2d=EPS,
                                          radius_clip=3.0, absgrad=True)
        vox = explicit.explicit_voxelize(state, m.means, self.ranges, self.centers,
                                         dim2=self.dim, dim1=self.dim, dim0=self.dim,
                                         tile_size=8, eps3d=EPS, radius_clip=3.0)
        hier = loss.compute_hierarchy_loss(m.means, m.parent, m.history_means, m.history_scales,
                                           m.history_quats, m.activate_scale, 1.0)
        out = self.loss(res.image.unsqueeze(-1), self.targets, self.edge_mask, vox.volume,
                        hierarchy_loss=hier)
        out["total"].backward()
        explicit.explicit_backward(state, m.means, m.quats, m.scales, m.opacities)
        optim.step_all(self.opts)
        for t in m.param_dict().values():
            t.grad = None
        if self.step_i % 100 == 99:
            keys = m.trainable_param_keys
            n = m.means.shape[0]
            grow = torch.rand(n, device=m.means.device, generator=self.mask_gen) < 0.01
            densify.split(m, self.opts, self.state, grow, keys)
            n = m.means.shape[0]
            prune = torch.rand(n, device=m.means.device, generator=self.mask_gen) < 0.01
            densify.remove(m, self.opts, self.state, prune, keys)
            self.refines += 1
        self.step_i += 1
        return state


class Voxelization:
    """Config-3 voxelization workload: the voxel branch at the op boundary."""

    def __init__(self, dev, n=N_VOX, dim=VOX_DIM, seed=1, needle_fraction=None):
        from r2splat import scenes
        from r2splat.cuda import _wrapper as W

        g = torch.Generator().manual_seed(seed)
        if needle_fraction is None:
            raw = scenes.random_gaussians(n, g, -4.5, 0.6)
        else:  # config 5 scales with a given share of needles
            raw = scenes.stress_gaussians(n, g, needle_fraction=needle_fraction)
        means = raw.means.to(dev)
        covars, max_scales, opac = W.prepare_gaussians(raw.quats.to(dev), raw.raw_scales.to(dev),
                                                       raw.raw_opacities.to(dev), SMIN, SMAX)
        self.means, self.covars, self.max_scales, self.opac = means, covars, max_scales, opac
        self.ranges = torch.full((3,), 2.0, device=dev)
        self.centers = torch.zeros(3, device=dev)
        self.v_volume = torch.randn(dim, dim, dim, generator=g).to(dev)
        self.dim = dim
        self.last = None

    def step(self):
        from r2splat.cuda import _wrapper as W

        d = self.dim
        nt = -(-d // 8)
        m3, con, r3 = W.world_to_volume_mapping_fwd(self.means, self.covars, self.max_scales,
                                                    self.ranges, self.centers, d, d, d, EPS, 3.0)
        _, ids, fl = W.isect_tiles_3d(m3, r3, 8, nt, nt, nt)
        off = W.isect_offset_encode_3d(ids, nt, nt, nt)
        vol = W.voxelize_to_voxels_fwd(m3, con, self.opac, off, fl, d, d, d, 8)
        vm3, vc3, vo = W.voxelize_to_voxels_bwd_per_gaussian(m3, con, self.opac, off, ids, fl,
                                                             self.v_volume, d, d, d, 8)
        W.world_to_volume_mapping_bwd(self.means, self.covars, self.ranges, self.centers, d, d, d,
                                      EPS, vm3, vc3)
        self.last = (m3, con, off, ids, fl, vol)
        return vol

    def step_ops(self):
        """The same voxelization through r2splat.ops (VolumePass: mapping, binning, the
        forward with its per-record reach masks, and the backward that reuses them)."""
        from r2splat.ops import _passes

        d = self.dim
        p = _passes.VolumePass.run(self.means, self.covars, self.max_scales, self.opac,
                                   self.ranges, self.centers, dim2=d, dim1=d, dim0=d,
                                   tile_size=8, eps3d=EPS, radius_clip=3.0)
        p.vjp(self.v_volume, self.means, self.covars)
        return p.volume


class SlabVoxelization:
    """Config-5 volume at the stated 5 % needles: 2M Gaussians whose brick
    list (7.46e9 records at 512^3) exceeds one list's int32 offsets, so
    r2splat.ops voxelizes it in z-slabs (forward) and re-bins each slab for
    the backward.  One step = VolumePass.run + vjp."""

    def __init__(self, dev, seed=5):
        from r2splat import scenes
        from r2splat.cuda import _ops
        from r2splat.cuda import _wrapper as W

        g = torch.Generator().manual_seed(seed)
        raw = scenes.stress_gaussians(2_000_000, g, needle_fraction=0.05)
        self.means = raw.means.to(dev)
        self.covars, self.max_scales, self.opac = W.prepare_gaussians(
            raw.quats.to(dev), raw.raw_scales.to(dev), raw.raw_opacities.to(dev), SMIN, SMAX)
        self.ranges = torch.full((3,), 2.0, device=dev)
        self.centers = torch.zeros(3, device=dev)
        self.v_volume = torch.randn(512, 512, 512, generator=g).to(dev)
        self.limit = _ops.SLAB_RECORDS
        self.slabs, self.records = (), 0

    def step(self):
        from r2splat.cuda import _ops
        from r2splat.ops import _passes

        p = _passes.VolumePass.run(self.means, self.covars, self.max_scales, self.opac,
                                   self.ranges, self.centers, dim2=512, dim1=512, dim0=512,
                                   tile_size=8, eps3d=EPS, radius_clip=3.0)
        p.vjp(self.v_volume, self.means, self.covars)
        if not self.records:
            self.slabs = p.slabs
            self.records = sum(_ops.layer_counts_3d(p.means3d, p.radii, 8, 64, 64, 64))
        return p


class DensifyTable:
    """Config-4 densify/prune workload: the binary-tree model table at
    N = 500k (params, Adam moments, parent / level, three strategy
    statistics) with the N - 1 archived ancestors, and 1 % masks."""

    def __init__(self, proj: Projection, seed=3):
        from r2splat.cuda import _lib as L

        dev = proj.viewmats.device
        g = torch.Generator().manual_seed(seed)
        n = N_PROJ
        means, quats, scales, opac = (t.detach() for t in proj.params)
        f32 = lambda *shape: torch.randn(*shape, generator=g).to(dev)  # noqa: E731
        i32 = lambda k: torch.randint(0, 20, (k,), generator=g, dtype=torch.int32).to(dev)  # noqa
        params = [(means, L.COL_MEANS), (scales, L.COL_RAW_SCALES), (quats, L.COL_COPY),
                  (opac, L.COL_RAW_OPACITIES)]
        moments = [f32(*t.shape) for t, _ in params for _ in range(2)]
        state = [f32(n) for _ in range(3)]
        parent, level = i32(n), i32(n)
        h = n - 1
        hist_src = [means, scales, quats, opac, parent, level]
        hist = [torch.zeros((h,) + tuple(t.shape[1:]), dtype=t.dtype, device=dev)
                for t in hist_src]
        self.history_rows = h
        self.hist_cols = [(a, L.COL_HISTORY, b) for a, b in zip(hist, hist_src)]
        self.tree = [(parent, L.COL_PARENT, None), (level, L.COL_LEVEL, None)]
        self.params = params
        self.moments = moments
        self.state = state
        self.geometry = (quats, scales, [SMIN] * 3, [SMAX] * 3, 1e-5, True)
        self.masks = [torch.rand(n, generator=g).to(dev) < 0.01 for _ in range(3)]
        self.words = sum(int(t[0].numel() // t[0].shape[0]) for t in self.tree)
        self.words += sum(int(t.numel() // t.shape[0]) for t, _ in params)
        self.words += sum(int(t.numel() // t.shape[0]) for t in moments + state)
        self.hist_words = sum(int(t.numel() // t.shape[0]) for t in hist_src)

    def columns(self, op):
        from r2splat.cuda import _lib as L

        cols = [] if op == "remove" else list(self.hist_cols)
        cols += [(t, L.COL_COPY if op == "remove" else r, None) for t, r, _ in self.tree]
        cols += [(t, r if op == "split" else L.COL_COPY, None) for t, r in self.params]
        moment_role = L.COL_COPY if op == "remove" else L.COL_ZERO_NEW
        cols += [(t, moment_role, None) for t in self.moments]
        cols += [(t, L.COL_COPY, None) for t in self.state]
        return cols

    def run(self, op):
        from r2splat.cuda import _wrapper as W

        if op == "split":
            return W.densify_split(self.masks[0], self.columns(op), self.history_rows,
                                   self.geometry)
        if op == "duplicate":
            return W.densify_duplicate(self.masks[1], self.columns(op), self.history_rows)
        return W.densify_remove(self.masks[2], self.columns(op))

    def algorithmic_bytes(self, op, n_sel):
        """Each source row read once, each destination row written once, the
        8-byte index lists read once; the archive copied and appended."""
        n, h, w, hw = N_PROJ, self.history_rows, self.words, self.hist_words
        if op == "remove":
            return 4 * w * (n + (n - n_sel)) + 8 * n
        rows_out = n + n_sel
        hist = 4 * hw * (2 * h + 2 * n_sel)
        return 4 * w * (n + rows_out) + 8 * n + hist + (n if op == "duplicate" else 0)


def torch_projection_loss(renders, targets, edge_mask, window):
    """The reference's projection terms as plain torch ops (2-D conv2d SSIM of
    metric.py:36-54, L1, masked edge L1), for timing beside the fused path."""
    import torch.nn.functional as F

    c1, c2 = 0.01 ** 2, 0.03 ** 2
    r = renders.permute(0, 3, 1, 2).contiguous()
    t = targets.permute(0, 3, 1, 2).contiguous()
    pad = window.shape[-1] // 2
    mu1, mu2 = F.conv2d(r, window, padding=pad), F.conv2d(t, window, padding=pad)
    s11 = F.conv2d(r * r, window, padding=pad) - mu1 * mu1
    s22 = F.conv2d(t * t, window, padding=pad) - mu2 * mu2
    s12 = F.conv2d(r * t, window, padding=pad) - mu1 * mu2
    ssim = (((2 * mu1 * mu2 + c1) * (2 * s12 + c2)) /
            ((mu1 * mu1 + mu2 * mu2 + c1) * (s11 + s22 + c2))).mean()
    l1 = (renders - targets).abs().mean()
    edge = (edge_mask * (renders - targets).abs()).mean()
    return l1 + 0.25 * (1 - ssim) + edge


def torch_tv(vol):
    """loss.py:10-21 as plain torch ops, for timing beside the fused path."""
    dx = (vol[1:] - vol[:-1]).abs()
    dy = (vol[:, 1:] - vol[:, :-1]).abs()
    dz = (vol[:, :, 1:] - vol[:, :, :-1]).abs()
    return (dx.sum() + dy.sum() + dz.sum()) / (dx.numel() + dy.numel() + dz.numel())


def time_losses(dev, reps, det=DET):
    """Loss forward + backward at the config-4 shapes, fused kernels beside
    the same terms as plain torch ops: the 512^2 projection loss (L1, SSIM,
    edge) and TV over 32^3 (the trainer's sampled volume) and 128^3."""
    from r2splat.ops import loss

    g = torch.Generator().manual_seed(5)
    renders = torch.rand(1, det, det, 1, generator=g).to(dev).requires_grad_(True)
    targets = torch.rand(1, det, det, 1, generator=g).to(dev)
    edge_mask = (torch.rand(1, det, det, 1, generator=g) < 0.1).float().to(dev)
    taps = torch.exp(-(torch.arange(11, dtype=torch.float32) - 5) ** 2 / 4.5)
    taps = taps / taps.sum()
    window = (taps[:, None] @ taps[None, :])[None, None].to(dev)

    def fused():
        renders.grad = None
        l1, sl, ed = loss.projection_losses(renders, targets, edge_mask, targets)
        (l1 + 0.25 * sl + ed).backward()

    def composed():
        renders.grad = None
        torch_projection_loss(renders, targets, edge_mask, window).backward()

    out = {"projection_loss_fused_ms": time_kernel(fused, reps) * 1e3,
           "projection_loss_torch_ms": time_kernel(composed, reps) * 1e3}
    for d in (32, 128):
        vol = torch.randn(d, d, d, generator=g).to(dev).requires_grad_(True)

        def tv_fused(vol=vol):
            vol.grad = None
            loss.compute_tv_loss(vol).backward()

        def tv_composed(vol=vol):
            vol.grad = None
            torch_tv(vol).backward()

        out[f"tv_{d}_fused_ms"] = time_kernel(tv_fused, reps) * 1e3
        out[f"tv_{d}_torch_ms"] = time_kernel(tv_composed, reps) * 1e3
    return out


def time_adam(proj: Projection, reps):
    """The Adam step of the four config-4 parameter groups: one fused launch
    (r2splat.optim.step_all) beside four torch.optim.Adam.step() calls."""
    from r2splat import optim

    out = {}
    g = torch.Generator().manual_seed(6)
    for name, cls in (("fused", optim.Adam), ("torch", torch.optim.Adam)):
        params = {k: torch.nn.Parameter(t.detach().clone())
                  for k, t in zip(("means", "quats", "scales", "opacities"), proj.params)}
        opts = {k: cls([{"params": p, "name": k}], lr=LRS[k], eps=1e-15)
                for k, p in params.items()}
        for p in params.values():
            p.grad = torch.randn(p.shape, generator=g).to(p.device)
        if name == "fused":
            fn = lambda: optim.step_all(opts)  # noqa: E731
        else:
            def fn():
                for o in opts.values():
                    o.step()
        out[f"adam_{name}_ms"] = time_kernel(fn, reps) * 1e3
    n_elem = sum(int(t.numel()) for t in proj.params)
    out["adam_algorithmic_bytes"] = 4 * n_elem * 7  # read p, g, m, v; write p, m, v
    out["adam_fused_hbm_frac"] = (out["adam_algorithmic_bytes"] / (out["adam_fused_ms"] * 1e-3)
                                  / (HBM_PEAK_GBS * 1e9))
    return out


def time_steps(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    # The objects built so far leave the collector's view: a full collection
    # over them (about 270k objects: torch's and the workloads') stalls the
    # host some 80 ms every ~150 training steps, which a long training
    # process avoids the same way.
    gc.collect()
    gc.freeze()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def time_kernel(fn, reps):
    """Average device time of fn() bracketed by events on the current stream."""
    fn()
    torch.cuda.synchronize()
    s, e = _events()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    e.synchronize()
    return s.elapsed_time(e) / reps * 1e-3


def kernel_breakdown(proj: Projection, reps):
    """Event timings of each projection stage at the config-4 inputs of the
    headline's 20 orbit views (each stage timed ``reps`` times per view, on
    the stream its kernels run on), averaged over the views.

    Entries other than ``binning_2d`` (count, scan, one host read, emit,
    sort passes, offsets), ``rasterize_bwd_op`` (pack and both passes) and
    the forwards (the rows kernel, then the combine of a heavy tile's
    partial tiles) are single kernel launches: r2splat.ops' pack, packed
    forward and the two backward passes over the packed payload are timed
    apart through their C entry points; ``rasterize_fwd`` is the
    reference-signature forward (four-array gathers).  Returns per-stage
    mean seconds, the per-view times of the raster kernels, and the record
    count of each view."""
    from r2splat.cuda import _backend, _ops
    from r2splat.cuda import _wrapper as W

    lib = _backend.library()
    means, quats, scales, opac = (t.detach() for t in proj.params)
    det = proj.det
    nt = -(-det // 16)
    P = _ops._ptr
    cov, ms, op = W.prepare_gaussians(quats, scales, opac, SMIN, SMAX)
    per_view = {}
    counts = []
    for v in range(ORBIT_VIEWS):
        k = orbit_view(v)
        vm, Ks = proj.viewmats[k:k + 1], proj.Ks[k:k + 1]
        m2, c2, r, con, mu, opc = W.project_gaussians_fwd(means, cov, op, vm, Ks, det, det, EPS,
                                                          3.0)
        _, ids, fl = W.isect_tiles(m2, r, 16, nt, nt)
        off = W.isect_offset_encode(ids, 1, nt, nt)
        emit_ids, isect_src = _ops.emission_order(fl, nt * nt)
        v_img = proj.v_images[v % 4]
        n = int(fl.numel())
        counts.append(n)
        rows = torch.empty(lib.r2s_rasterize_bwd_workspace_bytes(n, 0, 4), dtype=torch.uint8,
                           device=m2.device)
        outs = [torch.zeros_like(m2), torch.zeros_like(m2), torch.zeros_like(con),
                torch.zeros_like(opc), torch.zeros_like(mu)]
        payload = torch.empty(lib.r2s_rasterize_payload_bytes(N_PROJ, 4) // 4, device=m2.device)
        fwd_ws = torch.empty(max(1, lib.r2s_rasterize_workspace_bytes(nt * nt, n, 16, 4)),
                             dtype=torch.uint8, device=m2.device)
        image = torch.empty((1, det, det), device=m2.device)

        def pack():
            # r2splat.ops' pack launch: the payload, and zeros into the
            # backward's five outputs.
            stream = torch.cuda.current_stream().cuda_stream
            rc = lib.r2s_rasterize_pack_f32(P(m2), P(con), P(opc), P(mu), 1, N_PROJ, P(payload),
                                            P(outs[0]), P(outs[1]), P(outs[2]), P(outs[3]),
                                            P(outs[4]), stream)
            assert rc == 0, lib.r2s_last_error()

        pack()
        proj_out = [torch.empty_like(t) for t in (m2, c2, r, con, mu, opc)]

        def project_pack():
            # r2splat.ops' projection launch: the projection, the payload and
            # the zeros of the backward's outputs in one kernel.
            stream = torch.cuda.current_stream().cuda_stream
            rc = lib.r2s_project_pack_fwd_f32(P(means), P(cov), P(op), P(vm), P(Ks), det, det,
                                              EPS, 3.0, *[P(t) for t in proj_out], P(payload),
                                              *[P(t) for t in outs], 1, N_PROJ, stream)
            assert rc == 0, lib.r2s_last_error()

        def fwd_packed():
            stream = torch.cuda.current_stream().cuda_stream
            rc = lib.r2s_rasterize_fwd_packed_f32(P(payload), P(off), P(fl), n, 1, N_PROJ, det,
                                                  det, 16, nt, nt, P(image), P(fwd_ws),
                                                  fwd_ws.numel(), stream)
            assert rc == 0, lib.r2s_last_error()

        # The rows pass as r2splat.ops calls it: no int64 keys (each wave's
        # keys come from the tile offsets).
        def bwd_rows():
            stream = torch.cuda.current_stream().cuda_stream
            rc = lib.r2s_rasterize_bwd_rows_packed_f32(P(payload), P(off), None, P(fl),
                                                       P(isect_src), n, P(v_img), 1, N_PROJ, det,
                                                       det, 16, nt, nt, 1, P(rows), rows.numel(),
                                                       stream)
            assert rc == 0, lib.r2s_last_error()

        def bwd_reduce():
            stream = torch.cuda.current_stream().cuda_stream
            rc = lib.r2s_rasterize_bwd_reduce_f32(P(rows), P(emit_ids), n, 1, N_PROJ, P(opc),
                                                  P(mu), P(outs[0]), P(outs[1]), P(outs[2]),
                                                  P(outs[3]), P(outs[4]), stream)
            assert rc == 0, lib.r2s_last_error()

        stages = {
            "prepare": lambda: W.prepare_gaussians(quats, scales, opac, SMIN, SMAX),
            "project_fwd": lambda: W.project_gaussians_fwd(means, cov, op, vm, Ks, det, det,
                                                           EPS, 3.0),
            "project_pack_fwd": project_pack,
            "binning_2d": lambda: W.isect_tiles(m2, r, 16, nt, nt),
            "rasterize_fwd": lambda: W.rasterize_to_pixels_fwd(m2, con, opc, mu, off, fl, det,
                                                               det, 16),
            "rasterize_pack": pack,
            "rasterize_fwd_packed": fwd_packed,
            "rasterize_bwd_rows": bwd_rows,
            "rasterize_bwd_reduce": bwd_reduce,
            "rasterize_bwd_op": lambda: W.rasterize_to_pixels_bwd_per_gaussian(
                m2, con, opc, mu, off, ids, fl, v_img, det, det, 16, True),
        }
        for name, fn in stages.items():
            per_view.setdefault(name, []).append(time_kernel(fn, reps))
        del rows, outs, payload, fwd_ws, image, proj_out
    mean = {k: sum(v) / len(v) for k, v in per_view.items()}
    return {"n_isects_2d": counts[0], "n_isects_per_view": counts, "seconds": mean,
            "per_view_seconds": {k: per_view[k] for k in ("rasterize_fwd", "rasterize_fwd_packed",
                                                          "rasterize_bwd_rows")}}


def voxel_breakdown(vox, reps):
    """Event timings of the voxelizer's kernels at the config-3 inputs,
    through their C entry points on the current stream: the forward
    (voxel_fwd_reach_kernel), the backward's rows pass (voxel_bwd_chunk_kernel)
    and its per-Gaussian reduce (row_reduce_kernel<10>)."""
    from r2splat.cuda import _backend, _ops

    lib = _backend.library()
    P = _ops._ptr
    m3, con, off, ids, fl, _ = vox.last
    d = vox.dim
    nb = -(-d // 8)
    n, N = int(fl.numel()), int(m3.shape[0])
    emit_ids, isect_src = _ops.emission_order(fl, nb ** 3)
    volume = torch.empty((d, d, d), device=m3.device)
    rows = torch.empty(lib.r2s_voxelize_bwd_workspace_bytes(n, 4), dtype=torch.uint8,
                       device=m3.device)
    outs = [torch.zeros_like(m3), torch.zeros_like(con), torch.zeros_like(vox.opac)]

    def stream():
        return torch.cuda.current_stream().cuda_stream

    def fwd():
        rc = lib.r2s_voxelize_fwd_f32(P(m3), P(con), P(vox.opac), P(off), P(fl), n, N, d, d, d,
                                      8, nb, nb, nb, P(volume), stream())
        assert rc == 0, lib.r2s_last_error()

    # The rows passes without int64 keys, as r2splat.ops calls them.
    def bwd_rows():
        rc = lib.r2s_voxelize_bwd_rows_f32(P(m3), P(con), P(vox.opac), P(off), None, P(fl),
                                           P(isect_src), n, P(vox.v_volume), N, d, d, d, 8, nb,
                                           nb, nb, P(rows), rows.numel(), stream())
        assert rc == 0, lib.r2s_last_error()

    def bwd_reduce():
        rc = lib.r2s_voxelize_bwd_reduce_f32(P(rows), P(emit_ids), n, N, P(outs[0]), P(outs[1]),
                                             P(outs[2]), stream())
        assert rc == 0, lib.r2s_last_error()

    reach = torch.empty(n, dtype=torch.int64, device=m3.device)

    def fwd_reach():
        rc = lib.r2s_voxelize_fwd_reach_f32(P(m3), P(con), P(vox.opac), P(off), P(fl), n, N, d,
                                            d, d, 8, nb, nb, nb, P(volume), P(reach), stream())
        assert rc == 0, lib.r2s_last_error()

    def bwd_rows_reach():
        rc = lib.r2s_voxelize_bwd_rows_reach_f32(P(m3), P(con), P(vox.opac), P(off), None,
                                                 P(fl), P(isect_src), n, P(vox.v_volume), N, d,
                                                 d, d, 8, nb, nb, nb, P(reach), P(rows),
                                                 rows.numel(), stream())
        assert rc == 0, lib.r2s_last_error()

    t = {"voxelize_fwd": time_kernel(fwd, reps), "voxelize_bwd_rows": time_kernel(bwd_rows, reps),
         "voxelize_bwd_reduce": time_kernel(bwd_reduce, reps)}
    # The r2splat.ops pair: the forward also stores the reach masks, the rows
    # pass takes them (the masks of the timed forward's last call).
    given = {"voxelize_fwd_reach": time_kernel(fwd_reach, reps),
             "voxelize_bwd_rows_given_reach": time_kernel(bwd_rows_reach, reps)}
    return {"n_isects_3d": n, "seconds": t, "given_reach_seconds": given}


# The reference's arithmetic per evaluated (pixel / voxel, record) pair, in
# flops (each add, subtract, multiply and negation; exp and compares not
# counted), from its loops: the forward evaluates sigma and alpha and adds
# alpha (RasterizeToPixelsFwd.cu:154-177, VoxelizeToVoxelsFwd.cu:186-214);
# the per-Gaussian backward evaluates sigma and alpha again (16 / 26) and,
# for a pixel that passes the alpha test, forms its gradient terms and adds
# them to the record's sums (35 in 2D: v_sigma, both mean components, their
# absolute values, three conic and the opacity and mu terms,
# RasterizeToPixelsBwd.cu:419-451; 51 in 3D: v_sigma, o e^-sigma, the
# opacity, six conic and three mean terms, VoxelizeToVoxelsBwd.cu:393-418).
# Charging every evaluation with the gradient terms makes the backward
# figures an upper bound of the reference's flops.
FLOPS_PER_EVALUATION = {"rasterize_fwd": 15, "rasterize_bwd_rows": 16 + 35,
                        "voxelize_fwd": 24, "voxelize_bwd_rows": 26 + 51}


def kernel_roofline(kernel, seconds, algorithmic_bytes, evaluations=None):
    """Roofline object of one kernel: its algorithmic bytes per launch over
    its average launch ``seconds`` (live) against MI355X's 8 TB/s HBM peak
    (``bound`` "hbm"), with the HBM bytes per launch its committed rocprofv3
    --pmc summary measured (``traffic``).  The raster and voxel kernels are
    limited by vector-ALU issue, not by HBM: ``valu`` gives that limit two
    ways, from the committed VALU counters (wave64 instructions issued per
    launch x 64 lanes x 2 flops, the fp32 FMA-equivalent issue rate) and
    from the reference's own arithmetic (FLOPS_PER_EVALUATION x the
    reference's evaluations per launch), both against MI355X's 157.3
    TFLOP/s fp32 vector peak."""
    gbs = algorithmic_bytes / seconds / 1e9
    traffic = measured_traffic(kernel)
    out = {"kernel": kernel, "bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS,
           "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS, "traffic": traffic,
           "algorithmic_bytes": int(algorithmic_bytes), "avg_launch_ms": seconds * 1e3,
           "source": f"profiles/pmc_{kernel}.txt"}
    valu, trans = measured_valu(kernel)
    fpe = FLOPS_PER_EVALUATION.get(kernel)
    if valu is None and fpe is None:
        return out
    v = {"limit": "fp32 vector ALU issue", "peak_tflops": VALU_PEAK_TFLOPS,
         "reference_evaluations": evaluations}
    if fpe is not None and evaluations is not None:
        flops = fpe * evaluations
        v.update({"reference_flops_per_evaluation": fpe,
                  "algorithmic_flops_per_launch": flops,
                  "algorithmic_tflops": flops / seconds / 1e12,
                  "algorithmic_flop_frac": flops / seconds / 1e12 / VALU_PEAK_TFLOPS})
    if valu is not None:
        rate = valu / seconds / 1e9
        v.update({"executed_evaluations": None if trans is None else trans * 64,
                  "wave_instructions_per_launch": valu,
                  "achieved_g_wave_instructions_per_s": rate,
                  "peak_g_wave_instructions_per_s": VALU_PEAK_G_WAVE_INSTR,
                  "issue_tflops": rate * 128 / 1e3,
                  "issue_frac": rate * 128 / 1e3 / VALU_PEAK_TFLOPS,
                  "source": f"profiles/pmc_valu_{kernel}.txt"})
    out["valu"] = v
    return out


def op_table(proj: Projection, vox, reps):
    """Every reference operator (r2splat/cuda/_wrapper.py:18-39) and the fused
    passes, timed at the config-4 (2D) and config-3 (3D) inputs with HIP
    events, with algorithmic bytes (inputs read once, outputs written once;
    per tile record: 12 B list + 28 B payload (2D) / 40 B (3D) + partials) and
    the resulting fraction of HBM peak.  The raster / voxel ops are
    VALU-bound, so their HBM fraction is low by construction."""
    from r2splat.cuda import _wrapper as W

    means, quats, scales, opac = (t.detach() for t in proj.params)
    vm, Ks, det = proj.viewmats[:1], proj.Ks[:1], proj.det
    N = means.shape[0]
    cov, ms, op = W.prepare_gaussians(quats, scales, opac, SMIN, SMAX)
    m2, c2, r2 = W.world_to_image_projection_fwd(means, cov, vm, Ks, det, det, EPS, 3.0)
    con, mu = W.conics_mu_fwd(c2, EPS)
    opc = op[None].contiguous()
    nt = -(-det // 16)
    _, ids, fl = W.isect_tiles(m2, r2, 16, nt, nt)
    off = W.isect_offset_encode(ids, 1, nt, nt)
    i2, P = int(fl.numel()), det * det
    v_img = proj.v_images[0]
    g = torch.Generator().manual_seed(7)
    rnd = lambda t: torch.randn(t.shape, generator=g).to(t.device)  # noqa: E731
    v_m2, v_c2, v_cov, v_con, v_mu = rnd(m2), rnd(c2), rnd(cov), rnd(con), rnd(mu)
    ops = {
        "parameter_transform_fwd": (lambda: W.parameter_transform_fwd(quats, scales, SMIN, SMAX),
                                    56 * N),
        "parameter_transform_bwd": (lambda: W.parameter_transform_bwd(quats, scales, SMIN, SMAX,
                                                                      v_cov), 80 * N),
        "prepare_gaussians": (lambda: W.prepare_gaussians(quats, scales, opac, SMIN, SMAX),
                              64 * N),
        "world_to_image_projection_fwd": (lambda: W.world_to_image_projection_fwd(
            means, cov, vm, Ks, det, det, EPS, 3.0), 76 * N),
        "world_to_image_projection_bwd": (lambda: W.world_to_image_projection_bwd(
            means, cov, vm, Ks, det, det, v_m2, v_c2), 104 * N),
        "conics_mu_fwd": (lambda: W.conics_mu_fwd(c2, EPS), 40 * N),
        "conics_mu_bwd": (lambda: W.conics_mu_bwd(c2, EPS, con, mu, v_con, v_mu), 80 * N),
        "project_gaussians_fwd": (lambda: W.project_gaussians_fwd(means, cov, op, vm, Ks, det,
                                                                  det, EPS, 3.0), 100 * N),
        "isect_tiles": (lambda: W.isect_tiles(m2, r2, 16, nt, nt), 16 * N + 12 * i2),
        "isect_offset_encode": (lambda: W.isect_offset_encode(ids, 1, nt, nt), 4 * nt * nt),
        "rasterize_to_pixels_fwd": (lambda: W.rasterize_to_pixels_fwd(
            m2, con, opc, mu, off, fl, det, det, 16), 32 * i2 + 4 * P),
        "rasterize_to_pixels_bwd_per_gaussian": (lambda: W.rasterize_to_pixels_bwd_per_gaussian(
            m2, con, opc, mu, off, ids, fl, v_img, det, det, 16, True), 76 * i2 + 4 * P + 36 * N),
        "rasterize_to_pixels_bwd (pixel mode)": (lambda: W.rasterize_to_pixels_bwd(
            m2, con, opc, mu, off, fl, v_img, det, det, 16, True), 76 * i2 + 4 * P + 36 * N),
    }
    if vox is not None:
        d = vox.dim
        nb3 = -(-d // 8)
        m3, con3, off3, ids3, fl3, _ = vox.last
        i3, V, N3 = int(fl3.numel()), d ** 3, vox.means.shape[0]
        r3 = W.world_to_volume_mapping_fwd(vox.means, vox.covars, vox.max_scales, vox.ranges,
                                           vox.centers, d, d, d, EPS, 3.0)[2]
        v_m3, v_c3 = rnd(m3), rnd(con3)
        ops.update({
            "world_to_volume_mapping_fwd": (lambda: W.world_to_volume_mapping_fwd(
                vox.means, vox.covars, vox.max_scales, vox.ranges, vox.centers, d, d, d, EPS, 3.0),
                84 * N3),
            "world_to_volume_mapping_bwd": (lambda: W.world_to_volume_mapping_bwd(
                vox.means, vox.covars, vox.ranges, vox.centers, d, d, d, EPS, v_m3, v_c3),
                108 * N3),
            "isect_tiles_3d": (lambda: W.isect_tiles_3d(m3, r3, 8, nb3, nb3, nb3),
                               24 * N3 + 12 * i3),
            "isect_offset_encode_3d": (lambda: W.isect_offset_encode_3d(ids3, nb3, nb3, nb3),
                                       4 * nb3 ** 3),
            "voxelize_to_voxels_fwd": (lambda: W.voxelize_to_voxels_fwd(
                m3, con3, vox.opac, off3, fl3, d, d, d, 8), 52 * i3 + 4 * V),
            "voxelize_to_voxels_bwd_per_gaussian": (lambda: W.voxelize_to_voxels_bwd_per_gaussian(
                m3, con3, vox.opac, off3, ids3, fl3, vox.v_volume, d, d, d, 8),
                92 * i3 + 4 * V + 40 * N3),
            "voxelize_to_voxels_bwd (pixel mode)": (lambda: W.voxelize_to_voxels_bwd(
                m3, con3, vox.opac, off3, fl3, vox.v_volume, d, d, d, 8),
                92 * i3 + 4 * V + 40 * N3),
        })
    table = {}
    for name, (fn, nbytes) in ops.items():
        sec = time_kernel(fn, reps)
        table[name] = {"ms": sec * 1e3, "algorithmic_bytes": int(nbytes),
                       "hbm_frac": nbytes / sec / (HBM_PEAK_GBS * 1e9)}
    return table


def measured_traffic(kernel: str):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 --pmc
    summary (profiles/pmc_<kernel>.txt, line ``hbm_bytes_per_launch: N``), or
    None when no such measurement is committed."""
    path = os.path.join(ROOT, "profiles", f"pmc_{kernel}.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def measured_valu(kernel: str):
    """VALU and transcendental wave64 instructions per launch of ``kernel``
    from the committed rocprofv3 --pmc summary (profiles/pmc_valu_<kernel>.txt,
    lines ``valu_wave_instructions_per_launch: N`` and
    ``trans_wave_instructions_per_launch: N``), or (None, None)."""
    path = os.path.join(ROOT, "profiles", f"pmc_valu_{kernel}.txt")
    vals = {}
    try:
        with open(path) as f:
            for line in f:
                key, _, v = line.partition(":")
                if key in ("valu_wave_instructions_per_launch",
                           "trans_wave_instructions_per_launch"):
                    vals[key] = float(v)
    except OSError:
        pass
    return (vals.get("valu_wave_instructions_per_launch"),
            vals.get("trans_wave_instructions_per_launch"))


def proj_bytes(n, i2, p):
    """Algorithmic bytes of one projection fwd+bwd call (B_proj)."""
    return 164 * n + 128 * i2 + 8 * p


def vox_bytes(n, i3, v):
    """Algorithmic bytes of one voxelization fwd+bwd call (B_vox)."""
    return 144 * n + 156 * i3 + 8 * v


def _config1_inputs():
    """BASELINE config 1 (seed 0): 4,096 Gaussians (means U[-1,1]^3,
    log-scales N(-4, 0.5), unit quaternions, densities U[0,1]), one
    cone-beam view at an angle U[0, 2 pi) from the same generator, a 64^2
    detector, a 64^3 volume over [-1,1]^3, N(0,1) upstream gradients."""
    from r2splat import geometry, scenes

    g = torch.Generator().manual_seed(0)
    raw = scenes.random_gaussians(4096, g, -4.0, 0.5)
    angle = float(torch.rand(1, generator=g)) * 2.0 * math.pi
    vm, Ks = geometry.cone_beam_views([angle], 64)
    v_image = torch.randn(1, 64, 64, generator=g)
    v_volume = torch.randn(64, 64, 64, generator=g)
    return raw, vm, Ks, v_image, v_volume


def config1_gpu(dev, steps, warmup):
    """The whole config-1 call on the GPU (prepare, projection, binning,
    rasterize, voxelize, explicit backward): (seconds per call, image, volume)."""
    from r2splat.ops import explicit

    raw, vm, Ks, v_image, v_volume = _config1_inputs()
    params = [t.clone().to(dev).requires_grad_(True) for t in
              (raw.means, raw.quats, raw.raw_scales, raw.raw_opacities)]
    vm, Ks, vi, vv = vm.to(dev), Ks.to(dev), v_image.to(dev), v_volume.to(dev)
    ranges = torch.full((3,), 2.0, device=dev)
    centers = torch.zeros(3, device=dev)

    def call():
        means, quats, scales, opac = params
        for p in params:
            p.grad = None
        st = explicit.prepare_explicit_gaussians(quats, scales, opac, scale_min=SMIN,
                                                 scale_max=SMAX)
        res = explicit.explicit_rasterize(st, means, vm, Ks, img_w=64, img_h=64, tile_size=16,
                                          eps2d=EPS, radius_clip=3.0, absgrad=True)
        vox = explicit.explicit_voxelize(st, means, ranges, centers, dim2=64, dim1=64, dim0=64,
                                         tile_size=8, eps3d=EPS, radius_clip=3.0)
        res.image.grad = vi
        vox.volume.grad = vv
        explicit.explicit_backward(st, means, quats, scales, opac)
        return res, vox

    t = time_steps(call, steps, warmup)
    res, vox = call()
    torch.cuda.synchronize()
    grads = [p.grad.detach().cpu() for p in params]
    return t, res.image.detach()[0].cpu(), vox.volume.detach().cpu(), grads


def cpu_threads():
    """Host threads for the CPU baseline: the process's CPU share (the
    OMP_NUM_THREADS the box sets, else the CPUs this process may run on)."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


def config1_cpu(runs=5):
    """The reference's dense PyTorch formulation of config 1 on the host
    (oracle/dense.py: preprocessing from the raw parameters, the dense
    alpha sums masked by the tile / brick cover, torch autograd for the
    backward, the voxel sums in chunks of 256 Gaussians), on all of the
    process's host threads: the median of ``runs`` calls after one warm-up.
    Returns (median seconds, every time, image, volume, grads)."""
    from oracle import dense

    raw, vm, Ks, v_image, v_volume = _config1_inputs()
    torch.set_num_threads(cpu_threads())
    times = []
    for i in range(runs + 1):
        params = [t.clone().requires_grad_(True) for t in
                  (raw.means, raw.quats, raw.raw_scales, raw.raw_opacities)]
        t0 = time.perf_counter()
        image, volume = dense.config1_call(params, vm[0], Ks[0], 64, 64, v_image[0],
                                           (64, 64, 64), v_volume, scale_min=SMIN,
                                           scale_max=SMAX, eps=EPS)
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
        log(f"config1 dense torch call {i}{' (warm-up)' if i == 0 else ''}: {dt:.2f} s")
    grads = [p.grad.detach() for p in params]
    return sorted(times)[len(times) // 2], times, image, volume, grads


def config1(dev, steps, warmup, runs=5):
    """Config 1 like for like: the GPU path and the dense CPU formulation,
    their times and how far their images, volumes and gradients differ."""
    t_gpu, img_g, vol_g, grads_g = config1_gpu(dev, steps, warmup)
    t_cpu, times, img_c, vol_c, grads_c = config1_cpu(runs)
    rel = lambda a, b: float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))  # noqa: E731
    return {"workload": "config1: 4096 Gaussians, one view on 64^2 + 64^3 voxelization, "
                        "fwd+bwd from the raw parameters",
            "gpu_ms_per_call": t_gpu * 1e3,
            "cpu_dense_torch_ms_per_call": t_cpu * 1e3,
            "cpu_dense_torch_ms_runs": [round(x * 1e3, 1) for x in times],
            "cpu_threads": torch.get_num_threads(),
            "gpu_speedup": t_cpu / t_gpu,
            "image_max_abs_diff": float((img_c - img_g).abs().max()),
            "volume_max_abs_diff": float((vol_c - vol_g).abs().max()),
            "grad_max_rel_diff": {n: rel(a, b) for n, a, b in
                                  zip(("means", "quats", "raw_scales", "raw_opacities"),
                                      grads_g, grads_c)}}


def oracle_projection_baseline(proj: Projection):
    """The CPU oracle (numpy, plus the C restatement over OpenMP threads) on
    the headline's own workload: config-4 projection fwd+bwd of all 500k
    Gaussians, 512^2, view 0.  Returns (calls/s, seconds, sample text)."""
    from oracle import compose

    raw = proj.raw
    means, quats = raw.means.numpy(), raw.quats.numpy()
    scales, opac = raw.raw_scales.numpy(), raw.raw_opacities.numpy()
    vm = proj.viewmats[:1].cpu().numpy()
    Ks = proj.Ks[:1].cpu().numpy()
    v_img = proj.v_images[0].cpu().numpy()
    t0 = time.perf_counter()
    covars, _, op = compose.prepare(quats, scales, opac, SMIN, SMAX)
    fwd = compose.rasterize_forward(means, covars, op, vm, Ks, DET, DET, 16, EPS, 3.0)
    compose.explicit_backward(covars, fwd, None, means, quats, scales, opac, SMIN, SMAX, v_img)
    dt = time.perf_counter() - t0
    sample = (f"oracle projection fwd+bwd (numpy + C over {cpu_threads()} OpenMP threads) on "
              f"all {raw.n} config-4 Gaussians, 512^2, view 0, {fwd['isect_ids'].size} tile "
              "records")
    return 1.0 / dt, dt, sample


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-voxel", action="store_true")
    ap.add_argument("--no-train", action="store_true")
    ap.add_argument("--no-densify", action="store_true")
    ap.add_argument("--no-losses", action="store_true")
    ap.add_argument("--no-stress", action="store_true")
    ap.add_argument("--kernel-reps", type=int, default=10)
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="also run a plain device copy of this many bytes 3 times (the "
                         "reference kernel for calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the r2splat path has no "
              "multi-GPU mode in this build.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from r2splat.cuda import _wrapper as W

    if not W.is_cuda_extension_available():
        raise RuntimeError("libr2splat_hip.so is not built or failed to load")
    dev = torch.device("cuda:0")

    log("building config-4 projection workload (500k binary-tree Gaussians, 512^2)")
    proj = Projection(dev)
    # The per-stage breakdown runs first, so the headline's W warm-up and K
    # timed steps follow a second or so of launches over the same inputs, as
    # inside a training loop (right after the host-side scene build, the first
    # ~40 steps of a process ran up to 8 % slower than later ones).
    kb = kernel_breakdown(proj, args.kernel_reps)
    i2 = kb["n_isects_2d"]
    log(f"kernel breakdown: { {k: round(v * 1e3, 3) for k, v in kb['seconds'].items()} } ms, "
        f"I2={i2}")
    t_proj = time_steps(proj.step, args.steps, args.warmup)
    log(f"projection fwd+bwd: {t_proj * 1e3:.3f} ms/call")

    result = {
        "metric": "proj fwd+bwd/s @500k Gauss 512² det; voxelize Mvox/s @256³; % HBM peak",
        "value": 1.0 / t_proj,
        "unit": "proj fwd+bwd calls/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_proj * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded binary-tree Gaussians, densities U[0,1], cone-beam views)",
        "config": {"workload": "config4 projection fwd+bwd", "n_gaussians": N_PROJ,
                   "detector": [DET, DET], "views_per_call": 1, "tile_size": 16,
                   "dso": 1.0, "dsd": 1.5, "s_detector": 3.0, "eps2d": EPS,
                   "radius_clip": 3.0, "backward_mode": "primitive", "absgrad": True},
    }
    # Means over the orbit views the headline cycles through.
    i2_mean = sum(kb["n_isects_per_view"]) / len(kb["n_isects_per_view"])
    b_proj = proj_bytes(N_PROJ, i2_mean, DET * DET)
    result["proj"] = {"n_isects_mean": i2_mean, "n_isects_per_view": kb["n_isects_per_view"],
                      "views_deg": [orbit_view(v) for v in range(ORBIT_VIEWS)],
                      "algorithmic_bytes": b_proj,
                      "hbm_frac": b_proj / t_proj / (HBM_PEAK_GBS * 1e9),
                      "kernel_ms": {k: v * 1e3 for k, v in kb["seconds"].items()},
                      "raster_kernel_ms_per_view": {
                          k: [round(x * 1e3, 4) for x in v]
                          for k, v in kb["per_view_seconds"].items()}}

    # Dominant single kernel and its roofline (binning_2d and the backward op
    # span several launches and are not candidates).
    secs = kb["seconds"]
    single = {k: v for k, v in secs.items()
              if k not in ("binning_2d", "rasterize_bwd_op", "rasterize_fwd")}
    dom = max(single, key=single.get)
    n_pix = DET * DET
    dom_bytes = {
        # per record: list (key 8 + id 4) + payload 28 (mean 8, conic 12, opacity 4,
        # mu 4) + partials 36 (8 + 8 + 12 + 4 + 4); v_image read once
        "rasterize_bwd_rows": 76 * i2_mean + 4 * n_pix,
        # rows 32 + emission id 4 per record; o, mu in, 36 B out per Gaussian
        "rasterize_bwd_reduce": 36 * i2_mean + 44 * N_PROJ,
        "rasterize_fwd_packed": 32 * i2_mean + 4 * n_pix,   # id 4 + payload 28; image write
        "rasterize_pack": 64 * N_PROJ,   # 28 in, 36 zeros out per Gaussian
        "project_fwd": 108 * N_PROJ,
        "project_pack_fwd": 176 * N_PROJ,  # the projection's 108, payload 32, zeros 36
        "prepare": 76 * N_PROJ,
    }[dom]
    result["roofline"] = kernel_roofline(dom, secs[dom], dom_bytes, 256 * i2_mean)

    if args.copy_bytes > 0:
        src = torch.ones(args.copy_bytes // 4, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # reads and writes copy_bytes each
        torch.cuda.synchronize()
        result["copy_calibration_bytes"] = args.copy_bytes

    if not args.no_train:
        log("config-4 training step (projection, voxelization, losses, Adam, densify / 100)")
        train = TrainStep(proj)
        n_train = max(100, args.steps)
        # 100 untimed steps first, one split + prune among them: the first
        # refine of a process takes about 15 ms (first launches of its
        # kernels, no new device memory), later ones about 2 ms.
        t_train = time_steps(train.step, n_train, max(100, args.warmup))
        result["train_step"] = {
            "workload": "config4 training step: projection fwd + 128^3 voxelize fwd over "
                        "[-1,1]^3 + L1/SSIM/edge/TV/hierarchy loss fwd+bwd + explicit backward + Adam "
                        "step of the 4 parameter groups + a 1% split and 1% prune of the model "
                        "table every 100 steps; timed after 100 untimed training steps",
            "refines": train.refines, "n_gaussians_after": int(train.model.means.shape[0]),
            "steps": n_train, "warmup_steps": max(100, args.warmup),
            "ms_per_step": t_train * 1e3, "steps_per_s": 1.0 / t_train}
        log(f"training-step shape: {t_train * 1e3:.3f} ms/step")

    if not args.no_voxel:
        log("building config-3 voxelization workload (200k Gaussians, 256^3)")
        vox = Voxelization(dev)
        t_vox = time_steps(vox.step, max(3, args.steps // 2), args.warmup)
        t_vox_ops = time_steps(vox.step_ops, max(3, args.steps // 2), args.warmup)
        m3, con, off, ids, fl, vol = vox.last
        i3 = int(fl.numel())
        n_vox = VOX_DIM ** 3
        b_vox = vox_bytes(N_VOX, i3, n_vox)
        vb = voxel_breakdown(vox, args.kernel_reps)
        vsec = vb["seconds"]
        vbytes = {
            # id 4 + offsets/keys 8 + payload 40 per record; volume write
            "voxelize_fwd": 52 * i3 + 4 * n_vox,
            # list 12 + payload 40 + row 40 per record; v_volume read
            "voxelize_bwd_rows": 92 * i3 + 4 * n_vox,
            # row 40 + emission id 4 per record; 40 B per Gaussian out
            "voxelize_bwd_reduce": 44 * i3 + 40 * N_VOX,
        }
        vdom = max(vsec, key=vsec.get)
        result["voxelize"] = {
            "workload": "config3 voxelization fwd+bwd", "n_gaussians": N_VOX, "grid": VOX_DIM,
            "n_isects": i3, "ms_per_call": t_vox * 1e3,
            "mvox_per_s": n_vox / t_vox / 1e6, "algorithmic_bytes": b_vox,
            "hbm_frac": b_vox / t_vox / (HBM_PEAK_GBS * 1e9),
            "kernel_ms": {k: v * 1e3 for k, v in vsec.items()},
            "roofline": kernel_roofline(vdom, vsec[vdom], vbytes[vdom], 512 * i3),
            # The same call through r2splat.ops (VolumePass), whose backward reuses the
            # forward's reach masks; the reference-signature operators above recompute them.
            "ms_per_call_ops": t_vox_ops * 1e3, "mvox_per_s_ops": n_vox / t_vox_ops / 1e6,
            "kernel_ms_given_reach": {k: v * 1e3 for k, v in vb["given_reach_seconds"].items()},
        }
        log(f"voxelization fwd+bwd: {t_vox * 1e3:.3f} ms/call (r2splat.ops: "
            f"{t_vox_ops * 1e3:.3f} ms), I3={i3}")

    log("per-operator table (config 4 / config 3 inputs)")
    result["ops"] = op_table(proj, None if args.no_voxel else vox, args.kernel_reps)

    if not args.no_losses:
        log("losses and Adam (fused vs torch ops)")
        result["losses"] = time_losses(dev, args.kernel_reps)
        result["losses"].update(time_adam(proj, args.kernel_reps))
        log("losses: " + ", ".join(f"{k} {v:.3f}" for k, v in result["losses"].items()))

    if not args.no_densify:
        log("config-4 densify / prune table (500k rows + 500k archived, 1% masks)")
        table = DensifyTable(proj)
        dens = {"workload": "config4 densify/prune: fused rewrite of params, Adam moments, "
                            "parent/level, strategy statistics and the history archive",
                "n_rows": N_PROJ, "history_rows": table.history_rows,
                "words_per_row": table.words, "history_words_per_row": table.hist_words}
        for op in ("split", "duplicate", "remove"):
            n_sel = table.run(op)[1]
            t_op = time_kernel(lambda: table.run(op), args.kernel_reps)
            b = table.algorithmic_bytes(op, n_sel)
            dens[op] = {"n_selected": n_sel, "ms_per_call": t_op * 1e3, "algorithmic_bytes": b,
                        "hbm_frac": b / t_op / (HBM_PEAK_GBS * 1e9)}
        result["densify"] = dens
        log("densify: " + ", ".join(f"{op} {dens[op]['ms_per_call']:.3f} ms"
                                    for op in ("split", "duplicate", "remove")))

    if not args.no_stress:
        log("config-5 stress shapes (2M Gaussians: 1024^2 projection, 512^3 voxelization)")
        sp = Projection(dev, n=2_000_000, det=1024, seed=5, stress=True)
        t_sp = time_steps(sp.step, 3, 1)
        with torch.no_grad():
            from r2splat.cuda import _wrapper as W2

            cov, _, op = W2.prepare_gaussians(sp.params[1].detach(), sp.params[2].detach(),
                                              sp.params[3].detach(), SMIN, SMAX)
            m2, _, rad, _, _, _ = W2.project_gaussians_fwd(sp.params[0].detach(), cov, op,
                                                          sp.viewmats[:1], sp.Ks[:1], 1024, 1024,
                                                          EPS, 3.0)
            i2_stress = int(W2.isect_tiles(m2, rad, 16, 64, 64)[1].numel())
        sv = Voxelization(dev, n=2_000_000, dim=512, seed=5, needle_fraction=0.0005)
        t_sv = time_steps(sv.step, 3, 1)
        n_sv = int(sv.last[4].numel())
        del sv
        torch.cuda.empty_cache()
        slab = SlabVoxelization(dev)
        t_slab = time_steps(slab.step, 1, 1)
        result["stress"] = {
            "projection": {"workload": "config5 projection fwd+bwd: 2M Gaussians (log-scale "
                                       "N(-5,1), 5% needles), 1024^2, one view",
                           "n_isects_view0": i2_stress, "ms_per_call": t_sp * 1e3},
            "voxelization": {"workload": "config5 voxelization fwd+bwd at 512^3 with 0.05% "
                                         "needles, one brick list",
                             "n_isects": n_sv, "ms_per_call": t_sv * 1e3,
                             "mvox_per_s": 512 ** 3 / t_sv / 1e6},
            "voxelization_5pct_needles": {
                "workload": "config5 voxelization fwd+bwd at 512^3 with the stated 5% needles "
                            "through r2splat.ops (VolumePass): z-slabs of at most "
                            f"{slab.limit} brick records, re-binned for the backward",
                "n_isects": slab.records, "slabs": len(slab.slabs),
                "ms_per_call": t_slab * 1e3, "mvox_per_s": 512 ** 3 / t_slab / 1e6}}
        log(f"stress: projection {t_sp * 1e3:.2f} ms, voxelization {t_sv * 1e3:.2f} ms "
            f"({n_sv} records); 5% needles {t_slab * 1e3:.1f} ms ({slab.records} records in "
            f"{len(slab.slabs)} slabs)")
        del sp, slab
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        log("config 1 like for like (GPU path vs the dense torch formulation on the host)")
        c1 = config1(dev, 20, 3)
        result["config1"] = c1
        log(f"config1: GPU {c1['gpu_ms_per_call']:.3f} ms, CPU dense torch "
            f"{c1['cpu_dense_torch_ms_per_call']:.1f} ms on {c1['cpu_threads']} threads, "
            f"max |diff| image {c1['image_max_abs_diff']:.2e} volume "
            f"{c1['volume_max_abs_diff']:.2e}")
        t_cpu = c1["cpu_dense_torch_ms_per_call"] * 1e-3
        result["cpu_baseline"] = {
            "value": 1.0 / t_cpu, "unit": "config-1 fwd+bwd calls/s (64^2 view + 64^3 volume)",
            "cores": c1["cpu_threads"], "kind": "port",
            "sample": "BASELINE config 1 in full: the reference's dense PyTorch formulation "
                      "(oracle/dense.py) from the raw parameters, torch autograd backward, "
                      f"median of 5 calls after 1 warm-up on {c1['cpu_threads']} host threads",
            "projections_per_s": 1.0 / t_cpu, "mvox_per_s": 64 ** 3 / t_cpu / 1e6,
            "seconds_per_call": t_cpu,
            "gpu_same_config_calls_per_s": 1e3 / c1["gpu_ms_per_call"]}
        log("timing the CPU oracle on the headline workload")
        cps, dt, sample = oracle_projection_baseline(proj)
        result["cpu_oracle"] = {"value": cps, "unit": "proj fwd+bwd calls/s",
                                "cores": cpu_threads(),
                                "kind": "port", "sample": sample, "sample_seconds": dt}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
