"""Training losses that feed the Gaussian backward, as fused HIP kernels.

Drop-in for the projection and volume terms of ``src/utils/loss.py`` and for
``ssim2d`` of ``src/utils/metric.py``:

* ``projection_losses`` returns the L1, 1 - SSIM and masked edge L1 terms of
  ``BinaryTreeLossComputer`` (loss.py:135-172) from one forward launch (plus
  a one-block reduction); autograd's backward is one launch that produces
  ``v_image`` directly.  The reference runs five 2-D convolutions and a few
  dozen element-wise kernels for the same values and as many again backward.
* ``compute_tv_loss`` (loss.py:10-21) is one reduction launch forward and one
  element-wise launch backward.
* ``compute_hierarchy_loss`` (loss.py:27-71) gathers each child's archived
  parent, measures it in the parent's scaled frame and stores its gradient
  in one launch; the backward scales it.
* ``LossComputer`` / ``BinaryTreeLossComputer`` keep the reference's
  constructor arguments and output dictionary (loss.py:74-172); their
  projection terms, TV term and weighted total are the outputs of one
  autograd node (``_TrainerLoss``), so the trainer's ``total.backward()``
  walks one node for them instead of one per term and sum.

Images and volumes are float32 CUDA tensors, as the trainer produces them;
gradients flow to the renders / volume only (targets, masks and edge
targets are data).
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch
from torch import Tensor

from ..cuda import _wrapper as W

__all__ = ["projection_losses", "ssim2d", "compute_tv_loss", "compute_edge_loss",
           "compute_hierarchy_loss", "LossComputer", "BinaryTreeLossComputer"]


_ZERO = {}


def _zero(device) -> Tensor:
    """A cached float32 zero scalar (never returned to callers)."""
    z = _ZERO.get(device)
    if z is None:
        z = _ZERO[device] = torch.zeros((), dtype=torch.float32, device=device)
    return z


def _grad_vector(grads, device) -> Tensor:
    """The upstream gradients of several scalar outputs as one float32 vector
    (zero for outputs that received none): one launch."""
    return torch.stack([_zero(device) if g is None else g.reshape(()).to(torch.float32)
                        for g in grads])


class _ProjectionLoss(torch.autograd.Function):
    """(l1, 1 - ssim, edge) as three outputs of one launch; the backward is
    one launch for any combination of their upstream gradients."""

    @staticmethod
    def forward(ctx, render, target, edge_target, edge_mask, window_size):
        ctx.set_materialize_grads(False)  # unused outputs' gradients stay None
        losses, ws = W.projection_loss_fwd(render, target, edge_target, edge_mask, window_size)
        ctx.save_for_backward(render, target, edge_target, edge_mask, ws)
        ctx.window_size = window_size
        return losses[0], losses[1], losses[2]

    @staticmethod
    def backward(ctx, g_l1, g_ssim, g_edge):
        if any(ctx.needs_input_grad[1:4]):
            raise NotImplementedError("gradients w.r.t. targets, edge targets or edge masks "
                                      "are not provided")
        render, target, edge_target, edge_mask, ws = ctx.saved_tensors
        scales = _grad_vector((g_l1, g_ssim, g_edge), render.device)
        g = W.projection_loss_bwd(render, target, edge_target, edge_mask, scales, ws,
                                  ctx.window_size)
        return g, None, None, None, None


_WEIGHTS = {}


class _TrainerLoss(torch.autograd.Function):
    """The loss computers' terms and weighted total as outputs of one graph
    node: forward = the projection-loss launch, the TV launch and one
    weighted sum; backward = the effective scale of each term (its own
    upstream gradient plus its weight times the total's), then one
    projection-loss launch and one TV launch.  Terms are ordered (l1, ssim,
    edge, tv, hierarchy); the hierarchy term is an input (computed by the
    caller), so its gradient is passed back."""

    @staticmethod
    def forward(ctx, weights, r, t, e, m, vol, hier, window_size, tv_mean):
        # Outputs that receive no gradient (the terms, in a trainer's
        # total.backward()) pass None instead of a zero tensor each.
        ctx.set_materialize_grads(False)
        losses, ws = W.projection_loss_fwd(r, t, e, m, window_size)
        z = _zero(r.device).reshape(1)
        tv = z if vol is None else W.tv_fwd(vol, tv_mean).reshape(1)
        terms = torch.cat((losses, tv, hier.detach().reshape(1).to(torch.float32)))
        total = torch.dot(terms, weights)
        ctx.save_for_backward(weights, r, t, e, m, ws, vol)
        ctx.window_size, ctx.tv_mean = window_size, tv_mean
        ctx.hier_dtype, ctx.hier_shape = hier.dtype, hier.shape
        return terms[0], terms[1], terms[2], terms[3], total

    @staticmethod
    def backward(ctx, g_l1, g_ssim, g_edge, g_tv, g_total):
        if any(ctx.needs_input_grad[2:5]):
            raise NotImplementedError("gradients w.r.t. targets, edge targets or edge masks "
                                      "are not provided")
        weights, r, t, e, m, ws, vol = ctx.saved_tensors
        dev = weights.device
        if g_total is None:
            g_total = _zero(dev)
        if g_l1 is None and g_ssim is None and g_edge is None and g_tv is None:
            eff = weights * g_total.to(torch.float32)
        else:
            own = _grad_vector((g_l1, g_ssim, g_edge, g_tv, None), dev)
            eff = torch.addcmul(own, weights, g_total.to(torch.float32))
        v_r = None
        if ctx.needs_input_grad[1]:
            v_r = W.projection_loss_bwd(r, t, e, m, eff[:3], ws, ctx.window_size)
        v_vol = None
        if vol is not None and ctx.needs_input_grad[5]:
            v_vol = W.tv_bwd(vol, eff[3:4], ctx.tv_mean)
        v_hier = None
        if ctx.needs_input_grad[6]:
            v_hier = eff[4].reshape(ctx.hier_shape).to(ctx.hier_dtype)
        return None, v_r, None, None, None, v_vol, v_hier, None, None


def _trainer_terms(renders, targets, edge_mask, edge_targets, volume_pred, hierarchy_loss,
                   weights, ssim_window, w_tv):
    """(l1, ssim, edge, tv, total) of the loss computers through _TrainerLoss;
    weights = (l1, ssim, edge, tv, hierarchy)."""
    if renders.shape != targets.shape:
        raise AssertionError("Input shapes must match for SSIM")
    if renders.dtype != torch.float32:
        raise TypeError(f"renders must be float32, got {renders.dtype}")
    dev = renders.device
    r = _planes(renders)
    t = _planes(_as_float(targets.detach()))
    e = m = None
    if edge_mask is not None:
        et = targets if edge_targets is None else edge_targets
        if torch.broadcast_shapes(edge_mask.shape, et.shape, renders.shape) != renders.shape:
            raise ValueError("edge_mask and edge_targets must broadcast to the renders' shape")
        e = _planes(_as_float(et.detach()).expand(renders.shape))
        m = _planes(_as_float(edge_mask.detach()).expand(renders.shape))
    vol = None
    if w_tv > 0 and volume_pred is not None:
        # loss.py:93-99 / 159-165: a volume that is not 3-D after squeezing gives 0.
        v = volume_pred.squeeze()
        if v.dim() == 4 and v.size(0) == 1:
            v = v[0]
        if v.dim() == 3 and v.is_cuda and v.dtype == torch.float32:
            vol = v.contiguous()
    if hierarchy_loss is None:
        hierarchy_loss = _zero(dev)
    elif not isinstance(hierarchy_loss, Tensor):  # a plain number
        hierarchy_loss = torch.tensor(float(hierarchy_loss), dtype=torch.float32, device=dev)
    key = (dev, weights)
    w = _WEIGHTS.get(key)
    if w is None:
        w = _WEIGHTS[key] = torch.tensor(weights, dtype=torch.float32, device=dev)
    return _TrainerLoss.apply(w, r, t, e, m, vol, hierarchy_loss, int(ssim_window), True)


def _planes(t: Tensor) -> Tensor:
    """[N, H, W, K] (the trainer's renders layout) -> [N*K, H, W] images."""
    if t.dim() != 4:
        raise ValueError(f"expected [N, H, W, C] images, got shape {tuple(t.shape)}")
    n, h, w, k = t.shape
    return t.permute(0, 3, 1, 2).reshape(n * k, h, w).contiguous()


def _as_float(t: Tensor) -> Tensor:
    return t if t.dtype == torch.float32 else t.to(torch.float32)


def projection_losses(renders: Tensor, targets: Tensor, edge_mask: Optional[Tensor] = None,
                      edge_targets: Optional[Tensor] = None,
                      ssim_window: int = 11) -> Tuple[Tensor, Tensor, Tensor]:
    """(mean |r - t|, 1 - ssim2d(r, t), mean(edge_mask |r - edge_targets|)) of
    renders / targets [N, H, W, C] (loss.py:143-158).  ``edge_targets``
    defaults to ``targets``; without an edge mask the edge term is zero."""
    if renders.shape != targets.shape:
        raise AssertionError("Input shapes must match for SSIM")
    if renders.dtype != torch.float32:
        raise TypeError(f"renders must be float32, got {renders.dtype}")
    r = _planes(renders)
    t = _planes(_as_float(targets.detach()))
    e = m = None
    if edge_mask is not None:
        et = targets if edge_targets is None else edge_targets
        if torch.broadcast_shapes(edge_mask.shape, et.shape, renders.shape) != renders.shape:
            raise ValueError("edge_mask and edge_targets must broadcast to the renders' shape")
        e = _planes(_as_float(et.detach()).expand(renders.shape))
        m = _planes(_as_float(edge_mask.detach()).expand(renders.shape))
    l1, ssim_loss, edge = _ProjectionLoss.apply(r, t, e, m, int(ssim_window))
    if edge_mask is None:
        edge = torch.zeros((), device=renders.device)
    return l1, ssim_loss, edge


def ssim2d(img1: Tensor, img2: Tensor, window_size: int = 11) -> Tensor:
    """metric.py:36-54: mean SSIM of [N, C, H, W] images (differentiable in img1)."""
    if img1.shape != img2.shape:
        raise AssertionError("Input shapes must match for SSIM")
    n, c, h, w = img1.shape
    a = img1.reshape(n * c, h, w).contiguous()
    b = _as_float(img2.detach()).reshape(n * c, h, w).contiguous()
    return 1.0 - _ProjectionLoss.apply(a, b, None, None, int(window_size))[1]


def compute_edge_loss(pred: Tensor, target: Tensor, edge_mask: Tensor) -> Tensor:
    """loss.py:23-24: (edge_mask * |pred - target|).mean()."""
    return projection_losses(pred, target, edge_mask, target)[2]


class _TV(torch.autograd.Function):
    @staticmethod
    def forward(ctx, vol, mean):
        ctx.save_for_backward(vol)
        ctx.mean = mean
        return W.tv_fwd(vol, mean)

    @staticmethod
    def backward(ctx, grad):
        (vol,) = ctx.saved_tensors
        return W.tv_bwd(vol, grad.to(torch.float32).reshape(1).contiguous(), ctx.mean), None


def compute_tv_loss(vol: Tensor, reduction: str = "mean") -> Tensor:
    """loss.py:10-21: anisotropic TV of a [D0, D1, D2] (or [1, D0, D1, D2]) volume."""
    if vol.dim() == 4 and vol.size(0) == 1:
        vol = vol[0]
    assert vol.dim() == 3, "tv_3d_loss expects 3D volume"
    return _TV.apply(vol.contiguous(), reduction == "mean")


class _Hierarchy(torch.autograd.Function):
    @staticmethod
    def forward(ctx, child_means, parent, history_means, parent_scales, history_quats,
                history_count, factor):
        out, ws = W.hierarchy_loss_fwd(child_means, parent, history_means, parent_scales,
                                       history_quats, history_count, factor)
        ctx.save_for_backward(out, ws)
        ctx.n = child_means.shape[0]
        return out[0]

    @staticmethod
    def backward(ctx, grad):
        out, ws = ctx.saved_tensors
        v = W.hierarchy_loss_bwd(ctx.n, grad.to(torch.float32).reshape(1).contiguous(), out, ws)
        return v, None, None, None, None, None, None


def compute_hierarchy_loss(child_means: Tensor, parent_indices: Tensor, history_means: Tensor,
                           history_scales: Tensor, history_quats: Tensor, scale_activation,
                           max_parent_distance_factor: float = 1.0) -> Tensor:
    """loss.py:27-71: mean squared excess of each child's distance from its
    archived parent, in the parent's scaled frame, over the allowed radius.
    The archive's scales go through ``scale_activation`` (the model's
    activation) as one element-wise pass; the rest is one fused launch."""
    if (child_means.numel() == 0 or parent_indices.numel() == 0 or history_means.numel() == 0
            or history_scales.numel() == 0 or history_quats.numel() == 0):
        return child_means.new_zeros(())
    history_count = min(history_means.shape[0], history_scales.shape[0],
                        history_quats.shape[0])
    parent_scales = scale_activation(history_scales[:history_count].detach())
    return _Hierarchy.apply(child_means, parent_indices, history_means.detach(),
                            parent_scales.to(torch.float32).contiguous(),
                            history_quats.detach(), int(history_count),
                            float(max_parent_distance_factor))


class LossComputer:
    """loss.py:74-103: weighted projection L1 / SSIM and volume TV."""

    def __init__(self, w_l1: float, w_ssim: float, w_tv: float, ssim_window: int = 11):
        self.w_l1 = w_l1
        self.w_ssim = w_ssim
        self.w_tv = w_tv
        self.ssim_window = ssim_window

    def __call__(self, renders: Tensor, targets: Tensor,
                 volume_pred: Optional[Tensor] = None) -> Dict[str, Tensor]:
        weights = (float(self.w_l1), float(self.w_ssim), 0.0, float(self.w_tv), 0.0)
        l1, ssim_loss, _, tv, total = _trainer_terms(renders, targets, None, None, volume_pred,
                                                     None, weights, self.ssim_window, self.w_tv)
        return {"proj_l1": l1, "proj_ssim": ssim_loss, "vol_tv": tv, "total": total}


class BinaryTreeLossComputer:
    """loss.py:105-172: projection L1 / SSIM, masked edge L1, volume TV and
    the hierarchy term (computed by the caller)."""

    def __init__(self, w_l1: float, w_ssim: float, w_tv: float, w_edge: float,
                 w_hierarchy: float = 0.0, ssim_window: int = 11):
        self.w_l1 = w_l1
        self.w_ssim = w_ssim
        self.w_tv = w_tv
        self.w_edge = w_edge
        self.w_hierarchy = w_hierarchy
        self.ssim_window = ssim_window

    def __call__(self, renders: Tensor, targets: Tensor, edge_mask: Optional[Tensor],
                 volume_pred: Optional[Tensor] = None,
                 hierarchy_loss: Optional[Tensor] = None,
                 edge_targets: Optional[Tensor] = None,
                 edge_weight_override: Optional[float] = None) -> Dict[str, Tensor]:
        if edge_targets is None:
            edge_targets = targets
        if hierarchy_loss is None:
            hierarchy_loss = torch.zeros((), device=renders.device)
        edge_weight = self.w_edge if edge_weight_override is None else float(edge_weight_override)
        weights = (float(self.w_l1), float(self.w_ssim), float(edge_weight), float(self.w_tv),
                   float(self.w_hierarchy))
        l1, ssim_loss, edge_loss, tv, total = _trainer_terms(
            renders, targets, edge_mask, edge_targets, volume_pred, hierarchy_loss, weights,
            self.ssim_window, self.w_tv)
        return {"proj_l1": l1, "proj_ssim": ssim_loss, "vol_tv": tv, "edge": edge_loss,
                "hierarchy": hierarchy_loss,
                "edge_weight": torch.full((), edge_weight, device=renders.device),
                "total": total}
