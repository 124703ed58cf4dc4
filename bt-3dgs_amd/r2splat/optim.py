"""Adam for the Gaussian parameter groups, stepped by one HIP launch.

The binary-tree trainer builds one ``torch.optim.Adam`` per parameter group
(``src/models/gaussian_model.py:514-530``) and steps them one after another
(``src/trainers/binary_tree.py:208-210``).  Two drop-ins:

* ``Adam``: a ``torch.optim.Adam`` whose ``step()`` is one launch
  (``r2s_adam_step_f32``) instead of torch's ten-odd element-wise kernels;
  same constructor, state layout (``step`` / ``exp_avg`` / ``exp_avg_sq``),
  ``state_dict`` and arithmetic.
* ``step_all(optimizers)``: one launch for several optimizers (ours or plain
  ``torch.optim.Adam`` with the supported options), replacing the trainer's
  ``for optimizer in optimizers.values(): optimizer.step()``.

Supported: float32 CUDA parameters, dense gradients, coupled weight decay;
not amsgrad, maximize, capturable, differentiable or fused -- those raise
``NotImplementedError`` (the reference uses none of them).
"""

from __future__ import annotations

import ctypes
from typing import Iterable, List

import torch
from torch.optim.optimizer import _get_scalar_dtype

from .cuda import _backend
from .cuda import _lib as L

__all__ = ["Adam", "step_all"]


def _check_group(group: dict) -> None:
    for key in ("amsgrad", "maximize", "capturable", "differentiable", "fused",
                "decoupled_weight_decay"):
        if group.get(key):
            raise NotImplementedError(f"the fused Adam step does not support {key}=True")
    for key in ("lr", "eps", "weight_decay"):
        if isinstance(group[key], torch.Tensor):
            raise NotImplementedError(f"the fused Adam step needs a float {key}")
    if any(isinstance(b, torch.Tensor) for b in group["betas"]):
        raise NotImplementedError("the fused Adam step needs float betas")


def _entries(optimizer: torch.optim.Optimizer, out: List[L.AdamTensor], keep: list) -> None:
    """Append one r2s_adam_tensor_t per parameter with a gradient; advances
    each parameter's step count as torch's Adam does."""
    for group in optimizer.param_groups:
        _check_group(group)
        lr, (beta1, beta2) = group["lr"], group["betas"]
        eps, wd = group["eps"], group["weight_decay"]
        for p in group["params"]:
            if p.grad is None:
                continue
            if p.grad.is_sparse:
                raise RuntimeError("Adam does not support sparse gradients, please consider "
                                   "SparseAdam instead")
            if not p.is_cuda or p.dtype != torch.float32:
                raise NotImplementedError("the fused Adam step needs float32 CUDA parameters")
            state = optimizer.state[p]
            if len(state) == 0:  # torch/optim/adam.py _init_group
                state["step"] = torch.tensor(0.0, dtype=_get_scalar_dtype())
                state["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                state["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)
            m, v = state["exp_avg"], state["exp_avg_sq"]
            if not (p.is_contiguous() and m.is_contiguous() and v.is_contiguous()):
                raise NotImplementedError("the fused Adam step needs contiguous tensors")
            if m.shape != p.shape or v.shape != p.shape:
                raise RuntimeError("Adam state does not match its parameter")
            grad = p.grad.contiguous()
            state["step"] += 1
            step = float(state["step"].item()) if isinstance(state["step"], torch.Tensor) \
                else float(state["step"])
            # torch/optim/adam.py _multi_tensor_adam, non-capturable branch.
            bias_correction1 = 1 - beta1 ** step
            bias_correction2 = 1 - beta2 ** step
            step_size = (lr / bias_correction1) * -1
            bias_correction2_sqrt = bias_correction2 ** 0.5
            out.append(L.AdamTensor(p.data_ptr(), grad.data_ptr(), m.data_ptr(), v.data_ptr(),
                                    p.numel(), 1 - beta1, beta2, 1 - beta2, wd,
                                    bias_correction2_sqrt, eps, step_size))
            keep.append(grad)


def _launch(entries: List[L.AdamTensor], device) -> None:
    if not entries:
        return
    lib = _backend.library()
    table = (L.AdamTensor * len(entries))(*entries)
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device).cuda_stream
        rc = lib.r2s_adam_step_f32(ctypes.cast(table, ctypes.c_void_p), len(entries), stream)
    if rc != 0:
        raise RuntimeError(f"r2s_adam_step_f32 failed ({rc}): "
                           f"{lib.r2s_last_error().decode(errors='replace')}")


def _device_of(optimizers) -> torch.device:
    for opt in optimizers:
        for group in opt.param_groups:
            for p in group["params"]:
                return p.device
    return torch.device("cuda")


def step_all(optimizers: Iterable[torch.optim.Optimizer]) -> None:
    """``optimizer.step()`` for every optimizer, as one launch."""
    opts = list(optimizers.values() if isinstance(optimizers, dict) else optimizers)
    for opt in opts:
        if not isinstance(opt, torch.optim.Adam):
            raise TypeError(f"step_all steps Adam optimizers, got {type(opt).__name__}")
    entries: List[L.AdamTensor] = []
    keep: list = []
    with torch.no_grad():
        for opt in opts:
            _entries(opt, entries, keep)
        _launch(entries, _device_of(opts))


class Adam(torch.optim.Adam):
    """torch.optim.Adam with a one-launch ``step()`` (see module docstring)."""

    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0,
                 amsgrad=False, **kwargs):
        super().__init__(params, lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                         amsgrad=amsgrad, **kwargs)
        for group in self.param_groups:
            _check_group(group)

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        entries: List[L.AdamTensor] = []
        keep: list = []
        _entries(self, entries, keep)
        _launch(entries, _device_of([self]))
        return loss
