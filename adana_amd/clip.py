"""Gradient-norm clipping on the HIP kernels, optionally fused into the step.

Reference: the training loop clips every step before ``opt.step()``
(src/optim/base.py:250-257) through ``distributed_backend.clip_grad_norm_``
(src/distributed/backend.py:33-35), i.e. ``torch.nn.utils.clip_grad_norm_``
with the default norm_type 2:

    norms = torch._foreach_norm(grads)                      # per tensor, grad dtype
    total = torch.linalg.vector_norm(torch.stack(norms))    # norm of the norms
    coef  = torch.clamp(max_norm / (total + 1e-6), max=1.0) # float / Tensor =
                                                            # reciprocal() * float
    torch._foreach_mul_(grads, coef)                        # in place

``clip_grad_norm_`` below has the same signature, return value (the total
norm as a 0-d tensor in the gradients' dtype) and effect.  The sums of
squares come from one read-only HIP pass over the gradients (binary64
accumulation), the total norm and the coefficient are computed on the device
(no host synchronisation), and the in-place scaling is either a separate HIP
pass or, with ``optimizer=`` an ADana / DANA_STAR_MK4 that owns exactly these
gradients, folded into that optimizer's next ``step()``: the step kernel
multiplies each gradient by the coefficient as it loads it and, with
``write_back=True`` (default), stores the clipped gradient back, so after
``step()`` every ``p.grad`` holds what the reference's in-place clipping
leaves there.  Between the clip call and ``step()`` the gradients are still
unscaled; ``optimizer.flush_clip()`` applies the pending scaling early, and
``zero_grad()`` drops it.
"""
from __future__ import annotations

import ctypes
from collections import OrderedDict
from typing import Iterable, List, Optional, Union

import numpy as np
import torch

from . import _hoststep, _lib
from ._layout import dense_layout

__all__ = ["clip_grad_norm_", "GradPlan"]


class GradPlan:
    """A laid-out gradient list on one device (the descriptors carry only the
    numel; the gradient pointers are the plan's separate array).  The layout
    is rebuilt when the tensor sizes change; the gradient pointers are
    re-uploaded only when an address moved."""

    def __init__(self, device: torch.device, bf16: bool):
        self.device = device
        self.bf16 = bf16
        self.flags = _lib.GRAD_BF16 if bf16 else 0
        self.numels = None
        self.ptrs = None
        self.grads: List[torch.Tensor] = []
        self.plan = _lib.Plan()
        self.dev_table = None
        self.dev_grad = None
        self.chunk_first = None
        self.workspace = None

    def prepare(self, grads: List[torch.Tensor]) -> None:
        n = len(grads)
        numels = np.fromiter((g.numel() for g in grads), dtype=np.int64, count=n)
        ptrs = np.frombuffer(_hoststep.data_ptrs(grads), dtype=np.uint64)
        relayout = self.numels is None or not np.array_equal(numels, self.numels)
        self.grads = grads
        with torch.cuda.device(self.device):
            if relayout:
                self.vstart, self.fold_first, self.n_chunks, self.n_folds = _lib.plan_layout(numels)
                self.numels = numels
                desc = np.zeros(n, dtype=_lib.DESC_DTYPE)
                desc["numel"] = numels
                table = np.concatenate([desc.view(np.uint8), self.vstart.view(np.uint8),
                                        self.fold_first.view(np.uint8)])
                self.dev_table = torch.from_numpy(table).pin_memory().to(self.device, non_blocking=True)
                self.dev_grad = torch.empty(max(n, 1), dtype=torch.int64, device=self.device)
                self.ptrs = None
                base = self.dev_table.data_ptr()
                pl = self.plan
                pl.desc = base
                pl.grad = self.dev_grad.data_ptr()
                pl.vstart = base + 64 * n
                pl.fold_first = base + 64 * n + 8 * (n + 1)
                pl.n_tensors = n
                pl.n_chunks = self.n_chunks
                pl.n_folds = self.n_folds
                self.chunk_first = torch.empty(max(self.n_chunks, 1), dtype=torch.int32, device=self.device)
                stream = torch.cuda.current_stream(self.device).cuda_stream
                _lib.check(_lib.lib().adana_plan_index(
                    ctypes.c_void_p(pl.vstart), n, self.n_chunks,
                    ctypes.c_void_p(self.chunk_first.data_ptr()), ctypes.c_void_p(stream)),
                    "adana_plan_index")
                pl.chunk_first = self.chunk_first.data_ptr()
                self.workspace = torch.empty(max(_lib.workspace_bytes(pl), 1), dtype=torch.uint8,
                                             device=self.device)
            if n and (self.ptrs is None or not np.array_equal(ptrs, self.ptrs)):
                self.dev_grad[:n].copy_(torch.from_numpy(ptrs.view(np.int64).copy()).pin_memory(),
                                        non_blocking=True)
                self.ptrs = ptrs.copy()

    def clip_norm(self, max_norm: float) -> torch.Tensor:
        """Launch the norm pass; returns a new device float32[2] = (total, coef)."""
        out = torch.empty(2, dtype=torch.float32, device=self.device)
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            _lib.check(_lib.lib().adana_grad_clip_norm(
                ctypes.byref(self.plan), self.flags, float(max_norm),
                ctypes.c_void_p(self.workspace.data_ptr()), self.workspace.numel(), None,
                ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream)), "adana_grad_clip_norm")
        return out

    def scale(self, clip: torch.Tensor) -> None:
        """In place g *= clip[1] for every gradient of the plan."""
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            _lib.check(_lib.lib().adana_grad_scale(
                ctypes.byref(self.plan), self.flags, ctypes.c_void_p(clip.data_ptr() + 4),
                ctypes.c_void_p(stream)), "adana_grad_scale")
        _hoststep.bump_versions(self.grads)                # g was scaled in place


_PLANS: "OrderedDict[tuple, GradPlan]" = OrderedDict()
_MAX_PLANS = 8


def _shared_plan(device, bf16: bool, grads) -> GradPlan:
    key = (device, bf16, len(grads), hash(tuple(g.numel() for g in grads)))
    plan = _PLANS.get(key)
    if plan is None:
        plan = _PLANS[key] = GradPlan(device, bf16)
        while len(_PLANS) > _MAX_PLANS:
            _PLANS.popitem(last=False)
    else:
        _PLANS.move_to_end(key)
    return plan


def _validate(grads: List[torch.Tensor]):
    g0 = grads[0]
    if g0.device.type != "cuda":
        raise RuntimeError(f"clip_grad_norm_: gradients must live on a ROCm GPU (got {g0.device}); "
                           "there is no CPU path")
    if g0.dtype not in (torch.float32, torch.bfloat16):
        raise NotImplementedError(f"clip_grad_norm_: gradient dtype {g0.dtype}")
    for g in grads:
        if g.device != g0.device or g.dtype != g0.dtype:
            raise NotImplementedError("clip_grad_norm_: all gradients must share one device and dtype "
                                      f"({g0.device}/{g0.dtype} vs {g.device}/{g.dtype})")
        if g.is_sparse or not dense_layout(g):
            raise NotImplementedError("clip_grad_norm_: sparse gradients, or gradients whose elements overlap "
                                      "or leave gaps in memory, are not supported")
    return g0.device, g0.dtype == torch.bfloat16


def clip_grad_norm_(parameters: Union[torch.Tensor, Iterable[torch.Tensor]], max_norm: float,
                    norm_type: float = 2.0, error_if_nonfinite: bool = False,
                    foreach: Optional[bool] = None, *, optimizer=None,
                    write_back: bool = True) -> torch.Tensor:
    """``torch.nn.utils.clip_grad_norm_`` (norm_type 2) on HIP kernels.

    ``foreach`` is accepted and ignored (there is one code path).  With
    ``optimizer`` (an ADana / DANA_STAR_MK4 whose parameters with gradients
    are exactly these), the scaling runs inside that optimizer's next
    ``step()``; ``write_back=False`` then leaves ``p.grad`` unscaled (the
    step still uses the clipped values) and saves one gradient write.
    """
    if isinstance(parameters, torch.Tensor):
        parameters = [parameters]
    else:
        parameters = list(parameters)
    if float(norm_type) != 2.0:
        raise NotImplementedError(f"clip_grad_norm_: norm_type {norm_type} (only 2.0 is implemented)")
    if optimizer is not None:
        optimizer.flush_clip()          # a pending scale applies before this norm is taken
    grads = [p.grad for p in parameters if p.grad is not None]
    if not grads:
        return torch.tensor(0.0)
    device, bf16 = _validate(grads)
    if optimizer is not None:
        plan = optimizer._clip_plan(device, bf16)
    else:
        plan = _shared_plan(device, bf16, grads)
    plan.prepare(grads)
    clip = plan.clip_norm(max_norm)
    total = clip[0]
    if bf16:
        total = total.to(torch.bfloat16)            # exact: the kernel rounded it to bfloat16
    if error_if_nonfinite and torch.logical_or(total.isnan(), total.isinf()):
        raise RuntimeError(
            f"The total norm of order {float(norm_type)} for gradients from `parameters` is "
            "non-finite, so it cannot be clipped. To disable this error and scale the gradients "
            "by the non-finite norm anyway, set `error_if_nonfinite=False`")
    if optimizer is None or not optimizer._arm_clip(grads, plan, clip, write_back):
        plan.scale(clip)
    return total
