"""Manau: Muon for 2-D weight matrices, Dana-Star-MK4 for everything else.

Drop-in for src/optim/manau.py:89-613 on one GPU: same constructor
arguments and defaults, group keys, parameter assignment (by ``param_names``),
state keys (``use_muon``, ``muon_buffer``, ``dana_m``, ``dana_v``,
``dana_tau``, ``step``, the diagnostics) and step order.

* The Dana-Star-MK4 branch (manau.py:504-613: embeddings, heads, 1-D
  parameters) is the HIP multi-tensor step with ADANA_VARIANT_MANAU: Manau's
  own op order (multiply-then-add moments, (|g| + sqrt v) + eps, maximum()
  regularisation, weight decay before the update, mk4A / mk4B powers,
  weighted time) in one launch over all of those tensors, state in slabs.
* The Muon half (momentum buffers, bfloat16 Newton-Schulz orthogonalisation,
  manau.py:320-500) is dense matrix work; it runs as torch operations (the
  products are library GEMMs), in the reference's order.

The distributed mode (``enable_distributed_mode``, all-gathers over a process
group) is not part of this single-GPU build and raises.
"""
from __future__ import annotations

import math
from typing import Dict, Tuple

import torch
from torch.optim import Optimizer

from . import _lib
from .optim import _DanaFamily


def zeropower_via_newtonschulz5(G: torch.Tensor, steps: int) -> torch.Tensor:
    """Newton-Schulz orthogonalisation of a 2-D matrix (manau.py:18-40), in
    G's dtype.  Transposed operands are made contiguous before each product
    (same values; the batched-product path has faulted on transposed bfloat16
    operands on this platform)."""
    assert len(G.shape) == 2
    a, b, c = (3.4445, -4.7750, 2.0315)
    X = G
    if G.size(0) > G.size(1):
        X = X.T.contiguous()
    X = X / (X.norm() + 1e-7)
    for _ in range(steps):
        A = X @ X.T.contiguous()
        B = b * A + c * A @ A
        X = a * X + B @ X
    if G.size(0) > G.size(1):
        X = X.T
    return X


def adjust_lr_wd_for_muon(lr, matched_adamw_rms, param_shape):
    """manau.py:81-86."""
    A, B = param_shape[:2]
    adjusted_ratio = math.sqrt(max(A, B)) * matched_adamw_rms
    return lr * adjusted_ratio


class Manau(_DanaFamily):
    """Manau (src/optim/manau.py:89-613).  ``param_groups`` must carry
    ``param_names``: names containing 'wte.weight', 'wpe.weight' or
    'lm_head.weight', and parameters of fewer than 2 dimensions, go to the
    Dana-Star-MK4 branch; the other parameters to Muon."""

    _STAR = True
    _VARIANT = _lib.VARIANT_MANAU
    _KEYS = ("dana_m", "dana_v", "dana_tau")
    _DIAG_COLUMNS = ((0, "current_alpha_factor"), (1, "gradient_norm"), (2, "auto_factor_mean"),
                     (4, "m_norm"))

    def __init__(self, param_groups, lr=2e-2, weight_decay=0.1, matched_adamw_rms=0.2, momentum=0.95,
                 nesterov=True, ns_steps=5, dana_momentum=False, delta=8.0, kappa=1.0, mk4A=0.0, mk4B=0.0,
                 clipsnr=1.0, epsilon=1e-8, weight_time=False, wd_decaying=False, wd_ts=1.0):
        defaults = dict(lr=lr, weight_decay=weight_decay, matched_adamw_rms=matched_adamw_rms,
                        momentum=momentum, nesterov=nesterov, ns_steps=ns_steps, dana_momentum=dana_momentum,
                        delta=delta, kappa=kappa, mk4A=mk4A, mk4B=mk4B, clipsnr=clipsnr, epsilon=epsilon,
                        weight_time=weight_time, wd_decaying=wd_decaying, wd_ts=wd_ts, weighted_step_count=0)
        Optimizer.__init__(self, param_groups, defaults)
        self.distributed_mode = False
        self.lr = lr
        self._engine_init(master_weights=False)

        muon_params, dana_params = [], []
        muon_total_params = dana_total_params = 0
        for group in self.param_groups:                                # manau.py:176-196
            param_names = group.get("param_names", None)
            if param_names is None:
                raise ValueError(
                    "Manau optimizer requires 'param_names' to be provided in param_groups. "
                    "This is needed to correctly identify embeddings and head layers."
                )
            for idx, p in enumerate(group["params"]):
                is_embedding_or_head = False
                if idx < len(param_names):
                    pname = param_names[idx]
                    if any(identifier in pname for identifier in ["wte.weight", "wpe.weight", "lm_head.weight"]):
                        is_embedding_or_head = True
                if not is_embedding_or_head and p.ndim >= 2:
                    self.state[p]["use_muon"] = True
                    muon_params.append((pname, p.shape, p.numel()))
                    muon_total_params += p.numel()
                else:
                    self.state[p]["use_muon"] = False
                    dana_params.append((pname, p.shape, p.numel()))
                    dana_total_params += p.numel()

        print("\n" + "=" * 80)                                          # manau.py:198-223
        print("Manau Optimizer Parameter Assignment")
        print("=" * 80)
        print(f"\nMuon (Newton-Schulz) parameters: {len(muon_params)}")
        print(f"Total Muon params: {muon_total_params:,} ({muon_total_params/1e6:.2f}M)")
        print("-" * 80)
        for pname, shape, numel in muon_params:
            print(f"  [Muon] {pname:50s} {str(shape):20s} {numel:>12,} params")
        print(f"\nDANA-STAR-MK4 parameters: {len(dana_params)}")
        print(f"Total DANA params: {dana_total_params:,} ({dana_total_params/1e6:.2f}M)")
        print("-" * 80)
        for pname, shape, numel in dana_params:
            print(f"  [DANA] {pname:50s} {str(shape):20s} {numel:>12,} params")
        print("\n" + "=" * 80)
        print(f"Total parameters: {muon_total_params + dana_total_params:,} "
              f"({(muon_total_params + dana_total_params)/1e6:.2f}M)")
        print(f"Muon ratio: {100*muon_total_params/(muon_total_params + dana_total_params):.1f}%")
        print(f"DANA ratio: {100*dana_total_params/(muon_total_params + dana_total_params):.1f}%")
        print("=" * 80 + "\n")

    def enable_distributed_mode(self, global_buffer_sizes, dist_group, tp_group,
                                dist_metas: Dict[torch.nn.Parameter, object]):
        """manau.py:225-271: sharded Muon over a process group -- not part of
        this single-GPU build."""
        raise NotImplementedError("Manau.enable_distributed_mode: this build runs one GPU per optimizer; "
                                  "the distributed Muon all-gathers are not implemented")

    # The fused clip path would scale only the Dana branch's gradients.
    def _arm_clip(self, grads, plan, clip, write_back: bool) -> bool:
        return False

    def _scalars(self, classes):
        hps, out = {}, []
        for gi, step, alpha, lr in classes:
            hp = hps.get(gi)
            if hp is None:
                g = self.param_groups[gi]
                hp = hps[gi] = _lib.ManauHParams(
                    delta=g["delta"], kappa=g["kappa"], mk4A=g["mk4A"], mk4B=g["mk4B"],
                    clipsnr=float(g["clipsnr"]), epsilon=g["epsilon"], weight_decay=g["weight_decay"],
                    wd_ts=g["wd_ts"], wd_decaying=1 if g["wd_decaying"] else 0)
            out.append(_lib.manau_scalars(hp, lr, step, alpha))
        return out

    @torch.no_grad()
    def step(self):
        for group in self.param_groups:             # the Dana branch has no CPU path: refuse first
            for p in group["params"]:
                if not self.state[p].get("use_muon", False) and p.device.type != "cuda":
                    raise RuntimeError(f"Manau: parameters must live on a ROCm GPU (got {p.device}); "
                                       "the Dana-Star-MK4 step has no CPU path")
        ns_inputs = {}
        for group in self.param_groups:                                 # manau.py:320-371
            momentum = group["momentum"]
            dana_momentum = group["dana_momentum"]
            delta = group["delta"]
            kappa = group["kappa"]
            weight_time = group["weight_time"]
            for p in group["params"]:
                if not self.state[p].get("use_muon", False):
                    continue
                g = p.grad
                assert g is not None
                assert self.distributed_mode or g.dim() == 2
                state = self.state[p]
                if "muon_buffer" not in state:
                    state["muon_buffer"] = torch.zeros_like(g)
                    state["step"] = 0
                buf = state["muon_buffer"]
                state["step"] += 1
                if dana_momentum:
                    step = state["step"]
                    time_factor = group["lr"] / self.lr if weight_time else 1.0
                    group["weighted_step_count"] += time_factor
                    if weight_time:
                        step = group["weighted_step_count"]
                        alpha = delta / (delta + step) * time_factor
                    else:
                        alpha = delta / (delta + step)
                    buf.mul_(1 - alpha).add_(g, alpha=alpha)
                else:
                    buf.mul_(momentum).add_(g)
                if dana_momentum:
                    step = state["step"]
                    time_scaling = step ** (1 - kappa)
                    g = g + buf * time_scaling
                else:
                    g = g.add(buf, alpha=momentum) if group["nesterov"] else buf
                ns_inputs[p] = g.bfloat16()

        for group in self.param_groups:                                 # manau.py:456-502
            lr = group["lr"]
            for p in group["params"]:
                if not self.state[p].get("use_muon", False):
                    continue
                ns_input = ns_inputs[p]
                update = zeropower_via_newtonschulz5(ns_input, steps=group["ns_steps"])
                p.data.mul_(1 - lr * group["weight_decay"])
                adjusted_lr = adjust_lr_wd_for_muon(lr, group["matched_adamw_rms"], ns_input.shape)
                p.data.add_(update, alpha=-adjusted_lr)

        self._dana_step()                                               # manau.py:504-613

    def _dana_step(self) -> None:
        """The Dana-Star-MK4 branch: the host bookkeeping of manau.py:520-578
        (per-parameter step, the group's weighted step count advanced once
        per parameter, alpha), then one kernel launch per launch set."""
        params, grads, states, keys = [], [], [], []
        fresh = []
        for gi, group in enumerate(self.param_groups):
            delta = group["delta"]
            weight_time = group["weight_time"]
            for p in group["params"]:
                st = self.state[p]
                if st.get("use_muon", False):
                    continue
                g = p.grad
                assert g is not None
                if "dana_m" not in st:                                  # :533-537
                    fresh.append((p, st))
                    st["step"] = 0
                st["step"] += 1
                time_factor = group["lr"] / self.lr if weight_time else 1.0
                group["weighted_step_count"] += time_factor
                if weight_time:
                    step = group["weighted_step_count"]
                    alpha = delta / (delta + step) * time_factor
                else:
                    step = st["step"]
                    alpha = delta / (delta + step)
                st["current_alpha"] = alpha                             # :578
                params.append(p)
                grads.append(g)
                states.append(st)
                keys.append((gi, step, alpha, group["lr"]))
        if not params:
            return
        for group in self.param_groups:
            if group["clipsnr"] is None:
                raise RuntimeError("Manau: clipsnr=None (torch.clamp needs a bound, manau.py:584-589)")
        if fresh:
            self._pack_states(fresh, None)
        cls_index: Dict[Tuple, int] = {}
        sclass = []
        for k in keys:
            c = cls_index.get(k)
            if c is None:
                c = cls_index[k] = len(cls_index)
            sclass.append(c)
        classes = list(cls_index)
        structure = (tuple(map(id, params)), tuple(sclass))
        if self._sets is None or structure != self._structure:
            flags = [self._validate(p, g) for p, g in zip(params, grads)]
            self._sets = self._build(params, grads, states, sclass, flags)
            self._structure = structure
        else:
            for ls in self._sets:
                ls.grads = grads if len(self._sets) == 1 else [grads[i] for i in ls.index]
                self._refresh_ptrs(ls)
        self._launch(params, grads, classes, None)
