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

import ctypes
import math
from typing import Dict, List, Tuple

import torch
from torch.optim import Optimizer

from . import _lib
from .optim import _DanaFamily

# Parameter names whose tensors stay on the Dana branch even when 2-D: token
# and position embeddings and the output head (src/optim/manau.py:186-189).
_DANA_NAME_MARKERS = ("wte.weight", "wpe.weight", "lm_head.weight")
# The quintic Newton-Schulz coefficients of Muon (K. Jordan's published
# orthogonalisation; src/optim/manau.py:23).
_NS_A, _NS_B, _NS_C = 3.4445, -4.7750, 2.0315


def _newton_schulz(m: torch.Tensor, iters: int) -> torch.Tensor:
    """Approximately orthogonalise a 2-D matrix (its U V^T) in its own dtype:
    normalise by the Frobenius norm, then ``iters`` rounds of
    X <- a X + (b A + (c A) A) X with A = X X^T, on the wide orientation of
    the matrix (rows <= columns), transposed back at the end.  This is the
    products' order of src/optim/manau.py:18-40, so bfloat16 results agree
    with the reference's.  Every product takes contiguous operands: torch's
    bfloat16 batched-product path is documented on this platform to fault
    the GPU with a transposed right operand, so none is ever passed."""
    if m.dim() != 2:
        raise ValueError(f"Newton-Schulz needs a matrix, got shape {tuple(m.shape)}")
    tall = m.shape[0] > m.shape[1]
    x = m.transpose(0, 1).contiguous() if tall else m
    x = x / (x.norm() + 1e-7)
    for _ in range(iters):
        gram = x @ x.transpose(0, 1).contiguous()
        poly = _NS_B * gram + _NS_C * gram @ gram
        x = _NS_A * x + poly @ x
    return x.transpose(0, 1) if tall else x


def _muon_lr(lr: float, matched_adamw_rms: float, shape) -> float:
    """Muon's step size for a matrix of ``shape``: lr scaled by
    sqrt(max(rows, cols)) * matched_adamw_rms, so the update's RMS matches an
    AdamW update's (src/optim/manau.py:81-86)."""
    return lr * (math.sqrt(max(shape[0], shape[1])) * matched_adamw_rms)


def _assignment_report(muon: List[Tuple[str, torch.Size, int]], dana: List[Tuple[str, torch.Size, int]]) -> str:
    """The parameter-assignment summary the reference's constructor prints
    (src/optim/manau.py:198-223), character for character."""
    rule, thin = "=" * 80, "-" * 80
    n_muon = sum(n for _, _, n in muon)
    n_dana = sum(n for _, _, n in dana)
    total = n_muon + n_dana
    out = ["", rule, "Manau Optimizer Parameter Assignment", rule]
    for tag, title, label, rows, count in (("Muon", "Muon (Newton-Schulz)", "Muon", muon, n_muon),
                                            ("DANA", "DANA-STAR-MK4", "DANA", dana, n_dana)):
        out += ["", f"{title} parameters: {len(rows)}", f"Total {label} params: {count:,} ({count / 1e6:.2f}M)",
                thin]
        out += [f"  [{tag}] {name:50s} {str(shape):20s} {numel:>12,} params" for name, shape, numel in rows]
    out += ["", rule, f"Total parameters: {total:,} ({total / 1e6:.2f}M)",
            f"Muon ratio: {100 * n_muon / total:.1f}%", f"DANA ratio: {100 * n_dana / total:.1f}%", rule, "", ""]
    return "\n".join(out)


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
        self._engine_init(master_weights=False, numerics="eager")   # the branch is eager ATen ops
        rows = {True: [], False: []}
        for group in self.param_groups:
            for name, p, to_muon in self._routes(group):
                self.state[p]["use_muon"] = to_muon
                rows[to_muon].append((name, p.shape, p.numel()))
        print(_assignment_report(rows[True], rows[False]), end="")

    @staticmethod
    def _routes(group):
        """(name, parameter, goes to Muon) for every parameter of a group:
        matrices go to Muon unless their name marks an embedding or the head
        (src/optim/manau.py:176-196).  Only a parameter with a name of its own
        can be marked by it: one past the end of the group's name list goes to
        Muon if it is a matrix (manau.py:185-190), and the printed report shows
        it under the previous name, as the reference's does."""
        names = group.get("param_names")
        if names is None:
            raise ValueError("Manau: every parameter group needs a 'param_names' list (one name per "
                             "parameter) to tell embeddings and the output head from the other matrices")
        name = ""
        out = []
        for i, p in enumerate(group["params"]):
            named = i < len(names)
            name = names[i] if named else name
            dana_by_name = named and any(marker in name for marker in _DANA_NAME_MARKERS)
            out.append((name, p, p.ndim >= 2 and not dana_by_name))
        return out

    def enable_distributed_mode(self, global_buffer_sizes, dist_group, tp_group,
                                dist_metas: Dict[torch.nn.Parameter, object]):
        """manau.py:225-271: sharded Muon over a process group -- not part of
        this single-GPU build."""
        raise NotImplementedError("Manau.enable_distributed_mode: this build runs one GPU per optimizer; "
                                  "the distributed Muon all-gathers are not implemented")

    # The fused clip path would scale only the Dana branch's gradients.
    def _arm_clip(self, grads, plan, clip, write_back: bool) -> bool:
        return False

    def _fill_scalars(self, ls, classes) -> int:
        """The launch set's scalar classes of the branch (adana_manau_scalars,
        the same 64-byte slots) written into ls.sc_arr; their count."""
        n_cls = min(_lib.MAX_CLASSES, len(classes) - ls.class_base)
        for k, sc in enumerate(self._scalars(classes[ls.class_base:ls.class_base + n_cls])):
            ctypes.memmove(ctypes.byref(ls.sc_arr[k]), ctypes.byref(sc), 64)
        return n_cls

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

    def _ema_alpha(self, group, own_step: int):
        """The EMA coefficient of one parameter's update and the step it was
        taken at: delta / (delta + t) with t the parameter's own step, or,
        with weight_time, the group's weighted step count (advanced here by
        lr / peak lr, once per parameter) and the coefficient scaled by that
        time factor (src/optim/manau.py:345-355, :541-555)."""
        weight_time = group["weight_time"]
        tf = group["lr"] / self.lr if weight_time else 1.0
        group["weighted_step_count"] += tf
        delta = group["delta"]
        if weight_time:
            t = group["weighted_step_count"]
            return t, delta / (delta + t) * tf
        return own_step, delta / (delta + own_step)

    def _muon_input(self, group, p) -> torch.Tensor:
        """Advance one Muon parameter's momentum buffer and return its
        Newton-Schulz input in bfloat16 (src/optim/manau.py:320-371):
        heavy-ball momentum, Nesterov by default, or with dana_momentum the
        Dana EMA of the gradient added to it with weight step^(1 - kappa)."""
        g = p.grad
        if g is None:
            raise AssertionError("Manau: a Muon parameter has no gradient")
        st = self.state[p]
        buf = st.get("muon_buffer")
        if buf is None:
            buf = st["muon_buffer"] = torch.zeros_like(g)
            st["step"] = 0
        st["step"] += 1
        if group["dana_momentum"]:
            _, a = self._ema_alpha(group, st["step"])
            buf.mul_(1 - a).add_(g, alpha=a)
            direction = g + buf * (st["step"] ** (1 - group["kappa"]))
        else:
            mu = group["momentum"]
            buf.mul_(mu).add_(g)
            direction = g.add(buf, alpha=mu) if group["nesterov"] else buf
        return direction.bfloat16()

    @torch.no_grad()
    def step(self):
        muon = [(group, p) for group in self.param_groups for p in group["params"]
                if self.state[p].get("use_muon", False)]
        for group in self.param_groups:             # the Dana branch has no CPU path: refuse first
            for p in group["params"]:
                if not self.state[p].get("use_muon", False) and p.device.type != "cuda":
                    raise RuntimeError(f"Manau: parameters must live on a ROCm GPU (got {p.device}); "
                                       "the Dana-Star-MK4 step has no CPU path")
        # every momentum first (they advance the weighted step counts the
        # Dana branch reads), then every orthogonalised update, then the
        # Dana branch (src/optim/manau.py:320-613)
        inputs = [self._muon_input(group, p) for group, p in muon]
        for (group, p), x in zip(muon, inputs):
            update = _newton_schulz(x, group["ns_steps"])
            lr = group["lr"]
            p.data.mul_(1 - lr * group["weight_decay"])
            p.data.add_(update, alpha=-_muon_lr(lr, group["matched_adamw_rms"], x.shape))
        self._dana_step()

    def _dana_step(self) -> None:
        """The Dana-Star-MK4 branch: the host bookkeeping of manau.py:520-578
        (per-parameter step, the group's weighted step count advanced once
        per parameter, alpha), then one kernel launch per launch set."""
        params, grads, states, keys = [], [], [], []
        fresh = []
        for gi, group in enumerate(self.param_groups):
            for p in group["params"]:
                st = self.state[p]
                if st.get("use_muon", False):
                    continue
                g = p.grad
                if g is None:
                    raise AssertionError("Manau: a Dana-branch parameter has no gradient")
                if "dana_m" not in st:                                  # :533-537
                    fresh.append((p, st))
                    st["step"] = 0
                st["step"] += 1
                step, alpha = self._ema_alpha(group, st["step"])
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
