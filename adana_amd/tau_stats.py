"""Tau order statistics of Dana-Star's state, selected on the GPU.

Reference: TauStatsCollector (src/optim/tau_stats_collector.py).  At
exponentially spaced eval steps it calls ``_extract_tau_statistics(opt)``
(:131-160), which copies every ``state['tau']`` to the host and runs
``compute_tau_order_statistics`` (:336-376): ``np.sort`` of the flattened
tensor, then the sorted values at indices ``unique(int32(1.1**k) - 1)``
(clamped to n - 1) from the smallest end and from the largest end.

Here the same indices are computed the same way on the host, and the values
at those ranks come from the library's exact multi-rank radix select
(``adana_order_stats``, adana_amd/csrc/adana_order_stats.hip): 4 to 8 passes
over each tensor in HBM, nothing copied to the host but the selected values.
Results equal the reference's (float32 values; NaN sorts last as in
np.sort).
"""
from __future__ import annotations

import ctypes
import functools
from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch

from . import _lib

__all__ = ["order_stat_indices", "order_values", "compute_tau_order_statistics",
           "extract_tau_statistics"]


def order_stat_indices(n: int) -> np.ndarray:
    """Sorted positions read by compute_tau_order_statistics for n >= 1
    elements (src/optim/tau_stats_collector.py:360-366)."""
    max_k = int(np.ceil(np.log(n) / np.log(1.1)))
    indices = np.int32(1.1 ** np.arange(max_k + 1)) - 1
    indices = np.unique(indices)
    return np.minimum(indices, n - 1)


def order_values(tensors: Sequence[torch.Tensor], ranks: Sequence[np.ndarray]) -> List[np.ndarray]:
    """Values at ``ranks[i]`` (ascending order, np.sort's) of each float32
    CUDA tensor, exactly, in one batched device selection."""
    if len(tensors) != len(ranks):
        raise ValueError("order_values: one rank array per tensor")
    flat, numel, rank_first, all_ranks = [], [], [0], []
    for t, r in zip(tensors, ranks):
        if t.device.type != "cuda" or t.dtype != torch.float32:
            raise RuntimeError(f"order_values: float32 ROCm tensors only (got {t.dtype} on {t.device})")
        f = t.detach().reshape(-1)
        if not f.is_contiguous():
            f = f.contiguous()
        flat.append(f)
        numel.append(f.numel())
        r = np.ascontiguousarray(r, dtype=np.int64)
        all_ranks.append(r)
        rank_first.append(rank_first[-1] + r.size)
    n = len(flat)
    if n == 0:
        return []
    ptrs = np.array([f.data_ptr() for f in flat], dtype=np.uint64)
    numel_a = np.array(numel, dtype=np.int64)
    rank_first_a = np.array(rank_first, dtype=np.int64)
    ranks_a = np.concatenate(all_ranks) if rank_first[-1] else np.zeros(1, np.int64)
    values = np.empty(max(rank_first[-1], 1), dtype=np.float32)
    L = _lib.lib()
    dev = flat[0].device
    for f in flat:
        if f.device != dev:
            raise NotImplementedError("order_values: tensors on more than one device")
    ws = torch.empty(max(int(L.adana_order_stats_workspace(n, rank_first[-1])), 1), dtype=torch.uint8,
                     device=dev)
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(L.adana_order_stats(ctypes.c_void_p(ptrs.ctypes.data), ctypes.c_void_p(numel_a.ctypes.data),
                                       n, ctypes.c_void_p(ranks_a.ctypes.data),
                                       ctypes.c_void_p(rank_first_a.ctypes.data),
                                       ctypes.c_void_p(values.ctypes.data), ctypes.c_void_p(ws.data_ptr()),
                                       ws.numel(), ctypes.c_void_p(stream)), "adana_order_stats")
    return [values[a:b].copy() for a, b in zip(rank_first[:-1], rank_first[1:])]


@functools.lru_cache(maxsize=1024)
def _rank_plan(n: int) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """For n >= 1 elements: the distinct ranks to select (both ends'
    positions, ascending) and where the smallest / largest order statistics
    sit among them.  Depends on n only, so it is cached (a model's tensors
    repeat a few shapes); the arrays are read-only."""
    idx = order_stat_indices(n)
    wanted = np.unique(np.concatenate([idx, (n - 1) - idx])).astype(np.int64)
    pos_small = np.searchsorted(wanted, idx)
    pos_large = np.searchsorted(wanted, (n - 1) - idx)
    for a in (wanted, pos_small, pos_large):
        a.flags.writeable = False
    return wanted, pos_small, pos_large


def _stats_for(tensors: Sequence[torch.Tensor]) -> List[Tuple[np.ndarray, np.ndarray]]:
    plans, ranks = [], []
    for t in tensors:
        n = t.numel()
        if n == 0:
            plans.append(None)
            ranks.append(np.zeros(0, np.int64))
            continue
        plan = _rank_plan(n)
        plans.append(plan)
        ranks.append(plan[0])
    vals = order_values(tensors, ranks)
    out = []
    for plan, v in zip(plans, vals):
        if plan is None:
            out.append((np.array([]), np.array([])))          # the reference's empty result
            continue
        _, pos_small, pos_large = plan
        out.append((v[pos_large], v[pos_small]))
    return out


def compute_tau_order_statistics(tau: torch.Tensor) -> Tuple[np.ndarray, np.ndarray]:
    """(largest_order_stats, smallest_order_stats) of a tau tensor on the GPU,
    equal to src/optim/tau_stats_collector.py:336-376 on ``tau.cpu().numpy()``."""
    return _stats_for([tau])[0]


def extract_tau_statistics(opt, param_name=None) -> Dict[str, Dict]:
    """TauStatsCollector._extract_tau_statistics (src/optim/tau_stats_collector.py:
    131-160) with one batched device selection for all tau tensors.
    ``param_name(param, group, param_idx)`` names the entries (default: the
    group's 'param_names' entry, else ``param_group_{id(group)}_idx_{i}``, as
    the reference's _get_param_name)."""
    def default_name(param, group, idx):
        if "param_names" in group and idx < len(group["param_names"]):
            return group["param_names"][idx]
        return f"param_group_{id(group)}_idx_{idx}"

    name_of = param_name or default_name
    entries = []
    for group in opt.param_groups:
        for idx, param in enumerate(group["params"]):
            if param not in opt.state:
                continue
            state = opt.state[param]
            if "tau" not in state:
                continue
            entries.append((name_of(param, group, idx), state["tau"]))
    stats = _stats_for([t for _, t in entries])
    out = {}
    for (name, tau), (largest, smallest) in zip(entries, stats):
        out[name] = {"shape": tuple(tau.shape), "largest_order_stats": largest,
                     "smallest_order_stats": smallest, "num_elements": tau.numel()}
    return out
