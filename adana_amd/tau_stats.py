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

from . import _hoststep, _lib

__all__ = ["order_stat_indices", "order_values", "compute_tau_order_statistics",
           "extract_tau_statistics"]


def order_stat_indices(n: int) -> np.ndarray:
    """Sorted positions read by compute_tau_order_statistics for n >= 1
    elements (src/optim/tau_stats_collector.py:360-366)."""
    max_k = int(np.ceil(np.log(n) / np.log(1.1)))
    indices = np.int32(1.1 ** np.arange(max_k + 1)) - 1
    indices = np.unique(indices)
    return np.minimum(indices, n - 1)


def _select(flat: Sequence[torch.Tensor], numel: np.ndarray, ranks: np.ndarray,
            rank_first: np.ndarray, compact: bool = True) -> np.ndarray:
    """One adana_order_stats call: the values at ``ranks[rank_first[i]:
    rank_first[i + 1]]`` of each contiguous float32 tensor ``flat[i]``,
    concatenated.  ``compact``: give it the workspace with which its late
    passes read only the values that can still match (about 1/8 of the
    tensors' bytes more; same results)."""
    dev = flat[0].device
    for f in flat:
        if f.device.type != "cuda" or f.dtype != torch.float32:
            raise RuntimeError(f"order_values: float32 ROCm tensors only (got {f.dtype} on {f.device})")
        if f.device != dev:
            raise NotImplementedError("order_values: tensors on more than one device")
    n = len(flat)
    total = int(rank_first[-1])
    ptrs = np.frombuffer(_hoststep.data_ptrs(list(flat)), dtype=np.uint64)
    values = np.empty(max(total, 1), dtype=np.float32)
    ranks = ranks if total else np.zeros(1, np.int64)
    L = _lib.lib()
    if compact:
        nbytes = int(L.adana_order_stats_workspace_compact(ctypes.c_void_p(numel.ctypes.data),
                                                             ctypes.c_void_p(rank_first.ctypes.data), n))
    else:
        nbytes = int(L.adana_order_stats_workspace(n, total))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        _lib.check(L.adana_order_stats(ctypes.c_void_p(ptrs.ctypes.data), ctypes.c_void_p(numel.ctypes.data),
                                       n, ctypes.c_void_p(ranks.ctypes.data),
                                       ctypes.c_void_p(rank_first.ctypes.data),
                                       ctypes.c_void_p(values.ctypes.data), ctypes.c_void_p(ws.data_ptr()),
                                       ws.numel(), ctypes.c_void_p(stream)), "adana_order_stats")
    return values


def _contiguous(t: torch.Tensor) -> torch.Tensor:
    t = t.detach()
    return t if t.is_contiguous() else t.contiguous()


def order_values(tensors: Sequence[torch.Tensor], ranks: Sequence[np.ndarray],
                 compact: bool = True) -> List[np.ndarray]:
    """Values at ``ranks[i]`` (ascending order, np.sort's) of each float32
    CUDA tensor, exactly, in one batched device selection (``compact``: see
    _select)."""
    if len(tensors) != len(ranks):
        raise ValueError("order_values: one rank array per tensor")
    if not tensors:
        return []
    flat = [_contiguous(t) for t in tensors]
    all_ranks = [np.ascontiguousarray(r, dtype=np.int64).ravel() for r in ranks]
    rank_first = np.zeros(len(flat) + 1, dtype=np.int64)
    np.cumsum([r.size for r in all_ranks], out=rank_first[1:])
    numel = np.array([f.numel() for f in flat], dtype=np.int64)
    values = _select(flat, numel, np.concatenate(all_ranks), rank_first, compact)
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


@functools.lru_cache(maxsize=16)
def _batch_plan(sizes: Tuple[int, ...]):
    """For a list of tensor sizes: the sizes, the concatenated ranks and their
    offsets for one _select call, and the positions of every tensor's largest
    and smallest order statistics in its result (global indices, with the
    offsets where each tensor's share starts).  Depends on the sizes only, so
    repeated collections over one model reuse it; arrays are read-only."""
    plans = [_rank_plan(n) if n else None for n in sizes]
    counts = [p[0].size if p else 0 for p in plans]
    rank_first = np.zeros(len(sizes) + 1, dtype=np.int64)
    np.cumsum(counts, out=rank_first[1:])
    ranks = (np.concatenate([p[0] for p in plans if p]) if rank_first[-1]
             else np.zeros(0, np.int64))
    large, small, out_first = [], [], [0]
    for p, base in zip(plans, rank_first[:-1]):
        if p is not None:
            large.append(p[2] + base)
            small.append(p[1] + base)
        out_first.append(out_first[-1] + (p[1].size if p else 0))
    large = np.concatenate(large) if large else np.zeros(0, np.int64)
    small = np.concatenate(small) if small else np.zeros(0, np.int64)
    numel = np.array(sizes, dtype=np.int64)
    for a in (numel, ranks, rank_first, large, small):
        a.flags.writeable = False
    return numel, ranks, rank_first, large, small, out_first


def _stats_for(tensors: Sequence[torch.Tensor]) -> List[Tuple[np.ndarray, np.ndarray]]:
    """(largest, smallest) order statistics of each tensor, from one selection."""
    if not tensors:
        return []
    flat = [_contiguous(t) for t in tensors]
    numel, ranks, rank_first, large, small, out_first = _batch_plan(tuple(f.numel() for f in flat))
    values = _select(flat, numel, ranks, rank_first)
    vl, vs = values[large], values[small]
    out = []
    for n, a, b in zip(numel, out_first[:-1], out_first[1:]):
        if n == 0:
            out.append((np.array([]), np.array([])))          # the reference's empty result
        else:
            out.append((vl[a:b], vs[a:b]))
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
