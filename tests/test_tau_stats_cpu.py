"""Tau order statistics: the oracle's restatement of
compute_tau_order_statistics (src/optim/tau_stats_collector.py:336-376)
pinned by brute force (pure-Python sort and index formula on small inputs)
and by invariants; the product's host-side index computation and argument
checks without a GPU."""
import math

import numpy as np
import pytest
import torch


def _brute(values):
    """Pure Python: sort with NaN last; indices floor(1.1**k) - 1 for
    k = 0..ceil(log n / log 1.1), deduplicated, clamped to n - 1."""
    n = len(values)
    s = sorted(values, key=lambda v: (math.isnan(v), v if not math.isnan(v) else 0.0))
    max_k = math.ceil(math.log(n) / math.log(1.1))
    idx = sorted({int(1.1 ** k) - 1 for k in range(max_k + 1)})
    idx = [min(i, n - 1) for i in idx]
    return [s[n - 1 - i] for i in idx], [s[i] for i in idx]


def _same(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return a.shape == b.shape and bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


@pytest.mark.parametrize("n", [1, 2, 3, 10, 11, 37, 100, 1000, 4097])
def test_oracle_matches_brute_force(oracle_mod, n):
    rng = np.random.default_rng(n)
    for dist in ("uniform", "dups", "special"):
        if dist == "uniform":
            x = rng.random(n).astype(np.float32)
        elif dist == "dups":
            x = rng.integers(0, 5, n).astype(np.float32) / 4
        else:
            x = rng.normal(0, 1, n).astype(np.float32)
            x[::7] = np.nan
            x[1::11] = 0.0
            x[2::13] = -0.0
            x[3::17] = np.inf
        largest, smallest = oracle_mod.tau_order_statistics(x)
        bl, bs = _brute([float(v) for v in x])
        assert _same(largest, bl) and _same(smallest, bs), (n, dist)


def test_oracle_invariants(oracle_mod):
    rng = np.random.default_rng(0)
    x = rng.random(50000).astype(np.float32)
    largest, smallest = oracle_mod.tau_order_statistics(x)
    assert smallest[0] == x.min() and largest[0] == x.max()
    assert np.all(np.diff(smallest) >= 0) and np.all(np.diff(largest) <= 0)
    assert smallest.dtype == np.float32 and largest.size == smallest.size
    assert smallest[-1] == largest[-1] == np.sort(x)[-1] or smallest.size > 0
    e = oracle_mod.tau_order_statistics(np.zeros(0, np.float32))
    assert e[0].size == 0 and e[1].size == 0


@pytest.mark.parametrize("n", [1, 2, 5, 64, 1000, 65536, 10 ** 8])
def test_product_indices_match_oracle_formula(n):
    from adana_amd.tau_stats import order_stat_indices

    idx = order_stat_indices(n)
    max_k = math.ceil(math.log(n) / math.log(1.1))
    want = sorted({min(int(1.1 ** k) - 1, n - 1) for k in range(max_k + 1)})
    assert sorted(set(idx.tolist())) == want
    assert idx.dtype.kind == "i" and idx.max() <= n - 1 and idx.min() >= 0


def test_batch_plan_places_every_statistic(oracle_mod):
    """The cached batch plan of a mixed list (empty and one-element tensors
    among others): selecting its ranks from each tensor's np.sort and reading
    its large / small positions gives the oracle's statistics per tensor."""
    from adana_amd.tau_stats import _batch_plan

    rng = np.random.default_rng(5)
    sizes = (5, 0, 1000, 1, 77, 1000, 65537)
    xs = [rng.normal(0, 1, n).astype(np.float32) for n in sizes]
    numel, ranks, rank_first, large, small, out_first = _batch_plan(sizes)
    assert _batch_plan(sizes)[1] is ranks                      # cached per size list
    assert list(numel) == list(sizes) and rank_first[0] == 0 and rank_first[-1] == ranks.size
    values = np.concatenate([np.sort(x)[ranks[a:b]] for x, a, b in zip(xs, rank_first[:-1], rank_first[1:])])
    vl, vs = values[large], values[small]
    for x, a, b in zip(xs, out_first[:-1], out_first[1:]):
        wl, ws = oracle_mod.tau_order_statistics(x)
        assert np.array_equal(vl[a:b], wl) and np.array_equal(vs[a:b], ws)


def test_order_values_rejects_cpu_tensors():
    from adana_amd.tau_stats import order_values

    with pytest.raises(RuntimeError, match="ROCm"):
        order_values([torch.zeros(4)], [np.array([0])])
    assert order_values([], []) == []


def test_order_stats_library_validates_before_device_work():
    """adana_order_stats checks every size and rank before it touches the
    device (fake device pointers here): ranks outside a tensor, negative
    sizes, and tensors of 2^32 or more elements (its histogram bins are
    32-bit counters) are refused."""
    import ctypes

    from adana_amd import _lib

    L = _lib.lib()
    fake = (ctypes.c_void_p * 1)(0x1000)
    vals = (ctypes.c_float * 2)()

    def call(numel, ranks):
        nm = (ctypes.c_int64 * 1)(numel)
        rk = (ctypes.c_int64 * len(ranks))(*ranks)
        rf = (ctypes.c_int64 * 2)(0, len(ranks))
        return L.adana_order_stats(fake, nm, 1, rk, rf, vals, None, 0, None)

    assert call(10, [10]) == -1 and "outside tensor" in _lib.last_error()
    assert call(-1, []) == -1 and "bad sizes" in _lib.last_error()
    assert call(1 << 32, [0]) == -3 and "2^32" in _lib.last_error()          # ADANA_E_UNSUPPORTED
    assert call(10, [3]) == -1 and "workspace" in _lib.last_error()
    assert L.adana_order_stats_workspace(1, 2) > L.adana_order_stats_workspace(1, 1) > 0
    # the compacting workspace: the plain one plus 32 rows of 256 values, 256
    # counts and a word per 65,536-element tile of every tensor with ranks
    nm = (ctypes.c_int64 * 2)(1 << 20, 5)
    rf = (ctypes.c_int64 * 3)(0, 2, 2)
    plain = L.adana_order_stats_workspace(2, 2)
    assert L.adana_order_stats_workspace_compact(nm, rf, 2) >= plain + 16 * (32 * 256 * 4 + 256 + 4)
    bad = (ctypes.c_int64 * 3)(0, 2, 1)
    assert L.adana_order_stats_workspace_compact(nm, bad, 2) == 0


def test_index_formula_fails_past_2_31_elements_as_the_reference():
    """src/optim/tau_stats_collector.py:360-366 casts 1.1^k to int32 and
    clamps with n - 1; for a tensor of more than 2^31 elements numpy 2
    refuses that clamp.  The restatement keeps the reference's behaviour
    (the GPU select itself handles such tensors: order_values with int64
    ranks, tests/test_gpu_tau_stats.py)."""
    import warnings

    from adana_amd.tau_stats import order_stat_indices

    with warnings.catch_warnings():
        warnings.simplefilter("ignore", RuntimeWarning)   # the int32 cast's "invalid value"
        with pytest.raises(OverflowError):
            order_stat_indices((1 << 31) + 1027)
        assert order_stat_indices((1 << 31) - 1)[-1] == (1 << 31) - 2   # still fine below
