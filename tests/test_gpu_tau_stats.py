"""GPU parity of the tau order statistics (adana_order_stats through
adana_amd.tau_stats) against the oracle's np.sort-based restatement of
compute_tau_order_statistics (src/optim/tau_stats_collector.py:336-376):
bit-identical float32 values (NaN equal to NaN; -0 and +0 equal as values,
as np.sort ranks them), for value distributions and sizes that exercise every
pass width, and for a real DANA_STAR_MK4 state through
extract_tau_statistics (:131-160)."""
import time

import numpy as np
import pytest
import torch

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"


def _same(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return a.shape == b.shape and bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


def _cases(rng):
    out = []
    for n in (1, 2, 3, 17, 1000, 16384, 16385, 100_003):
        out.append((f"uniform{n}", rng.random(n).astype(np.float32)))
    out.append(("tau_like", np.clip(rng.beta(2, 5, 300_000), 0, 1).astype(np.float32)))
    out.append(("dups", (rng.integers(0, 7, 200_000) / 8).astype(np.float32)))
    out.append(("constant", np.full(50_000, 0.25, np.float32)))
    x = rng.normal(0, 1, 123_457).astype(np.float32)
    x[::97] = np.nan
    x[1::101] = 0.0
    x[2::103] = -0.0
    x[3::107] = np.inf
    x[4::109] = -np.inf
    x[5::113] = 1e-42                                   # denormals
    out.append(("special", x))
    out.append(("wide", (10.0 ** rng.uniform(-30, 30, 200_000)).astype(np.float32)))
    return out


def test_order_statistics_match_oracle(oracle_mod):
    from adana_amd.tau_stats import _stats_for

    rng = np.random.default_rng(3)
    cases = _cases(rng)
    print("case: order statistics,", len(cases), "tensors in one batch", flush=True)
    tensors = [torch.from_numpy(x).to(DEV) for _, x in cases]
    got = _stats_for(tensors)
    for (name, x), (gl, gs) in zip(cases, got):
        wl, ws = oracle_mod.tau_order_statistics(x)
        assert _same(gl, wl) and _same(gs, ws), name
        assert gl.dtype == np.float32


def test_ranks_in_any_order():
    """order_values takes each tensor's ranks in any order, repeats included:
    the values equal np.sort(x)[ranks] position by position (shuffled ranks
    take the library's sorting path, ascending ones its linear scan)."""
    from adana_amd.tau_stats import order_values

    rng = np.random.default_rng(11)
    print("case: order_values with shuffled and repeated ranks", flush=True)
    xs = [rng.normal(0, 1, 300_001).astype(np.float32), np.clip(rng.beta(2, 5, 70_000), 0, 1).astype(np.float32),
          (rng.integers(0, 5, 40_000) / 4).astype(np.float32)]
    ranks = []
    for x in xs:
        r = np.unique(np.concatenate([np.int64(1.1 ** np.arange(120)) - 1, rng.integers(0, x.size, 300)]))
        r = r[r < x.size]
        ranks.append(r)
    shuffled = [rng.permutation(np.concatenate([r, r[:17]])) for r in ranks]
    tensors = [torch.from_numpy(x).to(DEV) for x in xs]
    for rs in (ranks, shuffled):
        got = order_values(tensors, rs)
        for x, r, g in zip(xs, rs, got):
            assert _same(g, np.sort(x)[r])


def test_many_ranks_in_one_tensor():
    """3,000 ranks of one tensor of distinct values: the late passes hold
    3,000 active prefixes, so the digits narrow to 1 bit past the LDS budget
    and the prefix lookup falls back to the binary search (tables too large);
    a second tensor with 600 ranks uses the cuckoo tables in the same passes."""
    from adana_amd.tau_stats import order_values

    rng = np.random.default_rng(13)
    print("case: 3000 and 600 ranks per tensor", flush=True)
    xs = [rng.permutation(np.arange(200_000, dtype=np.float32) * np.float32(0.5) - 7),
          rng.normal(0, 1, 150_000).astype(np.float32)]
    ranks = [np.sort(rng.choice(x.size, k, replace=False)) for x, k in zip(xs, (3000, 600))]
    got = order_values([torch.from_numpy(x).to(DEV) for x in xs], ranks)
    for x, r, g in zip(xs, ranks, got):
        assert _same(g, np.sort(x)[r])


def test_unaligned_and_empty_tensors(oracle_mod):
    import adana_amd

    print("case: order statistics unaligned/empty", flush=True)
    base = torch.rand(10_001, device=DEV)
    view = base[1:]                                     # 4-byte offset: element-wise loads
    wl, ws = oracle_mod.tau_order_statistics(view.cpu().numpy())
    gl, gs = adana_amd.compute_tau_order_statistics(view)
    assert _same(gl, wl) and _same(gs, ws)
    e = adana_amd.compute_tau_order_statistics(torch.zeros(0, device=DEV))
    assert e[0].size == 0 and e[1].size == 0


def test_extract_tau_statistics_from_optimizer(oracle_mod):
    import adana_amd

    print("case: extract_tau_statistics", flush=True)
    torch.manual_seed(0)
    shapes = [(256, 64), (64,), (1000, 33), (5,)]
    for named in (True, False):
        params = [torch.nn.Parameter(torch.randn(s, device=DEV) * 0.02) for s in shapes]
        if named:     # src/main.py:367 adds param_names to every group
            groups = [{"params": params[:2], "param_names": ["w0", "b0"]},
                      {"params": params[2:], "param_names": ["w1", "b1"]}]
        else:
            groups = [{"params": params[:2]}, {"params": params[2:]}]
        opt = adana_amd.DANA_STAR_MK4(groups, lr=1e-3, kappa=0.85)
        for _ in range(5):
            for p in params:
                p.grad = torch.randn_like(p) * 1e-3
            opt.step()
        stats = adana_amd.extract_tau_statistics(opt)
        g0, g1 = opt.param_groups
        names = (["w0", "b0", "w1", "b1"] if named else
                 [f"param_group_{id(g)}_idx_{i}" for g in (g0, g1) for i in range(2)])
        assert list(stats) == names
        for name, p in zip(names, params):
            tau = opt.state[p]["tau"]
            wl, ws = oracle_mod.tau_order_statistics(tau.cpu().numpy())
            e = stats[name]
            assert e["shape"] == tuple(tau.shape) and e["num_elements"] == tau.numel()
            assert _same(e["largest_order_stats"], wl) and _same(e["smallest_order_stats"], ws), name


def test_large_tensor_timing(oracle_mod):
    """A 64M-element tau-like tensor: equal to the oracle; prints the GPU
    selection time and the host path's (copy + np.sort) time."""
    import adana_amd

    print("case: order statistics 64M", flush=True)
    n = 1 << 26
    t = torch.rand(n, device=DEV).pow_(2)
    adana_amd.compute_tau_order_statistics(t[:100_000])    # warm-up
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gl, gs = adana_amd.compute_tau_order_statistics(t)
    t1 = time.perf_counter()
    x = t.cpu().numpy()
    wl, ws = oracle_mod.tau_order_statistics(x)
    t2 = time.perf_counter()
    assert _same(gl, wl) and _same(gs, ws)
    print(f"64M elements: GPU select {1e3 * (t1 - t0):.1f} ms, copy + np.sort {1e3 * (t2 - t1):.1f} ms", flush=True)


def test_order_stats_beyond_2_31_elements():
    """A tensor of 2^31 + 1027 values x[i] = i mod 2^24 (exact in float32):
    value v occurs 129 times for v < 1027 and 128 times otherwise, so the
    value at every rank, including ranks past 2^31, has a closed form.  The
    reference's index set is int32 and cannot address this tensor (its
    formula raises there, see test_tau_stats_cpu.py), so the ranks are the
    same positions 1.1^k - 1 from both ends, computed in int64, through
    order_values."""
    from adana_amd.tau_stats import order_values

    n, M, extra = (1 << 31) + 1027, 1 << 24, 1027
    print(f"case: order statistics of {n} values", flush=True)
    x = torch.empty(n, dtype=torch.float32, device=DEV)
    block = 1 << 27
    for a in range(0, n, block):
        b = min(n, a + block)
        x[a:b] = (torch.arange(a, b, dtype=torch.int64, device=DEV) % M).to(torch.float32)

    def value_at(r):
        r = np.asarray(r, dtype=np.int64)
        head = extra * 129
        return np.where(r < head, r // 129, extra + (r - head) // 128).astype(np.float32)

    max_k = int(np.ceil(np.log(n) / np.log(1.1)))
    idx = np.minimum(np.unique((1.1 ** np.arange(max_k + 1)).astype(np.int64) - 1), n - 1)
    ranks = np.unique(np.concatenate([idx, (n - 1) - idx]))
    assert ranks.max() > (1 << 31) and ranks.min() == 0
    (vals,) = order_values([x], [ranks])
    assert np.array_equal(vals, value_at(ranks))
    assert vals[-1] == M - 1
    del x
    torch.cuda.empty_cache()


def _select_raw(xs, ranks, compact):
    """adana_order_stats through ctypes with a zeroed workspace (of the
    compacting size when ``compact``): the values, and the per-tile words
    the compaction wrote (the last block of that workspace: one word per
    65,536-element tile, rows kept or 0x80000000 for a tile read whole)."""
    import ctypes

    from adana_amd import _hoststep, _lib

    L = _lib.lib()
    flat = [torch.from_numpy(x).to(DEV) if isinstance(x, np.ndarray) else x for x in xs]
    numel = np.array([f.numel() for f in flat], np.int64)
    rank_first = np.zeros(len(flat) + 1, np.int64)
    np.cumsum([r.size for r in ranks], out=rank_first[1:])
    rk = np.concatenate(ranks).astype(np.int64)
    ptrs = np.frombuffer(_hoststep.data_ptrs(flat), dtype=np.uint64)
    P = ctypes.c_void_p
    if compact:
        nbytes = L.adana_order_stats_workspace_compact(P(numel.ctypes.data), P(rank_first.ctypes.data), len(flat))
    else:
        nbytes = L.adana_order_stats_workspace(len(flat), int(rank_first[-1]))
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
    vals = np.empty(rk.size, np.float32)
    rc = L.adana_order_stats(P(ptrs.ctypes.data), P(numel.ctypes.data), len(flat), P(rk.ctypes.data),
                             P(rank_first.ctypes.data), P(vals.ctypes.data), P(ws.data_ptr()), nbytes,
                             P(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "adana_order_stats")
    tiles = int(sum((n + 65535) // 65536 for n, a, b in zip(numel, rank_first[:-1], rank_first[1:]) if b > a))
    meta_bytes = (4 * tiles + 255) // 256 * 256
    meta = ws[nbytes - meta_bytes:nbytes - meta_bytes + 4 * tiles].cpu().numpy().view(np.uint32) if compact else None
    return [vals[a:b] for a, b in zip(rank_first[:-1], rank_first[1:])], meta


def test_compaction_gives_the_same_values():
    """Late passes over compacted values (the larger workspace) against the
    plain passes and np.sort: a uniform tensor, whose active prefixes soon
    hold few values (every tile compacted, none overflowing); a sorted one,
    whose matching values crowd into a few tiles (threads there overflow their
    32 rows, so those tiles are read whole); an unaligned view; a tensor of
    mostly equal values (never compacted); and a tiny one, in one batch."""
    from adana_amd.tau_stats import _rank_plan

    rng = np.random.default_rng(17)
    print("case: order statistics with and without compaction", flush=True)
    base = rng.random(3_000_001).astype(np.float32)
    mostly_equal = np.zeros(400_000, np.float32)
    mostly_equal[::50] = rng.random(8_000).astype(np.float32)
    xs = [rng.random(2_500_000).astype(np.float32), np.sort(rng.random(2_000_000).astype(np.float32)),
          torch.from_numpy(base).to(DEV)[1:], mostly_equal, rng.random(100).astype(np.float32)]
    hosts = [x if isinstance(x, np.ndarray) else base[1:] for x in xs]
    ranks = [_rank_plan(h.size)[0] for h in hosts]
    got_c, meta = _select_raw(xs, ranks, True)
    got_p, _ = _select_raw(xs, ranks, False)
    for h, r, gc, gp in zip(hosts, ranks, got_c, got_p):
        want = np.sort(h)[r]
        assert _same(gc, want) and _same(gp, want)
    tiles = [(h.size + 65535) // 65536 for h in hosts]
    first = np.concatenate([[0], np.cumsum(tiles)])
    m = [meta[a:b] for a, b in zip(first[:-1], first[1:])]
    assert np.all((m[0] > 0) & (m[0] < 0x80000000)), "uniform: every tile compacted, none overflowing"
    assert np.any(m[1] == 0x80000000) and np.any((m[1] > 0) & (m[1] < 0x80000000)), "sorted: both kinds of tile"
    assert np.all(m[2] != 0), "unaligned view compacted"
    assert np.all(m[3] == 0), "mostly equal values: never compacted"


def test_compaction_with_special_values_and_shuffled_ranks():
    """Compaction on values with NaN, +-0, +-inf and denormals mixed in, and
    with ranks given out of order and repeated (the host's other slot path):
    the same values as np.sort and as the uncompacted passes, with every tile
    of both tensors compacted."""
    from adana_amd.tau_stats import _rank_plan

    rng = np.random.default_rng(19)
    print("case: compaction with special values and shuffled ranks", flush=True)
    x = rng.normal(0, 1, 2_000_000).astype(np.float32)
    x[::97] = np.nan
    x[1::101] = 0.0
    x[2::103] = -0.0
    x[3::107] = np.inf
    x[4::109] = -np.inf
    x[5::113] = 1e-42
    y = rng.random(1_500_000).astype(np.float32)
    ry = _rank_plan(y.size)[0]
    ry = rng.permutation(np.concatenate([ry, ry[:40]]))          # out of order, with repeats
    ranks = [_rank_plan(x.size)[0], ry]
    got_c, meta = _select_raw([x, y], ranks, True)
    got_p, _ = _select_raw([x, y], ranks, False)
    for h, r, gc, gp in zip((x, y), ranks, got_c, got_p):
        want = np.sort(h)[r]
        assert _same(gc, want) and _same(gp, want)
    tx = (x.size + 65535) // 65536
    assert np.all(meta[:tx] != 0), "special values: every tile compacted"
    assert np.all(meta[tx:] != 0), "shuffled ranks: every tile compacted"


def _random_values(rng, n):
    kind = int(rng.integers(7))
    if kind == 0:
        x = rng.random(n)
    elif kind == 1:
        x = rng.normal(0, float(10 ** rng.uniform(-3, 3)), n)
    elif kind == 2:
        x = 1.0 + rng.normal(0, 1e-6, n)                          # one narrow cluster
    elif kind == 3:
        x = rng.integers(0, int(rng.integers(1, 20)), n) / 7.0    # few distinct values
    elif kind == 4:
        x = rng.beta(2, 5, n)
    elif kind == 5:
        x = 10.0 ** rng.uniform(-40, 38, n) * rng.choice([-1.0, 1.0], n)
    else:
        x = np.sort(rng.random(n))                                 # sorted: values crowd into few tiles
    x = x.astype(np.float32)
    if n and rng.random() < 0.4:                                   # sprinkle special values
        for v in (np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-42, -1e-42):
            x[rng.integers(0, n, int(rng.integers(0, 4)))] = v
    return x


@pytest.mark.parametrize("seed", range(24))
def test_random_lists_and_ranks(seed):
    """Seeded random tensor lists (0 to 400,000 elements; uniform, normal,
    one narrow cluster, few distinct values, beta, 78 decades of both signs,
    sorted; NaN, infinities, signed zeros and denormals sprinkled in) and rank
    sets (sorted and distinct, or shuffled with repeats; up to 600 per
    tensor), with and without compaction: every value equals
    np.sort(x)[rank]."""
    from adana_amd import tau_stats

    rng = np.random.default_rng(5000 + seed)
    xs, ranks = [], []
    for _ in range(int(rng.integers(1, 11))):
        u = rng.random()
        n = 0 if u < 0.08 else int(rng.integers(1, 50)) if u < 0.3 else int(np.exp(rng.uniform(np.log(50), np.log(400_000))))
        xs.append(_random_values(rng, n))
        if n == 0:
            ranks.append(np.zeros(0, np.int64))
            continue
        k = int(rng.integers(1, min(n, 600) + 1))
        if rng.random() < 0.5:
            r = np.sort(rng.choice(n, k, replace=False))
        else:
            r = rng.integers(0, n, k)
        ranks.append(r.astype(np.int64))
    compact = bool(rng.integers(2))
    print(f"case: random order statistics seed {seed}: {len(xs)} tensors, sizes {[x.size for x in xs]}, "
          f"compact {compact}", flush=True)
    got = tau_stats.order_values([torch.from_numpy(x).to(DEV) for x in xs], ranks, compact=compact)
    for i, (x, r, g) in enumerate(zip(xs, ranks, got)):
        assert _same(g, np.sort(x)[r]), f"seed {seed} tensor {i} (n={x.size}, {r.size} ranks)"
