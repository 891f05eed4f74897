"""StepTable.scan, the step's one-pass host bookkeeping (adana_amd/csrc/hoststep.cpp),
on CPU tensors: the same results from the calling thread alone and with helper
threads, and nothing modified when a row does not fit or a step counter cannot
be advanced.

The scan restates the reference's per-parameter walk (src/optim/adana.py:184-197,
src/optim/dana_star_mk4.py:243-262): skip parameters without a gradient,
``state['step'] += 1``, and the in-place update that bumps each parameter's
version counter."""
import multiprocessing as mp
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from adana_amd import _hoststep

N = 5000          # long enough for the helper threads (2048 rows and more)


def _rows(n, seed=0, dtype=torch.float32):
    rng = np.random.default_rng(seed)
    params = [torch.nn.Parameter(torch.zeros(int(rng.integers(1, 9)), 3, dtype=dtype)) for _ in range(n)]
    for p in params:
        p.grad = torch.zeros_like(p)
    states = [{"step": 7, "m": None} for _ in params]
    return params, states


@pytest.fixture(params=[0, 3], ids=["calling_thread", "helpers3"])
def threads(request):
    before = _hoststep.scan_threads(request.param)
    yield request.param
    _hoststep.scan_threads(before)


def _scan(table, out):
    return table.scan(out.ctypes.data)


def test_scan_gathers_counts_and_bumps(threads):
    params, states = _rows(N)
    table = _hoststep.step_table(params, states, [], False)
    out = np.zeros(N, np.uint64)
    v0 = [p._version for p in params]
    assert _scan(table, out) == (0, N)                       # every pointer is new to the table
    assert list(out) == [p.grad.data_ptr() for p in params]
    assert all(st["step"] == 8 and type(st["step"]) is int for st in states)
    assert [p._version for p in params] == [v + 1 for v in v0]
    assert _scan(table, out) == (0, 0)                       # nothing moved
    assert all(st["step"] == 9 for st in states)
    for i in (100, 4000):
        params[i].grad = torch.ones_like(params[i])
    assert _scan(table, out) == (100, 4001)
    assert out[100] == params[100].grad.data_ptr() and out[4000] == params[4000].grad.data_ptr()
    table.forget()
    assert _scan(table, out) == (0, N)
    assert [p._version for p in params] == [v + 4 for v in v0]


def _break_row(kind, params, i):
    p = params[i]
    if kind == "dtype":
        p.grad_dtype = None                       # torch checks gradient dtypes unless told not to
        p.grad = torch.zeros_like(p, dtype=torch.float64)
    elif kind == "none":
        p.grad = None
    elif kind == "shape":                         # torch refuses such a p.grad; set_ reshapes it in place
        p.grad.set_(torch.zeros(p.shape[0] + 1, 3))
    elif kind == "strides":
        p.grad = torch.zeros(3, p.shape[0]).t() if p.shape[0] > 1 else torch.zeros(5, 3)
    elif kind == "param_storage":
        p.data = torch.zeros_like(p)


@pytest.mark.parametrize("kind", ["dtype", "none", "shape", "strides", "param_storage"])
@pytest.mark.parametrize("row", [0, 2600, N - 1])
def test_scan_rejects_with_nothing_modified(threads, kind, row):
    params, states = _rows(N, seed=row)
    if kind == "strides":
        params[row] = torch.nn.Parameter(torch.zeros(4, 3))
        params[row].grad = torch.zeros(4, 3)
    table = _hoststep.step_table(params, states, [], False)
    out = np.zeros(N, np.uint64)
    assert _scan(table, out) == (0, N)
    _break_row(kind, params, row)
    before_out = out.copy()
    v0 = [p._version for p in params]
    assert _scan(table, out) is None
    assert all(st["step"] == 8 for st in states)
    assert [p._version for p in params] == v0
    assert np.array_equal(out, before_out)


def test_scan_rejects_new_gradient_on_inactive(threads):
    params, states = _rows(N)
    idle = torch.nn.Parameter(torch.zeros(2))
    table = _hoststep.step_table(params, states, [idle], False)
    out = np.zeros(N, np.uint64)
    assert _scan(table, out) == (0, N)
    idle.grad = torch.zeros(2)
    assert _scan(table, out) is None
    assert all(st["step"] == 8 for st in states)


@pytest.mark.parametrize("row", [0, 3000, N - 1])
def test_scan_missing_counter_rolls_back(threads, row):
    params, states = _rows(N)
    table = _hoststep.step_table(params, states, [], False)
    out = np.zeros(N, np.uint64)
    del states[row]["step"]
    v0 = [p._version for p in params]
    with pytest.raises(KeyError):
        _scan(table, out)
    assert all(st["step"] == 7 for j, st in enumerate(states) if j != row)
    assert "step" not in states[row]
    assert [p._version for p in params] == v0


def test_scan_counts_of_other_types(threads):
    """Counts that are not exact ints (a float, an int subclass) advance like
    the reference's ``state['step'] += 1``."""
    class Count(int):
        def __add__(self, other):
            return Count(int(self) + other)

    params, states = _rows(N)
    states[1]["step"] = 2.5
    states[2500]["step"] = Count(40)
    table = _hoststep.step_table(params, states, [], False)
    out = np.zeros(N, np.uint64)
    assert _scan(table, out) == (0, N)
    assert states[1]["step"] == 3.5 and states[2500]["step"] == 41 and type(states[2500]["step"]) is Count
    assert states[0]["step"] == 8 and states[N - 1]["step"] == 8
    # a failing row still rolls every count back, whatever its type
    params[4999].grad = None
    assert _scan(table, out) is None
    assert states[1]["step"] == 3.5 and states[2500]["step"] == 41 and states[0]["step"] == 8


def test_scan_threads_setting():
    before = _hoststep.scan_threads()
    try:
        assert _hoststep.scan_threads(5) == before
        assert _hoststep.scan_threads() == 5
        with pytest.raises(ValueError):
            _hoststep.scan_threads(9)
        with pytest.raises(ValueError):
            _hoststep.scan_threads(-2)
        assert _hoststep.scan_threads() == 5
    finally:
        _hoststep.scan_threads(before)


def test_scan_threads_default_follows_the_cpus():
    """At import the helper count is the CPUs the process may run on, less
    two, within [0, 8] (checked in a fresh interpreter, whose value no other
    test has changed)."""
    code = ("import os, torch; from adana_amd import _hoststep; "
            "print(_hoststep.scan_threads(), min(8, max(0, len(os.sched_getaffinity(0)) - 2)))")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    out = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    got, want = map(int, out.stdout.split())
    assert got == want


def _child_scan(q):
    params, states = _rows(N, seed=3)
    table = _hoststep.step_table(params, states, [], False)
    out = np.zeros(N, np.uint64)
    span = table.scan(out.ctypes.data)
    q.put((span, all(st["step"] == 8 for st in states)))


@pytest.mark.skipif(not hasattr(os, "fork"), reason="fork() only")
def test_scan_after_fork():
    """A process forked after the helper threads started gets a pool of its own
    (the parent's threads do not exist in the child)."""
    before = _hoststep.scan_threads(3)
    try:
        params, states = _rows(N)
        table = _hoststep.step_table(params, states, [], False)
        assert table.scan(np.zeros(N, np.uint64).ctypes.data) == (0, N)     # helpers running
        ctx = mp.get_context("fork")
        q = ctx.Queue()
        child = ctx.Process(target=_child_scan, args=(q,))
        child.start()
        child.join(60)
        assert child.exitcode == 0
        assert q.get(timeout=5) == ((0, N), True)
    finally:
        _hoststep.scan_threads(before)


def test_scan_reentered_from_a_step_counter(threads):
    """A step counter whose ``+ 1`` runs Python code that scans again: the same
    table declines (None, the caller's general path), another table scans on
    the calling thread (the helpers are serving the outer scan), and the
    outer scan completes."""
    params, states = _rows(N)
    other_params, other_states = _rows(3000, seed=9)
    table = _hoststep.step_table(params, states, [], False)
    other = _hoststep.step_table(other_params, other_states, [], False)
    seen = []

    class Count(int):
        def __add__(self, k):
            seen.append(table.scan(np.zeros(N, np.uint64).ctypes.data))
            seen.append(other.scan(np.zeros(3000, np.uint64).ctypes.data))
            return Count(int(self) + k)

    states[N // 2]["step"] = Count(7)
    out = np.zeros(N, np.uint64)
    assert _scan(table, out) == (0, N)
    assert seen == [None, (0, 3000)]
    assert states[N // 2]["step"] == 8 and type(states[N // 2]["step"]) is Count
    assert all(st["step"] == 8 for st in states) and all(st["step"] == 8 for st in other_states)
    assert _scan(table, out) == (0, 0)                # and the table scans again afterwards
