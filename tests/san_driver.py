"""Drives the host code under the sanitizers: the step-table extension
(adana_amd/csrc/hoststep.cpp) and the host functions of the kernel library
(adana_amd/csrc/adana_mta.hip).  tests/test_sanitizers_cpu.py builds
instrumented copies of both and runs this file in a child process with the
matching sanitizer runtime preloaded:

    python tests/san_driver.py hoststep <dir holding the instrumented _hoststep*.so>
    python tests/san_driver.py mta <instrumented libadana_mta.so>

Every check here is an assert (a failure exits non-zero); the sanitizers stop
the process on their own findings.  CPU tensors only: no GPU is needed."""
import ctypes
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _rows(rng, torch, n, dtype):
    params = [torch.nn.Parameter(torch.randn(int(rng.integers(1, 6)), 2, dtype=dtype)) for _ in range(n)]
    for p in params:
        p.grad = torch.randn_like(p)
    return params, [{"step": 3} for _ in params]


def hoststep(ext_dir: str) -> None:
    sys.path.insert(0, ext_dir)
    import numpy as np
    import torch
    import _hoststep as H
    assert os.path.dirname(os.path.abspath(H.__file__)) == os.path.abspath(ext_dir), H.__file__

    rng = np.random.default_rng(0)
    cols = [(0, "current_alpha"), (1, "gradient_norm"), (3, "current_kappa_factor")]
    for helpers in (0, 3):
        assert 0 <= H.scan_threads(helpers) <= 8
        for n in (0, 1, 7, 2600):
            for dtype, bf16 in ((torch.float32, False), (torch.bfloat16, True)):
                params, states = _rows(rng, torch, n, dtype)
                idle = torch.nn.Parameter(torch.zeros(3))
                t = H.step_table(params, states, [idle], bf16)
                out = np.zeros(max(n, 1), np.uint64)
                assert t.scan(out.ctypes.data) == ((0, n) if n else (0, 0))
                assert t.scan(out.ctypes.data) == (0, 0)
                assert t.grads_are([p.grad for p in params])
                if n:
                    params[n - 1].grad = torch.zeros_like(params[n - 1])
                    assert t.scan(out.ctypes.data) == (n - 1, n)
                    assert out[n - 1] == params[n - 1].grad.data_ptr()
                    t.forget()
                    assert t.scan(out.ctypes.data) == (0, n)
                    assert all(st["step"] == 7 for st in states)
                    # a row that does not fit, a missing counter, counters of other types
                    keep = params[n // 2].grad
                    params[n // 2].grad = None
                    assert t.scan(out.ctypes.data) is None
                    params[n // 2].grad = keep
                    del states[0]["step"]
                    try:
                        t.scan(out.ctypes.data)
                        raise AssertionError("missing step counter accepted")
                    except KeyError:
                        pass
                    states[0]["step"] = 7.0
                    assert t.scan(out.ctypes.data) == (0, 0)
                    assert states[0]["step"] == 8.0 and states[-1]["step"] == 8
                    idle.grad = torch.zeros(3)
                    assert t.scan(out.ctypes.data) is None
                    idle.grad = None
                # diagnostics bound into the states, one held elsewhere, one dropped
                buf = torch.arange(5 * max(n, 1), dtype=torch.float32)
                t.diag_bind(buf, cols)
                if n:
                    kept = states[n - 1]["gradient_norm"]
                    del states[0]["current_alpha"]
                    held, lost = t.diag_check()
                    assert (n - 1) * len(cols) + 1 in held and 0 in lost, (held, lost)
                    flat = [(k // len(cols)) * 5 + cols[k % len(cols)][0] for k in held]
                    copy = buf.index_select(0, torch.tensor(flat, dtype=torch.int64))
                    t.diag_rehome(held, copy, lost, buf)
                    assert float(kept) == float(buf[5 * (n - 1) + 1])
                    assert t.diag_check() == ([], [])
                    del kept
                    # the same lists taken by the scan itself (helpers on long plans)
                    kept = states[n // 2]["current_alpha"]
                    view = states[n - 1]["current_kappa_factor"].detach()
                    states[n // 3]["gradient_norm"] = torch.zeros(())
                    want = t.diag_check()
                    got = t.scan(out.ctypes.data, True)
                    assert got is not None and (got[2], got[3]) == want, (got, want)
                    assert t.scan(out.ctypes.data, False) == (0, 0)
                    del view, kept
                del t
    H.scan_threads(3)

    # the module's other entry points
    params, states = _rows(rng, torch, 40, torch.float32)
    grads = [p.grad for p in params]
    got, absent = H.grads_of(params)
    assert got == grads and absent == bytes(40)
    assert H.grads_match(params, grads, False) and not H.grads_match(params, grads, True)
    g2, absent2, gp, pp, match = H.grads_scan(params, False)
    assert g2 == grads and match and len(gp) == len(pp) == 8 * 40
    assert np.frombuffer(H.data_ptrs(grads + [None]), np.uint64)[-1] == 0
    v0 = [p._version for p in params]
    H.bump_versions(params)
    assert [p._version for p in params] == [v + 1 for v in v0]
    assert H.advance_if_same(params, grads, states, pp, gp)
    assert all(st["step"] == 4 for st in states)
    params[3].grad = torch.zeros_like(params[3])
    assert not H.advance_if_same(params, grads, states)
    H.advance_steps(states)
    assert all(st["step"] == 5 for st in states)
    buf = torch.zeros(5 * 40)
    H.bind_diag(buf, states, cols)
    assert states[39]["current_kappa_factor"].data_ptr() == buf.data_ptr() + 4 * (5 * 39 + 3)
    groups = [{"params": params[:10]}, {"params": params[10:]}]
    assert H.same_params(groups, params) and not H.same_params(groups, params[::-1])
    print("hoststep: ok")


def mta(libpath: str) -> None:
    sys.path.insert(0, ROOT)
    from adana_amd import _lib

    L = ctypes.CDLL(libpath)
    _lib._declare(L)
    assert L.adana_abi_version() == _lib.ABI_VERSION

    # scalars over the hyperparameter cases the optimizers meet
    sc = _lib.StepScalars()
    for kappa in (0.0, 0.5, 0.85, 1.0, 2.0, -3.0):
        for eager in (0, 1):
            for has_clip, wd_decaying in ((0, 0), (1, 1)):
                hp = _lib.HParams(peak_lr=1e-3, delta=8.0, kappa=kappa, epsilon=1e-8, weight_decay=0.4,
                                  clipsnr=2.0, wd_ts=10.0, gamma_3_factor=1.0, has_clip=has_clip,
                                  wd_decaying=wd_decaying, eager=eager)
                for step in (1, 2, 1000, 1 << 40):
                    assert L.adana_step_scalars_init(ctypes.byref(sc), ctypes.byref(hp), 1e-3, step) == 0
    assert L.adana_step_scalars_init(None, None, 1e-3, 1) != 0
    ms = _lib.ManauScalars()
    mh = _lib.ManauHParams(delta=8.0, kappa=0.85, mk4A=0.0, mk4B=0.0, clipsnr=2.0, epsilon=1e-8,
                           weight_decay=0.1, wd_ts=10.0, wd_decaying=1)
    for step in (1.0, 7.5, 1e6):
        assert L.adana_manau_scalars_init(ctypes.byref(ms), ctypes.byref(mh), 2e-3, step, 0.5) == 0

    # layouts: empty, tiny, chunk edges, many tensors, a tensor past 2^31 elements, bad input
    i64 = ctypes.c_int64
    for numel in ([], [0], [1], [1023, 1024, 1025, 0, 7], [3] * 3000, [(1 << 31) + 5, 1 << 20]):
        n = len(numel)
        nm = (i64 * max(n, 1))(*numel)
        vstart = (i64 * (n + 1))()
        fold_first = (ctypes.c_int32 * (n + 1))()
        n_folds = i64(-1)
        chunks = L.adana_plan_layout(nm, n, vstart, fold_first, ctypes.byref(n_folds))
        assert chunks >= 0 and n_folds.value >= 0 and vstart[n] >= sum(numel)
        plan = _lib.Plan(n_tensors=n, n_chunks=chunks, n_folds=n_folds.value)
        assert L.adana_workspace_bytes(ctypes.byref(plan)) >= 0
    bad = (i64 * 2)(5, -1)
    assert L.adana_plan_layout(bad, 2, (i64 * 3)(), (ctypes.c_int32 * 3)(), ctypes.byref(i64())) < 0
    assert L.adana_plan_layout(None, 2, None, None, None) < 0
    assert L.adana_order_stats_workspace(194, 1 << 20) > 0
    rf = (i64 * 3)(0, 5, 12)
    assert L.adana_order_stats_workspace_compact((i64 * 2)(5, 7), rf, 2) > 0

    # the step entry points' argument checks (they return before any device call)
    plan = _lib.Plan(n_tensors=1, n_chunks=1, n_folds=0)
    scs = (_lib.StepScalars * 2)()
    assert L.adana_mta_step(None, scs, 1, 0, None, 0, None, None) != 0
    assert L.adana_mta_step(ctypes.byref(plan), scs, 1, 1 << 30, None, 0, None, None) != 0
    assert L.adana_mta_step(ctypes.byref(plan), scs, 0, 0, None, 0, None, None) != 0
    assert L.adana_mta_step_scaled(ctypes.byref(plan), scs, 1, 0, None, None, 0, None, None) != 0
    assert L.adana_mta_step_noalloc(ctypes.byref(plan), scs, 1, 0, None, None) != 0
    empty = _lib.Plan(n_tensors=0, n_chunks=0, n_folds=0)
    assert L.adana_grad_scale(None, 0, None, None) != 0
    assert L.adana_plan_index(None, -1, 0, None, None) != 0
    del empty
    # the last error message: whole, truncated, and into no buffer
    for size in (512, 9, 1):
        buf = ctypes.create_string_buffer(size)
        need = L.adana_last_error(buf, size)
        assert need > 0 and len(buf.value) == min(need, size - 1)
    assert L.adana_last_error(None, 0) > 0
    print("mta host: ok")


if __name__ == "__main__":
    {"hoststep": hoststep, "mta": mta}[sys.argv[1]](sys.argv[2])
