"""The C ABI driven directly, as a non-Python caller (or a plain ctypes
binding) would: plan layout, device table, chunk index, workspace,
one adana_mta_step per step -- against the oracle, bit-exact for m, v and
tau and under the Dana-Star pow bar for p; diagnostics rtol 1e-5."""
import ctypes
import os

import numpy as np
import pytest
import torch

from helpers import bf16_ulp_diff, ulp_diff
from test_gpu_parity import STAR_HARD_CASES

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def test_integration_example_through_the_c_abi(oracle_mod):
    from adana_amd import _lib

    print("case: raw C ABI, Dana-Star-MK4, 1M + 3 + 70000 elements", flush=True)
    O = oracle_mod
    L = _lib.lib()
    rng = np.random.default_rng(4)
    sizes = [1 << 20, 3, 70_000]
    p_np = [rng.normal(0, 0.02, n).astype(np.float32) for n in sizes]
    p = [torch.from_numpy(x.copy()).cuda() for x in p_np]
    m = [torch.zeros_like(x) for x in p]
    v = [torch.zeros_like(x) for x in p]
    tau = [torch.zeros_like(x) for x in p]
    g = [torch.empty_like(x) for x in p]

    numel = np.array(sizes, dtype=np.int64)
    vstart, fold_first, n_chunks, n_folds = _lib.plan_layout(numel)
    desc = np.zeros(len(sizes), _lib.DESC_DTYPE)
    for i in range(len(sizes)):
        desc[i] = (p[i].data_ptr(), 0, m[i].data_ptr(), v[i].data_ptr(), tau[i].data_ptr(), 0,
                   sizes[i], 0, _lib.DESC_VEC_OK)
    table = torch.from_numpy(np.concatenate([desc.view(np.uint8), vstart.view(np.uint8),
                                             fold_first.view(np.uint8)])).cuda()
    gtab = torch.tensor([x.data_ptr() for x in g], dtype=torch.int64, device="cuda")
    n = len(sizes)
    plan = _lib.Plan(desc=table.data_ptr(), grad=gtab.data_ptr(), vstart=table.data_ptr() + 64 * n,
                     fold_first=table.data_ptr() + 64 * n + 8 * (n + 1), n_tensors=n,
                     n_chunks=n_chunks, n_folds=n_folds)
    chunk_first = torch.empty(n_chunks, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.adana_plan_index(ctypes.c_void_p(plan.vstart), n, n_chunks,
                                  ctypes.c_void_p(chunk_first.data_ptr()), ctypes.c_void_p(stream)), "plan_index")
    plan.chunk_first = chunk_first.data_ptr()
    ws = torch.empty(_lib.workspace_bytes(plan), dtype=torch.uint8, device="cuda")
    diag = torch.empty(5 * n, device="cuda")
    hp = _lib.HParams(peak_lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=0.4, clipsnr=2.0,
                      wd_ts=10.0, gamma_3_factor=1.0, has_clip=1, wd_decaying=1)

    cpu = {k: [x.copy() if k == "p" else np.zeros_like(x) for x in p_np] for k in ("p", "m", "v", "tau")}
    for t in range(1, 6):
        g_np = [rng.normal(0, 1e-3, nn).astype(np.float32) for nn in sizes]
        for gi, x in zip(g, g_np):
            gi.copy_(torch.from_numpy(x))
        sc = (_lib.StepScalars * 1)(_lib.step_scalars(hp, 1e-3, t))
        _lib.check(L.adana_mta_step(ctypes.byref(plan), ctypes.cast(sc, ctypes.c_void_p), 1, _lib.VARIANT_STAR,
                                    ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(diag.data_ptr()),
                                    ctypes.c_void_p(stream)), "mta_step")
        osc = O.step_scalars(lr=1e-3, peak_lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=0.4,
                             clipsnr=2.0, wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0, t=t)
        sums = [O.element_step(True, cpu["p"][i], g_np[i], cpu["m"][i], cpu["v"][i], cpu["tau"][i], osc)
                for i in range(n)]
        torch.cuda.synchronize()
        d = diag.cpu().numpy().reshape(n, 5)
        for i in range(n):
            for key, arr in (("m", m), ("v", v), ("tau", tau)):
                assert ulp_diff(arr[i].cpu().numpy(), cpu[key][i]).max() == 0, (t, i, key)
            bad = int(np.count_nonzero(ulp_diff(p[i].cpu().numpy(), cpu["p"][i])))
            assert bad <= STAR_HARD_CASES, (t, i, bad)
            cpu["p"][i][...] = p[i].cpu().numpy()
            ref = O.finalize_diag(sums[i], sizes[i])
            np.testing.assert_allclose(d[i], [ref[k] for k in O.DIAG_KEYS], rtol=1e-5, atol=1e-30, equal_nan=True)


def test_cpp_host_drives_the_c_abi():
    """tests/c_abi_driver (C++, built by tests/Makefile): its own HIP
    allocations, adana_plan_layout / adana_plan_index / adana_workspace_bytes,
    then adana_mta_step for 6 Dana-Star-MK4 steps over 5 tensors, each step
    checked against the C oracle (m, v, tau bit-exact, p under the pow bar,
    diagnostics 1e-5).  Runs as a child process, with no Python in the step."""
    import subprocess

    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c_abi_driver")
    print("case: C++ host program over the C ABI", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout[-2000:], flush=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert r.stdout.strip().splitlines()[-1] == "c_abi_driver: ok"


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("kappas", [(0.85, 0.85), (0.85, 0.6)], ids=["one_exponent", "two_exponents"])
def test_bf16_state_classes_through_the_c_abi(oracle_mod, kappas, numerics):
    """bfloat16 state (ADANA_STATE_BF16) through the raw C ABI with two scalar
    classes, in both numerics.  Eager: one shared exponent takes the
    launch's pow table; two exponents (reachable only through the C ABI: the
    Python classes share one kappa) take the binary64 pow per element.
    Compiled: the binary32 update with the binary64 pow either way.  All
    bit-exact against the oracle's bfloat16 modes (Dana-Star p: the pow
    allowance), 12 steps so that tau * t passes 1 and alpha passes 0.5."""
    from adana_amd import _lib

    print("case: raw C ABI, bf16 state, kappas", kappas, numerics, flush=True)
    O = oracle_mod
    L = _lib.lib()
    rng = np.random.default_rng(11)
    sizes = [70_000, 4099, 1 << 16]
    cls = [0, 1, 0]
    p_h = [O.f32_to_bf16(rng.normal(0, 0.02, n).astype(np.float32)) for n in sizes]

    def dev(h):
        return torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).cuda()

    p = [dev(h) for h in p_h]
    m = [torch.zeros_like(x) for x in p]
    v = [torch.zeros_like(x) for x in p]
    tau = [torch.zeros_like(x) for x in p]
    g = [torch.empty_like(x) for x in p]
    n = len(sizes)
    vstart, fold_first, n_chunks, n_folds = _lib.plan_layout(np.array(sizes, dtype=np.int64))
    desc = np.zeros(n, _lib.DESC_DTYPE)
    for i in range(n):
        desc[i] = (p[i].data_ptr(), 0, m[i].data_ptr(), v[i].data_ptr(), tau[i].data_ptr(), 0,
                   sizes[i], cls[i], _lib.DESC_VEC_OK)
    table = torch.from_numpy(np.concatenate([desc.view(np.uint8), vstart.view(np.uint8),
                                             fold_first.view(np.uint8)])).cuda()
    gtab = torch.tensor([x.data_ptr() for x in g], dtype=torch.int64, device="cuda")
    plan = _lib.Plan(desc=table.data_ptr(), grad=gtab.data_ptr(), vstart=table.data_ptr() + 64 * n,
                     fold_first=table.data_ptr() + 64 * n + 8 * (n + 1), n_tensors=n,
                     n_chunks=n_chunks, n_folds=n_folds)
    chunk_first = torch.empty(n_chunks, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.adana_plan_index(ctypes.c_void_p(plan.vstart), n, n_chunks,
                                  ctypes.c_void_p(chunk_first.data_ptr()), ctypes.c_void_p(stream)), "plan_index")
    plan.chunk_first = chunk_first.data_ptr()
    ws = torch.empty(_lib.workspace_bytes(plan), dtype=torch.uint8, device="cuda")
    diag = torch.empty(5 * n, dtype=torch.bfloat16, device="cuda")
    kw = dict(peak_lr=1e-3, delta=8.0, epsilon=1e-8, weight_decay=0.4, clipsnr=2.0, wd_ts=10.0,
              gamma_3_factor=1.0)
    eager = numerics == "eager"
    hps = [_lib.HParams(kappa=k, has_clip=1, wd_decaying=1, eager=int(eager), **kw) for k in kappas]
    cpu = {"p": [h.copy() for h in p_h]}
    for key in ("m", "v", "tau"):
        cpu[key] = [np.zeros(nn, np.uint16) for nn in sizes]
    flags = _lib.VARIANT_STAR | _lib.GRAD_BF16 | _lib.STATE_BF16 | (_lib.NUMERICS_EAGER if eager else 0)
    for t in range(1, 13):
        g_h = [O.f32_to_bf16(rng.normal(0, 1e-3, nn).astype(np.float32)) for nn in sizes]
        for gi, h in zip(g, g_h):
            gi.copy_(dev(h))
        sc = (_lib.StepScalars * 2)(*[_lib.step_scalars(hp, 1e-3, t) for hp in hps])
        _lib.check(L.adana_mta_step(ctypes.byref(plan), ctypes.cast(sc, ctypes.c_void_p), 2, flags,
                                    ctypes.c_void_p(ws.data_ptr()), ws.numel(), ctypes.c_void_p(diag.data_ptr()),
                                    ctypes.c_void_p(stream)), "mta_step")
        for i in range(n):
            osc = O.step_scalars(lr=1e-3, kappa=kappas[cls[i]], wd_decaying=True, t=t, compiled=not eager, **kw)
            O.element_step(True, cpu["p"][i], g_h[i], cpu["m"][i], cpu["v"][i], cpu["tau"][i], osc)
        torch.cuda.synchronize()
        for i in range(n):
            for key, arr in (("m", m), ("v", v), ("tau", tau)):
                got = arr[i].cpu().view(torch.int16).numpy().view(np.uint16)
                assert np.array_equal(got, cpu[key][i]), (t, i, key)
            got = p[i].cpu().view(torch.int16).numpy().view(np.uint16)
            d = bf16_ulp_diff(got, cpu["p"][i])
            bad = int(np.count_nonzero(d))
            assert bad <= STAR_HARD_CASES and (bad == 0 or d.max() <= 1), (t, i, bad, d.max())
            cpu["p"][i][...] = got


def test_integration_example_runs(oracle_mod):
    """The ctypes example of the integration guide's section 2 runs as written against the built
    library (a plan with its gradient pointer array) and steps its tensor: the
    diagnostics are finite and match the oracle's over the same ten steps."""
    import contextlib
    import io
    import os
    import re

    O = oracle_mod
    print("case: integration guide ctypes example", flush=True)
    text = open(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "INTEGRATION.md")).read()
    section = text[text.index("## 2. C ABI"):]
    code = re.search(r"```python\n(.*?)```", section, re.S).group(1)
    ns = {}
    torch.manual_seed(0)
    with contextlib.redirect_stdout(io.StringIO()):
        exec(compile(code, "INTEGRATION.md", "exec"), ns)
    torch.cuda.synchronize()
    diag = ns["diag"].cpu().numpy()
    assert np.isfinite(diag).all(), diag
    # the same ten steps on the oracle, from the example's own inputs
    assert ns["p"].shape == (1 << 20,)
    g = ns["g"].cpu().numpy()
    torch.manual_seed(0)
    p0 = torch.randn(1 << 20, device="cuda").cpu().numpy()
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=[p0], lr=1e-3, weight_decay=0.4)], star=True, peak_lr=1e-3,
                            kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=10.0)
    for _ in range(10):
        orc.step([[g]])
    ost = orc.state[id(p0)]
    np.testing.assert_allclose(diag, [ost[k] for k in O.DIAG_KEYS], rtol=1e-5)
    np.testing.assert_array_equal(ns["m"].cpu().numpy(), ost["m"])
