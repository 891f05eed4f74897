"""CPU checks of Manau's Dana-Star-MK4 branch (src/optim/manau.py:504-613).

The oracle's restatement (oracle.OracleManau, adana_oracle_manau_step) is
pinned by the reference's own Manau.step() run in this container
(tests/golden/make_golden_manau.py) over a named GPT-like list: the branch's
state and diagnostics, and the weighted step count that Manau advances once
per parameter (and, with dana_momentum, once per Muon parameter before it).
Bars: dana_m and dana_v bit-exact (no sqrt or pow on their path); dana_tau
within 2 ulp and p within a few ulp of the tensor's scale (the reference's
CPU sqrt and pow are Sleef approximations of the correctly rounded values
the oracle takes); current_alpha and weighted_step_count exactly equal
(binary64 host arithmetic); the other diagnostics rtol 2e-5.  Also closed
forms for a constant gradient and the host scalars' binary32 bits against
the product's adana_manau_scalars_init.
"""
import json
import os

import numpy as np
import pytest

from helpers import ulp_diff

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ("manau", "manau_wt", "manau_mk4")
DIAG = ("current_alpha", "current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")


def _inputs(name="manau.inputs"):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    meta = json.loads(str(z["meta"]))
    n = len(meta["params"])
    p0 = [z[f"p0_{i}"] for i in range(n)]
    grads = [[z[f"g_{k}_{i}"] for i in range(n)] for k in range(1, meta["n_steps"] + 1)]
    return meta, p0, grads


def _gold(case):
    return np.load(os.path.join(GOLDEN, f"manau.{case}.npz"))


def _oracle(O, meta, case, params, use_muon):
    kw = meta["cases"][case]
    groups = []
    for gi, scale in enumerate(meta["group_wd_scale"]):
        idx = [i for i, (_, _, g) in enumerate(meta["params"]) if g == gi]
        groups.append(O.OracleManauGroup(
            params=[params[i] for i in idx], use_muon=[bool(use_muon[i]) for i in idx], lr=kw["lr"],
            weight_decay=kw["weight_decay"] * scale, delta=kw.get("delta", 8.0), kappa=kw.get("kappa", 1.0),
            mk4A=kw.get("mk4A", 0.0), mk4B=kw.get("mk4B", 0.0), clipsnr=kw.get("clipsnr", 1.0),
            epsilon=kw.get("epsilon", 1e-8), weight_time=kw.get("weight_time", False),
            wd_decaying=kw.get("wd_decaying", False), wd_ts=kw.get("wd_ts", 1.0),
            dana_momentum=kw.get("dana_momentum", False)))
    order = [[i for i, (_, _, g) in enumerate(meta["params"]) if g == gi] for gi in range(len(groups))]
    return O.OracleManau(groups=groups, peak_lr=kw["lr"]), kw, order


def _scaled_err(x, ref, scale):
    scale = np.maximum(np.abs(scale), np.float32(1e-30)).astype(np.float32)
    return np.abs(x.astype(np.float64) - ref.astype(np.float64)) / np.spacing(scale).astype(np.float64)


@pytest.mark.parametrize("case", CASES)
def test_oracle_manau_follows_reference_trajectory(oracle_mod, case):
    O = oracle_mod
    meta, p0, grads = _inputs()
    gold = _gold(case)
    use_muon = gold["use_muon"]
    names = [n for n, _, _ in meta["params"]]
    assert [bool(u) for u in use_muon] == [("wte" not in n and "lm_head" not in n and len(s) >= 2)
                                          for n, s, _ in meta["params"]]
    params = [x.copy() for x in p0]
    opt, kw, order = _oracle(O, meta, case, params, use_muon)
    for k in range(1, meta["n_steps"] + 1):
        for g in opt.groups:
            g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        opt.step([[grads[k - 1][i] for i in idx] for idx in order])
        assert [g.weighted_step_count for g in opt.groups] == list(gold["weighted_step_count"][k - 1]), k
        for i, p in enumerate(params):
            if use_muon[i]:
                continue
            st = opt.state[id(p)]
            ref = gold["diag"][k - 1, i]
            assert st["current_alpha"] == ref[0], (case, k, names[i])
            got = np.array([st[key] for key in DIAG[1:]])
            np.testing.assert_allclose(got, ref[1:], rtol=2e-5, atol=1e-12, err_msg=f"{case} t={k} {names[i]}")
        if k not in meta["checkpoints"]:
            continue
        for i, p in enumerate(params):
            if use_muon[i]:
                continue
            st = opt.state[id(p)]
            assert st["step"] == int(gold[f"step{i}_t{k}"])
            assert ulp_diff(st["dana_m"], gold[f"dana_m{i}_t{k}"]).max() == 0, (case, k, names[i])
            assert ulp_diff(st["dana_v"], gold[f"dana_v{i}_t{k}"]).max() == 0, (case, k, names[i])
            # tau is an EMA of a value the reference computes through Sleef's
            # sqrt: 1-ulp differences enter each step and accumulate (the
            # single-step test below holds each step to 2 ulp)
            assert ulp_diff(st["dana_tau"], gold[f"dana_tau{i}_t{k}"]).max() <= max(2, k // 2), (case, k, names[i])
            scale = np.full(p.shape, np.abs(gold[f"p{i}_t{k}"]).max(), np.float32)
            assert _scaled_err(p, gold[f"p{i}_t{k}"], scale).max() <= 2 * k, (case, k, names[i])


@pytest.mark.parametrize("case", ["manau", "manau_mk4"])
def test_oracle_manau_nonfinite_gradients(oracle_mod, case):
    """NaN, +inf and -inf gradient entries in Dana-branch tensors
    (make_golden_manau.py --nonfinite, the reference's own run): the oracle
    puts NaN and inf where the reference does in dana_m, dana_v, dana_tau and
    p; the other elements meet the trajectory bars; diagnostics NaN alike."""
    O = oracle_mod
    meta, p0, grads = _inputs("manau.nonfinite.inputs")
    gold = np.load(os.path.join(GOLDEN, f"manau.{case}.nonfinite.npz"))
    use_muon = gold["use_muon"]
    params = [x.copy() for x in p0]
    opt, kw, order = _oracle(O, meta, case, params, use_muon)
    hit = set()
    for k in range(1, meta["n_steps"] + 1):
        for g in opt.groups:
            g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        opt.step([[grads[k - 1][i] for i in idx] for idx in order])
        for i, p in enumerate(params):
            if use_muon[i]:
                continue
            st = opt.state[id(p)]
            got = np.array([st[key] for key in DIAG[1:]])
            np.testing.assert_allclose(got, gold["diag"][k - 1, i][1:], rtol=2e-5, atol=1e-12, equal_nan=True,
                                       err_msg=f"{case} t={k} tensor {i}")
        if k not in meta["checkpoints"]:
            continue
        for i, p in enumerate(params):
            if use_muon[i]:
                continue
            st = opt.state[id(p)]
            for key, bound in (("dana_m", 0), ("dana_v", 0), ("dana_tau", max(2, k // 2))):
                ref = gold[f"{key}{i}_t{k}"]
                assert np.array_equal(np.isnan(st[key]), np.isnan(ref)), (case, key, k, i)
                assert ulp_diff(st[key], ref).max() <= bound, (case, key, k, i)
            ref = gold[f"p{i}_t{k}"]
            assert np.array_equal(np.isnan(p), np.isnan(ref)) and np.array_equal(np.isinf(p), np.isinf(ref))
            if not np.isfinite(ref).all():
                hit.add(i)
            fin = np.isfinite(ref)
            scale = np.full(fin.sum(), np.abs(ref[fin]).max(), np.float32)
            assert _scaled_err(p[fin], ref[fin], scale).max() <= 2 * k, (case, k, i)
    assert hit == {0, 5, 7, 8}                                  # every injected tensor went non-finite


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("t0", [0, 8])
def test_oracle_manau_single_step_from_reference_state(oracle_mod, case, t0):
    """From the reference's own state at step t0, one oracle step lands on the
    reference's state at t0 + 1: dana_m, dana_v bit-exact, dana_tau within 2
    ulp, p within 4 ulp (6 with general mk4 exponents: two more Sleef pows)
    of max(|p_before|, |p_after|, |update|)."""
    O = oracle_mod
    meta, p0, grads = _inputs()
    gold = _gold(case)
    use_muon = gold["use_muon"]
    k = t0 + 1
    params = [(p0[i] if t0 == 0 else gold[f"p{i}_t{t0}"]).copy() for i in range(len(p0))]
    opt, kw, order = _oracle(O, meta, case, params, use_muon)
    if t0 > 0:
        for g, w in zip(opt.groups, gold["weighted_step_count"][t0 - 1]):
            g.weighted_step_count = float(w)
        for i, p in enumerate(params):
            if not use_muon[i]:
                opt.state[id(p)] = {"step": int(gold[f"step{i}_t{t0}"]),
                                    **{n: gold[f"{n}{i}_t{t0}"].copy() for n in ("dana_m", "dana_v", "dana_tau")}}
    prev = [p.copy() for p in params]
    for g in opt.groups:
        g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
    opt.step([[grads[k - 1][i] for i in idx] for idx in order])
    bound = 6 if case == "manau_mk4" else 4
    for i, p in enumerate(params):
        if use_muon[i]:
            continue
        st = opt.state[id(p)]
        assert ulp_diff(st["dana_m"], gold[f"dana_m{i}_t{k}"]).max() == 0
        assert ulp_diff(st["dana_v"], gold[f"dana_v{i}_t{k}"]).max() == 0
        assert ulp_diff(st["dana_tau"], gold[f"dana_tau{i}_t{k}"]).max() <= 2
        ref = gold[f"p{i}_t{k}"]
        scale = np.maximum(np.maximum(np.abs(prev[i]), np.abs(ref)), np.abs(ref - prev[i]))
        assert _scaled_err(p, ref, scale).max() <= bound, (case, t0, i)


def test_oracle_manau_constant_gradient_closed_form(oracle_mod):
    """Constant g from zero state: m_t = g (1 - P_t), v_t = g^2 (1 - P_t) with
    P_t = prod_k (1 - delta / (delta + k)); tau_t follows its scalar
    recursion.  Float64 references, a few ulp of binary32."""
    O = oracle_mod
    rng = np.random.default_rng(3)
    g = rng.normal(0, 1e-3, 500).astype(np.float32)
    p = rng.normal(0, 0.02, 500).astype(np.float32)
    m, v, tau = (np.zeros_like(p) for _ in range(3))
    delta, P = 8.0, 1.0
    tau64 = np.zeros(500)
    for t in range(1, 30):
        alpha = delta / (delta + t)
        sc = O.manau_scalars(lr=1e-3, step=t, alpha=alpha, kappa=0.85, mk4A=0.0, mk4B=0.0, clipsnr=1.0,
                             epsilon=1e-8, weight_decay=0.1, wd_decaying=False, wd_ts=1.0)
        O.manau_element_step(p, g, m, v, tau, sc)
        P *= 1 - alpha
        g64 = g.astype(np.float64)
        v64 = g64 * g64 * (1 - P)
        tu = np.abs(g64) / (np.abs(g64) + np.sqrt(v64) + 1e-8)
        tau64 = tau64 * (1 - alpha) + alpha * tu
        np.testing.assert_allclose(m, g64 * (1 - P), rtol=4e-6 * t, atol=0)
        np.testing.assert_allclose(v, v64, rtol=4e-6 * t, atol=0)
        np.testing.assert_allclose(tau, tau64, rtol=1e-5 * t, atol=0)


def test_manau_scalars_match_product_bitwise(oracle_mod):
    """The oracle's Python-float scalars and the product's
    adana_manau_scalars_init agree bit for bit (weight-time steps included)."""
    import ctypes

    from adana_amd import _lib

    O = oracle_mod
    for kw in (dict(kappa=0.85, mk4A=0.0, mk4B=0.0, clipsnr=1.0, weight_decay=0.1, wd_decaying=False, wd_ts=1.0),
               dict(kappa=0.5, mk4A=0.1, mk4B=0.25, clipsnr=2.0, weight_decay=0.03, wd_decaying=True, wd_ts=5.0),
               dict(kappa=1.0, mk4A=-0.5, mk4B=0.0, clipsnr=4.0, weight_decay=0.0, wd_decaying=True, wd_ts=7.0)):
        for step, alpha, lr in ((1, 8 / 9, 2e-2), (7, 8 / 15, 3e-3), (2.37, 8 / 10.37 * 0.4, 1e-2), (0.0, 0.0, 0.0)):
            ref = O.manau_scalars(lr=lr, step=step, alpha=alpha, epsilon=1e-8, **kw)
            hp = _lib.ManauHParams(delta=8.0, kappa=kw["kappa"], mk4A=kw["mk4A"], mk4B=kw["mk4B"],
                                   clipsnr=kw["clipsnr"], epsilon=1e-8, weight_decay=kw["weight_decay"],
                                   wd_ts=kw["wd_ts"], wd_decaying=int(kw["wd_decaying"]))
            got = _lib.manau_scalars(hp, lr, step, alpha)
            assert bytes(got) == bytes(ref), (kw, step)
            assert ctypes.sizeof(got) == 64


def _our_manau(meta, case):
    import contextlib
    import io

    import torch

    import adana_amd

    kw = meta["cases"][case]
    params = [torch.nn.Parameter(torch.zeros(s)) for _, s, _ in meta["params"]]
    groups = []
    for gi, scale in enumerate(meta["group_wd_scale"]):
        idx = [i for i, (_, _, g) in enumerate(meta["params"]) if g == gi]
        groups.append({"params": [params[i] for i in idx], "param_names": [meta["params"][i][0] for i in idx],
                       "weight_decay": kw["weight_decay"] * scale})
    printed = io.StringIO()
    with contextlib.redirect_stdout(printed):
        opt = adana_amd.Manau(groups, **kw)
    return opt, params, printed.getvalue()


@pytest.mark.parametrize("case", CASES)
def test_manau_constructor_matches_reference(case):
    """Same Muon / Dana assignment, group keys and printed summary as the
    reference's constructor (manau.py:121-223) on the same named list."""
    meta, _, _ = _inputs()
    gold = _gold(case)
    opt, params, printed = _our_manau(meta, case)
    assert printed == str(gold["ctor_stdout"])
    assert [opt.state[p]["use_muon"] for p in params] == [bool(u) for u in gold["use_muon"]]
    schema = json.loads(str(gold["schema"]))
    assert [sorted(k for k in g if k != "params") for g in opt.param_groups] == schema["param_groups"]


def test_manau_host_errors():
    import torch

    import adana_amd

    p = torch.nn.Parameter(torch.zeros(4))
    with pytest.raises(ValueError, match="param_names"):
        adana_amd.Manau([{"params": [p]}])
    meta, _, _ = _inputs()
    opt, params, _ = _our_manau(meta, "manau")
    with pytest.raises(NotImplementedError, match="distributed"):
        opt.enable_distributed_mode([], None, None, {})
    for q in params:
        q.grad = torch.zeros_like(q)
    before = [q.detach().clone() for q in params]
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()
    assert all(torch.equal(a, q) for a, q in zip(before, params))       # refused before any update


def test_manau_names_shorter_than_params():
    """A parameter past the end of its group's name list has no name of its
    own (manau.py:183-190 marks only ``idx < len(param_names)``): a matrix
    there goes to Muon even when the last listed name is the head's, and a
    vector to the Dana branch; the report lists it under that last name."""
    import contextlib
    import io

    import torch

    import adana_amd

    head = torch.nn.Parameter(torch.zeros(8, 4))
    extra_mat = torch.nn.Parameter(torch.zeros(4, 4))
    extra_vec = torch.nn.Parameter(torch.zeros(4))
    printed = io.StringIO()
    with contextlib.redirect_stdout(printed):
        opt = adana_amd.Manau([{"params": [head, extra_mat, extra_vec], "param_names": ["lm_head.weight"]}])
    assert opt.state[head]["use_muon"] is False
    assert opt.state[extra_mat]["use_muon"] is True
    assert opt.state[extra_vec]["use_muon"] is False
    assert printed.getvalue().count("lm_head.weight") == 3
