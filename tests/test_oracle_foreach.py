"""The oracle's foreach mode (adana_oracle_scalars.foreach) against the
reference's use_foreach=True path: src/optim/adana.py:229-370 and
src/optim/dana_star_mk4.py:298-536, whose kernel the constructor wraps in
torch.compile (adana.py:63-70).  Fixtures: tests/golden/<case>.foreach.npz
(compiled, float32), .foreach_eager.npz (eager, float32) and
.bf16_foreach.npz (compiled, bfloat16), written by the reference's own
step() (tests/golden/make_golden.py --foreach).

Pins, strongest first:
  * the torch restatement of the foreach path (oracle/torch_ref.py,
    update_foreach), which reproduces every foreach fixture at 0 ulp
    (tests/test_torch_restatement.py), with Dana-Star's element power made
    correctly rounded, equals the oracle bit for bit along every trajectory;
  * against the fixtures themselves: m, v and tau bit-exact; ADana's p
    bit-exact; Dana-Star's p within the bar of the SIMD power (compiled) or
    of torch's CPU sqrt and power (eager) -- the same causes, and the same
    bars, as the per-tensor path's fixtures in tests/test_oracle.py."""
import numpy as np
import pytest
import torch

from helpers import bf16_ulp_diff, golden_cases, load_golden_case, load_golden_inputs, ulp_diff
from test_oracle import _grads_for_step, _load_state, _scaled_err

CASES = golden_cases("foreach")


def _make(O, meta, case, params, numerics, bf16=False):
    kw = meta["cases"][case]["kwargs"]
    star = meta["cases"][case]["class"] == "DANA_STAR_MK4"
    groups = [O.OracleGroup(params=[params[i] for i in range(len(params)) if meta["group_of"][i] == gi],
                            lr=kw["lr"], delta=kw["delta"], epsilon=1e-8,
                            weight_decay=kw["weight_decay"] * meta["group_wd_scale"][gi]) for gi in range(2)]
    opt = O.OracleOptimizer(groups=groups, star=star, peak_lr=kw["lr"], kappa=kw["kappa"], clipsnr=kw["clipsnr"],
                            wd_decaying=kw["wd_decaying"], wd_ts=kw["wd_ts"], gamma_3_factor=kw["gamma_3_factor"],
                            numerics=numerics, bf16=bf16, foreach=True)
    return opt, kw, star


@pytest.mark.parametrize("mode", ["foreach", "bf16_foreach", "bf16_foreach_eager"])
@pytest.mark.parametrize("case", CASES)
def test_oracle_equals_foreach_restatement_with_correct_rounding(oracle_mod, case, mode):
    """torch_ref.update_foreach (the reference's bits, test_torch_restatement)
    with Dana-Star's element power correctly rounded gives the oracle's
    foreach mode bit for bit: p, m, v, tau after every one of the 20 steps,
    float32 and bfloat16 compiled; on bfloat16 eager (ATen's own sqrt and
    pow, which round like the correctly rounded ones at bfloat16 here) the
    same, diagnostics included."""
    from oracle.torch_ref import DIAG_KEYS, TorchRefGroup, TorchRefOptimizer
    from test_torch_restatement import _cr_pow, _cr_sqrt, _powf

    O = oracle_mod
    bf16 = mode.startswith("bf16")
    eager = mode.endswith("eager")
    meta, p0, grads, has_grad = load_golden_inputs()
    dt = torch.bfloat16 if bf16 else torch.float32
    o_params = [O.f32_to_bf16(x) if bf16 else x.copy() for x in p0]
    opt, kw, star = _make(O, meta, case, o_params, "eager" if eager else "compiled", bf16=bf16)
    t_params = [torch.from_numpy(x.copy()).to(dt) for x in p0]
    idx = [[i for i in range(len(p0)) if meta["group_of"][i] == gi] for gi in range(2)]
    tgroups = [TorchRefGroup(params=[t_params[i] for i in idx[gi]], lr=kw["lr"], delta=kw["delta"], epsilon=1e-8,
                             weight_decay=kw["weight_decay"] * meta["group_wd_scale"][gi]) for gi in range(2)]
    tref = TorchRefOptimizer(groups=tgroups, star=star, peak_lr=kw["lr"], kappa=kw["kappa"], clipsnr=kw["clipsnr"],
                             wd_decaying=kw["wd_decaying"], wd_ts=kw["wd_ts"], gamma_3_factor=kw["gamma_3_factor"])

    def bits(t):
        return t.view(torch.int16).numpy().view(np.uint16) if bf16 else t.numpy().view(np.uint32)

    for k in range(1, meta["n_steps"] + 1):
        lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        for g in opt.groups + tgroups:
            g.lr = lr
        og = _grads_for_step(meta, [[O.f32_to_bf16(x) if bf16 else x for x in gs] for gs in grads], has_grad, k)
        opt.step(og)
        tref.step([[torch.from_numpy(grads[k - 1][i].copy()).to(dt) if has_grad[k - 1, i] else None for i in idx[gi]]
                   for gi in range(2)], foreach=(None, None, None, False) if eager else (_cr_sqrt, _cr_pow, _powf, True))
        for i in range(len(p0)):
            assert np.array_equal(bits(t_params[i]), o_params[i].view(bits(t_params[i]).dtype)), (case, mode, k, i)
            tst, ost = tref.state.get(id(t_params[i])), opt.state.get(id(o_params[i]))
            if tst is None:
                continue
            for key in ("m", "v", "tau") if star else ("m", "v"):
                got = bits(tst[key])
                assert np.array_equal(got, ost[key].view(got.dtype)), (case, mode, key, k, i)
            if has_grad[k - 1, i]:
                np.testing.assert_allclose([float(tst[key]) for key in DIAG_KEYS], [ost[key] for key in O.DIAG_KEYS],
                                           rtol=8e-3 if bf16 else 1e-5, atol=0, equal_nan=True)


def _trajectory(O, case, mode, tau_bar=0):
    """The oracle's foreach mode over the fixture's 20 steps without
    re-synchronising; returns the worst p gap (ulps of the tensor's largest
    |p|) and checks m and v bit-exact, tau within ``tau_bar`` ulp, at every
    checkpoint."""
    bf16 = mode.startswith("bf16")
    meta, p0, grads, has_grad = load_golden_inputs()
    gold = load_golden_case(case, mode)
    params = [O.f32_to_bf16(x) if bf16 else x.copy() for x in p0]
    opt, kw, star = _make(O, meta, case, params, "eager" if mode.endswith("eager") else "compiled", bf16=bf16)
    worst, dworst = 0.0, 0.0
    for k in range(1, meta["n_steps"] + 1):
        for g in opt.groups:
            g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        opt.step(_grads_for_step(meta, [[O.f32_to_bf16(x) if bf16 else x for x in gs] for gs in grads], has_grad, k))
        for i, p in enumerate(params):
            st = opt.state.get(id(p))
            if st is None or not has_grad[k - 1, i]:
                continue
            got = np.array([st[key] for key in O.DIAG_KEYS], np.float64)
            ref = gold["diag"][k - 1, i].astype(np.float64)
            with np.errstate(invalid="ignore"):
                rel = np.where(np.isnan(got) & np.isnan(ref), 0.0, np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30))
            dworst = max(dworst, float(rel.max()))
        if k not in meta["checkpoints"]:
            continue
        for i, p in enumerate(params):
            st = opt.state.get(id(p), {})
            assert st.get("step", 0) == int(gold[f"step{i}_t{k}"])
            for key in ("m", "v", "tau") if star else ("m", "v"):
                if key in st:
                    d = (bf16_ulp_diff if bf16 else ulp_diff)(st[key], gold[f"{key}{i}_t{k}"])
                    assert d.max() <= (tau_bar if key == "tau" else 0), (case, mode, key, k, i, int(d.max()))
            ref = gold[f"p{i}_t{k}"]
            if bf16:
                worst = max(worst, float(bf16_ulp_diff(p, ref).max()))
            else:
                scale = np.full(p.shape, np.abs(ref).max(), np.float32)
                worst = max(worst, float(_scaled_err(p, ref, scale).max()))
    return star, worst, dworst


@pytest.mark.parametrize("mode", ["foreach", "bf16_foreach", "bf16_foreach_eager"])
@pytest.mark.parametrize("case", CASES)
def test_foreach_golden_trajectory(oracle_mod, case, mode):
    """Compiled, the reference's default for this path: m, v, tau bit-exact
    at every checkpoint, float32 and bfloat16; ADana's p bit-exact;
    Dana-Star's p within 2 ulp of the tensor's largest |p| (float32; the
    SIMD pow of the effective time, as on the per-tensor path; measured 1.5)
    and bit-exact on bfloat16; diagnostics within 2e-5 (float32) and 1
    bfloat16 ulp.  The eager ops on bfloat16 state: all bit-exact."""
    star, worst, dworst = _trajectory(oracle_mod, case, mode)
    bf16 = mode.startswith("bf16")
    assert worst <= (2 if star and not bf16 else 0), (case, mode, worst)
    assert dworst <= (2 ** -8 if bf16 else 2e-5), (case, mode, dworst)


@pytest.mark.parametrize("case", CASES)
def test_foreach_eager_golden_trajectory(oracle_mod, case):
    """Eager foreach ops (float32): m and v bit-exact; tau within 2 ulp and
    p within 3 ulp of the tensor's largest |p|, the eager per-tensor bars
    (torch's CPU sqrt and pow are not correctly rounded; the oracle's are)."""
    star, worst, dworst = _trajectory(oracle_mod, case, "foreach_eager", tau_bar=2)
    assert worst <= 3, (case, worst)
    assert dworst <= 2e-5, (case, dworst)


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("t0", [0, 7, 8])
def test_foreach_single_step(oracle_mod, case, t0):
    """From the reference's own foreach state at step t0, one oracle step:
    m, v, tau bit-exact; ADana's p bit-exact; Dana-Star's p within 1 ulp of
    max(|p_before|, |p_after|, |update|)."""
    O = oracle_mod
    meta, p0, grads, has_grad = load_golden_inputs()
    gold = load_golden_case(case, "foreach")
    k = t0 + 1
    params = [(p0[i] if t0 == 0 else gold[f"p{i}_t{t0}"]).copy() for i in range(len(p0))]
    opt, kw, star = _make(O, meta, case, params, "compiled")
    if t0 > 0:
        _load_state(opt, meta, gold, params, t0, star)
    prev = [p.copy() for p in params]
    for g in opt.groups:
        g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
    opt.step(_grads_for_step(meta, grads, has_grad, k))
    for i, p in enumerate(params):
        st = opt.state.get(id(p))
        if st is None:
            continue
        for key in ("m", "v", "tau") if star else ("m", "v"):
            assert ulp_diff(st[key], gold[f"{key}{i}_t{k}"]).max() == 0, (case, t0, key, i)
        ref = gold[f"p{i}_t{k}"]
        scale = np.maximum(np.maximum(np.abs(prev[i]), np.abs(ref)), np.abs(ref - prev[i]))
        assert _scaled_err(p, ref, scale).max() <= (1 if star else 0), (case, t0, i)


def test_foreach_scalars_alpha_and_step_dtype(oracle_mod):
    """The foreach path's scalars: alpha is the binary32 quotient of the
    binary32 delta and step (adana.py:175, :259).  For a delta exact in
    binary32 that is the per-tensor path's binary64 quotient rounded once (a
    correctly rounded quotient either way); for another delta the two
    differ.  A bfloat16 step above 256 is rounded (step_t has the parameters'
    dtype, adana.py:258)."""
    O = oracle_mod
    kw = dict(lr=1e-3, peak_lr=1e-3, kappa=0.85, epsilon=1e-8, weight_decay=0.1, clipsnr=None,
              wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0)
    for delta, expect_diff in ((8.0, False), (7.3, True)):
        diff = 0
        d32 = np.float32(delta)
        for t in range(1, 2000):
            fe, pt = O.foreach_scalars(**kw, delta=delta, t=t), O.step_scalars(**kw, delta=delta, t=t)
            assert fe.a == np.float32(d32 / (d32 + np.float32(t)))
            diff += fe.a != pt.a
        assert (diff > 0) == expect_diff, (delta, diff)
    sc = O.foreach_scalars(**kw, delta=8.0, t=257, step_bf16=True)
    assert sc.s == 256.0 and O.foreach_scalars(**kw, delta=8.0, t=257).s == 257.0


@pytest.mark.parametrize("case", golden_cases("foreach_nonfinite"))
def test_foreach_nonfinite_trajectory(oracle_mod, case):
    """The foreach path on NaN, +inf and -inf gradient entries (the
    reference's own compiled foreach run, make_golden.py --foreach): every
    element the reference turns NaN or inf is NaN or the same inf here, in p,
    m, v and tau; the finite elements meet the compiled foreach bars (m, v,
    tau bit-exact; p within 2 ulp of the tensor's largest finite |p|);
    diagnostics NaN where the reference's are, else within 2e-5."""
    O = oracle_mod
    meta, p0, grads, has_grad = load_golden_inputs("nonfinite.inputs")
    gold = load_golden_case(case, "foreach_nonfinite")
    params = [x.copy() for x in p0]
    opt, kw, star = _make(O, meta, case, params, "compiled")
    for k in range(1, meta["n_steps"] + 1):
        for g in opt.groups:
            g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        opt.step(_grads_for_step(meta, grads, has_grad, k))
        for i, p in enumerate(params):
            st = opt.state.get(id(p))
            if st is None or not has_grad[k - 1, i]:
                continue
            got = np.array([st[key] for key in O.DIAG_KEYS])
            np.testing.assert_allclose(got, gold["diag"][k - 1, i], rtol=2e-5, atol=1e-12, equal_nan=True,
                                       err_msg=f"{case} diag t={k} tensor {i}")
        if k not in meta["checkpoints"]:
            continue
        for i, p in enumerate(params):
            st = opt.state.get(id(p), {})
            if "m" not in st:
                continue
            for key in ("m", "v") + (("tau",) if star else ()):
                ref = gold[f"{key}{i}_t{k}"]
                assert np.array_equal(np.isnan(st[key]), np.isnan(ref)), (case, key, k, i)
                assert ulp_diff(st[key], ref).max() == 0, (case, key, k, i)
            ref = gold[f"p{i}_t{k}"]
            assert np.array_equal(np.isnan(p), np.isnan(ref)) and np.array_equal(np.isinf(p), np.isinf(ref))
            fin = np.isfinite(ref)
            assert np.array_equal(p[~fin & ~np.isnan(ref)], ref[~fin & ~np.isnan(ref)])
            if fin.any():
                scale = np.full(fin.sum(), np.abs(ref[fin]).max(), np.float32)
                assert _scaled_err(p[fin], ref[fin], scale).max() <= 2, (case, k, i)
