"""1,000 steps of the reference's own tensor ops against the oracle.

oracle/torch_ref.py runs the reference's update as torch CPU tensor ops, one
op per op of src/optim/adana.py:101-151 / src/optim/dana_star_mk4.py:137-203,
with torch's own sqrt and pow: the reference's bits (test_torch_restatement.py
pins it at 0 ulp against the golden fixtures of both of the reference's modes:
eager ATen ops, and the default torch.compile path with Inductor's forms).
The oracle differs from it only where torch's CPU sqrt (eager) and SIMD pow
(both modes) are not correctly rounded.  The same holds for the
use_foreach=True path (src/optim/adana.py:229-370,
src/optim/dana_star_mk4.py:298-536; torch_ref.update_foreach), run here in
both of its modes too.  Here both run the same 1,000 steps
on a small list (three tensors, gradients of scales 1e-5 .. 1e-1, a zero
gradient every 50 steps, an lr that moves), and the tests print the gap:

  * per step: before every step the oracle's state is set to the reference's,
    so the gap is one step's;
  * free-running: each side steps its own state for all 1,000 steps, so the
    gap is the accumulated drift.

Units: v and tau in ulps of each element; m in ulps of its tensor's largest
|m| (m crosses zero, where ulps of the element mean nothing); p per step in
ulps of max(|p before|, |p after|, |update|) per element, free-running in
ulps of its tensor's largest |p|.  The bars are the measured maxima of this
run, rounded up with headroom."""
import numpy as np
import pytest
import torch

from helpers import ulp_diff
from test_torch_restatement import _cr_sqrt, _powf, _simd_pow

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")

SHAPES = [(97,), (33, 5), (256,)]
N_STEPS = 1000
# Measured on this container's CPU (torch 2.10), max / median over the 1,000 steps:
#   per step     ADana eager p 3/0; compiled exact; Dana-Star eager p 3/0, tau 2/0; compiled p 2/0
#   free-running ADana eager p 2/1; compiled exact; Dana-Star eager p 2/1, tau 3/1; compiled p 2/1
# The foreach path (use_foreach=True), the same 1,000 steps:
#   per step     ADana compiled exact, eager p 2/0; Dana-Star compiled p 2/0, eager p 3/0, tau 2/0
#   free-running ADana compiled exact, eager p 2/1; Dana-Star compiled p 2/0.5, eager p 2/1, tau 3/1
# m and v are exact throughout (their ops have no sqrt or pow).  Bars: those, with headroom.
BARS = {
    ("eager", False): {"step": dict(p=4, m=0, v=0, tau=0), "free": dict(p=4, m=0, v=0, tau=0)},
    ("eager", True): {"step": dict(p=4, m=0, v=0, tau=3), "free": dict(p=4, m=0, v=0, tau=4)},
    ("compiled", False): {"step": dict(p=0, m=0, v=0, tau=0), "free": dict(p=0, m=0, v=0, tau=0)},
    ("compiled", True): {"step": dict(p=3, m=0, v=0, tau=0), "free": dict(p=4, m=0, v=0, tau=0)},
    ("foreach", False): {"step": dict(p=0, m=0, v=0, tau=0), "free": dict(p=0, m=0, v=0, tau=0)},
    ("foreach", True): {"step": dict(p=3, m=0, v=0, tau=0), "free": dict(p=4, m=0, v=0, tau=0)},
    ("foreach_eager", False): {"step": dict(p=4, m=0, v=0, tau=0), "free": dict(p=4, m=0, v=0, tau=0)},
    ("foreach_eager", True): {"step": dict(p=4, m=0, v=0, tau=3), "free": dict(p=4, m=0, v=0, tau=4)},
}


def _m_ulps(got, ref):
    scale = np.float32(max(float(np.abs(ref).max()), 1e-30))
    return np.abs(got.astype(np.float64) - ref.astype(np.float64)) / float(np.spacing(scale))


def _p_ulps(got, ref, prev):
    """ulps of max(|p before|, |p after|, |update|) per element (the update's
    own rounding is on that scale; a p near zero is not)."""
    ref64, prev64 = ref.astype(np.float64), prev.astype(np.float64)
    scale = np.maximum(np.maximum(np.abs(prev64), np.abs(ref64)), np.abs(ref64 - prev64))
    scale = np.maximum(scale, 1e-30).astype(np.float32)
    return np.abs(got.astype(np.float64) - ref64) / np.spacing(scale).astype(np.float64)


def _gap(t_state, o_state, t_params, o_params, prev, star, resync):
    if resync:
        out = {"p": max(float(_p_ulps(o, t.numpy(), pv).max()) for t, o, pv in zip(t_params, o_params, prev))}
    else:
        out = {"p": max(float(_m_ulps(o, t.numpy()).max()) for t, o in zip(t_params, o_params))}
    out["m"] = max(float(_m_ulps(t_state[id(t)]["m"].numpy(), o_state[id(o)]["m"]).max())
                   for t, o in zip(t_params, o_params))
    for key in ("v", "tau") if star else ("v",):
        out[key] = max(int(ulp_diff(t_state[id(t)][key].numpy(), o_state[id(o)][key]).max())
                       for t, o in zip(t_params, o_params))
    if not star:
        out["tau"] = 0
    return out


def _run(O, star, mode, resync):
    from oracle.torch_ref import TorchRefGroup, TorchRefOptimizer

    rng = np.random.default_rng(2024)
    p0 = [rng.normal(0.0, 0.02, s).astype(np.float32) for s in SHAPES]
    t_params = [torch.from_numpy(x.copy()) for x in p0]
    o_params = [x.copy() for x in p0]
    hp = dict(kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0)
    tref = TorchRefOptimizer(groups=[TorchRefGroup(params=t_params, lr=1e-3, weight_decay=0.1)], star=star,
                             peak_lr=1e-3, **hp)
    foreach = mode.startswith("foreach")
    numerics = "eager" if mode.endswith("eager") else "compiled"
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=o_params, lr=1e-3, weight_decay=0.1)], star=star,
                            peak_lr=1e-3, numerics=numerics, foreach=foreach, **hp)
    compiled = (_cr_sqrt, _simd_pow, _powf) if mode == "compiled" else None
    fe = None
    if foreach:
        fe = (_cr_sqrt, _simd_pow, _powf, True) if numerics == "compiled" else (None, None, None, False)
    per_step = {k: [] for k in ("p", "m", "v", "tau")}
    for k in range(N_STEPS):
        lr = 1e-3 * (0.5 + 0.5 * np.cos(np.pi * k / N_STEPS))
        tref.groups[0].lr = orc.groups[0].lr = lr
        grads = [rng.normal(0.0, 10.0 ** rng.uniform(-5, -1), s).astype(np.float32) for s in SHAPES]
        if k % 50 == 49:
            grads[1][...] = 0.0
        if resync and k:
            for t, o in zip(t_params, o_params):
                o[...] = t.numpy()
                for key in ("m", "v", "tau") if star else ("m", "v"):
                    orc.state[id(o)][key][...] = tref.state[id(t)][key].numpy()
        prev = [t.numpy().copy() for t in t_params]
        tref.step([[torch.from_numpy(g.copy()) for g in grads]], compiled=compiled, foreach=fe)
        orc.step([grads])
        gap = _gap(tref.state, orc.state, t_params, o_params, prev, star, resync)
        for key, val in gap.items():
            per_step[key].append(val)
    return {key: (float(np.max(v)), float(np.median(v))) for key, v in per_step.items()}


@pytest.mark.parametrize("mode", ["eager", "compiled", "foreach", "foreach_eager"])
@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
@pytest.mark.parametrize("resync", [True, False], ids=["per_step", "free_running"])
def test_thousand_steps_against_reference_ops(oracle_mod, star, mode, resync):
    stats = _run(oracle_mod, star, mode, resync)
    kind = "step" if resync else "free"
    print(f"\n{'Dana-Star-MK4' if star else 'ADana'} {mode} {N_STEPS} steps, {kind} gap (max, median): "
          + ", ".join(f"{k} {mx:g} / {md:g}" for k, (mx, md) in stats.items()))
    bars = BARS[(mode, star)][kind]
    for key, (mx, _) in stats.items():
        assert mx <= bars[key], (key, stats)
