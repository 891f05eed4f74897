"""Seeded random configurations of the step against the oracle.

Each case draws, from its seed: the variant (ADana / Dana-MK4 or
Dana-Star-MK4), fp32 parameters or the bf16-master extension, 1-3 parameter
groups with their own lr, delta, epsilon and weight decay, 1-10 tensors per
group (empty, tiny, ragged and up to 70,000-element sizes, 1-D and 2-D), kappa
from the values that select each pow kind (0, 0.5, 0.85, 1, 1.5, 2, 3),
clipsnr, decaying weight decay, wd_ts, gamma_3_factor and the numerics
(the reference's compiled path or its eager ops).  It then takes 7
steps (crossing t = delta for the smallest deltas) with a new lr per group
each step, gradients of random scale with some all-zero tensors, and some
gradients None (that tensor skips the step and keeps its state), and checks
every step against the oracle (src/optim/adana.py:101-153,
src/optim/dana_star_mk4.py:137-203) to the bars of test_gpu_parity.py: m, v
and tau bit-exact, p bit-exact (Dana-Star: at most 2 hard-case elements per
tensor, within 2 scaled ulp), diagnostics rtol 1e-5.  A second sweep runs
the same draws on the reference's own bfloat16 path, a third with
clip_grad_norm_ fused into every step, and a fourth with use_foreach=True
(the reference's foreach path, src/optim/adana.py:229-370,
src/optim/dana_star_mk4.py:298-536) on float32, bf16-master and bfloat16
state.
"""
import numpy as np
import pytest
import torch  # noqa: F401  (the GPU test session's torch)

from test_gpu_parity import Pair, _normal

pytestmark = pytest.mark.gpu

KAPPAS = (0.0, 0.5, 0.85, 1.0, 1.5, 2.0, 3.0)


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    star = bool(rng.integers(2))
    master = bool(rng.random() < 0.3)
    groups = []
    for _ in range(int(rng.integers(1, 4))):
        shapes = []
        for _ in range(int(rng.integers(1, 11))):
            kind = rng.random()
            if kind < 0.08:
                shapes.append((0,))
            elif kind < 0.25:
                shapes.append((int(rng.integers(1, 9)),))
            elif kind < 0.6:
                shapes.append((int(np.exp(rng.uniform(np.log(9), np.log(70000)))),))
            else:
                shapes.append((int(rng.integers(1, 300)), int(rng.integers(1, 200))))
        gkw = {"lr": float(10 ** rng.uniform(-4, -2.5)), "delta": float(rng.choice([1.0, 2.0, 4.0, 8.0])),
               "epsilon": float(rng.choice([1e-8, 1e-6])), "weight_decay": float(rng.choice([0.0, 0.1, 0.4]))}
        groups.append((shapes, gkw))
    hp = {"lr": float(groups[0][1]["lr"]), "kappa": float(rng.choice(KAPPAS)),
          "wd_decaying": bool(rng.integers(2)), "wd_ts": float(rng.choice([1.0, 10.0])),
          "gamma_3_factor": float(rng.choice([1.0, 0.5]))}
    if star:
        hp["clipsnr"] = float(rng.choice([0.5, 1.0, 2.0]))
    else:
        hp["clipsnr"] = None if rng.random() < 0.5 else float(rng.choice([0.5, 2.0]))
    hp["numerics"] = "eager" if rng.random() < 0.4 else "compiled"
    return rng, star, master, groups, hp


@pytest.mark.parametrize("seed", range(48))
def test_random_configuration(oracle_mod, seed):
    _random_configuration(oracle_mod, seed, foreach=False)


@pytest.mark.parametrize("seed", range(16))
def test_random_configuration_foreach(oracle_mod, seed):
    """Other draws with use_foreach=True, against the oracle's foreach mode."""
    _random_configuration(oracle_mod, 300 + seed, foreach=True)


def _random_configuration(oracle_mod, seed, foreach):
    O = oracle_mod
    rng, star, master, groups, hp = _draw(seed)
    hp["foreach"] = foreach
    shapes = [s for ss, _ in groups for s in ss]
    print(f"case: random configuration seed {seed}: star {star} master {master} groups {len(groups)} "
          f"tensors {len(shapes)} elements {sum(int(np.prod(s)) for s in shapes)} {hp}", flush=True)

    def param(s):
        x = _normal(rng, s, 0.02)
        return O.f32_to_bf16(x) if master else x

    groups_np = [([param(s) for s in ss], gkw) for ss, gkw in groups]
    pair = Pair(O, star, groups_np, master=master, **hp)
    for k in range(7):
        pair.set_lr([g["lr"] * float(rng.uniform(0.5, 1.5)) for _, g in groups])
        grads = []
        for ss, _ in groups:
            gs = []
            for s in ss:
                u = rng.random()
                if u < 0.12:
                    gs.append(None)
                    continue
                g = _normal(rng, s, float(10 ** rng.uniform(-5, -1)))
                if u < 0.18:
                    g = np.zeros_like(g)
                gs.append(O.f32_to_bf16(g) if master else g)
            grads.append(gs)
        pair.step(grads)
        pair.compare(where=f"seed {seed} k={k}")
    pair.opt._check_slab_guards()     # nothing written outside the state tensors


@pytest.mark.parametrize("seed", range(24))
def test_random_configuration_bf16_state(oracle_mod, seed):
    """The same draws on the reference's own bfloat16 path (bfloat16
    parameters, m, v, tau; every op rounded to bfloat16), against the
    oracle's bfloat16 restatement to the bars of test_gpu_bf16.py: m, v, tau
    bit-exact, p bit-exact (Dana-Star: at most 2 elements per tensor within 1
    bfloat16 ulp), diagnostics within 1 bfloat16 ulp."""
    _random_configuration_bf16_state(oracle_mod, 100 + seed, foreach=False)


@pytest.mark.parametrize("seed", range(8))
def test_random_configuration_bf16_state_foreach(oracle_mod, seed):
    """Other draws on bfloat16 state with use_foreach=True (either numerics),
    against the oracle's foreach mode."""
    _random_configuration_bf16_state(oracle_mod, 400 + seed, foreach=True)


def _random_configuration_bf16_state(oracle_mod, seed, foreach):
    import adana_amd
    from test_gpu_bf16 import _bits, _check, _diag_close, _to_gpu16
    from test_gpu_parity import STAR_HARD_CASES

    O = oracle_mod
    rng, star, _, groups, hp = _draw(seed)
    shapes = [s for ss, _ in groups for s in ss]
    print(f"case: random bf16-state configuration seed {seed} foreach {foreach}: star {star} groups {len(groups)} "
          f"tensors {len(shapes)} elements {sum(int(np.prod(s)) for s in shapes)} {hp}", flush=True)
    host = [[O.f32_to_bf16(_normal(rng, s, 0.02)) for s in ss] for ss, _ in groups]
    gpu = [[torch.nn.Parameter(_to_gpu16(h)) for h in hs] for hs in host]
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls([dict(params=ps, **gkw) for ps, (_, gkw) in zip(gpu, groups)], use_foreach=foreach, **hp)
    orc = O.OracleOptimizer(
        groups=[O.OracleGroup(params=hs, lr=gkw["lr"], delta=gkw["delta"], epsilon=gkw["epsilon"],
                              weight_decay=gkw["weight_decay"]) for hs, (_, gkw) in zip(host, groups)],
        star=star, peak_lr=hp["lr"], kappa=hp["kappa"], clipsnr=hp["clipsnr"], wd_decaying=hp["wd_decaying"],
        wd_ts=hp["wd_ts"], gamma_3_factor=hp["gamma_3_factor"], bf16=True, numerics=hp["numerics"],
        foreach=foreach)
    keys = ("m", "v", "tau") if star else ("m", "v")
    for k in range(7):
        for g, og, (_, gkw) in zip(opt.param_groups, orc.groups, groups):
            g["lr"] = og.lr = gkw["lr"] * float(rng.uniform(0.5, 1.5))
        grads = []
        for ps, ss in zip(gpu, (ss for ss, _ in groups)):
            gs = []
            for p, s in zip(ps, ss):
                u = rng.random()
                if u < 0.12:
                    p.grad = None
                    gs.append(None)
                    continue
                g = _normal(rng, s, float(10 ** rng.uniform(-5, -1)))
                g16 = O.f32_to_bf16(np.zeros_like(g) if u < 0.18 else g)
                p.grad = _to_gpu16(g16)
                gs.append(g16)
            grads.append(gs)
        opt.step()
        orc.step(grads)
        torch.cuda.synchronize()
        for gi, (ps, hs) in enumerate(zip(gpu, host)):
            for pi, (p, h) in enumerate(zip(ps, hs)):
                st, ost = opt.state[p], orc.state.get(id(h))
                tag = f"seed {seed} k={k} group {gi} tensor {pi} shape {h.shape}"
                if ost is None:
                    assert len(st) == 0, tag
                    continue
                assert st["step"] == ost["step"], tag
                for key in keys:
                    _check(_bits(st[key]), ost[key], f"{tag} {key}")
                got = _bits(p)
                _check(got, h, f"{tag} p", STAR_HARD_CASES if star else 0)
                h[...] = got.reshape(h.shape)
                _diag_close([float(st[key]) for key in O.DIAG_KEYS], [float(ost[key]) for key in O.DIAG_KEYS], tag)
    opt._check_slab_guards()          # nothing written outside the state tensors


@pytest.mark.parametrize("seed", range(16))
def test_random_configuration_with_clipping(oracle_mod, seed):
    """The same draws (fp32 or bf16 master) with clip_grad_norm_ through the
    optimizer before every step, its scaling fused into the step: max_norm
    drawn around the gradients' norm (clipping or not), the clipped gradient
    written back or not; the total norm, the written-back gradients and the
    step checked against the oracle's clip (torch's formula) and step; every
    fourth seed with use_foreach=True."""
    from test_gpu_clip import _clipped_pair_step

    O = oracle_mod
    rng, star, master, groups, hp = _draw(200 + seed)
    hp["foreach"] = seed % 4 == 3
    if sum(int(np.prod(s)) for ss, _ in groups for s in ss) == 0:
        groups[0][0].append((100,))                      # something to clip
    write_back = bool(rng.integers(2))
    print(f"case: random clipped configuration seed {seed}: star {star} master {master} "
          f"write_back {write_back} {hp}", flush=True)

    def param(s):
        x = _normal(rng, s, 0.02)
        return O.f32_to_bf16(x) if master else x

    pair = Pair(O, star, [([param(s) for s in ss], gkw) for ss, gkw in groups], master=master, **hp)
    for k in range(5):
        std = float(10 ** rng.uniform(-4, -1))
        grads = [[_normal(rng, s, std) for s in ss] for ss, _ in groups]
        norm = float(np.sqrt(sum(float(np.sum(np.square(g, dtype=np.float64))) for gs in grads for g in gs)))
        max_norm = max(norm, 1e-12) * float(10 ** rng.uniform(-1, 0.5))
        if master:
            grads = [[O.f32_to_bf16(g).reshape(g.shape) for g in gs] for gs in grads]
        _clipped_pair_step(pair, O, grads, max_norm, write_back, bf16=master)
        pair.compare(where=f"seed {seed} k={k}")
