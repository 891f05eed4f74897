"""Seeded random configurations of the step against the oracle.

Each case draws, from its seed: the variant (ADana / Dana-MK4 or
Dana-Star-MK4), fp32 parameters or the bf16-master extension, 1-3 parameter
groups with their own lr, delta, epsilon and weight decay, 1-10 tensors per
group (empty, tiny, ragged and up to 70,000-element sizes, 1-D and 2-D), kappa
from the values that select each pow kind (0, 0.5, 0.85, 1, 1.5, 2, 3),
clipsnr, decaying weight decay, wd_ts and gamma_3_factor.  It then takes 7
steps (crossing t = delta for the smallest deltas) with a new lr per group
each step, gradients of random scale with some all-zero tensors, and some
gradients None (that tensor skips the step and keeps its state), and checks
every step against the oracle (src/optim/adana.py:101-153,
src/optim/dana_star_mk4.py:137-203) to the bars of test_gpu_parity.py: m, v
and tau bit-exact, p bit-exact (Dana-Star: at most 2 hard-case elements per
tensor, within 2 scaled ulp), diagnostics rtol 1e-5.
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
    return rng, star, master, groups, hp


@pytest.mark.parametrize("seed", range(48))
def test_random_configuration(oracle_mod, seed):
    O = oracle_mod
    rng, star, master, groups, hp = _draw(seed)
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
