"""Parity at the headline configuration's full size: Dana-Star-MK4 over the
north-star parameter list (2,645,527,040 fp32 parameters in 194 tensors:
d_model 2560, 32 layers, MLP 4x, vocab 50304, tied embedding; two weight-decay
groups as src/models/base.py:503-561; launcher hyper-parameters as
scripts/launch.sh:36-40,188-223), with row-sparse embedding gradients.

The oracle cannot run 2.6 G elements in seconds, but the update is
element-wise, so it replays a random sample of every tensor's elements from
their inputs exactly.  Bars:
  * sampled m, v, tau: bit-exact;
  * sampled p: bit-exact except the Dana-Star pow's rare rounding-boundary
    cases (at most STAR_HARD_CASES per tensor per step, each within
    STAR_P_ULPS ulps of max(|p_before|, |p_after|));
  * gradient_norm and m_norm of every tensor (reductions over all of its
    elements): rtol 1e-5 against binary64 reductions of the full tensors.
"""
import os
import sys

import numpy as np
import pytest
import torch

from helpers import ulp_diff
from test_gpu_parity import STAR_HARD_CASES, STAR_P_ULPS

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"
SAMPLES = 1024          # per tensor, plus its first and last element


def test_north_star_list_sampled_parity(oracle_mod):
    import adana_amd
    from bench import gpt_shapes

    O = oracle_mod
    decay, nodecay = gpt_shapes(50304, 2560, 32)
    assert sum(int(np.prod(s)) for s in decay + nodecay) == 2_645_527_040
    print("case: north-star list at full size, 3 steps, sampled oracle replay", flush=True)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(0)
    p_d = [torch.nn.Parameter(torch.empty(s, device=DEV).normal_(0, 0.02, generator=gen)) for s in decay]
    p_n = [torch.nn.Parameter(torch.empty(s, device=DEV).normal_(0, 0.02, generator=gen)) for s in nodecay]
    hp = dict(lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, clipsnr=2.0, wd_decaying=True, wd_ts=10.0)
    wd = {0: 0.4, 1: 0.0}
    opt = adana_amd.DANA_STAR_MK4([{"params": p_d, "weight_decay": wd[0]},
                                   {"params": p_n, "weight_decay": wd[1]}], **hp)
    params = p_d + p_n
    group = [0] * len(p_d) + [1] * len(p_n)
    rng = np.random.default_rng(7)
    idx = []
    for p in params:
        n = p.numel()
        pick = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, size=min(n, SAMPLES))]))
        idx.append(torch.from_numpy(pick).to(DEV))

    def gather(ts):
        return [t.detach().reshape(-1).index_select(0, ix).cpu().numpy() for t, ix in zip(ts, idx)]

    host_p = gather(params)
    host_m = [np.zeros_like(x) for x in host_p]
    host_v = [np.zeros_like(x) for x in host_p]
    host_tau = [np.zeros_like(x) for x in host_p]
    emb = len(p_d)                                       # the tied embedding opens the no-decay group
    assert tuple(params[emb].shape) == (50304, 2560)
    for t in range(1, 4):
        gen.manual_seed(1000 + t)
        for p in params:
            p.grad = torch.empty_like(p).normal_(0, 1e-3, generator=gen)
        rows = (torch.rand((50304, 1), device=DEV, generator=gen) < 0.1).float()
        params[emb].grad.mul_(rows)                      # row-sparse embedding gradient
        host_g = gather([p.grad for p in params])
        gnorm = [float(torch.linalg.vector_norm(p.grad.double())) for p in params]
        p_before = [x.copy() for x in host_p]
        opt.step()
        torch.cuda.synchronize()
        got_p = gather(params)
        got_m = gather([opt.state[p]["m"] for p in params])
        got_v = gather([opt.state[p]["v"] for p in params])
        got_tau = gather([opt.state[p]["tau"] for p in params])
        for i in range(len(params)):
            osc = O.step_scalars(lr=hp["lr"], peak_lr=hp["lr"], delta=hp["delta"], kappa=hp["kappa"],
                                 epsilon=hp["epsilon"], weight_decay=wd[group[i]], clipsnr=hp["clipsnr"],
                                 wd_decaying=hp["wd_decaying"], wd_ts=hp["wd_ts"], gamma_3_factor=1.0, t=t)
            O.element_step(True, host_p[i], host_g[i], host_m[i], host_v[i], host_tau[i], osc)
            where = (t, i, tuple(params[i].shape))
            assert ulp_diff(got_m[i], host_m[i]).max() == 0, where
            assert ulp_diff(got_v[i], host_v[i]).max() == 0, where
            assert ulp_diff(got_tau[i], host_tau[i]).max() == 0, where
            d = ulp_diff(got_p[i], host_p[i])
            bad = np.nonzero(d)[0]
            assert bad.size <= STAR_HARD_CASES, (where, bad.size)
            for j in bad:
                scale = max(abs(float(p_before[i][j])), abs(float(host_p[i][j])))
                assert abs(float(got_p[i][j]) - float(host_p[i][j])) <= STAR_P_ULPS * np.spacing(np.float32(scale)), where
            host_p[i][...] = got_p[i]                    # continue from the GPU's p
            st = opt.state[params[i]]
            np.testing.assert_allclose(float(st["gradient_norm"]), gnorm[i], rtol=1e-5, err_msg=str(where))
            mnorm = float(torch.linalg.vector_norm(st["m"].double()))
            np.testing.assert_allclose(float(st["m_norm"]), mnorm, rtol=1e-5, err_msg=str(where))
            assert st["step"] == t
    del opt, params, p_d, p_n
    torch.cuda.empty_cache()
