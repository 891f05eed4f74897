"""Parity at the full sizes of the benchmarked configurations, with the
workloads' own lists and hyper-parameters (bench.workload):
  * north_star: Dana-Star-MK4, 2,645,527,040 fp32 parameters in 194 tensors
    (d_model 2560, 32 layers, MLP 4x, vocab 50304, tied), row-sparse
    embedding gradients;
  * c4: ADana on the same list with bf16 parameters, fp32 master/m/v and
    bf16 gradients;
  * c3: Dana-Star-MK4, 1,311,082,496 parameters (d_model 2048, 24 layers).
Two weight-decay groups as src/models/base.py:503-561; launcher
hyper-parameters as scripts/launch.sh:36-40,188-223.

The oracle cannot run billions of elements in seconds, but the update is
element-wise, so it replays a random sample of every tensor's elements from
their inputs exactly.  Bars:
  * sampled m, v, tau, ADana's master: bit-exact; bf16 params: equal to
    RNE(master) (ADana);
  * sampled Dana-Star p: bit-exact except the pow's rare rounding-boundary
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
STEPS = 3
ELEMENTS = {"north_star": 2_645_527_040, "c4": 2_645_527_040, "c3": 1_311_082_496}


@pytest.mark.parametrize("name", ["north_star", "c4", "c3"])
def test_full_size_sampled_parity(oracle_mod, name):
    import adana_amd
    from bench import workload

    O = oracle_mod
    w = workload(name)
    star, master, hp = w["star"], w["master"], w["hp"]
    shapes = [s for g in w["groups"] for s in g]
    assert sum(int(np.prod(s)) for s in shapes) == ELEMENTS[name]
    print(f"case: {name} at full size ({ELEMENTS[name]} params), {STEPS} steps, sampled oracle replay", flush=True)
    pdtype = torch.bfloat16 if master else torch.float32
    gen = torch.Generator(device=DEV)
    gen.manual_seed(0)
    groups, params, wd_of = [], [], []
    for gi, gshapes in enumerate(w["groups"]):
        ps = [torch.nn.Parameter(torch.empty(s, device=DEV).normal_(0, 0.02, generator=gen).to(pdtype))
              for s in gshapes]
        wd = hp["weight_decay"] * w["group_wd"][gi]
        groups.append({"params": ps, "weight_decay": wd})
        params += ps
        wd_of += [wd] * len(ps)
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(groups, master_weights=master, **hp)
    sparse_emb = name in ("north_star", "c3")
    emb = len(w["groups"][0])                            # the tied embedding opens the no-decay group
    rng = np.random.default_rng(7)
    idx = []
    for p in params:
        n = p.numel()
        pick = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, size=min(n, SAMPLES))]))
        idx.append(torch.from_numpy(pick).to(DEV))

    def gather(ts):
        return [t.detach().reshape(-1).index_select(0, ix).float().cpu().numpy() for t, ix in zip(ts, idx)]

    host_p = gather(params)                              # master mode: the master starts as float(p_bf16)
    host_m = [np.zeros_like(x) for x in host_p]
    host_v = [np.zeros_like(x) for x in host_p]
    host_tau = [np.zeros_like(x) for x in host_p] if star else [None] * len(params)
    for t in range(1, STEPS + 1):
        gen.manual_seed(1000 + t)
        for p in params:
            p.grad = torch.empty(p.shape, device=DEV).normal_(0, 1e-3, generator=gen).to(pdtype)
        if sparse_emb:
            rows = (torch.rand((params[emb].shape[0], 1), device=DEV, generator=gen) < 0.1).to(pdtype)
            params[emb].grad.mul_(rows)                  # row-sparse embedding gradient
        host_g = gather([p.grad for p in params])
        gnorm = [float(torch.linalg.vector_norm(p.grad.double())) for p in params]
        p_before = [x.copy() for x in host_p]
        opt.step()
        torch.cuda.synchronize()
        got_p = gather([opt.state[p]["master"] for p in params] if master else params)
        got_lp = gather(params) if master else None
        got_m = gather([opt.state[p]["m"] for p in params])
        got_v = gather([opt.state[p]["v"] for p in params])
        got_tau = gather([opt.state[p]["tau"] for p in params]) if star else None
        for i in range(len(params)):
            osc = O.step_scalars(lr=hp["lr"], peak_lr=hp["lr"], delta=hp["delta"], kappa=hp["kappa"],
                                 epsilon=hp["epsilon"], weight_decay=wd_of[i], clipsnr=hp["clipsnr"],
                                 wd_decaying=hp["wd_decaying"], wd_ts=hp["wd_ts"], gamma_3_factor=1.0, t=t)
            O.element_step(star, host_p[i], host_g[i], host_m[i], host_v[i], host_tau[i], osc)
            where = (name, t, i, tuple(params[i].shape))
            assert ulp_diff(got_m[i], host_m[i]).max() == 0, where
            assert ulp_diff(got_v[i], host_v[i]).max() == 0, where
            if star:
                assert ulp_diff(got_tau[i], host_tau[i]).max() == 0, where
                d = ulp_diff(got_p[i], host_p[i])
                bad = np.nonzero(d)[0]
                assert bad.size <= STAR_HARD_CASES, (where, bad.size)
                for j in bad:
                    scale = max(abs(float(p_before[i][j])), abs(float(host_p[i][j])))
                    assert (abs(float(got_p[i][j]) - float(host_p[i][j]))
                            <= STAR_P_ULPS * np.spacing(np.float32(scale))), where
            else:
                assert ulp_diff(got_p[i], host_p[i]).max() == 0, where
                if master:                               # the bf16 parameter is RNE(master)
                    want = O.bf16_to_f32(O.f32_to_bf16(host_p[i])).reshape(host_p[i].shape)
                    assert np.array_equal(got_lp[i].view(np.uint32), want.view(np.uint32)), where
            host_p[i][...] = got_p[i]                    # continue from the GPU's p
            st = opt.state[params[i]]
            np.testing.assert_allclose(float(st["gradient_norm"]), gnorm[i], rtol=1e-5, err_msg=str(where))
            mnorm = float(torch.linalg.vector_norm(st["m"].double()))
            np.testing.assert_allclose(float(st["m_norm"]), mnorm, rtol=1e-5, err_msg=str(where))
            assert st["step"] == t
    del opt, params, groups
    torch.cuda.empty_cache()
