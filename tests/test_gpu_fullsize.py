"""Parity at the full sizes of the benchmarked configurations, with the
workloads' own lists and hyper-parameters (bench.workload):
  * north_star: Dana-Star-MK4, 2,645,527,040 fp32 parameters in 194 tensors
    (d_model 2560, 32 layers, MLP 4x, vocab 50304, tied), row-sparse
    embedding gradients;
  * c4: ADana on the same list with bf16 parameters, fp32 master/m/v and
    bf16 gradients;
  * c3: Dana-Star-MK4, 1,311,082,496 parameters (d_model 2048, 24 layers);
  * c2: Dana-MK4, 50,938,880 parameters in 67 tensors, 1-D gradients x 0.1,
    under the bench's lr schedule, the reference's cos_inf through LambdaLR (a new group lr every step);
  * c5: Dana-Star-MK4 over 10,000 log-uniform tensors (94,406,322
    parameters), 5% of them with all-zero gradients.
Ten steps each, so every run crosses t = delta = 8, where alpha = 0.5 and
ATen's lerp takes its second branch.
Two weight-decay groups as src/models/base.py:503-561; launcher
hyper-parameters as scripts/launch.sh:36-40,188-223.

The oracle cannot run billions of elements in seconds, but the update is
element-wise, so for north_star, c4 and c3 it replays a random sample of
every tensor's elements (1,024 and the first and last) from their inputs
exactly; c2 and c5 (at most FULL_REPLAY elements) are replayed whole, every
element of every tensor at every step.  Bars:
  * replayed m, v, tau, ADana's master: bit-exact; bf16 params: equal to
    RNE(master) (ADana);
  * replayed Dana-Star p: bit-exact except the pow's rare rounding-boundary
    cases (at most STAR_HARD_CASES per tensor per step, each within
    STAR_P_ULPS ulps of max(|p_before|, |p_after|));
  * all five diagnostics of every tensor, reductions over all of its
    elements, rtol 1e-5: gradient_norm and m_norm against binary64 norms of
    the full gradient and m; current_alpha and auto_factor_mean against
    binary64 means of alpha_factor and mfac recomputed from the full
    post-step m, v (and tau) by torch ops on the device (each element's m,
    v, tau is the oracle's, as the samples show); current_kappa_factor
    against their ratio (NaN for all-zero gradients).
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
FULL_REPLAY = 100_000_000   # configurations of at most this many elements: every element replayed
STEPS = 10
ELEMENTS = {"north_star": 2_645_527_040, "c4": 2_645_527_040, "c3": 1_311_082_496, "c2": 50_938_880,
            "c5": 94_406_322}


@pytest.mark.parametrize("name", ["north_star", "c4", "c3", "c2", "c5"])
def test_full_size_parity(oracle_mod, name):
    import adana_amd
    from bench import workload

    O = oracle_mod
    w = workload(name)
    star, master, hp = w["star"], w["master"], w["hp"]
    shapes = [s for g in w["groups"] for s in g]
    assert sum(int(np.prod(s)) for s in shapes) == ELEMENTS[name]
    full = ELEMENTS[name] <= FULL_REPLAY
    print(f"case: {name} at full size ({ELEMENTS[name]} params), {STEPS} steps, "
          f"{'full' if full else 'sampled'} oracle replay", flush=True)
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
    zero = np.random.default_rng(1).random(len(params)) < 0.05
    emb = len(w["groups"][0])                            # the tied embedding opens the no-decay group
    rng = np.random.default_rng(7)
    idx = []
    for p in params:
        n = p.numel()
        pick = np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, size=min(n, SAMPLES))]))
        idx.append(None if full else torch.from_numpy(pick).to(DEV))

    def gather(ts):
        if full:
            return [t.detach().reshape(-1).float().cpu().numpy() for t in ts]
        return [t.detach().reshape(-1).index_select(0, ix).float().cpu().numpy() for t, ix in zip(ts, idx)]

    host_p = gather(params)                              # master mode: the master starts as float(p_bf16)
    host_m = [np.zeros_like(x) for x in host_p]
    host_v = [np.zeros_like(x) for x in host_p]
    host_tau = [np.zeros_like(x) for x in host_p] if star else [None] * len(params)
    from bench import C2_SCHEDULE, cos_inf_schedule

    sched, factor = None, None
    if w["schedule"] == "cos_inf":
        # as the bench and src/main.py:411-423: LambdaLR over the reference's cos_inf factor
        factor = cos_inf_schedule(**C2_SCHEDULE)
        sched = torch.optim.lr_scheduler.LambdaLR(opt, factor)
    for t in range(1, STEPS + 1):
        lr = opt.param_groups[0]["lr"]
        assert all(g["lr"] == lr for g in opt.param_groups)
        assert lr == (hp["lr"] * factor(t - 1) if sched is not None else hp["lr"])
        gen.manual_seed(1000 + t)
        for i, p in enumerate(params):
            p.grad = torch.empty(p.shape, device=DEV).normal_(0, 1e-3, generator=gen).to(pdtype)
            if name == "c2" and p.dim() == 1:
                p.grad.mul_(0.1)                         # the bench's C2: 1-D gradients x 0.1
            if name == "c5" and zero[i]:
                p.grad.zero_()                           # the bench's C5: 5% all-zero gradients
        if sparse_emb:
            rows = (torch.rand((params[emb].shape[0], 1), device=DEV, generator=gen) < 0.1).to(pdtype)
            params[emb].grad.mul_(rows)                  # row-sparse embedding gradient
        host_g = gather([p.grad for p in params])
        gnorm = [float(torch.linalg.vector_norm(p.grad.double())) for p in params]
        p_before = [x.copy() for x in host_p]
        opt.step()
        if sched is not None:
            sched.step()
        torch.cuda.synchronize()
        got_p = gather([opt.state[p]["master"] for p in params] if master else params)
        got_lp = gather(params) if master else None
        got_m = gather([opt.state[p]["m"] for p in params])
        got_v = gather([opt.state[p]["v"] for p in params])
        got_tau = gather([opt.state[p]["tau"] for p in params]) if star else None
        for i in range(len(params)):
            osc = O.step_scalars(lr=lr, peak_lr=hp["lr"], delta=hp["delta"], kappa=hp["kappa"],
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
            ca, afm = _alpha_mfac_means(star, st["m"], st["v"], st.get("tau"), t, hp)
            got = [float(st[k]) for k in ("current_alpha", "auto_factor_mean", "current_kappa_factor")]
            np.testing.assert_allclose(got, [ca, afm, ca / afm if afm else float("nan")], rtol=1e-5,
                                       atol=0, equal_nan=True, err_msg=str(where))
            assert st["step"] == t
    del opt, params, groups
    torch.cuda.empty_cache()


def _alpha_mfac_means(star, m, v, tau, t, hp, block=1 << 26):
    """Binary64 means of alpha_factor and mfac over a whole tensor, from its
    post-step m, v (and tau) at step t (src/optim/adana.py:107-123;
    src/optim/dana_star_mk4.py:143-174), block by block on the device."""
    mf, vf = m.detach().reshape(-1), v.detach().reshape(-1)
    tf = tau.detach().reshape(-1) if star else None
    e = 1.0 - hp["kappa"]
    clip = hp["clipsnr"]
    s_af = s_mf = 0.0
    for a in range(0, mf.numel(), block):
        mm, vv = mf[a:a + block].double(), vf[a:a + block].double()
        se = torch.sqrt(vv) + hp["epsilon"]
        if star:
            ta = tf[a:a + block].double()
            ct = torch.clamp(ta, max=0.5)
            treg = torch.clamp(ct / (1.0 - ct), min=1.0 / (1.0 + t))
            mfac = torch.abs(mm) * torch.sqrt(treg) / se / treg
            af = torch.clamp(ta * t, min=1.0) ** e * mfac
        else:
            mfac = torch.abs(mm) / se
            af = (1.0 + t) ** e * mfac
        if clip is not None:
            af = torch.clamp(af, max=clip)
        s_af += float(af.sum())
        s_mf += float(mfac.sum())
    n = mf.numel()
    return s_af / n, s_mf / n


def _norm64(t: torch.Tensor, block: int = 1 << 28) -> float:
    """Binary64 2-norm of a large tensor, block by block (no full-size copy)."""
    f = t.detach().reshape(-1)
    s = 0.0
    for a in range(0, f.numel(), block):
        s += float(torch.sum(f[a:a + block].double() ** 2))
    return s ** 0.5


def test_single_tensor_beyond_2_31_elements(oracle_mod):
    """One Dana-Star-MK4 tensor of 2^31 + 1027 elements (per-tensor offsets,
    chunk indices and fold ranges past 2^31; a ragged last chunk), 2 steps.
    Sampled oracle replay as above, with the elements around index 2^31 and
    the last ones always in the sample; gradient_norm and m_norm against
    binary64 reductions of the whole tensor."""
    import adana_amd

    O = oracle_mod
    n = (1 << 31) + 1027
    print(f"case: one tensor of {n} elements, 2 steps", flush=True)
    hp = dict(lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=0.4, clipsnr=2.0, wd_decaying=True,
              wd_ts=10.0)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(3)
    p = torch.nn.Parameter(torch.empty(n, device=DEV).normal_(0, 0.02, generator=gen))
    opt = adana_amd.DANA_STAR_MK4([p], **hp)
    rng = np.random.default_rng(11)
    edge = [0, 1, (1 << 31) - 4, (1 << 31) - 1, 1 << 31, (1 << 31) + 1, n - 1027, n - 3, n - 2, n - 1]
    pick = np.unique(np.concatenate([edge, rng.integers(0, n, size=SAMPLES)]))
    ix = torch.from_numpy(pick).to(DEV)

    def gather(t):
        return t.detach().reshape(-1).index_select(0, ix).float().cpu().numpy()

    hp_, hg = gather(p), None
    hm, hv, ht = (np.zeros_like(hp_) for _ in range(3))
    for t in (1, 2):
        gen.manual_seed(2000 + t)
        p.grad = torch.empty(n, device=DEV).normal_(0, 1e-3, generator=gen)
        hg = gather(p.grad)
        gnorm = _norm64(p.grad)
        before = hp_.copy()
        opt.step()
        torch.cuda.synchronize()
        st = opt.state[p]
        osc = O.step_scalars(lr=hp["lr"], peak_lr=hp["lr"], delta=hp["delta"], kappa=hp["kappa"],
                             epsilon=hp["epsilon"], weight_decay=hp["weight_decay"], clipsnr=hp["clipsnr"],
                             wd_decaying=True, wd_ts=hp["wd_ts"], gamma_3_factor=1.0, t=t)
        O.element_step(True, hp_, hg, hm, hv, ht, osc)
        for key, want in (("m", hm), ("v", hv), ("tau", ht)):
            assert ulp_diff(gather(st[key]), want).max() == 0, (t, key)
        got = gather(p)
        d = ulp_diff(got, hp_)
        bad = np.nonzero(d)[0]
        assert bad.size <= STAR_HARD_CASES, (t, bad.size)
        for j in bad:
            scale = max(abs(float(before[j])), abs(float(hp_[j])))
            assert abs(float(got[j]) - float(hp_[j])) <= STAR_P_ULPS * np.spacing(np.float32(scale)), t
        hp_[...] = got
        np.testing.assert_allclose(float(st["gradient_norm"]), gnorm, rtol=1e-5)
        np.testing.assert_allclose(float(st["m_norm"]), _norm64(st["m"]), rtol=1e-5)
        assert st["step"] == t
    del opt, p
    torch.cuda.empty_cache()


def test_clip_single_tensor_beyond_2_31_elements(oracle_mod):
    """clip_grad_norm_ over one gradient of 2^31 + 1027 elements: the total
    within 2e-6 of the binary64 norm of the whole tensor, and the sampled
    clipped gradients (around index 2^31 and at the end included) equal to
    torch's binary32 product with the coefficient of that total."""
    import adana_amd

    O = oracle_mod
    n = (1 << 31) + 1027
    print(f"case: clip_grad_norm_ over one gradient of {n} elements", flush=True)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(5)
    p = torch.nn.Parameter(torch.zeros(1, device=DEV).expand(n))     # no storage needed for p
    p.grad = torch.empty(n, device=DEV).normal_(0, 1e-3, generator=gen)
    rng = np.random.default_rng(13)
    edge = [0, (1 << 31) - 1, 1 << 31, (1 << 31) + 1, n - 1]
    ix = torch.from_numpy(np.unique(np.concatenate([edge, rng.integers(0, n, size=SAMPLES)]))).to(DEV)
    g0 = p.grad.index_select(0, ix).cpu().numpy()
    want = _norm64(p.grad)
    total = adana_amd.clip_grad_norm_([p], 0.5)
    torch.cuda.synchronize()
    assert abs(float(total) - want) <= 2e-6 * want
    coef = O.clip_coef(np.float32(float(total)), 0.5)
    assert coef < 1.0                                              # the norm (~46) is above max_norm
    got = p.grad.index_select(0, ix).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), O.clip_scale(g0, coef).view(np.uint32))
    del p
    torch.cuda.empty_cache()


def test_manau_dana_branch_full_size(oracle_mod):
    """Manau on the north-star model (bench.manau_model: 2,516,582,400 Muon and
    128,944,640 Dana-Star-MK4 parameters), 2 steps with new gradients each:
    the Dana branch's sampled m, v, tau bit-exact against the oracle's Manau
    restatement replayed on the same elements, p under the pow bar, and
    gradient_norm / m_norm of every branch tensor against binary64
    reductions of the whole tensor."""
    import contextlib
    import io

    import adana_amd
    from bench import manau_grads, manau_model

    O = oracle_mod
    print("case: Manau's Dana branch on the north-star model, 2 steps", flush=True)
    groups, params, hp = manau_model(seed=0)
    with contextlib.redirect_stdout(io.StringIO()):
        opt = adana_amd.Manau(groups, **hp)
    rng = np.random.default_rng(17)
    dana, picks, ogroups, host = [], [], [], []
    for g in groups:
        mine = [p for p in g["params"] if not opt.state[p]["use_muon"]]
        if not mine:
            continue
        hs = []
        for p in mine:
            n = p.numel()
            ix = torch.from_numpy(np.unique(np.concatenate([[0, n - 1], rng.integers(0, n, size=SAMPLES)]))).to(DEV)
            dana.append(p)
            picks.append(ix)
            hs.append(p.detach().reshape(-1).index_select(0, ix).cpu().numpy())
        host.append(hs)
        ogroups.append(O.OracleManauGroup(params=hs, use_muon=[False] * len(hs), lr=hp["lr"],
                                          weight_decay=g["weight_decay"], delta=hp["delta"], kappa=hp["kappa"],
                                          clipsnr=hp["clipsnr"], wd_decaying=hp["wd_decaying"], wd_ts=hp["wd_ts"]))
    orc = O.OracleManau(groups=ogroups, peak_lr=hp["lr"])
    flat_host = [h for hs in host for h in hs]
    assert sum(p.numel() for p in dana) == 128_944_640

    def gather(ts):
        return [t.detach().reshape(-1).index_select(0, ix).float().cpu().numpy() for t, ix in zip(ts, picks)]

    for t in (1, 2):
        if t > 1:
            manau_grads(params, groups[1]["params"][0], 100 + t)
        gs = gather([p.grad for p in dana])
        gnorm = [_norm64(p.grad) for p in dana]
        before = [x.copy() for x in flat_host]
        opt.step()
        torch.cuda.synchronize()
        k = 0
        og = []
        for hs in host:
            og.append(gs[k:k + len(hs)])
            k += len(hs)
        orc.step(og)
        got = {key: gather([opt.state[p][key] for p in dana]) for key in ("dana_m", "dana_v", "dana_tau")}
        got_p = gather(dana)
        for i, p in enumerate(dana):
            ost = orc.state[id(flat_host[i])]
            where = (t, i, tuple(p.shape))
            for key in ("dana_m", "dana_v", "dana_tau"):
                assert ulp_diff(got[key][i], ost[key]).max() == 0, (where, key)
            d = ulp_diff(got_p[i], flat_host[i])
            bad = np.nonzero(d)[0]
            assert bad.size <= STAR_HARD_CASES, (where, bad.size)
            for j in bad:
                scale = max(abs(float(before[i][j])), abs(float(flat_host[i][j])))
                assert abs(float(got_p[i][j]) - float(flat_host[i][j])) <= STAR_P_ULPS * np.spacing(np.float32(scale))
            flat_host[i][...] = got_p[i]                     # continue from the GPU's p
            st = opt.state[p]
            np.testing.assert_allclose(float(st["gradient_norm"]), gnorm[i], rtol=1e-5, err_msg=str(where))
            np.testing.assert_allclose(float(st["m_norm"]), _norm64(st["dana_m"]), rtol=1e-5, err_msg=str(where))
    del opt, params, groups
    torch.cuda.empty_cache()
