"""The step kernel's foreach instances (ADANA_FOREACH: the reference's
use_foreach=True path, src/optim/adana.py:229-370 and
src/optim/dana_star_mk4.py:298-536) against the oracle's foreach mode, which
tests/test_oracle_foreach.py pins to the reference's own foreach runs: the
golden scenarios in both of the reference's modes (and, at the checkpoints,
against the reference's fixtures themselves), C1's size, float32 and
bf16-master lists that take the two-group launches, and the reference's
bfloat16 path in both modes, including a tensor on the element-wise path.
Bars as in tests/test_gpu_parity.py and tests/test_gpu_bf16.py: m, v, tau
bit-exact; ADana's p bit-exact; Dana-Star's p bit-exact but for the pow's
hard cases (at most STAR_HARD_CASES elements per tensor per step)."""
import numpy as np
import pytest
import torch

from helpers import load_golden_case, load_golden_inputs, ulp_diff
from test_gpu_bf16 import _bits, _check, _diag_close, _to_gpu16
from test_gpu_parity import STAR_HARD_CASES, Pair, _normal, _scaled_ulps

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("case", ["adana", "dana_mk4", "adana_k1_nowd", "dana_star", "dana_star_mk4",
                                  "dana_star_mk4_k05"])
def test_foreach_golden_on_gpu(oracle_mod, case, numerics):
    """The golden scenario with use_foreach=True: every step against the
    oracle's foreach mode, and every checkpoint against the reference's own
    foreach run (tests/golden/<case>.foreach[_eager].npz): m and v
    bit-exact; tau bit-exact (compiled) or within 2 ulp (eager: torch's CPU
    sqrt); p within 2 (compiled) or 3 (eager) ulp of the tensor's largest
    |p|, ADana's compiled p bit-exact."""
    print("case: foreach golden", case, numerics, flush=True)
    meta, p0, grads, has_grad = load_golden_inputs()
    gold = load_golden_case(case, "foreach" if numerics == "compiled" else "foreach_eager")
    kw = dict(meta["cases"][case]["kwargs"])
    star = meta["cases"][case]["class"] == "DANA_STAR_MK4"
    idx = [[i for i in range(len(p0)) if meta["group_of"][i] == gi] for gi in range(2)]
    groups = [([p0[i] for i in idx[gi]], {"weight_decay": kw["weight_decay"] * meta["group_wd_scale"][gi]})
              for gi in range(2)]
    pair = Pair(oracle_mod, star, groups, numerics=numerics, foreach=True, **kw)
    order = [i for gi in range(2) for i in idx[gi]]
    for k in range(1, meta["n_steps"] + 1):
        lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        pair.set_lr([lr, lr])
        pair.step([[grads[k - 1][i] if has_grad[k - 1, i] else None for i in idx[gi]] for gi in range(2)])
        if k in meta["checkpoints"]:
            for p, i in zip([p for tp in pair.gpu_params for p in tp], order):
                st = pair.opt.state[p]
                for key in ("m", "v", "tau") if star else ("m", "v"):
                    if key in st:
                        bar = 2 if (key == "tau" and numerics == "eager") else 0
                        d = ulp_diff(st[key].cpu().numpy(), gold[f"{key}{i}_t{k}"])
                        assert d.max() <= bar, (case, numerics, k, i, key, int(d.max()))
                ref = gold[f"p{i}_t{k}"]
                err = _scaled_ulps(p.detach().cpu().numpy(), ref, np.full(ref.shape, np.abs(ref).max(), np.float32))
                bar = 3 if numerics == "eager" else (2 if star else 0)
                assert err.max() <= bar, (case, numerics, k, i, err.max())
        pair.compare(where=f"foreach {case} {numerics} t={k}")


@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
def test_foreach_c1_size(oracle_mod, star):
    """C1's tensor (1024 x 4096) and a 1-D tensor of odd length in one list,
    use_foreach=True, 10 steps crossing t = delta, against the oracle without
    re-synchronising (ADana bit-exact)."""
    print("case: foreach C1 size star", star, flush=True)
    rng = np.random.default_rng(5)
    pair = Pair(oracle_mod, star, [([_normal(rng, (1024, 4096), 0.02), _normal(rng, (4099,), 0.02)], {})],
                foreach=True, lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=0.4,
                clipsnr=2.0 if star else None, wd_decaying=True, wd_ts=10.0, gamma_3_factor=0.7)
    for t in range(1, 11):
        pair.step([[_normal(rng, (1024, 4096), 1e-3), _normal(rng, (4099,), 1e-3)]])
        pair.compare(resync=star, where=f"t={t}")


SIZES = [9_000_000, 6_000_003, 5_000_001, 1027]     # 19,540 chunks: two-group launches on a 256-CU MI355X


@pytest.mark.parametrize("master", [False, True], ids=["fp32", "master"])
@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
def test_foreach_two_group_grid(oracle_mod, star, master):
    """~20M elements (the two-group launch range), float32 and bf16-master,
    2 steps, use_foreach=True, every element against the oracle."""
    O = oracle_mod
    print(f"case: foreach grid star {star} master {master} sizes {SIZES}", flush=True)
    rng = np.random.default_rng(33)

    def arr(n, std):
        x = _normal(rng, (n,), std)
        return O.f32_to_bf16(x) if master else x

    pair = Pair(O, star, [([arr(n, 0.02) for n in SIZES], {})], master=master, foreach=True, lr=1e-3,
                delta=8.0, kappa=0.85, weight_decay=0.1, clipsnr=2.0, wd_decaying=True, wd_ts=10.0)
    for k in range(2):
        pair.step([[arr(n, 1e-3) for n in SIZES]])
        pair.compare(where=f"foreach grid k={k}")


BF16_SIZES = [[37, 3 * 129, 40 * 17, 4099, 70_001], [9_000_000, 6_000_003, 5_000_001, 1027]]


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("sizes", BF16_SIZES, ids=["small", "grid"])
@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
def test_foreach_bf16_state(oracle_mod, star, sizes, numerics):
    """The reference's bfloat16 path with use_foreach=True, compiled and
    eager: m, v, tau bit-exact, p bit-exact but for Dana-Star's pow hard
    cases, the five bfloat16 diagnostics within 1 bfloat16 ulp; 3 steps with
    the lr moving, one tensor a view 2 bytes into a buffer (the element-wise
    path), two groups (weight decay on the first)."""
    import adana_amd

    O = oracle_mod
    print(f"case: foreach bf16 state star {star} sizes {sizes} {numerics}", flush=True)
    rng = np.random.default_rng(34)
    host = [O.f32_to_bf16(rng.normal(0, 0.02, n).astype(np.float32)) for n in sizes]
    gpu = []
    flat = torch.empty(sizes[1] + 1, dtype=torch.bfloat16, device=DEV)
    for i, h in enumerate(host):
        if i == 1:
            v = flat[1:]
            v.copy_(_to_gpu16(h))
            gpu.append(torch.nn.Parameter(v))
        else:
            gpu.append(torch.nn.Parameter(_to_gpu16(h)))
    hp = dict(lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=10.0, gamma_3_factor=0.7)
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls([dict(params=gpu[:3], weight_decay=0.1), dict(params=gpu[3:], weight_decay=0.0)],
              use_foreach=True, numerics=numerics, **hp)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=host[:3], lr=hp["lr"], weight_decay=0.1),
                                    O.OracleGroup(params=host[3:], lr=hp["lr"], weight_decay=0.0)],
                            star=star, peak_lr=hp["lr"], kappa=hp["kappa"], clipsnr=hp["clipsnr"], wd_decaying=True,
                            wd_ts=hp["wd_ts"], gamma_3_factor=hp["gamma_3_factor"], bf16=True, foreach=True,
                            numerics=numerics)
    for t in range(1, 4):
        lr = 1e-3 * (1.0 - 0.2 * t)
        for g, og in zip(opt.param_groups, orc.groups):
            g["lr"] = og.lr = lr
        g16 = [O.f32_to_bf16(rng.normal(0, 1e-3, n).astype(np.float32)) for n in sizes]
        for p, g in zip(gpu, g16):
            p.grad = _to_gpu16(g)
        opt.step()
        orc.step([g16[:3], g16[3:]])
        torch.cuda.synchronize()
        for i, p in enumerate(gpu):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"foreach bf16 {numerics} star {star} t={t} tensor {i} (n={sizes[i]})"
            for key in ("m", "v", "tau") if star else ("m", "v"):
                _check(_bits(st[key]), ost[key], f"{tag} {key}")
            got = _bits(p)
            _check(got, host[i], f"{tag} p", STAR_HARD_CASES if star else 0)
            host[i][...] = got.reshape(host[i].shape)
            _diag_close([float(st[key]) for key in O.DIAG_KEYS], [float(ost[key]) for key in O.DIAG_KEYS], tag)




@pytest.mark.parametrize("case", ["adana", "dana_mk4", "adana_k1_nowd", "dana_star", "dana_star_mk4",
                                  "dana_star_mk4_k05"])
def test_foreach_bf16_eager_golden_on_gpu(oracle_mod, case):
    """The golden scenario on bfloat16 parameters with use_foreach=True and
    the eager ops: every checkpoint bit-exact against the reference's own run
    (tests/golden/<case>.bf16_foreach_eager.npz) for m, v and tau, and for p
    but for Dana-Star's pow hard cases, 20 steps without re-synchronising."""
    import adana_amd

    O = oracle_mod
    print("case: foreach bf16 eager golden", case, flush=True)
    meta, p0, grads, has_grad = load_golden_inputs()
    gold = load_golden_case(case, "bf16_foreach_eager")
    kw = dict(meta["cases"][case]["kwargs"])
    star = meta["cases"][case]["class"] == "DANA_STAR_MK4"
    gpu = [torch.nn.Parameter(_to_gpu16(O.f32_to_bf16(x))) for x in p0]
    idx = [[i for i in range(len(p0)) if meta["group_of"][i] == gi] for gi in range(2)]
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    wd = kw.pop("weight_decay")
    opt = cls([dict(params=[gpu[i] for i in idx[gi]], weight_decay=wd * meta["group_wd_scale"][gi]) for gi in range(2)],
              use_foreach=True, numerics="eager", **kw)
    for k in range(1, meta["n_steps"] + 1):
        for g in opt.param_groups:
            g["lr"] = kw["lr"] * meta["lr_multiplier"][k - 1]
        for i, p in enumerate(gpu):
            p.grad = _to_gpu16(O.f32_to_bf16(grads[k - 1][i])) if has_grad[k - 1, i] else None
        opt.step()
        if k not in meta["checkpoints"]:
            continue
        torch.cuda.synchronize()
        for i, p in enumerate(gpu):
            _check(_bits(p), gold[f"p{i}_t{k}"], f"{case} p t={k} tensor {i}", STAR_HARD_CASES if star else 0)
            st = opt.state[p]
            for key in (("m", "v", "tau") if star else ("m", "v")) if st else ():
                _check(_bits(st[key]), gold[f"{key}{i}_t{k}"], f"{case} {key} t={k} tensor {i}")


@pytest.mark.parametrize("case", ["adana", "dana_mk4", "dana_star", "dana_star_mk4"])
def test_foreach_nonfinite_gradients_on_gpu(oracle_mod, case):
    """The golden scenario's NaN, +inf and -inf gradient entries
    (nonfinite.inputs.npz) with use_foreach=True: every step against the
    oracle's foreach mode (NaN where the oracle's NaNs are, the usual bars
    elsewhere), and every checkpoint's NaN and inf positions against the
    reference's own foreach run (<case>.foreach_nonfinite.npz)."""
    print("case: foreach non-finite gradients", case, flush=True)
    meta, p0, grads, has_grad = load_golden_inputs("nonfinite.inputs")
    gold = load_golden_case(case, "foreach_nonfinite")
    kw = dict(meta["cases"][case]["kwargs"])
    star = meta["cases"][case]["class"] == "DANA_STAR_MK4"
    idx = [[i for i in range(len(p0)) if meta["group_of"][i] == gi] for gi in range(2)]
    groups = [([p0[i] for i in idx[gi]], {"weight_decay": kw["weight_decay"] * meta["group_wd_scale"][gi]})
              for gi in range(2)]
    pair = Pair(oracle_mod, star, groups, foreach=True, **kw)
    order = [i for gi in range(2) for i in idx[gi]]
    for k in range(1, meta["n_steps"] + 1):
        lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        pair.set_lr([lr, lr])
        pair.step([[grads[k - 1][i] if has_grad[k - 1, i] else None for i in idx[gi]] for gi in range(2)])
        if k in meta["checkpoints"]:
            for p, i in zip([p for tp in pair.gpu_params for p in tp], order):
                got, ref = p.detach().cpu().numpy(), gold[f"p{i}_t{k}"]
                assert np.array_equal(np.isnan(got), np.isnan(ref)) and np.array_equal(np.isinf(got), np.isinf(ref)), \
                    (case, k, i)
        pair.compare(where=f"foreach non-finite {case} t={k}")
