"""GPU parity of the HIP step (through the C ABI) against the CPU oracle.

Bars (stated per assertion):
  * m, v, tau: bit-exact (their path has only correctly rounded ops and the
    FMAs ATen's lerp/addcmul use);
  * p for ADana / Dana-MK4: bit-exact;
  * p for Dana-Star(-MK4): bit-exact, except elements whose per-element pow
    x ** (1 - kappa) lies within ~2^-52 of a binary32 rounding boundary (the
    GPU's binary64 pow and the C library's may round those differently; rate
    ~4e-9): at most STAR_HARD_CASES such elements per tensor per step, each
    within 2 ulps of max(|p_before|, |p_after|, |update|);
  * bf16 params (master mode): master and RNE(master) exactly equal for ADana;
    Dana-Star's master as its fp32 p above, its bf16 copy within 1 bf16 ulp;
  * diagnostics: rtol 1e-5 against the oracle's binary64 sums.
"""
import math

import numpy as np
import pytest
import torch

from helpers import bf16_ulp_diff, golden_cases, load_golden_inputs, ulp_diff

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"
STAR_HARD_CASES = 2      # per tensor per step
STAR_P_ULPS = 2          # bound on those elements


def _check_star_p(got, ref, prev, tag):
    """Bit-exact except <= STAR_HARD_CASES elements within STAR_P_ULPS."""
    d = ulp_diff(got, ref)
    bad = np.nonzero(d)[0]
    assert bad.size <= STAR_HARD_CASES, f"{tag}: {bad.size} elements of p differ (max {d.max()} ulp)"
    if bad.size:
        e = _scaled_ulps(np.ravel(got)[bad], np.ravel(ref)[bad], np.ravel(prev)[bad])
        assert e.max() <= STAR_P_ULPS, f"{tag}: p differs by {e.max()} scaled ulp"
    return int(bad.size)


def _scaled_ulps(x, ref, prev):
    x = np.asarray(x, np.float64).ravel()
    ref_ = np.asarray(ref, np.float64).ravel()
    prev = np.asarray(prev, np.float64).ravel()
    scale = np.maximum(np.maximum(np.abs(prev), np.abs(ref_)), np.abs(ref_ - prev))
    scale = np.maximum(scale, 1e-30).astype(np.float32)
    return np.abs(x - ref_) / np.spacing(scale).astype(np.float64)


class Pair:
    """The GPU optimizer and the oracle driven in lock step on equal inputs."""

    def __init__(self, O, star, groups_np, master=False, numerics="compiled", foreach=False, **hp):
        import adana_amd

        self.O = O
        self.star = star
        self.master = master
        self.groups_np = groups_np            # [(list of np arrays, group kwargs)]
        self.cpu_params = [[x.copy() for x in ps] for ps, _ in groups_np]
        self.gpu_params = []
        torch_groups = []
        for ps, gkw in groups_np:
            tp = []
            for x in ps:
                if master:
                    t = torch.from_numpy(x.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
                else:
                    t = torch.from_numpy(x.copy()).to(DEV)
                tp.append(torch.nn.Parameter(t))
            self.gpu_params.append(tp)
            torch_groups.append(dict(params=tp, **gkw))
        cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
        self.opt = cls(torch_groups, master_weights=master, numerics=numerics, use_foreach=foreach, **hp)
        self.oracle = O.OracleOptimizer(
            groups=[O.OracleGroup(params=cp, lr=gkw.get("lr", hp["lr"]),
                                  delta=gkw.get("delta", hp.get("delta", 8.0)),
                                  epsilon=gkw.get("epsilon", hp.get("epsilon", 1e-8)),
                                  weight_decay=gkw.get("weight_decay", hp.get("weight_decay", 0.0)))
                    for cp, (_, gkw) in zip(self.cpu_params, groups_np)],
            star=star, peak_lr=hp["lr"], kappa=hp.get("kappa", 1.0),
            clipsnr=hp.get("clipsnr", 1.0 if star else None),
            wd_decaying=hp.get("wd_decaying", False), wd_ts=hp.get("wd_ts", 1.0),
            gamma_3_factor=hp.get("gamma_3_factor", 1.0), master=master, numerics=numerics, foreach=foreach)

    def set_lr(self, lrs):
        for g, og, lr in zip(self.opt.param_groups, self.oracle.groups, lrs):
            g["lr"] = lr
            og.lr = lr

    def step(self, grads):
        """grads[gi][pi]: float32 array (uint16 bf16 bits in master mode) or None."""
        for tp, gs in zip(self.gpu_params, grads):
            for p, g in zip(tp, gs):
                if g is None:
                    p.grad = None
                elif self.master:
                    p.grad = torch.from_numpy(g.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
                else:
                    p.grad = torch.from_numpy(g.copy()).to(DEV)
        self.prev = [[x.copy() for x in cp] for cp in self.cpu_params]
        self.opt.step()
        self.oracle.step(grads)
        torch.cuda.synchronize()

    def compare(self, resync=True, check_diag=True, where=""):
        """Compare every tensor; return the number of Dana-Star hard-case elements."""
        worst = 0
        for gi, (tp, cp) in enumerate(zip(self.gpu_params, self.cpu_params)):
            for pi, (p, c) in enumerate(zip(tp, cp)):
                st = self.opt.state[p]
                ost = self.oracle.state.get(id(c))
                tag = f"{where} group {gi} tensor {pi} shape {tuple(c.shape)}"
                if ost is None:
                    assert len(st) == 0, tag
                    continue
                assert st["step"] == ost["step"], tag
                if c.size == 0:                  # nothing to compare but the step and diagnostics
                    assert all(st[k].numel() == 0 for k in ("m", "v") + (("tau",) if self.star else ())), tag
                    if check_diag:
                        got = np.array([float(st[k]) for k in self.O.DIAG_KEYS])
                        ref = np.array([ost[k] for k in self.O.DIAG_KEYS])
                        np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30, equal_nan=True,
                                                   err_msg=tag + " diagnostics")
                    continue
                for key in ("m", "v") + (("tau",) if self.star else ()):
                    d = ulp_diff(st[key].cpu().numpy(), ost[key])
                    assert d.max() == 0, f"{tag}: {key} differs by {d.max()} ulp at {d.argmax()}"
                if self.master:
                    gm = st["master"].cpu().numpy()
                    g16 = p.detach().cpu().view(torch.int16).numpy().view(np.uint16)
                    if not self.star:
                        assert ulp_diff(gm, ost["master"]).max() == 0, f"{tag}: master"
                        assert np.array_equal(g16, c), f"{tag}: bf16 param"
                    else:
                        _check_star_p(gm, ost["master"], self.O.bf16_to_f32(self.prev[gi][pi]),
                                      tag + " master")
                        assert bf16_ulp_diff(g16, c).max() <= 1, f"{tag}: bf16 param"
                    if resync:
                        ost["master"][...] = gm
                        c[...] = g16.reshape(c.shape)
                else:
                    gp = p.detach().cpu().numpy()
                    if not self.star:
                        d = ulp_diff(gp, c)
                        assert d.max() == 0, f"{tag}: p differs by {d.max()} ulp at {d.argmax()}"
                    else:
                        worst += _check_star_p(gp, c, self.prev[gi][pi], tag)
                    if resync:
                        c[...] = gp
                if check_diag:
                    got = np.array([float(st[k]) for k in self.O.DIAG_KEYS])
                    ref = np.array([ost[k] for k in self.O.DIAG_KEYS])
                    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30, equal_nan=True,
                                               err_msg=tag + " diagnostics")
        return worst


def _normal(rng, shape, std):
    return rng.normal(0.0, std, shape).astype(np.float32)


# --------------------------------------------------------------------------

@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("clipsnr", [None, 2.0])
def test_c1_adana_single_tensor(oracle_mod, clipsnr, numerics):
    """Config C1 (1024x4096 fp32, delta 8, omega 4, kappa 0.85, lr 1e-3,
    wd_ts 10): bit-exact p, m, v for 12 steps (t crosses delta), in both of
    the reference's numerics."""
    print("case: C1 ADana 1024x4096 clipsnr", clipsnr, numerics, flush=True)
    rng = np.random.default_rng(0)
    pair = Pair(oracle_mod, False, [([_normal(rng, (1024, 4096), 0.02)], {})], lr=1e-3,
                delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=4.0 / 10.0, clipsnr=clipsnr,
                wd_decaying=True, wd_ts=10.0, numerics=numerics)
    for t in range(1, 13):
        g = np.random.default_rng(1000 + t).normal(0, 1e-3, (1024, 4096)).astype(np.float32)
        pair.step([[g]])
        pair.compare(resync=False, where=f"t={t}")


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("case", golden_cases("eager"))
def test_golden_cases_on_gpu(oracle_mod, case, numerics):
    """The golden-vector scenarios (two groups, grad None every other step,
    all-zero and row-sparse grads, warm-up/cosine lr) on the GPU vs the
    oracle, in both numerics; and, for the compiled numerics, every
    checkpoint against the reference's own torch.compile run
    (tests/golden/<case>.compiled.npz): m, v, tau bit-exact, ADana's p
    bit-exact, Dana-Star's p within 1 ulp of the tensor's largest value (the
    reference's SIMD pow is not correctly rounded)."""
    print("case: golden", case, numerics, flush=True)
    _golden_on_gpu(oracle_mod, case, "inputs", numerics)


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("case", ["adana", "dana_mk4", "dana_star", "dana_star_mk4"])
def test_nonfinite_gradients_on_gpu(oracle_mod, case, numerics):
    """The same scenarios with NaN, +inf and -inf gradient entries at steps 3
    and 6 (tests/golden/nonfinite.inputs.npz; the oracle follows the
    reference's own run there): the elements they reach turn NaN (v: inf)
    exactly where the oracle's do, the other elements keep the usual bars,
    and the tensors' diagnostics are NaN."""
    print("case: non-finite gradients", case, numerics, flush=True)
    _golden_on_gpu(oracle_mod, case, "nonfinite.inputs", numerics)


def _golden_on_gpu(oracle_mod, case, inputs, numerics):
    from helpers import load_golden_case

    gold = load_golden_case(case, "compiled") if (inputs == "inputs" and numerics == "compiled") else None
    meta, p0, grads, has_grad = load_golden_inputs(inputs)
    c = meta["cases"][case]
    kw = dict(c["kwargs"])
    star = c["class"] == "DANA_STAR_MK4"
    groups = []
    for gi in range(2):
        idx = [i for i in range(len(p0)) if meta["group_of"][i] == gi]
        groups.append(([p0[i] for i in idx],
                       {"weight_decay": kw["weight_decay"] * meta["group_wd_scale"][gi]}))
    pair = Pair(oracle_mod, star, groups, numerics=numerics, **kw)
    for k in range(1, meta["n_steps"] + 1):
        lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        pair.set_lr([lr, lr])
        gl = []
        for gi in range(2):
            idx = [i for i in range(len(p0)) if meta["group_of"][i] == gi]
            gl.append([grads[k - 1][i] if has_grad[k - 1, i] else None for i in idx])
        pair.step(gl)
        if gold is not None and k in meta["checkpoints"]:
            flat = [p for tp in pair.gpu_params for p in tp]
            order = [i for gi in range(2) for i in range(len(p0)) if meta["group_of"][i] == gi]
            for p, i in zip(flat, order):
                st = pair.opt.state[p]
                for key in ("m", "v", "tau") if star else ("m", "v"):
                    if key in st:
                        assert ulp_diff(st[key].cpu().numpy(), gold[f"{key}{i}_t{k}"]).max() == 0, (case, k, i, key)
                ref = gold[f"p{i}_t{k}"]
                err = _scaled_ulps(p.detach().cpu().numpy(), ref, np.full(ref.shape, np.abs(ref).max(), np.float32))
                assert err.max() <= (1 if star else 0), (case, k, i, err.max())
        pair.compare(where=f"{case} t={k}")
        for g, og in zip(pair.opt.param_groups, pair.oracle.groups):
            assert g["weighted_step_count"] == og.weighted_step_count


def _gpt_list(rng, vocab, d, layers, mlp=4):
    """Tied-embedding GPT parameter list split into (decay, no-decay) groups
    the way src/models/base.py:503-561 splits it."""
    decay, nodecay = [], [_normal(rng, (vocab, d), 0.02)]
    for _ in range(layers):
        decay += [_normal(rng, (3 * d, d), 0.02), _normal(rng, (d, d), 0.02),
                  _normal(rng, (mlp * d, d), 0.02), _normal(rng, (d, mlp * d), 0.02)]
        nodecay += [np.ones(d, np.float32), np.zeros(d, np.float32),
                    np.ones(d, np.float32), np.zeros(d, np.float32)]
    nodecay += [np.ones(d, np.float32), np.zeros(d, np.float32)]
    return decay, nodecay


def _cos_inf(k):
    """The reference's cos_inf lr factor (src/optim/schedule.py:70-98, restated
    in bench.py) over a 40-iteration run with a 4-step warm-up."""
    from bench import cos_inf_schedule

    return cos_inf_schedule(n_iterations=40, n_warmup=4, div_factor=1e2, final_div_factor=1e-1, n_inf=0)(k)


@pytest.mark.parametrize("star", [False, True])
def test_gpt_list_two_groups(oracle_mod, star):
    """C2-shaped list (smaller dims): mixed 2-D / 1-D tensors, 1-D grads x0.1,
    two weight-decay groups, SNR clipping, warm-up + cosine lr."""
    print("case: GPT list star", star, flush=True)
    rng = np.random.default_rng(2)
    decay, nodecay = _gpt_list(rng, vocab=1003, d=96, layers=2)
    peak = 3e-3
    pair = Pair(oracle_mod, star, [(decay, {"weight_decay": 4.0 / 20}), (nodecay, {"weight_decay": 0.0})],
                lr=peak, delta=8.0, kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=20.0)
    for k in range(12):
        pair.set_lr([peak * _cos_inf(k)] * 2)
        gl = [[_normal(rng, x.shape, 1e-3) * (np.float32(0.1) if x.ndim == 1 else 1) for x in ps]
              for ps in (decay, nodecay)]
        pair.step(gl)
        pair.compare(where=f"k={k}")


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("kappa", [1.0, 0.0, 1.5, 2.0, -1.0, -2.0, 3.0, 0.3, -3.0])
def test_star_pow_modes(oracle_mod, kappa, numerics):
    """Every kind of the per-element pow eff_time ** (1 - kappa)
    (src/optim/dana_star_mk4.py:168-170) through the kernel, in both
    numerics: exponent 0 (kappa 1: no pow), 1 (kappa 0: identity), -0.5
    (eager: 1/sqrt; compiled: a general pow), -1, 2, 3, 4 and -2 (eager:
    ATen's specialisations or a general pow; compiled: Inductor's integer
    powering by products), and a general one (0.5 and 0.15 run in the
    golden cases).  No SNR clip, so the pow reaches p unclamped; 12 steps,
    so that tau * t passes 1 and the pow sees arguments above 1."""
    print("case: Dana-Star pow mode kappa", kappa, numerics, flush=True)
    rng = np.random.default_rng(int(100 + 10 * kappa))
    shapes = [(37, 19), (1024,), (5,), (4096 + 3,)]
    params = [_normal(rng, s, 0.02) for s in shapes]
    pair = Pair(oracle_mod, True, [(params, {})], lr=1e-3, delta=4.0, kappa=kappa, clipsnr=None,
                weight_decay=0.1, wd_decaying=True, wd_ts=5.0, numerics=numerics)
    for k in range(12):
        gl = [[_normal(rng, x.shape, 1e-3) for x in params]]
        pair.step(gl)
        pair.compare(where=f"kappa={kappa} k={k}")
    taus = np.concatenate([pair.opt.state[p]["tau"].cpu().numpy().ravel() for p in pair.gpu_params[0]])
    assert (taus * 12 > 1).mean() > 0.3                      # the pow saw arguments above 1


def test_many_tiny_tensors(oracle_mod):
    """C5-shaped list (fewer tensors): log-uniform sizes incl. non-multiples of
    4 and 1-element tensors, 5% all-zero grads, chunks spanning many tensors."""
    print("case: many tiny tensors", flush=True)
    rng = np.random.default_rng(5)
    sizes = np.floor(np.exp(rng.uniform(math.log(1), math.log(65536), 700))).astype(int)
    sizes[:5] = [1, 2, 3, 5, 7]
    params = [_normal(rng, (int(n),), 0.02) for n in sizes]
    zero = rng.random(len(sizes)) < 0.05
    pair = Pair(oracle_mod, True, [(params, {})], lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0,
                weight_decay=0.1, wd_decaying=False)
    for k in range(10):
        gl = [[np.zeros_like(x) if z else _normal(rng, x.shape, 1e-3) for x, z in zip(params, zero)]]
        pair.step(gl)
        pair.compare(where=f"k={k}")


@pytest.mark.parametrize("star", [False, True])
def test_unaligned_views(oracle_mod, star):
    """Parameters and grads that are views at odd offsets of flat buffers run
    the element-wise (non-vector) path; results are unchanged."""
    import adana_amd

    print("case: unaligned views star", star, flush=True)
    rng = np.random.default_rng(7)
    sizes = [37, 4099, 1, 20000]
    flat = torch.from_numpy(_normal(rng, (sum(sizes) + 3,), 0.02)).to(DEV)
    views, off = [], 1
    for n in sizes:
        views.append(flat[off:off + n])
        off += n
    params = [torch.nn.Parameter(v) for v in views]
    cpu = [v.detach().cpu().numpy().copy() for v in views]
    O = oracle_mod
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(params, lr=1e-3, kappa=0.85, clipsnr=1.0, weight_decay=0.2)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=cpu, lr=1e-3, weight_decay=0.2)],
                            star=star, peak_lr=1e-3, kappa=0.85, clipsnr=1.0)
    gflat = torch.zeros(sum(sizes) + 1, device=DEV)
    for k in range(6):
        gs = [_normal(rng, (n,), 1e-3) for n in sizes]
        o = 1
        for p, g in zip(params, gs):
            gflat[o:o + g.size].copy_(torch.from_numpy(g))
            p.grad = gflat[o:o + g.size]
            o += g.size
        prev = [c.copy() for c in cpu]
        opt.step()
        orc.step([gs])
        for p, c, pv in zip(params, cpu, prev):
            st, ost = opt.state[p], orc.state[id(c)]
            assert ulp_diff(st["m"].cpu().numpy(), ost["m"]).max() == 0
            assert ulp_diff(st["v"].cpu().numpy(), ost["v"]).max() == 0
            gp = p.detach().cpu().numpy()
            if star:
                assert ulp_diff(st["tau"].cpu().numpy(), ost["tau"]).max() == 0
                _check_star_p(gp, c, pv, "unaligned")
            else:
                assert ulp_diff(gp, c).max() == 0
            c[...] = gp
    # the guard elements around the views (one before the first, two after the
    # last) and the gradient buffer's leading guard stay untouched
    start = _normal(np.random.default_rng(7), (sum(sizes) + 3,), 0.02)
    for i in (0, sum(sizes) + 1, sum(sizes) + 2):
        assert flat[i].item() == float(start[i]), i
    assert gflat[0].item() == 0.0


@pytest.mark.parametrize("star", [False, True])
def test_bf16_master_weights(oracle_mod, star):
    """C4 mode: bf16 params + fp32 master/m/v(/tau) + bf16 grads."""
    print("case: bf16 master star", star, flush=True)
    rng = np.random.default_rng(11)
    O = oracle_mod
    shapes = [(257, 64), (1000,), (33,)]
    p16 = [O.f32_to_bf16(_normal(rng, s, 0.02)) for s in shapes]
    pair = Pair(O, star, [(p16, {})], master=True, lr=1e-3, delta=8.0, kappa=0.85,
                clipsnr=None, weight_decay=0.1, wd_decaying=True, wd_ts=10.0)
    for k in range(10):
        gl = [[O.f32_to_bf16(_normal(rng, s, 1e-3)) for s in shapes]]
        pair.step(gl)
        pair.compare(where=f"k={k}")


def test_more_classes_than_one_launch(oracle_mod):
    """More (group, step) classes than one launch carries: 11 groups with
    different lr, plus lagging per-tensor steps."""
    print("case: many classes", flush=True)
    rng = np.random.default_rng(13)
    groups = [([_normal(rng, (300 + 17 * i,), 0.02), _normal(rng, (64, 9), 0.02)],
               {"lr": 1e-3 * (1 + i), "weight_decay": 0.01 * i}) for i in range(11)]
    pair = Pair(oracle_mod, True, groups, lr=1e-3, kappa=0.8, clipsnr=1.5)
    for k in range(6):
        gl = [[None if (k % 2 and pi == 1 and gi % 3 == 0) else _normal(rng, x.shape, 1e-3)
               for pi, x in enumerate(ps)] for gi, (ps, _) in enumerate(groups)]
        pair.step(gl)
        pair.compare(where=f"k={k}")


def test_empty_tensor_and_zero_grads(oracle_mod):
    """numel 0 tensors: no work, diagnostics NaN/0 as torch's mean/norm give;
    all-zero grads: kappa factor 0/0 = NaN (src/optim/adana.py:224)."""
    import adana_amd

    p_empty = torch.nn.Parameter(torch.zeros(0, device=DEV))
    p_zero = torch.nn.Parameter(torch.linspace(-1, 1, 100, device=DEV))
    opt = adana_amd.ADana([p_empty, p_zero], lr=1e-3, kappa=0.85)
    p_empty.grad = torch.zeros(0, device=DEV)
    p_zero.grad = torch.zeros(100, device=DEV)
    before = p_zero.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    st = opt.state[p_empty]
    assert math.isnan(float(st["current_alpha"])) and float(st["gradient_norm"]) == 0.0
    assert float(st["m_norm"]) == 0.0
    st = opt.state[p_zero]
    assert math.isnan(float(st["current_kappa_factor"]))
    assert float(st["current_alpha"]) == 0.0
    assert torch.equal(p_zero.detach(), before)


@pytest.mark.parametrize("star", [False, True])
def test_state_dict_resume_is_bit_identical(star):
    """stop -> state_dict -> fresh optimizer -> load_state_dict -> continue
    gives the same bits as an uninterrupted run."""
    import adana_amd

    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    rng = np.random.default_rng(17)
    init = [_normal(rng, s, 0.02) for s in [(128, 33), (77,)]]
    grads = [[_normal(rng, x.shape, 1e-3) for x in init] for _ in range(10)]

    def run(split):
        ps = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in init]
        opt = cls(ps, lr=2e-3, kappa=0.85, clipsnr=2.0, weight_decay=0.1, wd_decaying=True,
                  wd_ts=5.0)
        for k in range(10):
            if k == split:
                sd = opt.state_dict()
                opt = cls(ps, lr=2e-3, kappa=0.85, clipsnr=2.0, weight_decay=0.1,
                          wd_decaying=True, wd_ts=5.0)
                opt.load_state_dict(sd)
            for p, g in zip(ps, grads[k]):
                p.grad = torch.from_numpy(g).to(DEV)
            opt.step()
        torch.cuda.synchronize()
        return [p.detach().cpu().numpy() for p in ps], opt

    a, oa = run(split=None)
    b, ob = run(split=5)
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.int32), y.view(np.int32))
    for pa, pb in zip(oa.param_groups[0]["params"], ob.param_groups[0]["params"]):
        assert oa.state[pa]["step"] == ob.state[pb]["step"] == 10
        assert torch.equal(oa.state[pa]["m"], ob.state[pb]["m"])


def test_run_twice_is_deterministic():
    """Same inputs twice -> identical bits, diagnostics included (no atomics)."""
    import adana_amd

    rng = np.random.default_rng(19)
    init = [_normal(rng, s, 0.02) for s in [(3000, 40), (5,), (16384 * 3 + 1,)]]
    g = [_normal(rng, x.shape, 1e-3) for x in init]
    outs = []
    for _ in range(2):
        ps = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in init]
        opt = adana_amd.DANA_STAR_MK4(ps, lr=1e-3, kappa=0.85, clipsnr=2.0)
        for _ in range(3):
            for p, gg in zip(ps, g):
                p.grad = torch.from_numpy(gg).to(DEV)
            opt.step()
        torch.cuda.synchronize()
        outs.append(([p.detach().cpu() for p in ps],
                     [[float(opt.state[p][k]) for k in adana_amd.DIAG_KEYS] for p in ps]))
    for x, y in zip(outs[0][0], outs[1][0]):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))
    assert np.array_equal(np.array(outs[0][1]), np.array(outs[1][1]), equal_nan=True)


@pytest.mark.parametrize("foreach", [False, True], ids=["per_tensor", "foreach"])
@pytest.mark.parametrize("star", [False, True])
def test_drift_over_1000_steps(oracle_mod, star, foreach):
    """1,000 steps at config C1's shape (1024 x 4096) without re-synchronising
    the oracle: m, v, tau stay bit-exact (they never read p); ADana p stays
    bit-exact; Dana-Star p differs only where a pow hard case (rate ~4e-9 per
    element and step) left a trace, by at most a few ulp of the tensor's
    scale.  Reports max / median ulp and the max relative difference.  Both
    of the reference's paths: per tensor and use_foreach=True."""
    print("case: 1000-step drift at 1024x4096, star", star, "foreach", foreach, flush=True)
    rng = np.random.default_rng(23)
    shape = (1024, 4096)
    n = shape[0] * shape[1]
    pair = Pair(oracle_mod, star, [([_normal(rng, shape, 0.02)], {})], lr=1e-3, delta=8.0,
                kappa=0.85, clipsnr=2.0 if star else None, weight_decay=0.4, wd_decaying=True,
                wd_ts=100.0, foreach=foreach)
    gen = torch.Generator(device=DEV)
    gpu_p = pair.gpu_params[0][0]
    c = pair.cpu_params[0][0]
    worst, worst_rel, med = 0.0, 0.0, 0.0
    for t in range(1, 1001):
        gen.manual_seed(5000 + t)
        g = torch.empty(shape, device=DEV).normal_(0.0, 1e-3, generator=gen)
        gpu_p.grad = g
        pair.opt.step()
        pair.oracle.step([[g.cpu().numpy()]])
        if t % 100 == 0 or t in (1, 8, 9):
            torch.cuda.synchronize()
            p = gpu_p.detach().cpu().numpy()
            st, ost = pair.opt.state[gpu_p], pair.oracle.state[id(c)]
            for key in ("m", "v") + (("tau",) if star else ()):
                assert ulp_diff(st[key].cpu().numpy(), ost[key]).max() == 0, (t, key)
            d = ulp_diff(p, c)
            nz = d[d > 0]
            scale = np.full(p.shape, np.abs(c).max(), np.float32)
            err = np.abs(p.astype(np.float64) - c) / np.spacing(scale).astype(np.float64)
            rel = np.abs(p.astype(np.float64) - c) / np.maximum(np.abs(c.astype(np.float64)), 1e-30)
            worst, worst_rel = max(worst, float(err.max())), max(worst_rel, float(rel.max()))
            med = float(np.median(nz)) if nz.size else 0.0
            print(f"t={t}: {nz.size} elements differ, max {int(d.max())} ulp, median {med:.1f} ulp of the "
                  f"differing ones, max rel {float(rel.max()):.2e}", flush=True)
            if not star:
                assert d.max() == 0, t
            else:
                # a pow hard case leaves a <=1-ulp trace in p that later steps carry
                assert nz.size <= 8 + math.ceil(2e-8 * n * t), (t, nz.size)
    print(f"max drift of p over 1000 steps: {worst:.2f} ulp of max|p|, max rel {worst_rel:.2e}", flush=True)
    assert worst <= 4


@pytest.mark.parametrize("star", [False, True])
def test_large_tensor_fold_path(oracle_mod, star):
    """Tensors of more than ADANA_DIRECT_CHUNKS chunks go through the fold
    workgroups (two folds or more; the last to finish finalizes the tensor,
    and 512 * 1024 + 1 elements leave a fold of one chunk); smaller ones are
    summed directly: all kinds in one list, diagnostics against the oracle
    (and the clip norm path)."""
    import adana_amd

    print("case: large tensor fold path star", star, flush=True)
    rng = np.random.default_rng(9)
    sizes = [9_000_000, 5, 512 * 1024, 512 * 1024 + 1, 70_000, 4096 * 1024, 4096 * 1024 + 1, 3000 * 1024 + 7]
    params = [_normal(rng, (n,), 0.02) for n in sizes]
    pair = Pair(oracle_mod, star, [(params, {})], lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0,
                weight_decay=0.1, wd_decaying=True, wd_ts=10.0)
    for k in range(3):
        gl = [[_normal(rng, x.shape, 1e-3) for x in params]]
        pair.step(gl)
        pair.compare(where=f"k={k}")
    grads = [p.grad for p in pair.gpu_params[0]]
    total = adana_amd.clip_grad_norm_(pair.gpu_params[0], 1e9)
    want = float(np.sqrt(sum(float(np.sum(np.square(g.cpu().numpy().astype(np.float64)))) for g in grads)))
    assert abs(float(total) - want) <= 2e-6 * want


@pytest.mark.parametrize("fresh_grads", [False, True])
def test_parameter_storage_rebound_is_followed(oracle_mod, fresh_grads):
    """``p.data = other`` between steps (a new storage for the parameter) is
    picked up without invalidate_plan(): the step updates the new storage and
    leaves the old one alone, with gradients that persist between steps and
    with new gradient tensors every step (zero_grad(set_to_none=True))."""
    print("case: parameter storage rebound, fresh grads", fresh_grads, flush=True)
    rng = np.random.default_rng(41)
    shapes = [(300,), (64, 33), (7,)]
    params = [_normal(rng, s, 0.02) for s in shapes]
    pair = Pair(oracle_mod, True, [(params, {})], lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0,
                weight_decay=0.1)
    gl = [[_normal(rng, x.shape, 1e-3) for x in params]]
    gpu_grads = [torch.from_numpy(g.copy()).to(DEV) for g in gl[0]]
    for k in range(6):
        if k == 3:
            p = pair.gpu_params[0][1]
            old = p.data
            p.data = old.clone()                                   # same values, new storage
            snapshot = old.clone()
        for p, g in zip(pair.gpu_params[0], gpu_grads):
            p.grad = g.clone() if fresh_grads else g
        pair.prev = [[x.copy() for x in cp] for cp in pair.cpu_params]
        pair.opt.step()
        pair.oracle.step(gl)
        torch.cuda.synchronize()
        pair.compare(where=f"k={k}")
        if k >= 3:
            assert torch.equal(old, snapshot)                      # the old storage is not written


@pytest.mark.parametrize("drop_other_grad", [False, True])
def test_parameter_rebound_to_another_shape_raises(drop_other_grad):
    """``p.data = x`` with x of another shape (and a gradient of that shape)
    raises at the next step, before any launch, whether the plan is reused
    (same tensors have gradients) or rebuilt (another tensor's gradient is
    None); the other tensors' state is left as it was."""
    import adana_amd

    print("case: parameter rebound to another shape, drop other grad", drop_other_grad, flush=True)
    ps = [torch.nn.Parameter(torch.full((300,), 0.5, device=DEV)),
          torch.nn.Parameter(torch.full((64, 33), 0.5, device=DEV))]
    opt = adana_amd.DANA_STAR_MK4(ps, lr=1e-3, kappa=0.85)
    for _ in range(2):
        for p in ps:
            p.grad = torch.full_like(p, 1e-3)
        opt.step()
    torch.cuda.synchronize()
    m_before = opt.state[ps[0]]["m"].clone()
    ps[1].data = torch.zeros(65, 33, device=DEV)
    ps[1].grad = torch.full_like(ps[1], 1e-3)
    ps[0].grad = None if drop_other_grad else torch.full_like(ps[0], 1e-3)
    with pytest.raises(RuntimeError, match="must match the size"):
        opt.step()
    torch.cuda.synchronize()
    assert torch.equal(opt.state[ps[0]]["m"], m_before)


@pytest.mark.parametrize("star", [False, True])
def test_new_gradient_buffers_every_step(oracle_mod, star):
    """New gradient tensors at new addresses every step, alternating between
    16-byte-aligned buffers and views 4 bytes into a flat buffer (so the
    kernel's gradient alignment test flips each step between the vector and
    the element-wise path): the re-pointed gradient array gives the oracle's
    results every step, and every step after the first takes the one-pass
    host scan."""
    print("case: new gradient buffers every step, star", star, flush=True)
    rng = np.random.default_rng(43)
    shapes = [(1000,), (64, 33), (5,), (4096 + 8,)]
    params = [_normal(rng, s, 0.02) for s in shapes]
    pair = Pair(oracle_mod, star, [(params, {})], lr=1e-3, delta=8.0, kappa=0.85,
                clipsnr=2.0 if star else None, weight_decay=0.1)
    total = sum(int(np.prod(s)) for s in shapes)
    for k in range(8):
        gl = [[_normal(rng, x.shape, 1e-3) for x in params]]
        if k % 2:
            flat = torch.empty(total + 1, device=DEV)
            off = 1                                             # 4 bytes in: not 16-byte aligned
            views = []
            for g in gl[0]:
                v = flat[off:off + g.size].view(g.shape)
                v.copy_(torch.from_numpy(g))
                views.append(v)
                off += g.size
        else:
            views = [torch.from_numpy(g.copy()).to(DEV) for g in gl[0]]
        for p, v in zip(pair.gpu_params[0], views):
            p.grad = v
        pair.prev = [[x.copy() for x in cp] for cp in pair.cpu_params]
        pair.opt.step()
        pair.oracle.step(gl)
        torch.cuda.synchronize()
        pair.compare(where=f"k={k}")
        ls = pair.opt._sets[0]
        assert (ls.host_desc["flags"] != 0).all()               # the other pointers stay aligned
        assert (ls.host_grad % 16 == 0).all() == (k % 2 == 0), (k, ls.host_grad % 16)
        assert pair.opt._fast


def test_gradient_storage_swapped_in_place(oracle_mod):
    """The same gradient objects every step, but ``g.set_(other)`` moves their
    storage between steps: the step reads the new storage (the object-identity
    fast path also compares data pointers)."""
    print("case: gradient storage swapped under the same objects", flush=True)
    rng = np.random.default_rng(45)
    shapes = [(1000,), (64, 33), (5,)]
    params = [_normal(rng, s, 0.02) for s in shapes]
    pair = Pair(oracle_mod, True, [(params, {})], lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0,
                weight_decay=0.1)
    grads = [torch.zeros(s, device=DEV) for s in shapes]
    for p, g in zip(pair.gpu_params[0], grads):
        p.grad = g
    for k in range(6):
        gl = [[_normal(rng, x.shape, 1e-3) for x in params]]
        for g, new in zip(grads, gl[0]):
            if k % 2:
                g.set_(torch.from_numpy(new.copy()).to(DEV))       # same object, new storage
            else:
                g.copy_(torch.from_numpy(new))
        pair.prev = [[x.copy() for x in cp] for cp in pair.cpu_params]
        pair.opt.step()
        pair.oracle.step(gl)
        torch.cuda.synchronize()
        pair.compare(where=f"k={k}")


@pytest.mark.parametrize("star", [False, True])
def test_closure_and_group_added_mid_run(oracle_mod, star):
    """step(closure): the closure runs with gradients enabled, its loss is
    returned, and the gradients it leaves are the ones stepped
    (src/optim/adana.py:155-160).  add_param_group after 3 steps: the new
    group joins with fresh state and both groups match the oracle."""
    O = oracle_mod
    print("case: closure and add_param_group, star", star, flush=True)
    rng = np.random.default_rng(47)
    a = [_normal(rng, (300,), 0.02), _normal(rng, (17, 9), 0.02)]
    pair = Pair(O, star, [(a, {"weight_decay": 0.1})], lr=1e-3, delta=8.0, kappa=0.85,
                clipsnr=2.0 if star else None, weight_decay=0.1)
    for k in range(6):
        if k == 3:
            b = [_normal(rng, (1000,), 0.02), _normal(rng, (5,), 0.02)]
            tb = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in b]
            pair.opt.add_param_group({"params": tb, "weight_decay": 0.0})
            cb = [x.copy() for x in b]
            pair.gpu_params.append(tb)
            pair.cpu_params.append(cb)
            pair.oracle.groups.append(O.OracleGroup(params=cb, lr=1e-3, weight_decay=0.0))
        gl = [[_normal(rng, x.shape, 1e-3) for x in cp] for cp in pair.cpu_params]
        seen = {}

        def closure():
            seen["grad_enabled"] = torch.is_grad_enabled()
            for tp, gs in zip(pair.gpu_params, gl):
                for p, g in zip(tp, gs):
                    p.grad = torch.from_numpy(g.copy()).to(DEV)
            return torch.tensor(float(k) + 0.5)

        pair.prev = [[x.copy() for x in cp] for cp in pair.cpu_params]
        loss = pair.opt.step(closure)
        pair.oracle.step(gl)
        torch.cuda.synchronize()
        assert seen["grad_enabled"] and float(loss) == k + 0.5
        pair.compare(where=f"k={k}")
    assert [g["weighted_step_count"] for g in pair.opt.param_groups] == [6.0, 3.0]


@pytest.mark.parametrize("star", [False, True])
def test_permuted_parameters(oracle_mod, star):
    """Parameters with dense non-contiguous layouts (a transposed matrix, a
    permuted 3-D tensor) and gradients of the same strides, as autograd
    produces them: the state is zeros_like(p) with p's strides, the step runs
    in storage order, and every element matches the oracle's (run on the
    logical arrays); 8 steps crossing t = delta.  (Gradients of other strides
    and parameters with gaps: test_staged_layouts.)"""
    import adana_amd

    O = oracle_mod
    print("case: permuted parameter layouts, star", star, flush=True)
    rng = np.random.default_rng(77)
    base = [torch.from_numpy(_normal(rng, (64, 33), 0.02)).to(DEV).t(),
            torch.from_numpy(_normal(rng, (4, 5, 6), 0.02)).to(DEV).permute(2, 0, 1),
            torch.from_numpy(_normal(rng, (1000,), 0.02)).to(DEV)]
    ps = [torch.nn.Parameter(b) for b in base]
    assert not ps[0].is_contiguous() and not ps[1].is_contiguous()
    host = [p.detach().cpu().numpy().copy() for p in ps]                   # logical order
    hp = dict(lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0, weight_decay=0.1, wd_decaying=True, wd_ts=10.0)
    opt = (adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana)(ps, **hp)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=host, lr=1e-3, weight_decay=0.1)], star=star,
                            peak_lr=1e-3, kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=10.0)
    for t in range(1, 9):
        gl = [_normal(rng, h.shape, 1e-3) for h in host]
        for p, g in zip(ps, gl):
            gt = torch.empty_strided(p.shape, p.stride(), device=DEV)
            gt.copy_(torch.from_numpy(g))
            p.grad = gt
        prev = [h.copy() for h in host]
        opt.step()
        orc.step([gl])
        torch.cuda.synchronize()
        for i, p in enumerate(ps):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"t={t} tensor {i} shape {tuple(p.shape)} strides {p.stride()}"
            for key in ("m", "v") + (("tau",) if star else ()):
                assert st[key].stride() == p.stride(), tag
                assert ulp_diff(st[key].cpu().numpy(), ost[key]).max() == 0, f"{tag} {key}"
            gp = p.detach().cpu().numpy()
            if star:
                _check_star_p(gp, host[i], prev[i], tag)
            else:
                assert ulp_diff(gp, host[i]).max() == 0, tag
            host[i][...] = gp
            got = np.array([float(st[k]) for k in O.DIAG_KEYS])
            np.testing.assert_allclose(got, [ost[k] for k in O.DIAG_KEYS], rtol=1e-5, atol=1e-30, err_msg=tag)


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().contiguous()
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32)


@pytest.mark.parametrize("mode", ["f32", "master", "bf16"])
@pytest.mark.parametrize("star", [False, True])
def test_staged_layouts(star, mode):
    """Parameters with gaps in memory (slices of larger tensors, whose state
    zeros_like makes contiguous) and gradients whose strides differ from
    their state's are staged through buffers of the state's layout.  Every
    step equals, bit for bit (p, m, v, tau, the five diagnostics), the same
    optimizer's step on twins of the state's layout with gradients of that
    layout (nothing staged; their parity with the oracle the other tests
    pin).  The memory between a gapped parameter's elements is untouched; a
    gradient's layout changes between steps; 10 steps cross t = delta.  On
    clip_grad_norm_ steps the coefficient is fused into the staged load and
    written back through the staging buffer: every gradient then equals
    RN(g * coef), and the twins step on those products.  A parameter whose
    elements share memory (expanded) is refused."""
    import adana_amd

    print("case: staged layouts, star", star, "mode", mode, flush=True)
    dt = torch.float32 if mode == "f32" else torch.bfloat16
    gen = torch.Generator().manual_seed(91)

    def rnd(*shape, std=0.02):
        return (torch.randn(*shape, generator=gen) * std).to(dt).to(DEV)

    def transposed(g):          # g's values in the reverse-strided dense layout
        return torch.empty(g.shape[::-1], dtype=dt, device=DEV).t().copy_(g)

    big0, big1 = rnd(12, 40), rnd(3001)
    keep0, keep1 = big0.clone(), big1.clone()
    views = [big0[:, 5:21],                       # gapped rows: contiguous state
             big1[::3],                           # stride 3: contiguous state
             rnd(64, 33).t(),                     # permuted: state of its strides
             rnd(30, 20).t()[2:17],               # permuted and gapped: contiguous state
             rnd(5000)]                           # contiguous, never staged
    ps = [torch.nn.Parameter(v) for v in views]
    twins = [torch.nn.Parameter(v.detach().clone()) for v in views]   # clone: the state's layout
    assert not any(p.is_contiguous() for p in ps[:4])
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    hp = dict(lr=1e-3, delta=8.0, kappa=0.85, clipsnr=2.0, weight_decay=0.1, wd_decaying=True, wd_ts=10.0,
              master_weights=mode == "master")
    opt, ref = cls(ps, **hp), cls(twins, **hp)
    keys = ("m", "v") + (("tau",) if star else ()) + (("master",) if mode == "master" else ())
    for t in range(1, 11):
        gl = [rnd(*p.shape, std=1e-3) for p in ps]                    # contiguous values
        ps[0].grad = transposed(gl[0])                                # staged
        ps[1].grad = gl[1].clone()                                    # p staged, g not
        ps[2].grad = gl[2].clone() if t % 2 else torch.empty_like(ps[2]).copy_(gl[2])   # staged on odd t
        ps[3].grad = transposed(gl[3])                                # both staged
        ps[4].grad = gl[4].clone()
        clip = t in (5, 7, 9)
        if clip:
            opt.clip_grad_norm_(1e-3)
            coef = opt._pending_clip[2][1]
            assert float(coef) < 1.0
            gl = [(g.float() * coef).to(dt) for g in gl]              # _foreach_mul_(grads, coef)
        for q, g in zip(twins, gl):
            q.grad = torch.empty_like(q).copy_(g)
        opt.step()
        ref.step()
        torch.cuda.synchronize()
        for i, (p, q) in enumerate(zip(ps, twins)):
            tag = f"t={t} tensor {i} shape {tuple(p.shape)} strides {p.stride()}"
            assert torch.equal(_bits(p), _bits(q)), tag
            for k in keys:
                assert same_layout_as(opt.state[p][k], ref.state[q][k]), f"{tag} {k}"
                assert torch.equal(_bits(opt.state[p][k]), _bits(ref.state[q][k])), f"{tag} {k}"
            for k in adana_amd.optim.DIAG_KEYS:
                assert torch.equal(_bits(opt.state[p][k]), _bits(ref.state[q][k])), f"{tag} {k}"
            if clip:
                assert torch.equal(_bits(p.grad), _bits(gl[i])), f"{tag} clipped grad"
    gap0 = torch.ones_like(big0, dtype=torch.bool)
    gap0[:, 5:21] = False
    gap1 = torch.ones_like(big1, dtype=torch.bool)
    gap1[::3] = False
    assert torch.equal(big0[gap0], keep0[gap0]) and torch.equal(big1[gap1], keep1[gap1])
    assert not torch.equal(big0[~gap0], keep0[~gap0])                # the slice itself was stepped
    shared = torch.nn.Parameter(torch.zeros(1, 8, dtype=dt, device=DEV).expand(4, 8))
    shared.grad = torch.zeros(4, 8, dtype=dt, device=DEV)
    with pytest.raises(NotImplementedError, match="share memory"):
        cls([shared], **hp).step()


def same_layout_as(a: torch.Tensor, b: torch.Tensor) -> bool:
    return a.shape == b.shape and a.stride() == b.stride()


def test_step_hooks_profiler_and_scheduler():
    """step() keeps torch.optim.Optimizer's behaviour: per-optimizer and global
    pre/post hooks run (a pre-hook may replace the arguments), the profiler
    records the ``Optimizer.step#ADana.step`` range, an LR scheduler sees the
    steps, and the update is the same as without any of them."""
    import adana_amd
    from torch.optim.optimizer import register_optimizer_step_post_hook, register_optimizer_step_pre_hook

    print("case: step hooks, profiler, scheduler", flush=True)
    torch.manual_seed(3)
    ref = torch.nn.Parameter(torch.randn(5000, device=DEV) * 0.02)
    hooked = torch.nn.Parameter(ref.detach().clone())
    opt_ref = adana_amd.ADana([ref], lr=1e-3, kappa=0.85)
    opt = adana_amd.ADana([hooked], lr=1e-3, kappa=0.85)
    g = torch.randn(5000, device=DEV) * 1e-3
    ref.grad, hooked.grad = g.clone(), g.clone()
    opt_ref.step()                                                  # before any hook is registered
    calls = []
    h1 = opt.register_step_pre_hook(lambda o, a, k: calls.append(("pre", o is opt)))
    h2 = opt.register_step_post_hook(lambda o, a, k: calls.append(("post", o is opt)))
    h3 = register_optimizer_step_pre_hook(lambda o, a, k: calls.append(("gpre", o is opt)))
    h4 = register_optimizer_step_post_hook(lambda o, a, k: calls.append(("gpost", o is opt)))
    swapped = lambda: torch.tensor(7.0)                              # noqa: E731
    h5 = opt.register_step_pre_hook(lambda o, a, k: ((o,), {"closure": swapped}))
    loss = opt.step(closure=lambda: torch.tensor(1.0))
    assert float(loss) == 7.0                                       # the pre-hook's closure ran
    assert calls == [("gpre", True), ("pre", True), ("post", True), ("gpost", True)]
    for h in (h1, h2, h3, h4, h5):
        h.remove()
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda k: 1.0)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
        ref.grad, hooked.grad = g.clone(), g.clone()
        opt_ref.step()
        opt.step()
        sched.step()
    assert any(e.name == "Optimizer.step#ADana.step" for e in prof.events())
    assert sched.last_epoch == 1
    for _ in range(2):
        ref.grad, hooked.grad = g.clone(), g.clone()
        opt_ref.step()
        opt.step()
    torch.cuda.synchronize()
    assert torch.equal(ref, hooked)
    assert opt.state[hooked]["step"] == opt_ref.state[ref]["step"] == 4


@pytest.mark.parametrize("fresh", [None, False])
def test_diagnostics_kept_from_a_step_keep_their_value(fresh):
    """As the reference binds new 0-d tensors each step (src/optim/adana.py:
    221-225), a diagnostic kept from one step -- a reference to it, or a
    tensor sharing its storage (detach(), a view) -- keeps its value after
    the next step, and the state holds a new tensor (the default); entries
    nothing else refers to are refreshed in place.  Each has a storage of its own (a deepcopy copies 4 bytes); the
    packed read-out and .item() agree.  With fresh_diagnostics=False every
    entry is refreshed in place."""
    import copy

    import adana_amd

    print("case: kept diagnostics", fresh, flush=True)
    torch.manual_seed(8)
    ps = [torch.nn.Parameter(torch.randn(n, device=DEV) * 0.02) for n in (3000, 70_000)]
    opt = adana_amd.DANA_STAR_MK4(ps, lr=1e-3, kappa=0.85, clipsnr=2.0, fresh_diagnostics=fresh)
    for p in ps:
        p.grad = torch.randn_like(p) * 1e-3
    opt.step()
    kept = opt.state[ps[1]]["gradient_norm"]
    first = float(kept)
    detached = opt.state[ps[0]]["m_norm"].detach()               # shares the entry's storage
    first_d = float(detached)
    untouched = opt.state[ps[0]]["current_alpha"]
    untouched_id = id(untouched)
    del untouched
    assert kept.untyped_storage().nbytes() == 4
    assert copy.deepcopy(opt.state[ps[1]])["m_norm"].untyped_storage().nbytes() == 4
    for p in ps:
        p.grad = torch.randn_like(p) * 5e-3
    opt.step()
    now = opt.state[ps[1]]["gradient_norm"]
    want = float(torch.linalg.vector_norm(ps[1].grad.double()))
    assert float(now) == pytest.approx(want, rel=1e-5)
    if fresh is None:
        assert now is not kept and float(kept) == first             # the kept tensor holds step 1's value
        assert float(detached) == first_d                            # and so does a tensor over its storage
        assert float(opt.state[ps[0]]["m_norm"]) != first_d
        assert id(opt.state[ps[0]]["current_alpha"]) == untouched_id  # refreshed in place
    else:
        assert now is kept and float(kept) == float(now)            # one tensor, refreshed in place
    params, vals = opt.diagnostics_host()
    for p, row in zip(params, vals):
        st = opt.state[p]
        assert list(row) == pytest.approx([float(st[k]) for k in adana_amd.optim.DIAG_KEYS], rel=0, nan_ok=True)


@pytest.mark.parametrize("fresh", [None, False])
def test_diagnostics_kept_on_long_lists(fresh):
    """A list of 5,000 tensors, long enough for the step table's helper
    threads: by default a diagnostic kept from the first step (the general
    path's check) and one kept from the second (the check the fast path's
    scan takes in the same pass) both keep their values, no warning is
    raised; with fresh_diagnostics=False the entries are refreshed in place."""
    import warnings

    import adana_amd

    print("case: kept diagnostics on 5,000 tensors, fresh", fresh, flush=True)
    ps = [torch.nn.Parameter(torch.full((4,), 0.01 * (i % 7 + 1), device=DEV)) for i in range(5000)]
    opt = adana_amd.ADana(ps, lr=1e-3, fresh_diagnostics=fresh)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        for p in ps:
            p.grad = torch.full_like(p, 1e-3)
        opt.step()
        assert opt._fast                              # the next steps take the table's scan
        kept1 = opt.state[ps[5]]["gradient_norm"]
        first = float(kept1)
        for p in ps:
            p.grad = torch.full_like(p, 2e-3)
        opt.step()
        kept2 = opt.state[ps[4000]]["gradient_norm"]
        view2 = opt.state[ps[2500]]["m_norm"].detach()
        second, second_m = float(kept2), float(view2)
        for p in ps:
            p.grad = torch.full_like(p, 4e-3)
        opt.step()
        torch.cuda.synchronize()
    now = float(opt.state[ps[4000]]["gradient_norm"])
    assert now == pytest.approx(2 * second)
    if fresh is None:
        assert float(kept1) == first and float(kept2) == second and float(view2) == second_m
        assert opt.state[ps[5]]["gradient_norm"] is not kept1 and opt.state[ps[4000]]["gradient_norm"] is not kept2
    else:
        assert opt.state[ps[4000]]["gradient_norm"] is kept2 and float(kept2) == now
        assert float(kept1) == pytest.approx(4 * first)


@pytest.mark.parametrize("master", [False, True])
@pytest.mark.parametrize("star", [False, True])
def test_state_slab_guards(star, master):
    """The state slabs' elements outside every state tensor -- a canary bit
    pattern before the first tensor and after the last, zero padding between
    tensors -- are untouched after steps over tensors that end on, before and
    after chunk boundaries; and the check sees a changed canary."""
    import adana_amd

    print("case: state slab guards star", star, "master", master, flush=True)
    rng = np.random.default_rng(11)
    sizes = [1, 1023, 1024, 1025, 5000, 3]
    dt = torch.bfloat16 if master else torch.float32
    params = [torch.nn.Parameter(torch.from_numpy(_normal(rng, (n,), 0.02)).to(DEV).to(dt)) for n in sizes]
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(params, lr=1e-3, kappa=0.85, weight_decay=0.1, master_weights=master)
    for _ in range(3):
        for p, n in zip(params, sizes):
            p.grad = torch.from_numpy(_normal(rng, (n,), 1e-3)).to(DEV).to(dt)
        opt.step()
    torch.cuda.synchronize()
    families = (3 if star else 2) + (1 if master else 0)
    assert opt._check_slab_guards() == families
    ref, fam, base, total, _ = opt._slab_guards[0]
    slab = ref()
    bits = slab.view(torch.int16 if slab.dtype == torch.bfloat16 else torch.int32)
    bits[base + total] = 0
    with pytest.raises(RuntimeError, match="overwritten"):
        opt._check_slab_guards()
