"""GPU parity of the reference's own bfloat16 path (ADANA_STATE_BF16):
bfloat16 parameters without ``master_weights`` keep bfloat16 m, v, tau (the
reference's ``zeros_like(p)``, src/optim/adana.py:191-195;
src/optim/dana_star_mk4.py:251-255), in both of the reference's numerics:
its default torch.compile path (binary32 arithmetic, each tensor rounded to
bfloat16 where it is stored) and its eager ops (every op rounded to
bfloat16).

Bars:
  * p, m, v, tau bit-exact against the C oracle's bfloat16 modes
    (oracle/adana_oracle.c, adana_oracle_step_bf16), which reproduce the
    reference's own bfloat16 compiled and eager runs bit for bit
    (tests/test_oracle.py); Dana-Star's p additionally allows
    STAR_HARD_CASES elements per tensor per step within 1 bfloat16 ulp (a
    pow result within ~2^-52 of a binary32 rounding boundary may round
    either way);
  * against the reference's bfloat16 fixtures directly: every checkpoint of
    every golden case bit for bit (same allowance), compiled and eager;
  * diagnostics: bfloat16 0-d tensors as the reference's, within 1 bfloat16
    ulp of the oracle's (the reductions' order differs before the rounding).
"""
import numpy as np
import pytest
import torch

from helpers import bf16_ulp_diff, golden_cases, load_golden_case, load_golden_inputs
from test_gpu_parity import STAR_HARD_CASES

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"


def _to_gpu16(h: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(h).view(np.int16).copy()).view(torch.bfloat16).to(DEV)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def _check(got, want, tag, allow=0):
    d = bf16_ulp_diff(got, want)
    bad = int((d > 0).sum())
    assert bad <= allow and (bad == 0 or d.max() <= 1), f"{tag}: {bad} values differ (max {d.max()} bf16 ulp)"


def _diag_close(got, want, tag):
    """Within 1 bfloat16 ulp (NaN equal to NaN)."""
    for g, w, key in zip(got, want, ("current_alpha", "gradient_norm", "auto_factor_mean",
                                     "current_kappa_factor", "m_norm")):
        if np.isnan(w):
            assert np.isnan(g), (tag, key)
            continue
        tol = np.spacing(np.float32(abs(w))) * (1 << 16) if w else 0.0     # one bfloat16 ulp
        assert abs(g - w) <= tol, (tag, key, g, w)


def _golden_run(case, O, numerics):
    """The golden scenario on bfloat16 parameters: the HIP step and the
    oracle in lock step; yields after every step."""
    import adana_amd

    meta, p0, grads, has_grad = load_golden_inputs()
    kw = meta["cases"][case]["kwargs"]
    star = meta["cases"][case]["class"] == "DANA_STAR_MK4"
    host = [O.f32_to_bf16(x) for x in p0]
    idx = [[i for i in range(len(p0)) if meta["group_of"][i] == gi] for gi in range(2)]
    gpu = [torch.nn.Parameter(_to_gpu16(h)) for h in host]
    groups = [{"params": [gpu[i] for i in idx[gi]], "weight_decay": kw["weight_decay"] * meta["group_wd_scale"][gi]}
              for gi in range(2)]
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(groups, numerics=numerics, **kw)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=[host[i] for i in idx[gi]], lr=kw["lr"], delta=kw["delta"],
                                                  epsilon=1e-8, weight_decay=groups[gi]["weight_decay"])
                                    for gi in range(2)],
                            star=star, peak_lr=kw["lr"], kappa=kw["kappa"], clipsnr=kw["clipsnr"],
                            wd_decaying=kw["wd_decaying"], wd_ts=kw["wd_ts"], gamma_3_factor=kw["gamma_3_factor"],
                            bf16=True, numerics=numerics)
    for k in range(1, meta["n_steps"] + 1):
        lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        for g in opt.param_groups:
            g["lr"] = lr
        for g in orc.groups:
            g.lr = lr
        gl16 = [O.f32_to_bf16(grads[k - 1][i]) if has_grad[k - 1, i] else None for i in range(len(p0))]
        for p, g in zip(gpu, gl16):
            p.grad = None if g is None else _to_gpu16(g)
        opt.step()
        orc.step([[gl16[i] for i in idx[gi]] for gi in range(2)])
        torch.cuda.synchronize()
        yield k, meta, star, opt, orc, gpu, host, has_grad


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("case", golden_cases("eager"))
def test_bf16_golden_against_oracle_and_reference(oracle_mod, case, numerics):
    print("case: bf16 state golden scenario", case, numerics, flush=True)
    gold = load_golden_case(case, "bf16_compiled" if numerics == "compiled" else "bf16_eager")
    for k, meta, star, opt, orc, gpu, host, has_grad in _golden_run(case, oracle_mod, numerics):
        for i, p in enumerate(gpu):
            st = opt.state[p]
            ost = orc.state.get(id(host[i]))
            tag = f"{case} t={k} tensor {i}"
            if ost is None:
                assert len(st) == 0, tag
                continue
            assert st["step"] == ost["step"], tag
            keys = ("m", "v", "tau") if star else ("m", "v")
            for key in keys:
                assert st[key].dtype == torch.bfloat16, tag
                _check(_bits(st[key]), ost[key], f"{tag} {key}")
            got = _bits(p)
            _check(got, host[i], f"{tag} p", STAR_HARD_CASES if star else 0)
            host[i][...] = got.reshape(host[i].shape)                        # continue from the GPU's p
            if has_grad[k - 1, i]:
                assert all(st[key].dtype == torch.bfloat16 and st[key].dim() == 0 for key in oracle_mod.DIAG_KEYS)
                _diag_close([float(st[key]) for key in oracle_mod.DIAG_KEYS],
                            [ost[key] for key in oracle_mod.DIAG_KEYS], tag)
            if k in meta["checkpoints"]:
                # the reference's own bfloat16 run in the same numerics
                _check(got, gold[f"p{i}_t{k}"], f"{tag} p vs reference", STAR_HARD_CASES if star else 0)
                for key in keys:
                    _check(_bits(st[key]), gold[f"{key}{i}_t{k}"], f"{tag} {key} vs reference")


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("star", [False, True])
def test_bf16_mixed_list_views_and_clip(oracle_mod, star, numerics):
    """Tensors of 1 to 70,000 elements, one 2-byte-offset view (scalar path),
    two groups, 12 steps crossing t = delta, a fused clip every third step:
    bit-exact against the oracle (the clip coefficient applied to the bf16
    gradient as torch's in-place clipping leaves it)."""
    import adana_amd

    O = oracle_mod
    print("case: bf16 state mixed list, star", star, numerics, flush=True)
    rng = np.random.default_rng(21)
    sizes = [70_000, 1, 3, 1024, 4099, 33 * 65]
    host = [O.f32_to_bf16(rng.normal(0, 0.02, n).astype(np.float32)) for n in sizes]
    flat = torch.empty(sizes[4] + 1, dtype=torch.bfloat16, device=DEV)
    gpu = []
    for i, h in enumerate(host):
        if i == 4:
            v = flat[1:]                                                  # 2 bytes in: not 8-byte aligned
            v.copy_(_to_gpu16(h))
            gpu.append(torch.nn.Parameter(v))
        else:
            gpu.append(torch.nn.Parameter(_to_gpu16(h)))
    hp = dict(lr=2e-3, delta=8.0, kappa=0.85, weight_decay=0.2, clipsnr=2.0, wd_decaying=True, wd_ts=5.0)
    groups = [{"params": gpu[:3]}, {"params": gpu[3:], "weight_decay": 0.0}]
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(groups, numerics=numerics, **hp)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=host[:3], lr=hp["lr"], weight_decay=0.2),
                                    O.OracleGroup(params=host[3:], lr=hp["lr"], weight_decay=0.0)],
                            star=star, peak_lr=hp["lr"], kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=5.0,
                            bf16=True, numerics=numerics)
    for t in range(1, 13):
        g16 = [O.f32_to_bf16(rng.normal(0, 1e-3 * (30 if t % 3 == 0 else 1), n).astype(np.float32)) for n in sizes]
        for p, g in zip(gpu, g16):
            p.grad = _to_gpu16(g)
        if t % 3 == 0:
            total = opt.clip_grad_norm_(0.05)
            gf = [O.bf16_to_f32(g) for g in g16]
            _, want_total = O.clip_norms(gf, bf16=True)
            assert float(total) == pytest.approx(float(want_total), rel=2 ** -7)   # within 1 bf16 ulp
            coef = np.float32(float(opt._pending_clip[2][1]))                     # the device's coefficient
            assert coef == pytest.approx(float(O.clip_coef(want_total, 0.05, bf16=True)), rel=2 ** -7)
            g16 = [O.f32_to_bf16(O.clip_scale(g, coef, bf16=True)) for g in gf]
        opt.step()
        orc.step([g16[:3], g16[3:]])
        torch.cuda.synchronize()
        for i, p in enumerate(gpu):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"star {star} t={t} tensor {i} (n={sizes[i]})"
            for key in ("m", "v", "tau") if star else ("m", "v"):
                _check(_bits(st[key]), ost[key], f"{tag} {key}")
            got = _bits(p)
            _check(got, host[i], f"{tag} p", STAR_HARD_CASES if star else 0)
            host[i][...] = got
            if t % 3 == 0:
                _check(_bits(p.grad), g16[i], f"{tag} clipped grad written back")


def test_bf16_state_dict_matches_reference_schema():
    """state_dict() of the bfloat16 path has the reference's schema: m, v,
    tau bfloat16 shaped like p, an int step, and bfloat16 0-d diagnostics;
    a torch.save round trip resumes bit-identically."""
    import io

    import adana_amd

    print("case: bf16 state_dict", flush=True)
    torch.manual_seed(0)
    ps = [torch.nn.Parameter((torch.randn(300, device=DEV) * 0.02).bfloat16()) for _ in range(2)]
    opt = adana_amd.DANA_STAR_MK4(ps, lr=1e-3, kappa=0.85, clipsnr=2.0)
    grads = [[(torch.randn(300, device=DEV) * 1e-3).bfloat16() for _ in ps] for _ in range(6)]
    for k in range(3):
        for p, g in zip(ps, grads[k]):
            p.grad = g.clone()
        opt.step()
    sd = opt.state_dict()
    st = sd["state"][0]
    assert isinstance(st["step"], int) and st["step"] == 3
    for key in ("m", "v", "tau"):
        assert st[key].dtype == torch.bfloat16 and st[key].shape == (300,)
    for key in ("current_alpha", "gradient_norm", "auto_factor_mean", "current_kappa_factor", "m_norm"):
        assert st[key].dtype == torch.bfloat16 and st[key].dim() == 0
    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    qs = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    opt2 = adana_amd.DANA_STAR_MK4(qs, lr=1e-3, kappa=0.85, clipsnr=2.0)
    opt2.load_state_dict(torch.load(buf, weights_only=True))
    for k in range(3, 6):
        for p, q, g in zip(ps, qs, grads[k]):
            p.grad = g.clone()
            q.grad = g.clone()
        opt.step()
        opt2.step()
    torch.cuda.synchronize()
    for p, q in zip(ps, qs):
        assert torch.equal(_bits_t(p), _bits_t(q))
        for key in ("m", "v", "tau"):
            assert torch.equal(_bits_t(opt.state[p][key]), _bits_t(opt2.state[q][key]))


def _bits_t(t):
    return t.detach().view(torch.int16)



@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("star", [False, True])
def test_bf16_nonfinite_gradients(oracle_mod, star, numerics):
    """NaN, +inf and -inf gradient entries (and huge and subnormal ones) on the
    bfloat16 path: p, m, v, tau bit-exact against the oracle's bfloat16
    restatement wherever it is finite, and NaN where it is NaN (the IEEE arms
    of the bf16 division and square root, and the pow table's NaN entry)."""
    import adana_amd

    O = oracle_mod
    print("case: bf16 state, non-finite gradients, star", star, numerics, flush=True)
    rng = np.random.default_rng(5)
    sizes = [4096, 777]
    host = [O.f32_to_bf16(rng.normal(0, 0.02, n).astype(np.float32)) for n in sizes]
    gpu = [torch.nn.Parameter(_to_gpu16(h)) for h in host]
    hp = dict(lr=1e-3, delta=8.0, kappa=0.85, weight_decay=0.1, clipsnr=2.0)
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(gpu, numerics=numerics, **hp)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=host, lr=hp["lr"], weight_decay=0.1)],
                            star=star, peak_lr=hp["lr"], kappa=0.85, clipsnr=2.0, bf16=True, numerics=numerics)
    specials = np.array([np.nan, np.inf, -np.inf, 3e38, -3e38, 1e-40, -1e-40, 0.0], np.float32)
    for t in range(1, 11):
        gf = [rng.normal(0, 1e-3, n).astype(np.float32) for n in sizes]
        if t in (2, 5, 9):
            for g in gf:
                idx = rng.choice(g.size, 40, replace=False)
                g[idx] = rng.choice(specials, 40)
        g16 = [O.f32_to_bf16(g) for g in gf]
        for p, g in zip(gpu, g16):
            p.grad = _to_gpu16(g)
        opt.step()
        orc.step([g16])
        torch.cuda.synchronize()
        for i, p in enumerate(gpu):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"star {star} t={t} tensor {i}"
            for key in ("m", "v", "tau") if star else ("m", "v"):
                got, want = _bits(st[key]), ost[key]
                gn, wn = np.isnan(O.bf16_to_f32(got)), np.isnan(O.bf16_to_f32(want))
                assert np.array_equal(gn, wn), f"{tag} {key}: NaN in different places"
                _check(got[~gn], want[~wn], f"{tag} {key}")
            got, want = _bits(p), host[i]
            gn, wn = np.isnan(O.bf16_to_f32(got)), np.isnan(O.bf16_to_f32(want))
            assert np.array_equal(gn, wn), f"{tag} p: NaN in different places"
            _check(got[~gn], want[~wn], f"{tag} p", STAR_HARD_CASES if star else 0)
            host[i][...] = got
