"""GPU parity of adana_amd.Manau on the reference's own golden run
(tests/golden/make_golden_manau.py: src/optim/manau.py over a named GPT-like
list, 12 steps, three configurations).

Dana-Star-MK4 branch (the HIP kernel, ADANA_VARIANT_MANAU), against the
oracle driven in lock step on the same inputs:
  * dana_m, dana_v, dana_tau: bit-exact;
  * p: bit-exact except the pow's rare rounding-boundary cases (at most
    STAR_HARD_CASES per tensor per step, within STAR_P_ULPS scaled ulps);
  * current_alpha and the groups' weighted_step_count: exactly the
    reference's; the other diagnostics rtol 1e-5.
Muon half (torch operations), against the reference's recorded run:
  * muon_buffer: bit-exact (float32 multiply-add of the gradients);
  * parameters: within the bfloat16 Newton-Schulz products' tolerance
    (different GEMM accumulation orders on the GPU and the CPU).
Also the state_dict schema and a torch.save round trip.
"""
import io
import json
import os

import numpy as np
import pytest
import torch

from helpers import ulp_diff
from test_gpu_parity import _check_star_p

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ("manau", "manau_wt", "manau_mk4")


def _load(case, nonfinite=False):
    """Inputs and the reference's recorded run; ``nonfinite``: the inputs with
    NaN / inf gradient entries in Dana-branch tensors (make_golden_manau.py
    --nonfinite)."""
    tag = ".nonfinite" if nonfinite else ""
    z = np.load(os.path.join(GOLDEN, f"manau{tag}.inputs.npz"))
    meta = json.loads(str(z["meta"]))
    n = len(meta["params"])
    p0 = [z[f"p0_{i}"] for i in range(n)]
    grads = [[z[f"g_{k}_{i}"] for i in range(n)] for k in range(1, meta["n_steps"] + 1)]
    return meta, p0, grads, np.load(os.path.join(GOLDEN, f"manau.{case}{tag}.npz"))


def _build(meta, case, p0):
    import contextlib

    import adana_amd

    kw = meta["cases"][case]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in p0]
    groups = []
    for gi, scale in enumerate(meta["group_wd_scale"]):
        idx = [i for i, (_, _, g) in enumerate(meta["params"]) if g == gi]
        groups.append({"params": [params[i] for i in idx], "param_names": [meta["params"][i][0] for i in idx],
                       "weight_decay": kw["weight_decay"] * scale})
    with contextlib.redirect_stdout(io.StringIO()):
        opt = adana_amd.Manau(groups, **kw)
    return opt, params, kw


def _set_step_inputs(opt, params, meta, kw, grads, k):
    for g in opt.param_groups:
        g["lr"] = kw["lr"] * meta["lr_multiplier"][k - 1]
    for i, p in enumerate(params):
        p.grad = torch.from_numpy(grads[k - 1][i].copy()).to(DEV)


@pytest.mark.parametrize("case,nonfinite", [(c, False) for c in CASES] + [("manau", True), ("manau_mk4", True)])
def test_manau_matches_oracle_and_reference(oracle_mod, case, nonfinite):
    O = oracle_mod
    print("case: Manau", case, "non-finite gradients" if nonfinite else "", flush=True)
    meta, p0, grads, gold = _load(case, nonfinite)
    opt, params, kw = _build(meta, case, p0)
    use_muon = [bool(opt.state[p]["use_muon"]) for p in params]
    assert use_muon == [bool(u) for u in gold["use_muon"]]
    host = [x.copy() for x in p0]
    groups = []
    order = []
    for gi, scale in enumerate(meta["group_wd_scale"]):
        idx = [i for i, (_, _, g) in enumerate(meta["params"]) if g == gi]
        order.append(idx)
        groups.append(O.OracleManauGroup(
            params=[host[i] for i in idx], use_muon=[use_muon[i] for i in idx], lr=kw["lr"],
            weight_decay=kw["weight_decay"] * scale, delta=kw.get("delta", 8.0), kappa=kw.get("kappa", 1.0),
            mk4A=kw.get("mk4A", 0.0), mk4B=kw.get("mk4B", 0.0), clipsnr=kw.get("clipsnr", 1.0),
            epsilon=kw.get("epsilon", 1e-8), weight_time=kw.get("weight_time", False),
            wd_decaying=kw.get("wd_decaying", False), wd_ts=kw.get("wd_ts", 1.0),
            dana_momentum=kw.get("dana_momentum", False)))
    orc = O.OracleManau(groups=groups, peak_lr=kw["lr"])
    worst_muon = 0.0
    for k in range(1, meta["n_steps"] + 1):
        _set_step_inputs(opt, params, meta, kw, grads, k)
        for g in orc.groups:
            g.lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        prev = [x.copy() for x in host]
        opt.step()
        orc.step([[grads[k - 1][i] for i in idx] for idx in order])
        torch.cuda.synchronize()
        assert [g["weighted_step_count"] for g in opt.param_groups] == list(gold["weighted_step_count"][k - 1])
        for i, p in enumerate(params):
            st = opt.state[p]
            tag = f"{case} t={k} {meta['params'][i][0]}"
            if use_muon[i]:
                if k in meta["checkpoints"]:
                    assert ulp_diff(st["muon_buffer"].cpu().numpy(), gold[f"muon_buffer{i}_t{k}"]).max() == 0, tag
                    d = np.abs(p.detach().cpu().numpy() - gold[f"p{i}_t{k}"]).max()
                    worst_muon = max(worst_muon, d / kw["lr"])
                continue
            ost = orc.state[id(host[i])]
            assert st["step"] == ost["step"] == k
            for key in ("dana_m", "dana_v", "dana_tau"):
                d = ulp_diff(st[key].cpu().numpy(), ost[key])
                assert d.max() == 0, f"{tag}: {key} differs by {d.max()} ulp"
            gp = p.detach().cpu().numpy()
            _check_star_p(gp, host[i], prev[i], tag)
            host[i][...] = gp                                          # continue from the GPU's p
            assert st["current_alpha"] == ost["current_alpha"] == gold["diag"][k - 1, i, 0], tag
            got = [float(st[key]) for key in ("current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")]
            ref = [ost[key] for key in ("current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")]
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30, equal_nan=True, err_msg=tag)
    # Muon parameters after 12 steps of bfloat16 Newton-Schulz updates (each
    # about 0.2 * lr per entry) on the GPU vs the reference's CPU run
    print(f"max |p_muon - reference| / lr over the checkpoints: {worst_muon:.3g}", flush=True)
    assert worst_muon < 0.05


def test_manau_state_dict_schema_and_round_trip():
    print("case: Manau state_dict", flush=True)
    meta, p0, grads, gold = _load("manau")
    a, pa, kw = _build(meta, "manau", p0)
    for k in range(1, meta["state_at"] + 1):
        _set_step_inputs(a, pa, meta, kw, grads, k)
        a.step()
    torch.cuda.synchronize()
    sd = a.state_dict()
    schema = json.loads(str(gold["schema"]))
    for idx, ent in schema["state"].items():
        ours = sd["state"][int(idx)]
        assert sorted(ours) == sorted(ent), idx
        for key, want in ent.items():
            v = ours[key]
            if want["type"] == "Tensor":
                assert isinstance(v, torch.Tensor) and str(v.dtype) == want["dtype"] and list(v.shape) == want["shape"]
            else:
                assert type(v).__name__ == want["type"], (idx, key)
    buf = io.BytesIO()
    torch.save({"optimizer": sd, "params": [p.detach().cpu() for p in pa]}, buf)
    buf.seek(0)
    ck = torch.load(buf, weights_only=True)
    b, pb, _ = _build(meta, "manau", [t.numpy() for t in ck["params"]])
    b.load_state_dict(ck["optimizer"])
    for k in range(meta["state_at"] + 1, meta["n_steps"] + 1):
        _set_step_inputs(a, pa, meta, kw, grads, k)
        _set_step_inputs(b, pb, meta, kw, grads, k)
        a.step()
        b.step()
    torch.cuda.synchronize()
    for x, y in zip(pa, pb):
        assert torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32))
        for key in ("dana_m", "dana_v", "dana_tau", "muon_buffer"):
            if key in a.state[x]:
                assert torch.equal(a.state[x][key].view(torch.int32), b.state[y][key].view(torch.int32)), key


def test_manau_weight_time_many_classes(oracle_mod):
    """weight_time gives every Dana parameter its own step and alpha (the
    group's counter advances once per parameter): 12 parameters make 12
    scalar classes, more than one launch carries, so the branch runs as two
    launch sets.  Against the oracle as above."""
    import contextlib

    import adana_amd

    O = oracle_mod
    print("case: Manau weight_time, 12 classes", flush=True)
    rng = np.random.default_rng(21)
    shapes = [(57,), (300,), (4,), (1000,), (33,), (64, 9), (5,), (17, 3), (2048,), (1,), (99,), (7, 7)]
    names = [f"block.{i}.norm.weight" if len(s) == 1 else f"wte.weight.{i}" for i, s in enumerate(shapes)]
    p0 = [rng.normal(0, 0.02, s).astype(np.float32) for s in shapes]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in p0]
    kw = dict(lr=1e-2, weight_decay=0.05, kappa=0.7, clipsnr=1.5, delta=8.0, weight_time=True, wd_decaying=True,
              wd_ts=4.0)
    with contextlib.redirect_stdout(io.StringIO()):
        opt = adana_amd.Manau([{"params": params, "param_names": names}], **kw)
    assert not any(opt.state[p]["use_muon"] for p in params)
    host = [x.copy() for x in p0]
    orc = O.OracleManau(groups=[O.OracleManauGroup(
        params=host, use_muon=[False] * len(host), lr=kw["lr"], weight_decay=kw["weight_decay"], delta=8.0,
        kappa=0.7, clipsnr=1.5, weight_time=True, wd_decaying=True, wd_ts=4.0)], peak_lr=kw["lr"])
    for k in range(1, 7):
        lr = kw["lr"] * (0.5 + 0.1 * k)
        opt.param_groups[0]["lr"] = lr
        orc.groups[0].lr = lr
        gs = [rng.normal(0, 1e-3, s).astype(np.float32) for s in shapes]
        for p, g in zip(params, gs):
            p.grad = torch.from_numpy(g.copy()).to(DEV)
        prev = [x.copy() for x in host]
        opt.step()
        orc.step([gs])
        torch.cuda.synchronize()
        assert opt.param_groups[0]["weighted_step_count"] == orc.groups[0].weighted_step_count
        assert len(opt._sets) == 2
        for i, p in enumerate(params):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"t={k} tensor {i}"
            for key in ("dana_m", "dana_v", "dana_tau"):
                assert ulp_diff(st[key].cpu().numpy(), ost[key]).max() == 0, f"{tag} {key}"
            gp = p.detach().cpu().numpy()
            _check_star_p(gp, host[i], prev[i], tag)
            host[i][...] = gp
            assert st["current_alpha"] == ost["current_alpha"], tag


@pytest.mark.parametrize("kappa,mk4", [(1.0, None), (2.0, None), (0.0, None), (0.3, None), (1.0, (0.2, 0.5))])
def test_manau_pow_kinds(oracle_mod, kappa, mk4):
    """Manau's branch instances the golden runs leave out: kappa 1 (no pow),
    special exponents -1 and 1, a general one, and the mk4 powers with
    kappa 1.  Against the oracle as above, 10 steps."""
    import contextlib

    import adana_amd

    O = oracle_mod
    print("case: Manau pow kind kappa", kappa, "mk4", mk4, flush=True)
    rng = np.random.default_rng(int(31 + 7 * kappa))
    shapes = [(97, 24), (24,), (1000,), (5,), (4096 + 3,)]
    names = ["transformer.wte.weight"] + [f"h.{i}.ln.weight" for i in range(len(shapes) - 1)]
    p0 = [rng.normal(0, 0.02, s).astype(np.float32) for s in shapes]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in p0]
    mk4A, mk4B = mk4 if mk4 else (0.0, 0.0)
    kw = dict(lr=1e-2, weight_decay=0.1, kappa=kappa, clipsnr=2.0, delta=4.0, mk4A=mk4A, mk4B=mk4B,
              wd_decaying=True, wd_ts=3.0)
    with contextlib.redirect_stdout(io.StringIO()):
        opt = adana_amd.Manau([{"params": params, "param_names": names}], **kw)
    host = [x.copy() for x in p0]
    orc = O.OracleManau(groups=[O.OracleManauGroup(
        params=host, use_muon=[False] * len(host), lr=kw["lr"], weight_decay=kw["weight_decay"], delta=4.0,
        kappa=kappa, mk4A=mk4A, mk4B=mk4B, clipsnr=2.0, wd_decaying=True, wd_ts=3.0)], peak_lr=kw["lr"])
    for k in range(1, 11):
        gs = [rng.normal(0, 1e-3, s).astype(np.float32) for s in shapes]
        for p, g in zip(params, gs):
            p.grad = torch.from_numpy(g.copy()).to(DEV)
        prev = [x.copy() for x in host]
        opt.step()
        orc.step([gs])
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"kappa={kappa} mk4={mk4} t={k} tensor {i}"
            for key in ("dana_m", "dana_v", "dana_tau"):
                assert ulp_diff(st[key].cpu().numpy(), ost[key]).max() == 0, f"{tag} {key}"
            gp = p.detach().cpu().numpy()
            _check_star_p(gp, host[i], prev[i], tag)
            host[i][...] = gp
            got = [float(st[key]) for key in ("current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")]
            ref = [ost[key] for key in ("current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")]
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30, err_msg=tag)


@pytest.mark.parametrize("seed", range(12))
def test_manau_random_configuration(oracle_mod, seed):
    """Seeded random Dana-branch configurations: an embedding matrix and 1-6
    vectors (1 to 70,000 elements), kappa from every pow kind's values, mk4A,
    mk4B, clipsnr, delta, weight_time, dana_momentum, decaying weight decay,
    a new lr every step and some all-zero gradients; 8 steps against the
    oracle as above."""
    import contextlib

    import adana_amd

    O = oracle_mod
    rng = np.random.default_rng(7000 + seed)
    shapes = [(int(rng.integers(1, 200)), int(rng.integers(1, 64)))]
    shapes += [(int(np.exp(rng.uniform(0, np.log(70000)))),) for _ in range(int(rng.integers(1, 7)))]
    names = ["transformer.wte.weight"] + [f"h.{i}.ln.weight" for i in range(len(shapes) - 1)]
    kw = dict(lr=float(10 ** rng.uniform(-3, -1.5)), weight_decay=float(rng.choice([0.0, 0.1])),
              kappa=float(rng.choice([0.0, 0.5, 0.85, 1.0, 2.0])), clipsnr=float(rng.choice([0.5, 1.0, 2.0])),
              delta=float(rng.choice([2.0, 4.0, 8.0])), mk4A=float(rng.choice([0.0, 0.1])),
              mk4B=float(rng.choice([0.0, 0.2])), weight_time=bool(rng.integers(2)),
              dana_momentum=bool(rng.integers(2)), wd_decaying=bool(rng.integers(2)),
              wd_ts=float(rng.choice([1.0, 3.0])))
    print(f"case: Manau random configuration seed {seed}: shapes {shapes} {kw}", flush=True)
    p0 = [rng.normal(0, 0.02, s).astype(np.float32) for s in shapes]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in p0]
    with contextlib.redirect_stdout(io.StringIO()):
        opt = adana_amd.Manau([{"params": params, "param_names": names}], **kw)
    host = [x.copy() for x in p0]
    okw = {k: v for k, v in kw.items() if k != "lr"}
    orc = O.OracleManau(groups=[O.OracleManauGroup(params=host, use_muon=[False] * len(host), lr=kw["lr"],
                                                   **okw)], peak_lr=kw["lr"])
    for k in range(1, 9):
        opt.param_groups[0]["lr"] = orc.groups[0].lr = kw["lr"] * float(rng.uniform(0.5, 1.5))
        gs = [(np.zeros(s, np.float32) if rng.random() < 0.1 else
               rng.normal(0, float(10 ** rng.uniform(-5, -2)), s).astype(np.float32)) for s in shapes]
        for p, g in zip(params, gs):
            p.grad = torch.from_numpy(g.copy()).to(DEV)
        prev = [x.copy() for x in host]
        opt.step()
        orc.step([gs])
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"seed {seed} t={k} tensor {i}"
            for key in ("dana_m", "dana_v", "dana_tau"):
                assert ulp_diff(st[key].cpu().numpy(), ost[key]).max() == 0, f"{tag} {key}"
            gp = p.detach().cpu().numpy()
            _check_star_p(gp, host[i], prev[i], tag)
            host[i][...] = gp
            got = [float(st[key]) for key in ("current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")]
            ref = [ost[key] for key in ("current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")]
            np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-30, equal_nan=True, err_msg=tag)
