"""Checkpoint interchange on the GPU (src/optim/utils.py:260-361 saves and
restores ``opt.state_dict()``):

  * a checkpoint the reference optimizer wrote at step 8
    (tests/golden/<case>.state8.npz) resumes in this build and follows the
    reference's own trajectory to step 20 (bars: resume_bars, shared with the
    oracle's CPU run of the same resume in tests/test_checkpoint_cpu.py);
  * this build's state_dict after 8 steps has the reference's schema (keys,
    Python types, dtypes, shapes, group entries) and its values (m, v
    bit-exact; tau within 2 ulp; diagnostics rtol 2e-5);
  * a torch.save / torch.load(weights_only=True) round trip mid-run resumes
    bit-identically;
  * a reference checkpoint (fp32 moments, no master copy) loads into the bf16
    master-weights extension and continues as the oracle does from the same
    state;
  * a deepcopy of a stepped optimizer keeps its configuration and steps on
    its own tensors, bit-identically to the original;
  * a loaded state missing a moment or its step counter fails with the
    reference's KeyError before anything changes.
"""
import io
import math

import numpy as np
import pytest
import torch

from helpers import (golden_cases, load_golden_case, load_golden_inputs, load_reference_state_dict,
                     state_dict_schema, ulp_diff)
from test_checkpoint_cpu import resume_bars

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"


def _build(case, p_init, dtype=torch.float32, **extra):
    import adana_amd

    meta, *_ = load_golden_inputs()
    c = meta["cases"][case]
    kw = dict(c["kwargs"])
    cls = adana_amd.DANA_STAR_MK4 if c["class"] == "DANA_STAR_MK4" else adana_amd.ADana
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV, dtype)) for x in p_init]
    groups = []
    for gi in range(2):
        groups.append({"params": [p for i, p in enumerate(params) if meta["group_of"][i] == gi],
                       "weight_decay": kw["weight_decay"] * meta["group_wd_scale"][gi]})
    # the checkpoints are the reference's eager run's: step in the same numerics
    return cls(groups, **kw, **{"numerics": "eager", **extra}), params, meta, kw, c["class"] == "DANA_STAR_MK4"


def _run(opt, params, meta, kw, grads, has_grad, k0, k1, dtype=torch.float32, on_step=None):
    for k in range(k0, k1 + 1):
        for g in opt.param_groups:
            g["lr"] = kw["lr"] * meta["lr_multiplier"][k - 1]
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grads[k - 1][i].copy()).to(DEV, dtype) if has_grad[k - 1, i] else None
        opt.step()
        if on_step:
            on_step(k)


@pytest.mark.parametrize("case", golden_cases("eager"))
def test_resume_from_reference_checkpoint(case):
    print("case: resume reference checkpoint", case, flush=True)
    meta, p0, grads, has_grad = load_golden_inputs()
    gold = load_golden_case(case, "eager")
    opt, params, meta, kw, star = _build(case, [gold[f"p{i}_t8"] for i in range(len(p0))])
    ref, _ = load_reference_state_dict(case, device=DEV)
    opt.load_state_dict(ref)

    def check(k):
        if k in (9, 20):
            torch.cuda.synchronize()
            got = []
            for p in params:
                st = opt.state[p]
                got.append({"step": st["step"], "m": st["m"].cpu().numpy(), "v": st["v"].cpu().numpy(),
                            "p": p.detach().cpu().numpy(),
                            **({"tau": st["tau"].cpu().numpy()} if star else {})})
            resume_bars(case, k, got, gold, star)

    _run(opt, params, meta, kw, grads, has_grad, 9, meta["n_steps"], on_step=check)
    for g, wsc in zip(opt.param_groups, gold["weighted_step_count"]):
        assert g["weighted_step_count"] == wsc
    for i, p in enumerate(params):                  # diagnostics of the last step
        st = opt.state[p]
        got = np.array([float(st[k]) for k in ("current_alpha", "gradient_norm", "auto_factor_mean",
                                                "current_kappa_factor", "m_norm")])
        np.testing.assert_allclose(got, gold["diag"][-1, i], rtol=2e-5, atol=1e-12, equal_nan=True)


@pytest.mark.parametrize("case", golden_cases("eager"))
def test_state_dict_matches_reference_schema(case):
    print("case: state_dict schema", case, flush=True)
    meta, p0, grads, has_grad = load_golden_inputs()
    opt, params, meta, kw, star = _build(case, p0)
    _run(opt, params, meta, kw, grads, has_grad, 1, 8)
    torch.cuda.synchronize()
    ours = opt.state_dict()
    ref, schema = load_reference_state_dict(case)
    assert state_dict_schema(ours) == state_dict_schema(ref)
    for gi, (g_ours, g_ref) in enumerate(zip(ours["param_groups"], schema["param_groups"])):
        for k, v in g_ref.items():
            assert g_ours[k] == v, (gi, k)
    for idx, st in ref["state"].items():
        o = ours["state"][idx]
        assert o["step"] == st["step"]
        assert ulp_diff(o["m"].cpu().numpy(), st["m"].numpy()).max() == 0
        assert ulp_diff(o["v"].cpu().numpy(), st["v"].numpy()).max() == 0
        if star:
            assert ulp_diff(o["tau"].cpu().numpy(), st["tau"].numpy()).max() <= 2
        for k in ("current_alpha", "gradient_norm", "auto_factor_mean", "current_kappa_factor", "m_norm"):
            np.testing.assert_allclose(float(o[k]), float(st[k]), rtol=2e-5, atol=1e-12, equal_nan=True)


@pytest.mark.parametrize("case", ["dana_mk4", "dana_star_mk4"])
def test_torch_save_round_trip_resumes_bit_identically(case):
    print("case: torch.save round trip", case, flush=True)
    meta, p0, grads, has_grad = load_golden_inputs()
    a, pa, meta, kw, star = _build(case, p0)
    _run(a, pa, meta, kw, grads, has_grad, 1, 8)
    buf = io.BytesIO()
    torch.save({"optimizer": a.state_dict(), "params": [p.detach().cpu() for p in pa]}, buf)
    buf.seek(0)
    ck = torch.load(buf, weights_only=True)
    b, pb, *_ = _build(case, [t.numpy() for t in ck["params"]])
    b.load_state_dict(ck["optimizer"])
    _run(a, pa, meta, kw, grads, has_grad, 9, meta["n_steps"])
    _run(b, pb, meta, kw, grads, has_grad, 9, meta["n_steps"])
    torch.cuda.synchronize()
    for x, y in zip(pa, pb):
        assert torch.equal(x.detach().view(torch.int32), y.detach().view(torch.int32))
        for k in ("m", "v") + (("tau",) if star else ()):
            assert torch.equal(a.state[x][k].view(torch.int32), b.state[y][k].view(torch.int32))
        assert a.state[x]["step"] == b.state[y]["step"]


def test_reference_checkpoint_into_bf16_master_mode(oracle_mod):
    """fp32-moment checkpoint without 'master' into master_weights=True bf16
    parameters: the master starts as float(p_bf16) and the run continues as
    the oracle's master-mode run from that state (ADana: bit-exact)."""
    print("case: reference checkpoint into bf16 master mode", flush=True)
    O = oracle_mod
    case = "dana_mk4"
    meta, p0, grads, has_grad = load_golden_inputs()
    gold = load_golden_case(case, "eager")
    p16 = [O.f32_to_bf16(gold[f"p{i}_t8"]).reshape(gold[f"p{i}_t8"].shape) for i in range(len(p0))]
    p_bf = [O.bf16_to_f32(x).reshape(x.shape) for x in p16]
    opt, params, meta, kw, star = _build(case, p_bf, dtype=torch.bfloat16, master_weights=True)
    ref, schema = load_reference_state_dict(case, device=DEV)
    opt.load_state_dict(ref)
    for p in params:
        st = opt.state[p]
        assert st["m"].dtype == torch.float32 and st["master"].dtype == torch.float32
        assert torch.equal(st["master"], p.detach().float())
    groups = []
    for gi in range(2):
        groups.append(O.OracleGroup(params=[p16[i] for i in range(len(p16)) if meta["group_of"][i] == gi],
                                    lr=kw["lr"], delta=kw["delta"], epsilon=1e-8,
                                    weight_decay=kw["weight_decay"] * meta["group_wd_scale"][gi],
                                    weighted_step_count=schema["param_groups"][gi]["weighted_step_count"]))
    orc = O.OracleOptimizer(groups=groups, star=False, peak_lr=kw["lr"], kappa=kw["kappa"],
                            clipsnr=kw["clipsnr"], wd_decaying=kw["wd_decaying"], wd_ts=kw["wd_ts"],
                            gamma_3_factor=kw["gamma_3_factor"], master=True, numerics="eager")
    for i, p in enumerate(p16):
        st = ref["state"][i]
        orc.state[id(p)] = {"step": st["step"], "m": st["m"].cpu().numpy().copy(),
                            "v": st["v"].cpu().numpy().copy(), "master": p_bf[i].copy()}
    g16 = [[O.f32_to_bf16(g).reshape(g.shape) for g in gs] for gs in grads]
    for k in range(9, 13):
        lr = kw["lr"] * meta["lr_multiplier"][k - 1]
        for g in opt.param_groups:
            g["lr"] = lr
        for g in orc.groups:
            g.lr = lr
        for i, p in enumerate(params):
            p.grad = (torch.from_numpy(g16[k - 1][i].view(np.int16).copy()).view(torch.bfloat16).to(DEV)
                      if has_grad[k - 1, i] else None)
        opt.step()
        gl = []
        for gi in range(2):
            idx = [i for i in range(len(p16)) if meta["group_of"][i] == gi]
            gl.append([g16[k - 1][i] if has_grad[k - 1, i] else None for i in idx])
        orc.step(gl)
    torch.cuda.synchronize()
    for i, p in enumerate(params):
        st, ost = opt.state[p], orc.state[id(p16[i])]
        assert ulp_diff(st["master"].cpu().numpy(), ost["master"]).max() == 0, i
        assert ulp_diff(st["m"].cpu().numpy(), ost["m"]).max() == 0, i
        assert np.array_equal(p.detach().cpu().view(torch.int16).numpy().view(np.uint16), p16[i]), i


def test_state_tensors_have_own_storages_in_family_slabs():
    """State tensors are laid out family by family (all m end to end, then
    all v, all tau; 4 KB aligned) but each has a storage of its own, so a
    per-parameter deepcopy (DynamicsLogger, src/logger/logger.py:93) and
    torch.save copy only that tensor's bytes."""
    import copy
    import adana_amd

    print("case: state slab layout", flush=True)
    shapes = [(300, 7), (5,), (4096,), (1, 1), (70000,)]
    params = [torch.nn.Parameter(torch.randn(s, device=DEV)) for s in shapes]
    opt = adana_amd.DANA_STAR_MK4(params, lr=1e-3, kappa=0.85)
    for p in params:
        p.grad = torch.randn_like(p) * 1e-3
    opt.step()
    torch.cuda.synchronize()
    for fam in ("m", "v", "tau"):
        ptrs = [opt.state[p][fam].data_ptr() for p in params]
        assert all(x % 4096 == 0 for x in ptrs), fam
        for a, b, p in zip(ptrs, ptrs[1:], params):
            assert b - a == (p.numel() + 1023) // 1024 * 4096, fam     # end to end in one slab
        for p in params:
            t = opt.state[p][fam]
            assert t._base is None and t.untyped_storage().nbytes() == 4 * p.numel()
            assert t.shape == p.shape and t.dtype == p.dtype and t.is_contiguous()
    snap = copy.deepcopy(opt.state[params[2]])
    assert snap["m"].untyped_storage().nbytes() == 4 * 4096
    assert torch.equal(snap["m"], opt.state[params[2]]["m"])
    buf = io.BytesIO()
    torch.save(opt.state_dict(), buf)
    assert len(buf.getvalue()) < 3 * 4 * sum(p.numel() for p in params) + 200_000


@pytest.mark.parametrize("star", [False, True])
def test_deepcopy_of_a_stepped_optimizer_steps_on_its_own(star):
    """copy.deepcopy of an optimizer after 3 steps copies its parameters and
    state and keeps its configuration (torch.optim.Optimizer alone would drop
    self.lr and the rest, and the copy's step() would fail); a clip pending
    at the copy is applied to the original's gradients first (a Parameter's
    copy has no gradient); the copy then steps on its own tensors,
    bit-identically to the original fed the same gradients, and leaves the
    original's tensors untouched."""
    import copy
    import adana_amd

    print("case: deepcopy of a stepped optimizer, star", star, flush=True)
    torch.manual_seed(5)
    params = [torch.nn.Parameter(torch.randn(s, device=DEV) * 0.02) for s in [(300, 7), (5,), (70000,)]]
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(params, lr=1e-3, kappa=0.85, clipsnr=2.0, weight_decay=0.1)
    for _ in range(3):
        for p in params:
            p.grad = torch.randn_like(p) * 1e-3
        opt.step()
    for p in params:                                   # a clip pending when the copy is taken
        p.grad = torch.randn_like(p) * 1e-1
    opt.clip_grad_norm_(1e-3)
    twin = copy.deepcopy(opt)
    tparams = twin.param_groups[0]["params"]
    assert all(a is not b and torch.equal(a, b) for a, b in zip(params, tparams))
    assert opt._pending_clip is None and all(q.grad is None for q in tparams)  # Parameter copies drop grads
    for p, q in zip(params, tparams):
        q.grad = p.grad.clone()                           # the clipped gradients
    opt.step()
    twin.step()
    torch.cuda.synchronize()
    assert all(torch.equal(p, q) for p, q in zip(params, tparams))
    keys = ("m", "v") + (("tau",) if star else ())
    for _ in range(6):
        grads = [torch.randn_like(p) * 1e-3 for p in params]
        for p, q, g in zip(params, tparams, grads):
            p.grad, q.grad = g.clone(), g.clone()
        opt.step()
        before = [p.detach().clone() for p in params]
        twin.step()
        torch.cuda.synchronize()
        for p, q, b in zip(params, tparams, before):
            assert torch.equal(p, b)                               # the original is not touched
            assert torch.equal(p, q)
            for k in keys:
                assert opt.state[p][k].data_ptr() != twin.state[q][k].data_ptr()
                assert torch.equal(opt.state[p][k], twin.state[q][k])
            assert opt.state[p]["step"] == twin.state[q]["step"]
            for k in adana_amd.optim.DIAG_KEYS:
                assert torch.equal(opt.state[p][k], twin.state[q][k]) or (
                    opt.state[p][k].isnan() and twin.state[q][k].isnan())


def test_diagnostics_have_own_storages_and_stay_live():
    """Each 0-d diagnostic is a tensor with a 4-byte storage of its own (a
    per-parameter deepcopy copies 4 bytes, not the list's buffer) that the
    kernel still writes every step; the packed read-out agrees with it."""
    import copy
    import adana_amd

    print("case: diagnostics storages", flush=True)
    shapes = [(300, 7), (5,), (4096,), (1, 1)]
    params = [torch.nn.Parameter(torch.randn(s, device=DEV)) for s in shapes]
    opt = adana_amd.DANA_STAR_MK4(params, lr=1e-3, kappa=0.85)
    seen = []
    for k in range(2):
        for p in params:
            p.grad = torch.randn_like(p) * 10.0 ** (-3 - k)
        opt.step()
        torch.cuda.synchronize()
        seen.append([[float(opt.state[p][key]) for key in adana_amd.DIAG_KEYS] for p in params])
    assert seen[0] != seen[1]                                # rewritten in place by the second step
    _, packed = opt.diagnostics_host()
    np.testing.assert_array_equal(packed, np.array(seen[1], np.float32))
    for p in params:
        st = opt.state[p]
        for key in adana_amd.DIAG_KEYS:
            t = st[key]
            assert t.dim() == 0 and t.dtype == torch.float32 and t.untyped_storage().nbytes() == 4
        snap = copy.deepcopy(st)
        for key in adana_amd.DIAG_KEYS:
            assert snap[key].untyped_storage().nbytes() == 4
            assert float(snap[key]) == float(st[key]) or (math.isnan(float(snap[key])) and math.isnan(float(st[key])))


def test_distributed_checkpoint_round_trip(tmp_path):
    """The reference's FSDP checkpoint path (src/optim/utils.py:276-290 save,
    :316-337 load): get_model/optimizer_state_dict and dcp.save, then, into a
    fresh model and optimizer (whose state torch first initialises with a
    zero-gradient, lr=0 step), dcp.load and set_model/optimizer_state_dict.
    Both runs then continue bit-identically."""
    import torch.distributed.checkpoint as dcp
    from torch.distributed.checkpoint.state_dict import (get_model_state_dict, get_optimizer_state_dict,
                                                         set_model_state_dict, set_optimizer_state_dict)
    import adana_amd

    print("case: torch.distributed.checkpoint round trip", flush=True)

    def make(seed):
        torch.manual_seed(seed)
        model = torch.nn.Sequential(torch.nn.Linear(64, 256), torch.nn.GELU(), torch.nn.Linear(256, 64),
                                    torch.nn.LayerNorm(64)).to(DEV)
        opt = adana_amd.DANA_STAR_MK4(model.parameters(), lr=1e-3, kappa=0.85, clipsnr=2.0, weight_decay=0.1,
                                      wd_decaying=True, wd_ts=10.0)
        return model, opt

    def train(model, opt, k0, k1):
        for k in range(k0, k1):
            gen = torch.Generator(device=DEV)
            gen.manual_seed(1000 + k)
            for p in model.parameters():
                p.grad = torch.randn(p.shape, device=DEV, generator=gen) * 1e-3
            opt.step()

    a_model, a_opt = make(0)
    train(a_model, a_opt, 0, 5)
    sd = {"model": get_model_state_dict(a_model), "optimizer": get_optimizer_state_dict(a_model, a_opt)}
    dcp.save(sd, checkpoint_id=str(tmp_path / "sharded"))

    b_model, b_opt = make(1)
    sd_b = {"model": get_model_state_dict(b_model), "optimizer": get_optimizer_state_dict(b_model, b_opt)}
    dcp.load(sd_b, checkpoint_id=str(tmp_path / "sharded"))
    set_model_state_dict(b_model, sd_b["model"])
    set_optimizer_state_dict(b_model, b_opt, sd_b["optimizer"])
    for ga, gb in zip(a_opt.param_groups, b_opt.param_groups):
        assert ga["weighted_step_count"] == gb["weighted_step_count"]

    train(a_model, a_opt, 5, 10)
    train(b_model, b_opt, 5, 10)
    torch.cuda.synchronize()
    for pa, pb in zip(a_model.parameters(), b_model.parameters()):
        assert torch.equal(pa.detach().view(torch.int32), pb.detach().view(torch.int32))
        sa, sb = a_opt.state[pa], b_opt.state[pb]
        assert sa["step"] == sb["step"] == 10
        for key in ("m", "v", "tau"):
            assert torch.equal(sa[key].view(torch.int32), sb[key].view(torch.int32)), key


@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
def test_state_missing_a_key_fails_before_any_change(star):
    """A loaded state without one of its moments (or its step counter) fails
    with the reference's KeyError (``m, v = state['m'], state['v']``,
    src/optim/adana.py:193-197) before any step counter, parameter or moment
    changes; restored, the same optimizer steps as an untouched copy does."""
    import copy

    import adana_amd

    torch.manual_seed(3)
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    ps = [torch.nn.Parameter(torch.randn(n, device=DEV) * 0.02) for n in (300, 17, 4099)]
    opt = cls(ps, lr=1e-3, kappa=0.85, weight_decay=0.1)
    for _ in range(3):
        for p in ps:
            p.grad = torch.randn_like(p) * 1e-3
        opt.step()
    twin = copy.deepcopy(opt)
    good = copy.deepcopy(opt.state_dict())
    keys = ("m", "v", "tau", "step") if star else ("m", "v", "step")
    for key in keys:
        sd = copy.deepcopy(good)
        del sd["state"][1][key]
        opt.load_state_dict(sd)
        before = [p.detach().clone() for p in ps]
        steps = [opt.state[p].get("step") for p in ps]
        m0 = opt.state[ps[0]]["m"].clone()
        with pytest.raises(KeyError, match=key):
            opt.step()
        torch.cuda.synchronize()
        assert all(torch.equal(a, p.detach()) for a, p in zip(before, ps)), key
        assert [opt.state[p].get("step") for p in ps] == steps, key
        assert torch.equal(opt.state[ps[0]]["m"], m0), key
    opt.load_state_dict(good)
    g = [torch.randn_like(p) * 1e-3 for p in ps]
    for o, params in ((opt, ps), (twin, [p for grp in twin.param_groups for p in grp["params"]])):
        for p, gg in zip(params, g):
            p.grad = gg.clone()
        o.step()
    torch.cuda.synchronize()
    for p, q in zip(ps, [p for grp in twin.param_groups for p in grp["params"]]):
        assert torch.equal(p.detach(), q.detach())
        for key in keys[:-1]:
            assert torch.equal(opt.state[p][key], twin.state[q][key])
