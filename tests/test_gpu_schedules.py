"""The packed diagnostics read-out (ADana / DANA_STAR_MK4
``diagnostics_host`` under ``log_optimizer_schedules``, src/optim/utils.py:
532-615) against the reference's value-by-value ``.item()`` path on the same
optimizer state: identical logged floats.  Also after load_state_dict (state
tensors not yet in a device buffer) and across plan rebuilds."""
import math
import time

import numpy as np
import pytest
import torch

from helpers import golden_cases, load_golden_case, load_golden_inputs, load_reference_state_dict

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"


class _ItemPath:
    """Hides diagnostics_host so log_optimizer_schedules reads value by value."""

    def __init__(self, opt):
        self.param_groups = opt.param_groups
        self.state = opt.state


def _same(a, b):
    assert set(a) == set(b)
    for k in a:
        assert (math.isnan(a[k]) and math.isnan(b[k])) or a[k] == b[k], (k, a[k], b[k])


def _build(case):
    import adana_amd

    meta, p0, grads, has_grad = load_golden_inputs()
    c = meta["cases"][case]
    kw = dict(c["kwargs"])
    cls = adana_amd.DANA_STAR_MK4 if c["class"] == "DANA_STAR_MK4" else adana_amd.ADana
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(DEV)) for x in p0]
    groups = [{"params": [p for i, p in enumerate(params) if meta["group_of"][i] == gi],
               "weight_decay": kw["weight_decay"] * meta["group_wd_scale"][gi]} for gi in range(2)]
    return cls(groups, **kw), params, meta, kw, grads, has_grad


@pytest.mark.parametrize("case", golden_cases("eager"))
def test_packed_readout_equals_item_path(case):
    import adana_amd

    print("case: packed diagnostics", case, flush=True)
    opt, params, meta, kw, grads, has_grad = _build(case)
    gold = load_golden_case(case, "eager")
    name = "dana-star-mk4" if "star" in case else "dana-mk4"
    for k in range(1, meta["n_steps"] + 1):
        for g in opt.param_groups:
            g["lr"] = kw["lr"] * meta["lr_multiplier"][k - 1]
        for i, p in enumerate(params):        # grad None on odd steps for tensor 5: plans alternate
            p.grad = torch.from_numpy(grads[k - 1][i].copy()).to(DEV) if has_grad[k - 1, i] else None
        opt.step()
        packed = adana_amd.log_optimizer_schedules(opt, name)
        _same(packed, adana_amd.log_optimizer_schedules(_ItemPath(opt), name))
        rows = gold["diag"][k - 1]
        want = [r for r in rows if not np.isnan(r[0])]
        np.testing.assert_allclose(packed["optimizer/alpha_schedule"],
                                   sum(float(r[0]) for r in want) / len(want), rtol=2e-5)


def test_packed_readout_after_load_state_dict():
    import adana_amd

    print("case: packed diagnostics after load_state_dict", flush=True)
    opt, params, *_ = _build("dana_star_mk4")
    ref, _ = load_reference_state_dict("dana_star_mk4", device=DEV)
    opt.load_state_dict(ref)
    _same(adana_amd.log_optimizer_schedules(opt, "dana-star-mk4"),
          adana_amd.log_optimizer_schedules(_ItemPath(opt), "dana-star-mk4"))


def test_packed_readout_many_tensors_timing():
    """C5-shaped list: 2,000 tensors.  Same result; prints both timings."""
    import adana_amd

    print("case: packed diagnostics timing", flush=True)
    rng = np.random.default_rng(0)
    sizes = np.floor(np.exp(rng.uniform(np.log(64), np.log(4096), 2000))).astype(int)
    params = [torch.nn.Parameter(torch.randn(int(n), device=DEV) * 0.02) for n in sizes]
    opt = adana_amd.DANA_STAR_MK4(params, lr=1e-3, kappa=0.85, clipsnr=2.0)
    for p in params:
        p.grad = torch.randn_like(p) * 1e-3
    opt.step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    a = adana_amd.log_optimizer_schedules(opt, "dana-star-mk4")
    t1 = time.perf_counter()
    b = adana_amd.log_optimizer_schedules(_ItemPath(opt), "dana-star-mk4")
    t2 = time.perf_counter()
    _same(a, b)
    print(f"2000 tensors: packed {1e3 * (t1 - t0):.2f} ms, value by value {1e3 * (t2 - t1):.2f} ms", flush=True)
