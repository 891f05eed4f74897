"""log_optimizer_schedules (src/optim/utils.py:532-615) on the reference's own
diagnostics: the golden runs' per-tensor values (tests/golden/<case>.eager.npz,
written by the reference's step()) placed in an optimizer's state as 0-d
tensors, read through the value-by-value path every non-package optimizer
takes.  Checks the logged keys (the reference's 'g2_gradient_norm' lookup
never matches, so that key is never logged), plain means in parameter order,
and NaN propagation from all-zero-gradient tensors."""
import math

import numpy as np
import pytest
import torch

from helpers import golden_cases, load_golden_case, load_golden_inputs


class _StateOnly:
    def __init__(self, params, diag):
        self.param_groups = [{"params": params[:3]}, {"params": params[3:]}]
        keys = ("current_alpha", "gradient_norm", "auto_factor_mean", "current_kappa_factor", "m_norm")
        self.state = {}
        for p, row in zip(params, diag):
            if not np.isnan(row[0]):
                self.state[p] = {k: torch.tensor(float(v), dtype=torch.float32) for k, v in zip(keys, row)}


@pytest.mark.parametrize("case", golden_cases("eager"))
@pytest.mark.parametrize("k", [1, 8, 20])
def test_schedule_logs_from_reference_diagnostics(case, k):
    import adana_amd

    meta, p0, _, _ = load_golden_inputs()
    gold = load_golden_case(case, "eager")
    params = [torch.nn.Parameter(torch.zeros(1)) for _ in p0]
    diag = gold["diag"][k - 1]
    opt = _StateOnly(params, diag)
    name = "dana-star-mk4" if "star" in case else "dana-mk4"
    logs = adana_amd.log_optimizer_schedules(opt, name)
    rows = [r for r in diag if not np.isnan(r[0])]
    assert set(logs) == {"optimizer/alpha_schedule", "optimizer/kappa_factor_schedule",
                         "optimizer/auto_factor", "optimizer/m_norm"}
    for key, col in (("optimizer/alpha_schedule", 0), ("optimizer/kappa_factor_schedule", 3),
                     ("optimizer/auto_factor", 2), ("optimizer/m_norm", 4)):
        vals = [float(np.float32(r[col])) for r in rows]
        want = sum(vals) / len(vals)
        got = logs[key]
        assert (math.isnan(got) and math.isnan(want)) or got == want, (key, got, want)
    # tensor 3 has all-zero gradients: its kappa factor is 0/0, the mean is NaN
    assert math.isnan(logs["optimizer/kappa_factor_schedule"])


def test_schedule_logs_other_names_and_empty():
    import adana_amd

    opt = _StateOnly([torch.nn.Parameter(torch.zeros(1)) for _ in range(6)], np.full((6, 5), np.nan))
    assert adana_amd.log_optimizer_schedules(opt, "dana-star") == {}
    assert adana_amd.log_optimizer_schedules(opt, "adamw") == {}
