"""``log_optimizer_schedules`` with one device-to-host copy.

Reference: src/optim/utils.py:532-615, called every logging step by the
training loop (src/optim/base.py:318).  For the Dana family it walks
``param_groups`` and calls ``.item()`` on four 0-d diagnostics of every
parameter with state -- one host synchronisation per value -- and logs their
plain means (Python ``sum(values) / len(values)``).  It looks up a
``"g2_gradient_norm"`` state key that neither optimizer writes, so that
entry is never logged.

Here the same dictionary is produced from ``optimizer.diagnostics_host()``
(ADana / DANA_STAR_MK4 of this package: one asynchronous copy of each
diagnostics buffer, one synchronisation), with the means computed exactly as
the reference computes them (sequential Python float sums in parameter
order), so the logged values are identical.  Other optimizers and names take
the reference's value-by-value path.
"""
from __future__ import annotations

__all__ = ["log_optimizer_schedules"]

_DANA = ("adana", "dana-mk4", "dana-star", "dana-star-mk4")


def _to_float(v):
    """A value as float, or None when it cannot be read (src/optim/utils.py:541-548)."""
    if isinstance(v, (int, float)):
        return float(v)
    try:
        return v.item() if hasattr(v, "item") else float(v)
    except (RuntimeError, ValueError):
        return None


def _mean(values):
    return sum(values) / len(values)


def _dana_values(optimizer):
    """(alpha, kappa_factor, auto_factor, g2_gradient_norm, m_norm) lists in
    parameter order."""
    if hasattr(optimizer, "diagnostics_host"):
        _, vals = optimizer.diagnostics_host()
        # columns as Python floats (binary32 values, as .item() gives them)
        col = lambda c: vals[:, c].tolist()                          # noqa: E731
        return col(0), col(3), col(2), [], col(4)
    alpha, kappa, auto, g2, mnorm = [], [], [], [], []
    for group in optimizer.param_groups:
        for param in group["params"]:
            if param in optimizer.state and "current_alpha" in optimizer.state[param]:
                state = optimizer.state[param]
                for key, out in (("current_alpha", alpha), ("current_kappa_factor", kappa),
                                 ("auto_factor_mean", auto), ("g2_gradient_norm", g2),
                                 ("m_norm", mnorm)):
                    if key in state:
                        v = _to_float(state[key])
                        if v is not None:
                            out.append(v)
    return alpha, kappa, auto, g2, mnorm


def log_optimizer_schedules(optimizer, optimizer_name):
    """Same signature and result as the reference's (src/optim/utils.py:532)."""
    logs = {}
    if optimizer_name in ["ademamix"]:
        alpha_values, omb3_values = [], []
        for group in optimizer.param_groups:
            for param in group["params"]:
                if param in optimizer.state and "current_alpha" in optimizer.state[param]:
                    state = optimizer.state[param]
                    v = _to_float(state["current_alpha"])
                    if v is not None:
                        alpha_values.append(v)
                    v = _to_float(state["current_one_minus_beta3"])
                    if v is not None:
                        omb3_values.append(v)
        if alpha_values:
            logs["optimizer/alpha_schedule"] = _mean(alpha_values)
            if omb3_values:
                logs["optimizer/one_minus_beta3_schedule"] = _mean(omb3_values)
    elif optimizer_name in _DANA:
        alpha, kappa, auto, g2, mnorm = _dana_values(optimizer)
        if alpha:
            logs["optimizer/alpha_schedule"] = _mean(alpha)
            if kappa:
                logs["optimizer/kappa_factor_schedule"] = _mean(kappa)
            if auto:
                logs["optimizer/auto_factor"] = _mean(auto)
            if g2:
                logs["optimizer/g2_gradient_norm"] = _mean(g2)
            if mnorm:
                logs["optimizer/m_norm"] = _mean(mnorm)
    return logs
