"""Torch-eager restatement of the reference step on CPU tensors.

TEST INFRASTRUCTURE ONLY: imported by tests/ (which pin it against the
reference's own golden bits) and by bench.py's cpu_baseline leg (which times
it on the GPU box's host cores as the reference's CPU step), never by the
product package ``adana_amd``.

``update`` is one tensor's update as torch tensor ops, one op for each tensor
op of ``ADana._update_param_compiled`` (src/optim/adana.py:101-151) and
``DANA_STAR_MK4._update_param_compiled`` (src/optim/dana_star_mk4.py:137-203)
in that order.  ``TorchRefOptimizer.step`` is the reference's host loop
around it (src/optim/adana.py:162-225; src/optim/dana_star_mk4.py:215-294):
group scalars, grad-None skip, lazy zero state, per-tensor step counter, the
six 0-d float32 tensors of adana.py:203-208, and the five diagnostics.

Run as the reference runs it with ``torch.compile`` disabled (its eager ops),
it reproduces the reference's golden vectors bit for bit.  Two hooks exist
for the tests that pin the CPU oracle: ``sqrt`` and ``epow`` replace torch's
square root and Dana-Star's element-wise power (to show that they alone
separate the oracle from the reference), and ``slip`` plants one plausible
op-order mistake (to show that the golden vectors catch it).

``update_compiled`` restates the same update the way the reference's
default torch.compile path computes it (Inductor's generated CPU code for
these ops): lerp_ as ``c * (end - self) + base`` and the second moment as
``v * (1 - alpha) + (g * g) * alpha`` (no fused multiply-adds), every
intermediate in binary32, bfloat16 tensors read as binary32 and rounded only
when m, v, tau and p are stored, ADana's 0-d pow evaluated by the C
library's powf with the exponent rounded to binary32.  It runs as eager
torch ops, so the caller passes the square root and element-wise power that
Inductor's code uses (the tests pin those against the reference's compiled
fixtures).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch

DIAG_KEYS = ("current_alpha", "gradient_norm", "auto_factor_mean", "current_kappa_factor", "m_norm")


def update(star: bool, p, g, m, v, tau, sc, hp: dict, sqrt=torch.sqrt, epow=None, slip: Optional[str] = None):
    """One tensor's update in place (p, m, v[, tau]); returns the diagnostics
    as 0-d tensors in DIAG_KEYS order except current_kappa_factor, which the
    caller divides (adana.py:224).  ``sc`` = (step, alpha, g2, g3,
    schedule_factor, wd) as 0-d float32 tensors; ``hp`` holds epsilon, kappa,
    clipsnr, wd_decaying, wd_ts and gamma_3_factor."""
    step_t, a_t, g2_t, g3_t, sf_t, wd_t = sc
    kappa, clip = hp["kappa"], hp["clipsnr"]
    if slip == "wd_first":
        p.mul_(1 + (-wd_t * sf_t))
    if slip == "lerp_one_branch":
        m.add_(a_t * (g - m))
    else:
        m.lerp_(g, a_t)                                       # adana.py:101
    if slip == "addcmul_unfused":
        v.mul_(1 - a_t).add_(a_t * (g * g))
    else:
        v.mul_(1 - a_t).addcmul_(g, g, value=a_t)             # :104
    se = sqrt(v).add_(hp["epsilon"])                          # :107
    if star:
        ag = torch.abs(g)                                     # dana_star_mk4.py:147
        tau.lerp_(ag / (ag + se), a_t)                        # :148-149
        ct = torch.clamp(tau, max=0.5)                        # :152
        pe = ct / (1.0 - ct)                                  # :153
        min_p = 1.0 / (1.0 + step_t)                          # :154
        treg = min_p + torch.relu(pe - min_p)                 # :156
        tt = step_t + 1 if slip == "time_plus_one" else step_t
        et = torch.clamp(tau * tt, min=1.0)                   # :159
        nt = sqrt(treg) / se                                  # :163-164
        mnt = torch.abs(m) * nt                               # :165
        mfac = mnt / treg                                     # :167
        pw = et ** (1 - kappa) if epow is None else epow(et, 1 - kappa)
        af = pw * mfac                                        # :170 / :174
        if clip is not None:
            af = torch.clamp(af, max=clip)
        g3t = (-g3_t) * hp["gamma_3_factor"] * (torch.sign(m) * (treg * af + mnt))   # :177
    else:
        nt = 1.0 / se                                         # adana.py:110
        mfac = torch.abs(m) * nt                              # :111, :115
        af = ((1.0 + step_t) ** (1 - kappa)) * mfac           # :114, :119 / :123
        if clip is not None:
            af = torch.clamp(af, max=clip)
        g3t = (-g3_t) * hp["gamma_3_factor"] * (torch.sign(m) * af + m * nt)         # :126
    g2t = (-g2_t) * (g * nt) if slip == "g2_assoc" else (-g2_t) * g * nt   # :129 / :180
    p.add_(g2t + g3t)                                         # :132-135
    if slip != "wd_first":
        if hp["wd_decaying"]:                                 # :139-142
            wdf = -wd_t / (1 + step_t / hp["wd_ts"]) * sf_t
        else:
            wdf = -wd_t * sf_t
        p.mul_(1 + wdf)                                       # :143
    return af.mean(), g.norm(), mfac.mean(), m.norm()         # :146-151


def update_compiled(star: bool, p, g, m, v, tau, sc, hp: dict, sqrt, epow, powf):
    """``update``'s ops as the compiled path computes them (module docstring):
    p, m, v[, tau] are updated in place from binary32 copies; returns the
    diagnostics (binary32 sums, rounded to p's dtype) as ``update`` does.
    ``sqrt(x)``, ``epow(x, e)`` (Dana-Star's element-wise power) and
    ``powf(x, e)`` (ADana's 0-d power, Python floats) are the functions
    Inductor's code calls."""
    step_t, a_t, g2_t, g3_t, sf_t, wd_t = sc
    kappa, clip = hp["kappa"], hp["clipsnr"]
    f32 = torch.float32
    P, G, M, V = p.to(f32), g.to(f32), m.to(f32), v.to(f32)
    small = bool(torch.abs(a_t) < 0.5)
    coef = a_t if small else a_t - 1.0                        # torch._refs.lerp

    def lerp(x, y):
        return coef * (y - x) + (x if small else y)

    M1 = lerp(M, G)                                           # adana.py:101
    V1 = V * (1 - a_t) + (G * G) * a_t                        # :104
    se = sqrt(V1) + hp["epsilon"]                             # :107
    if star:
        T = tau.to(f32)
        ag = torch.abs(G)                                     # dana_star_mk4.py:147
        T1 = lerp(T, ag / (ag + se))                          # :148-149
        ct = torch.clamp(T1, max=0.5)                         # :152
        pe = ct / (1.0 - ct)                                  # :153
        min_p = 1.0 / (1.0 + step_t)                          # :154
        treg = min_p + torch.relu(pe - min_p)                 # :156
        et = torch.clamp(T1 * step_t, min=1.0)                # :159
        nt = sqrt(treg) / se                                  # :163-164
        mnt = torch.abs(M1) * nt                              # :165
        mfac = mnt / treg                                     # :167
        af = epow(et, 1 - kappa) * mfac                       # :170 / :174
        if clip is not None:
            af = torch.clamp(af, max=clip)
        g3t = (-g3_t) * hp["gamma_3_factor"] * (torch.sign(M1) * (treg * af + mnt))   # :177
    else:
        nt = 1.0 / se                                         # adana.py:110
        mfac = torch.abs(M1) * nt                             # :111, :115
        pw = torch.tensor(powf(float(1.0 + step_t), 1 - kappa), dtype=f32)             # :114, :119
        af = pw * mfac
        if clip is not None:
            af = torch.clamp(af, max=clip)
        g3t = (-g3_t) * hp["gamma_3_factor"] * (torch.sign(M1) * af + M1 * nt)         # :126
    g2t = (-g2_t) * G * nt                                    # :129 / :180
    if hp["wd_decaying"]:                                     # :139-142
        wdf = -wd_t / (1 + step_t / hp["wd_ts"]) * sf_t
    else:
        wdf = -wd_t * sf_t
    P1 = (P + (g2t + g3t)) * (1 + wdf)                        # :132-143
    p.copy_(P1)
    m.copy_(M1)
    v.copy_(V1)
    if star:
        tau.copy_(T1)
    dt = p.dtype
    return (af.mean().to(dt), G.norm().to(dt), mfac.mean().to(dt), M1.norm().to(dt))   # :146-151


@dataclass
class TorchRefGroup:
    params: List[torch.Tensor]
    lr: float
    delta: float = 8.0
    epsilon: float = 1e-8
    weight_decay: float = 0.0
    weighted_step_count: float = 0.0


@dataclass
class TorchRefOptimizer:
    """The reference's step loop over float32 CPU tensors (``star`` selects
    Dana-Star(-MK4); ``clipsnr=None`` disables SNR clipping; ``peak_lr`` is the
    constructor's ``lr``)."""

    groups: List[TorchRefGroup]
    star: bool
    peak_lr: float
    kappa: float = 1.0
    clipsnr: Optional[float] = None
    wd_decaying: bool = False
    wd_ts: float = 1.0
    gamma_3_factor: float = 1.0
    state: Dict[int, dict] = field(default_factory=dict)

    @torch.no_grad()
    def step(self, grads: Sequence[Sequence[Optional[torch.Tensor]]], sqrt=torch.sqrt, epow=None,
             slip: Optional[str] = None, compiled=None, update_fn=None) -> None:
        """One step of the reference's loop.  ``compiled``: None for the eager
        ops (``update``), or (sqrt, epow, powf) for ``update_compiled``.
        ``update_fn(p)``, when given, returns the callable that replaces
        ``update`` for tensor p (bench.py passes ``update`` wrapped in
        torch.compile, one wrapper per shape, as src/optim/adana.py:72-79
        and src/optim/dana_star_mk4.py:88-96 do)."""
        f32 = dict(dtype=torch.float32)
        for gi, group in enumerate(self.groups):
            lr = group.lr
            sf = lr / self.peak_lr                            # adana.py:165
            group.weighted_step_count += sf                   # :167
            hp = dict(epsilon=group.epsilon, kappa=self.kappa, clipsnr=self.clipsnr,
                      wd_decaying=self.wd_decaying, wd_ts=self.wd_ts, gamma_3_factor=self.gamma_3_factor)
            for pi, p in enumerate(group.params):
                g = grads[gi][pi]
                if g is None:                                 # :186
                    continue
                st = self.state.get(id(p))
                if st is None:                                # :191-195
                    st = self.state[id(p)] = {"step": 0, "m": torch.zeros_like(p), "v": torch.zeros_like(p)}
                    if self.star:
                        st["tau"] = torch.zeros_like(p)
                st["step"] += 1                               # :197
                t = st["step"]
                sc = (torch.tensor(t, **f32), torch.tensor(group.delta / (group.delta + t), **f32),
                      torch.tensor(lr, **f32), torch.tensor(lr, **f32), torch.tensor(sf, **f32),
                      torch.tensor(group.weight_decay, **f32))                       # :199-208
                if update_fn is not None:
                    ca, gn, afm, mn = update_fn(p)(self.star, p, g, st["m"], st["v"], st.get("tau"), sc, hp)
                elif compiled is None:
                    ca, gn, afm, mn = update(self.star, p, g, st["m"], st["v"], st.get("tau"), sc, hp,
                                             sqrt=sqrt, epow=epow, slip=slip)
                else:
                    ca, gn, afm, mn = update_compiled(self.star, p, g, st["m"], st["v"], st.get("tau"), sc, hp,
                                                      *compiled)
                st["current_alpha"] = ca                      # :221-225
                st["gradient_norm"] = gn
                st["auto_factor_mean"] = afm
                st["current_kappa_factor"] = ca / afm
                st["m_norm"] = mn
