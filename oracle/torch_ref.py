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


def update_foreach(star: bool, p, g, m, v, tau, sc, hp: dict, sqrt, epow, powf, compiled: bool = True):
    """One tensor's share of the reference's foreach path
    (``_foreach_compute_kernel_impl``, src/optim/adana.py:310-370 and
    src/optim/dana_star_mk4.py:395-536), one op per ``torch._foreach_*`` op in
    that order: p, m, v[, tau] updated in place; returns the diagnostics as
    ``update`` does, computed as the reference's ``_foreach_step_group`` does
    after the kernel (.mean() / .norm() of the returned alpha factor and mfac
    and of grad and m, adana.py:280-285).

    ``sc`` = (step_t, alpha_t, g2, g3, schedule_factor, wd): step_t in p's
    dtype and alpha_t = delta / (delta + step_t) as 0-d tensors
    (adana.py:258-262), the rest binary32 0-d tensors.

    ``compiled`` False: the kernel's eager ops, literally, on the tensors'
    own dtype (ATen's lerp, sqrt and pow; bfloat16 tensors round every op).
    ``compiled`` True: the constructor's torch.compile of the kernel; every
    value in binary32 (bfloat16 tensors read as binary32 and rounded where
    they are stored), ``sqrt``, ``epow`` (Dana-Star's element-wise power) and
    ``powf`` (ADana's 0-d power of Python floats) as for update_compiled.
    Either way the foreach path has no addcmul, and its lerps are ATen's
    kernel on the tensors' own dtype: Inductor keeps a foreach lerp with a
    list of weight tensors as that kernel, so under torch.compile too m and
    tau come out of it rounded to their dtype, and tau's lerp reads the tau
    update stored in tau's dtype (the reference's bfloat16 fixtures fix
    this)."""
    step_t, a_t, g2_t, g3_t, sf_t, wd_t = sc
    kappa, clip, eps = hp["kappa"], hp["clipsnr"], hp["epsilon"]
    f32 = torch.float32
    if compiled:
        P, G, M, V = p.to(f32), g.to(f32), m.to(f32), v.to(f32)
        st = step_t.to(f32)
        T = tau.to(f32) if star else None
    else:
        P, G, M, V, T, st = p.clone(), g, m.clone(), v.clone(), (tau.clone() if star else None), step_t
        sqrt, epow = torch.sqrt, torch.pow
    # _foreach_lerp_(ms, grads, alpha): ATen's kernel in both modes, on m's dtype
    M = torch.lerp(m, g, a_t).to(f32) if compiled else torch.lerp(M, G, a_t)
    oma = torch.neg(a_t) + 1.0                                # _foreach_neg, _foreach_add_(., 1.0)
    V = V * oma                                               # _foreach_mul_(vs, .)
    V = V + (G * G) * a_t                                     # mul, mul, _foreach_add_
    sv = sqrt(V)                                              # sqrt_vs
    if star:
        ag = torch.abs(G)
        den = ag + sv                                         # dana_star_mk4.py:429-433
        if compiled:
            den = den + eps
        else:
            torch._foreach_add_([den], eps)                   # in place: eps in den's dtype
        tu = ag / den                                         # :436
        if compiled:                                          # :439, ATen's lerp on tau's dtype
            T = torch.lerp(tau, tu.to(tau.dtype), a_t).to(f32)
        else:
            T = torch.lerp(T, tu, a_t)
        ct = torch.clamp(T, max=0.5)                          # :444
        pe = ct / (torch.neg(ct) + 1.0)                       # :447-450
        min_p = torch.reciprocal(st + 1.0)                    # :455-456
        treg = torch.maximum(pe, min_p)                       # :457
        et = T * st                                           # :461
        et = torch.maximum(et, torch.ones_like(et))           # :462-463
        nt = sqrt(treg) / (sv + eps)                          # :468-470
        mfac = nt * (torch.abs(M) / treg)                     # :474-476
        af = epow(et, 1.0 - kappa) * mfac                     # :480-481
        if clip is not None:
            af = torch.clamp(af, max=clip)
        g3i = (treg * torch.sign(M)) * af + M * nt            # :490-497
    else:
        nt = torch.reciprocal(sv + eps)                       # adana.py:327-329
        mfac = torch.abs(M) * nt                              # :332-333
        et = st + 1.0                                         # :336
        ep = torch.tensor(powf(float(et), 1.0 - kappa), dtype=f32) if compiled else torch.pow(et, 1.0 - kappa)
        af = ep * mfac                                        # :339-340
        if clip is not None:
            af = torch.clamp(af, max=clip)
        g3i = torch.sign(M) * af + M * nt                     # :345-348
    if compiled:
        g3i = g3i * hp["gamma_3_factor"]
    else:
        torch._foreach_mul_([g3i], hp["gamma_3_factor"])     # in place: the factor in g3i's dtype
    g3t = g3i * g3_t                                          # _foreach_mul(., g3)
    g2t = (G * nt) * g2_t                                     # grad_norm, g2_term
    P = P + torch.neg(g2t + g3t)                              # add, neg_, add_
    nws = torch.neg(wd_t) * sf_t
    if hp["wd_decaying"]:                                     # adana.py:357-362
        wdf = torch.reciprocal(st / hp["wd_ts"] + 1.0) * nws
    else:
        wdf = nws if compiled else nws.to(p.dtype)
    P = P + P * wdf                                           # :367-368
    p.copy_(P)
    m.copy_(M)
    v.copy_(V)
    if star:
        tau.copy_(T)
    dt = p.dtype
    afd, mfd = af.to(dt), mfac.to(dt)
    return afd.mean(), g.norm(), mfd.mean(), m.norm()


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
             slip: Optional[str] = None, compiled=None, update_fn=None, foreach=None) -> None:
        """One step of the reference's loop.  ``compiled``: None for the eager
        ops (``update``), or (sqrt, epow, powf) for ``update_compiled``.
        ``update_fn(p)``, when given, returns the callable that replaces
        ``update`` for tensor p (bench.py passes ``update`` wrapped in
        torch.compile, one wrapper per shape, as src/optim/adana.py:72-79
        and src/optim/dana_star_mk4.py:88-96 do).  ``foreach``: (sqrt, epow,
        powf, compiled) runs ``update_foreach`` with the foreach path's
        scalars (src/optim/adana.py:245-262) instead."""
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
                if foreach is not None:
                    step_t = torch.tensor(t, dtype=p.dtype)                         # :258
                    delta_t = torch.tensor(group.delta, **f32)                      # :173
                    sc = (step_t, delta_t / (delta_t + step_t)) + sc[2:]            # :259
                    ca, gn, afm, mn = update_foreach(self.star, p, g, st["m"], st["v"], st.get("tau"), sc, hp,
                                                     *foreach)
                elif update_fn is not None:
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
