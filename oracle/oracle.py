"""CPU oracle for the ADana-family optimizer step.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU
baseline), never by the product package ``adana_amd``.

This module restates, independently of the product:

* the host-side scalar schedule of ``ADana.step`` (src/optim/adana.py:162-208)
  and ``DANA_STAR_MK4.step`` (src/optim/dana_star_mk4.py:215-272), including
  the 0-d tensor arithmetic the compiled update performs on those scalars
  (``1 - alpha``, ``1.0 + step``, ``(-g3) * gamma_3_factor``, the weight-decay
  factor, ``1.0 / (1.0 + step)``), each as one binary32 operation in numpy;
* the per-tensor step loop (grad-None skip, lazy state init, per-tensor step
  counter, diagnostics), src/optim/adana.py:184-225 and
  src/optim/dana_star_mk4.py:243-294;
* the element math itself lives in ``adana_oracle.c`` (same directory).
"""
from __future__ import annotations

import ctypes
import math
import os
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")

f32 = np.float32


class OracleScalars(ctypes.Structure):
    """Mirror of ``adana_oracle_scalars`` in adana_oracle.c."""

    _fields_ = [
        ("a", ctypes.c_float),
        ("oma", ctypes.c_float),
        ("s", ctypes.c_float),
        ("eps", ctypes.c_float),
        ("pw", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("clip", ctypes.c_float),
        ("has_clip", ctypes.c_int32),
        ("c3", ctypes.c_float),
        ("cg2", ctypes.c_float),
        ("opw", ctypes.c_float),
        ("star_exp", ctypes.c_float),
        ("pow_mode", ctypes.c_int32),
        ("compiled", ctypes.c_int32),
        ("pow_int", ctypes.c_int32),
        ("foreach", ctypes.c_int32),
        ("g3f", ctypes.c_float),
        ("lr", ctypes.c_float),
        ("wdf", ctypes.c_float),
    ]


class OracleManauScalars(ctypes.Structure):
    """Mirror of ``adana_oracle_manau_scalars`` in adana_oracle.c."""

    _fields_ = [
        ("a", ctypes.c_float), ("oma", ctypes.c_float), ("s", ctypes.c_float), ("eps", ctypes.c_float),
        ("min_p", ctypes.c_float), ("clip", ctypes.c_float), ("lr", ctypes.c_float), ("wdf", ctypes.c_float),
        ("e", ctypes.c_float * 3), ("mode", ctypes.c_int32 * 3), ("has_wd", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


_lib = None
ORACLE_ABI = 3


def lib():
    """Load (building first if needed) the oracle's shared library."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        i32 = ctypes.c_int32
        SP = ctypes.POINTER(OracleScalars)
        L.adana_oracle_adana_step.argtypes = [i64, P, P, P, P, SP, P]
        L.adana_oracle_star_step.argtypes = [i64, P, P, P, P, P, SP, P]
        L.adana_oracle_manau_step.argtypes = [i64, P, P, P, P, P, ctypes.POINTER(OracleManauScalars), P]
        L.adana_oracle_master_step.argtypes = [i64, i32, P, P, P, P, P, P, SP, P]
        L.adana_oracle_step_g16.argtypes = [i64, i32, P, P, P, P, P, SP, P]
        L.adana_oracle_step_bf16.argtypes = [i64, i32, P, P, P, P, P, SP, P]
        L.adana_oracle_f32_to_bf16.argtypes = [i64, P, P]
        L.adana_oracle_set_threads.argtypes = [ctypes.c_int]
        L.adana_oracle_set_threads.restype = None
        L.adana_oracle_get_threads.argtypes = []
        L.adana_oracle_get_threads.restype = ctypes.c_int
        for fn in (L.adana_oracle_adana_step, L.adana_oracle_star_step,
                   L.adana_oracle_master_step, L.adana_oracle_step_g16,
                   L.adana_oracle_step_bf16, L.adana_oracle_f32_to_bf16):
            fn.restype = None
        if L.adana_oracle_abi_version() != ORACLE_ABI:
            raise RuntimeError(f"{LIB_PATH}: oracle ABI {L.adana_oracle_abi_version()}, expected {ORACLE_ABI} "
                               f"(rebuild with oracle.build(force=True))")
        _lib = L
    return _lib


def build(force: bool = False) -> None:
    """Compile adana_oracle.c with the oracle's Makefile."""
    import subprocess

    subprocess.run(["make", "-s"] + (["-B"] if force else []) + ["-C", _HERE], check=True)


def set_threads(n: int) -> int:
    """Set the OpenMP thread count of the element loops; return the count in use."""
    L = lib()
    L.adana_oracle_set_threads(int(n))
    return int(L.adana_oracle_get_threads())


# --------------------------------------------------------------------------
# Host scalars
# --------------------------------------------------------------------------

def _pow0d(x: np.float32, e: float) -> np.float32:
    """``x ** e`` for a 0-d binary32 tensor and a Python-float exponent.

    ATen's pow(Tensor, Scalar) special-cases a few exponents (0 fills ones;
    1 copies; 0.5 sqrt; -0.5 rsqrt; -1 reciprocal; 2, 3, -2 by multiplication) and
    otherwise evaluates std::pow(float, double) in binary64 for a 0-d tensor
    (probed bitwise against torch 2.10; reference call site
    src/optim/adana.py:119,123).
    """
    x = f32(x)
    if e == 0.0:
        return f32(1.0)
    if e == 1.0:
        return x
    if e == 0.5:
        return f32(np.sqrt(x))
    if e == -0.5:
        return f32(1.0) / f32(np.sqrt(x))
    if e == -1.0:
        return f32(1.0) / x
    if e == 2.0:
        return x * x
    if e == 3.0:
        return (x * x) * x
    if e == -2.0:
        return f32(1.0) / (x * x)
    return f32(math.pow(float(x), e))


POW_GENERAL, POW_ONE, POW_SQRT, POW_RSQRT, POW_RECIP, POW_SQUARE, POW_CUBE, POW_INVSQ, POW_IDENTITY, POW_INT = range(10)


def pow_mode(e: float) -> int:
    """Which ATen pow specialisation an exponent selects (see _pow0d): torch's
    pow(Tensor, Scalar) returns ones for exponent 0 and a copy for exponent 1
    before its kernel's sqrt / rsqrt / reciprocal / square / cube cases."""
    return {0.0: POW_ONE, 1.0: POW_IDENTITY, 0.5: POW_SQRT, -0.5: POW_RSQRT, -1.0: POW_RECIP,
            2.0: POW_SQUARE, 3.0: POW_CUBE, -2.0: POW_INVSQ}.get(e, POW_GENERAL)


def pow_mode_compiled(e: float):
    """(mode, integer exponent) of x ** e under torch.compile: Inductor's pow
    lowering (torch/_inductor/lowering.py) turns an exponent equal to an
    integer k into pow(x, k) -- ones for 0, a copy for 1, products for any
    other |k| < 32 -- and 0.5 into sqrt; every other exponent, -0.5 included,
    stays a pow with the exponent rounded to binary32."""
    if e == 0.0:
        return POW_ONE, 0
    if e == 1.0:
        return POW_IDENTITY, 0
    if e == 0.5:
        return POW_SQRT, 0
    if e == math.floor(e) and abs(e) < 32:
        return POW_INT, int(e)
    return POW_GENERAL, 0


def pow_int(x: np.float32, k: int) -> np.float32:
    """x ** k for an integer k as Inductor's pow_recursive expands it: for
    k < 0 the powers of 1 / x; x ** 2j = (x ** j)(x ** j) and
    x ** (2j + 1) = (x ** j)(x ** j) x, every product one binary32 rounding."""
    x = f32(x)
    if k < 0:
        x, k = f32(1.0) / x, -k
    if k == 0:
        return f32(1.0)
    if k == 1:
        return x
    r = pow_int(x, k // 2)
    r = r * r
    return r * x if k % 2 else r


_libm = None


def _powf(x: np.float32, e: np.float32) -> np.float32:
    """The C library's binary32 pow (what Inductor's CPU code calls as
    std::pow(float, float) for a 0-d tensor)."""
    global _libm
    if _libm is None:
        _libm = ctypes.CDLL("libm.so.6")
        _libm.powf.restype = ctypes.c_float
        _libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return f32(_libm.powf(float(x), float(e)))


def _pow0d_compiled(x: np.float32, e: float) -> np.float32:
    """``x ** e`` for a 0-d binary32 tensor under torch.compile
    (src/optim/adana.py:119,123): Inductor's lowering, a general exponent
    evaluated by the C library's powf with the exponent rounded to binary32."""
    mode, k = pow_mode_compiled(e)
    x = f32(x)
    if mode == POW_ONE:
        return f32(1.0)
    if mode == POW_IDENTITY:
        return x
    if mode == POW_SQRT:
        return f32(np.sqrt(x))
    if mode == POW_INT:
        return pow_int(x, k)
    return _powf(x, f32(e))


def step_scalars(*, lr: float, peak_lr: float, delta: float, kappa: float, epsilon: float,
                 weight_decay: float, clipsnr: Optional[float], wd_decaying: bool,
                 wd_ts: float, gamma_3_factor: float, t: int, compiled: bool = True) -> OracleScalars:
    """Scalars of one tensor's update at per-tensor step ``t`` (already incremented).

    Follows src/optim/adana.py:163-208 (host) and :104-143 (0-d tensor ops
    inside the compiled update); Dana-Star uses the same host code
    (src/optim/dana_star_mk4.py:217-272) plus min_p (:154).  The scalars are
    the same binary32 values under torch.compile (Inductor computes these
    0-d ops in binary32 in the same order); ``compiled`` selects Inductor's
    forms of the element ops (adana_oracle.c).
    """
    sf = f32(lr / peak_lr)                       # :165 double divide, :207 fp32
    g2 = f32(lr)                                 # :205
    g3 = f32(lr)                                 # :206
    wd = f32(weight_decay)                       # :208
    a = f32(delta / (delta + t))                 # :200 double, :204 fp32
    s = f32(t)                                   # :203
    one_p_s = f32(1.0) + s                       # :114 ``1.0 + step``
    sc = OracleScalars()
    sc.a = a
    sc.oma = f32(1.0) - a                        # :104 ``1 - alpha``
    sc.s = s
    sc.eps = f32(epsilon)                        # :107 add_(epsilon)
    sc.pw = (_pow0d_compiled if compiled else _pow0d)(one_p_s, 1.0 - kappa)   # :119 / :123
    sc.min_p = f32(1.0) / one_p_s                # dana_star_mk4.py:154
    sc.has_clip = 0 if clipsnr is None else 1
    sc.clip = f32(clipsnr) if clipsnr is not None else f32(np.inf)
    sc.c3 = (-g3) * f32(gamma_3_factor)          # :126 ``(-g3) * gamma_3_factor``
    sc.cg2 = -g2                                 # :129 ``(-g2)``
    if wd_decaying:                              # :139-142
        wdf = ((-wd) / (f32(1.0) + s / f32(wd_ts))) * sf
    else:
        wdf = (-wd) * sf
    sc.opw = f32(1.0) + wdf                      # :143 ``1 + wd_factor``
    sc.star_exp = f32(1.0 - kappa)               # dana_star_mk4.py:170 (vectorised pow)
    if compiled:
        sc.pow_mode, sc.pow_int = pow_mode_compiled(1.0 - kappa)
    else:
        sc.pow_mode = pow_mode(1.0 - kappa)
    sc.compiled = 1 if compiled else 0
    return sc


def foreach_scalars(*, lr: float, peak_lr: float, delta: float, kappa: float, epsilon: float,
                    weight_decay: float, clipsnr: Optional[float], wd_decaying: bool,
                    wd_ts: float, gamma_3_factor: float, t: int, compiled: bool = True,
                    step_bf16: bool = False) -> OracleScalars:
    """Scalars of one tensor's update at step ``t`` on the reference's
    use_foreach=True path: the host code of src/optim/adana.py:171-176,
    :245-262 (dana_star_mk4.py:229-236, :327-340) and the 0-d tensor ops of
    ``_foreach_compute_kernel_impl`` (adana.py:316-365; dana_star_mk4.py:
    455-456, :520-528), all binary32.  step_t has the parameters' dtype
    (``step_bf16``: bfloat16, so a step above 256 is rounded); alpha is the
    binary32 quotient of the binary32 delta and that step."""
    st = f32(t)
    if step_bf16:
        st = bf16_to_f32(f32_to_bf16(np.array([st], np.float32)))[0]
    sf = f32(lr / peak_lr)                       # adana.py:165, :174
    d = f32(delta)                               # :175
    a = d / (d + st)                             # :259
    one_p_s = st + f32(1.0)                      # :336 / dana_star_mk4.py:455
    sc = OracleScalars()
    sc.a = a
    sc.oma = f32(1.0) - a                        # :317-318 neg, add_(1.0)
    sc.s = st
    sc.eps = f32(epsilon)
    sc.pw = (_pow0d_compiled if compiled else _pow0d)(one_p_s, 1.0 - kappa)   # :339
    sc.min_p = f32(1.0) / one_p_s                # dana_star_mk4.py:456
    sc.has_clip = 0 if clipsnr is None else 1
    sc.clip = f32(clipsnr) if clipsnr is not None else f32(np.inf)
    sc.star_exp = f32(1.0 - kappa)               # dana_star_mk4.py:480
    if compiled:
        sc.pow_mode, sc.pow_int = pow_mode_compiled(1.0 - kappa)
    else:
        sc.pow_mode = pow_mode(1.0 - kappa)
    sc.compiled = 1 if compiled else 0
    sc.foreach = 1
    sc.g3f = f32(gamma_3_factor)                 # :350
    sc.lr = f32(lr)                              # :172-173 g2, g3
    nws = (-f32(weight_decay)) * sf              # :360 / :363
    if step_bf16 and not compiled:
        # eager 0-d ops on the bfloat16 step tensor, each rounded to bfloat16
        def rb(x):
            return bf16_to_f32(f32_to_bf16(np.array([x], np.float32)))[0]
        ops = rb(st + f32(1.0))                  # :336 / dana_star_mk4.py:455
        sc.min_p = rb(f32(1.0) / ops)            # dana_star_mk4.py:456
        e16 = float(rb(f32(1.0 - kappa)))        # pow's exponent in bfloat16
        sc.pw = rb(_pow0d(ops, e16))             # :339
        if wd_decaying:                          # bfloat16 0-d quotient, float32 0-d product
            sc.wdf = f32(rb(f32(1.0) / rb(rb(st / f32(wd_ts)) + f32(1.0)))) * nws
        else:
            sc.wdf = rb(nws)                     # :364 .to(p.dtype)
    elif wd_decaying:                            # :357-361
        sc.wdf = (f32(1.0) / (st / f32(wd_ts) + f32(1.0))) * nws
    else:
        sc.wdf = nws
    return sc


# --------------------------------------------------------------------------
# Element kernels
# --------------------------------------------------------------------------

def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def element_step(star: bool, p: np.ndarray, g: np.ndarray, m: np.ndarray, v: np.ndarray,
                 tau: Optional[np.ndarray], sc: OracleScalars) -> np.ndarray:
    """Apply one element-wise update in place; return binary64 sums
    [sum(alpha_factor), sum(g^2), sum(mfac), sum(m^2)]."""
    L = lib()
    diag = np.zeros(4, dtype=np.float64)
    n = p.size
    if g.dtype == np.float32 and p.dtype == np.float32:
        if star:
            L.adana_oracle_star_step(n, _ptr(p), _ptr(g), _ptr(m), _ptr(v), _ptr(tau),
                                     ctypes.byref(sc), _ptr(diag))
        else:
            L.adana_oracle_adana_step(n, _ptr(p), _ptr(g), _ptr(m), _ptr(v),
                                      ctypes.byref(sc), _ptr(diag))
    elif g.dtype == np.uint16 and p.dtype == np.float32:
        L.adana_oracle_step_g16(n, int(star), _ptr(p), _ptr(g), _ptr(m), _ptr(v),
                                _ptr(tau) if star else None, ctypes.byref(sc), _ptr(diag))
    elif g.dtype == np.uint16 and p.dtype == np.uint16 and m.dtype == np.uint16:
        # the reference's own bfloat16 path: p, g, m, v, tau all bfloat16 bits
        L.adana_oracle_step_bf16(n, int(star), _ptr(p), _ptr(g), _ptr(m), _ptr(v),
                                 _ptr(tau) if star else None, ctypes.byref(sc), _ptr(diag))
    else:
        raise TypeError(f"oracle: unsupported dtypes p={p.dtype} g={g.dtype}")
    return diag


def master_step(star: bool, master: np.ndarray, p16: np.ndarray, g16: np.ndarray,
                m: np.ndarray, v: np.ndarray, tau: Optional[np.ndarray],
                sc: OracleScalars) -> np.ndarray:
    """bf16-parameter mode: fp32 math on ``master``; ``p16`` = RNE(master)."""
    L = lib()
    diag = np.zeros(4, dtype=np.float64)
    L.adana_oracle_master_step(master.size, int(star), _ptr(master), _ptr(p16), _ptr(g16),
                               _ptr(m), _ptr(v), _ptr(tau) if star else None,
                               ctypes.byref(sc), _ptr(diag))
    return diag


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().adana_oracle_f32_to_bf16(x.size, _ptr(x), _ptr(y))
    return y


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------
# Gradient-norm clipping (src/optim/base.py:250-257 -> torch.nn.utils.
# clip_grad_norm_ with norm_type 2, torch/nn/utils/clip_grad.py)
# --------------------------------------------------------------------------

def _round_to(x, bf16: bool) -> np.float32:
    x = np.float32(x)
    return bf16_to_f32(f32_to_bf16(np.array([x])))[0] if bf16 else x


def clip_norms(grads: Sequence[np.ndarray], bf16: bool = False):
    """(per-tensor norms, total norm) as torch._foreach_norm and
    torch.linalg.vector_norm(torch.stack(norms)) produce them: each norm in
    the gradient dtype (binary32, or bfloat16 for bfloat16 gradients), from
    binary64 sums of squares (torch accumulates in binary32; both are within
    a few binary32 ulps of the exact value)."""
    norms = [_round_to(math.sqrt(float(np.sum(np.square(np.asarray(g, dtype=np.float64)))))
                       , bf16) for g in grads]
    total = _round_to(math.sqrt(math.fsum(float(n) * float(n) for n in norms)), bf16)
    return norms, total


def clip_coef(total, max_norm: float, bf16: bool = False) -> np.float32:
    """torch's coefficient from the total norm (_clip_grads_with_norm_):
    ``clamp(max_norm / (total + 1e-6), max=1.0)`` where ``float / Tensor`` is
    ``Tensor.reciprocal() * float``; every op is one binary32 operation on
    binary32 operands (the Python floats 1e-6 and max_norm cast to binary32),
    rounded to bfloat16 after each op for bfloat16 norms.  NaN propagates."""
    den = _round_to(np.float32(total) + np.float32(1e-6), bf16)
    with np.errstate(divide="ignore", over="ignore", invalid="ignore"):
        rc = _round_to(np.float32(1.0) / den, bf16)
        coef = _round_to(rc * np.float32(max_norm), bf16)
    return np.float32(1.0) if coef > np.float32(1.0) else coef


def clip_scale(g: np.ndarray, coef, bf16: bool = False) -> np.ndarray:
    """torch._foreach_mul_(grads, coef): g * coef in binary32, rounded to
    bfloat16 for bfloat16 gradients (returned as float32 values)."""
    with np.errstate(over="ignore", invalid="ignore"):
        y = np.asarray(g, dtype=np.float32) * np.float32(coef)
    return bf16_to_f32(f32_to_bf16(y)).reshape(y.shape) if bf16 else y


# --------------------------------------------------------------------------
# Step loop (restates the reference optimizers' step() bookkeeping)
# --------------------------------------------------------------------------

DIAG_KEYS = ("current_alpha", "gradient_norm", "auto_factor_mean",
             "current_kappa_factor", "m_norm")


def finalize_diag(sums: np.ndarray, n: int, bf16: bool = False) -> Dict[str, float]:
    """Per-tensor diagnostics from binary64 sums (src/optim/adana.py:146-151,221-225).
    bf16: the reference's bfloat16 path, where each diagnostic is a bfloat16
    0-d tensor (binary32 reduction rounded to bfloat16) and the kappa factor
    is the quotient of the two rounded values, itself rounded."""
    with np.errstate(invalid="ignore", divide="ignore"):
        ca = sums[0] / n if n else float("nan")
        afm = sums[2] / n if n else float("nan")
        gn, mn = math.sqrt(sums[1]), math.sqrt(sums[3])
        if bf16:
            r = lambda x: float(bf16_to_f32(f32_to_bf16(np.array([x], np.float32)))[0])  # noqa: E731
            ca, afm, gn, mn = r(ca), r(afm), r(gn), r(mn)
            kf = r(np.float32(ca) / np.float32(afm))
        else:
            kf = np.float64(ca) / np.float64(afm)
    return {"current_alpha": float(ca), "gradient_norm": gn,
            "auto_factor_mean": float(afm), "current_kappa_factor": float(kf),
            "m_norm": mn}


@dataclass
class OracleGroup:
    params: List[np.ndarray]
    lr: float
    delta: float = 8.0
    epsilon: float = 1e-8
    weight_decay: float = 0.0
    weighted_step_count: float = 0.0


@dataclass
class OracleOptimizer:
    """Restatement of ADana / DANA_STAR_MK4 over numpy arrays.

    ``star`` selects Dana-Star(-MK4); ``clipsnr=None`` disables SNR clipping.
    ``peak_lr`` plays the part of the constructor's ``lr`` (``self.lr``).
    Params are float32 arrays (or, with ``master=True``, uint16 bf16 arrays
    with an fp32 master copy kept in the state; or, with ``bf16=True``, uint16
    bf16 arrays whose m, v, tau are bf16 too: the reference's own bfloat16
    path).  ``numerics`` is "compiled" (the reference's default torch.compile
    path, src/optim/adana.py:72-79, 210-216) or "eager" (its update run as
    ATen ops).  ``foreach``: the reference's use_foreach=True path
    (src/optim/adana.py:229-370, src/optim/dana_star_mk4.py:298-536), whose
    kernel the reference compiles by default (``numerics`` again selects
    that compiled form or the kernel's eager ops).
    """

    groups: List[OracleGroup]
    star: bool
    peak_lr: float
    kappa: float = 1.0
    clipsnr: Optional[float] = None
    wd_decaying: bool = False
    wd_ts: float = 1.0
    gamma_3_factor: float = 1.0
    master: bool = False
    bf16: bool = False
    numerics: str = "compiled"
    foreach: bool = False
    state: Dict[int, dict] = field(default_factory=dict)

    def step(self, grads: Sequence[Sequence[Optional[np.ndarray]]]) -> None:
        """``grads[gi][pi]`` is the gradient of group gi's param pi, or None."""
        for gi, group in enumerate(self.groups):
            sf = group.lr / self.peak_lr                       # adana.py:165
            group.weighted_step_count += sf                    # adana.py:167
            for pi, p in enumerate(group.params):
                g = grads[gi][pi]
                if g is None:                                  # adana.py:186
                    continue
                key = id(p)
                st = self.state.get(key)
                if st is None:                                 # adana.py:191-195
                    sdt = np.uint16 if self.bf16 else np.float32     # zeros_like(p)
                    st = {"step": 0,
                          "m": np.zeros(p.shape, sdt),
                          "v": np.zeros(p.shape, sdt)}
                    if self.star:
                        st["tau"] = np.zeros(p.shape, sdt)
                    if self.master:
                        st["master"] = bf16_to_f32(p).reshape(p.shape).copy()
                    self.state[key] = st
                st["step"] += 1                                # adana.py:197
                kw = dict(lr=group.lr, peak_lr=self.peak_lr, delta=group.delta,
                          kappa=self.kappa, epsilon=group.epsilon,
                          weight_decay=group.weight_decay, clipsnr=self.clipsnr,
                          wd_decaying=self.wd_decaying, wd_ts=self.wd_ts,
                          gamma_3_factor=self.gamma_3_factor, t=st["step"],
                          compiled=self.numerics == "compiled")
                sc = foreach_scalars(**kw, step_bf16=self.bf16) if self.foreach else step_scalars(**kw)
                if self.master:
                    sums = master_step(self.star, st["master"], p, g, st["m"], st["v"],
                                       st.get("tau"), sc)
                else:
                    sums = element_step(self.star, p, g, st["m"], st["v"], st.get("tau"), sc)
                st.update(finalize_diag(sums, p.size, bf16=self.bf16))


# --------------------------------------------------------------------------
# Manau's eager Dana-Star-MK4 branch (src/optim/manau.py:504-613)
# --------------------------------------------------------------------------

def manau_scalars(*, lr: float, step: float, alpha: float, kappa: float, mk4A: float, mk4B: float,
                  clipsnr: float, epsilon: float, weight_decay: float, wd_decaying: bool,
                  wd_ts: float) -> OracleManauScalars:
    """The branch's Python floats (manau.py:539-555, :606-610) rounded to
    binary32 where they meet float32 tensors."""
    sc = OracleManauScalars()
    sc.a = f32(alpha)                                     # add_(g, alpha=alpha)
    sc.oma = f32(1 - alpha)                               # mul_(1 - alpha)
    sc.s = f32(step)                                      # tau * step (:289)
    sc.eps = f32(epsilon)
    sc.min_p = f32(1.0 / (1.0 + step))                    # full_like(tau, 1.0 / (1.0 + step)) (:281)
    sc.clip = f32(clipsnr)                                # clamp(max=clipsnr) (:589)
    sc.lr = f32(lr)                                       # lr * tensor (:591, :600)
    if wd_decaying:                                       # :607-610 (binary64, then mul_)
        sc.wdf = f32(1 - weight_decay / (1 + step / wd_ts) * lr)
    else:
        sc.wdf = f32(1 - weight_decay * lr)
    sc.has_wd = 1 if weight_decay != 0 else 0
    for k, e in enumerate((1 - kappa, 2 * mk4B + 1, 2 * (-mk4A - mk4B))):
        sc.e[k] = f32(e)
        sc.mode[k] = pow_mode(e)
    return sc


def manau_element_step(p: np.ndarray, g: np.ndarray, m: np.ndarray, v: np.ndarray, tau: np.ndarray,
                       sc: OracleManauScalars) -> np.ndarray:
    """One Manau Dana-branch update in place; binary64 sums [sum(alpha_factor),
    sum(g^2), sum(mfac), sum(m^2)]."""
    diag = np.zeros(4, dtype=np.float64)
    lib().adana_oracle_manau_step(p.size, _ptr(p), _ptr(g), _ptr(m), _ptr(v), _ptr(tau), ctypes.byref(sc),
                                  _ptr(diag))
    return diag


@dataclass
class OracleManauGroup:
    params: List[np.ndarray]
    use_muon: List[bool]
    lr: float
    weight_decay: float = 0.1
    delta: float = 8.0
    kappa: float = 1.0
    mk4A: float = 0.0
    mk4B: float = 0.0
    clipsnr: float = 1.0
    epsilon: float = 1e-8
    weight_time: bool = False
    wd_decaying: bool = False
    wd_ts: float = 1.0
    dana_momentum: bool = False
    weighted_step_count: float = 0.0


@dataclass
class OracleManau:
    """Manau.step's Dana-Star-MK4 branch over numpy arrays (manau.py:504-613),
    with the weighted step count the Muon loop advances before it (:348-353
    when dana_momentum).  ``peak_lr`` is the constructor's lr (self.lr)."""

    groups: List[OracleManauGroup]
    peak_lr: float
    state: Dict[int, dict] = field(default_factory=dict)

    def step(self, grads: Sequence[Sequence[np.ndarray]]) -> None:
        for group in self.groups:                         # Muon loop (:329-353): counter only
            if group.dana_momentum:
                for use in group.use_muon:
                    if use:
                        group.weighted_step_count += group.lr / self.peak_lr if group.weight_time else 1.0
        for gi, group in enumerate(self.groups):          # :507-613
            for pi, p in enumerate(group.params):
                if group.use_muon[pi]:
                    continue
                g = grads[gi][pi]
                st = self.state.get(id(p))
                if st is None:                            # :533-537
                    st = self.state[id(p)] = {"dana_m": np.zeros(p.shape, np.float32),
                                              "dana_v": np.zeros(p.shape, np.float32),
                                              "dana_tau": np.zeros(p.shape, np.float32), "step": 0}
                st["step"] += 1                           # :542
                time_factor = group.lr / self.peak_lr if group.weight_time else 1.0
                group.weighted_step_count += time_factor  # :546
                if group.weight_time:                     # :548-554
                    step = group.weighted_step_count
                    alpha = group.delta / (group.delta + step) * time_factor
                else:
                    step = st["step"]
                    alpha = group.delta / (group.delta + step)
                sc = manau_scalars(lr=group.lr, step=step, alpha=alpha, kappa=group.kappa, mk4A=group.mk4A,
                                   mk4B=group.mk4B, clipsnr=group.clipsnr, epsilon=group.epsilon,
                                   weight_decay=group.weight_decay, wd_decaying=group.wd_decaying,
                                   wd_ts=group.wd_ts)
                sums = manau_element_step(p, g, st["dana_m"], st["dana_v"], st["dana_tau"], sc)
                n = p.size
                st["current_alpha"] = alpha                # :578
                st["current_alpha_factor"] = sums[0] / n if n else float("nan")
                st["gradient_norm"] = math.sqrt(sums[1])
                st["auto_factor_mean"] = sums[2] / n if n else float("nan")
                st["m_norm"] = math.sqrt(sums[3])


# --------------------------------------------------------------------------
# Tau order statistics (src/optim/tau_stats_collector.py:336-376)
# --------------------------------------------------------------------------

def tau_order_statistics(tau: np.ndarray):
    """(largest, smallest): np.sort of the flattened values, read at indices
    unique(int32(1.1**k) - 1) for k = 0..ceil(log n / log 1.1), clamped to
    n - 1, from the small end and from the large end (NaN sorts last)."""
    x = np.asarray(tau).reshape(-1)
    n = x.size
    if n == 0:
        return np.array([]), np.array([])
    s = np.sort(x)
    max_k = int(np.ceil(np.log(n) / np.log(1.1)))
    idx = np.minimum(np.unique(np.int32(1.1 ** np.arange(max_k + 1)) - 1), n - 1)
    return s[(n - 1) - idx], s[idx]
