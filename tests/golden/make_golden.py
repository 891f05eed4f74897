"""Write golden vectors for the ADana-family step from the reference itself.

Runs ONLY in the build container (the reference is not available on the GPU
boxes and never travels): it loads src/optim/adana.py and
src/optim/dana_star_mk4.py from the reference checkout by file path, drives
their own ``step()`` on CPU over small seeded inputs, and stores inputs and
outputs as ``.npz`` fixtures next to this script.

Why it is needed: closed forms and invariants pin the oracle's formulas but
not the exact binary32 rounding of the reference's composite ops (ATen's
lerp / addcmul association and FMA use); these vectors pin those bits.

Two modes of the reference are recorded:
  eager     -- ``_get_compiled_fn`` is replaced by the undecorated
               ``_update_param_compiled`` so each tensor runs as ATen eager ops
               (src/optim/adana.py:210-216 call the same function);
  compiled  -- the reference's default ``torch.compile`` path (Inductor-CPU),
               recorded when the container can compile it (--compiled).

A third output is the reference optimizer's own ``state_dict()`` at step
STATE_AT of the eager run (``<case>.state8.npz``: every tensor, plus a JSON
schema of keys, Python types, dtypes and shapes): the checkpoint interchange
tests load it into this build's optimizers and compare schemas
(src/optim/utils.py:283-310 saves exactly this dict).

A fifth output (--bf16) runs every case with the reference's own bfloat16
path: bfloat16 parameters and gradients (the float32 inputs rounded to
nearest even), so ``zeros_like(p)`` makes m, v and tau bfloat16 as well and
every tensor op rounds to bfloat16 (src/optim/adana.py:191-195;
src/optim/dana_star_mk4.py:251-255).  Both modes are recorded, eager and
``torch.compile``: ``<case>.bf16_eager.npz`` / ``<case>.bf16_compiled.npz``,
tensors stored as their 16-bit patterns (uint16), diagnostics as float32.

A sixth output (--foreach) runs every case with ``use_foreach=True``: the
reference's foreach path (src/optim/adana.py:229-370,
src/optim/dana_star_mk4.py:298-536), whose ``_foreach_compute_kernel_impl``
the constructor wraps in ``torch.compile(dynamic=True)``
(``<case>.foreach.npz``), and the same function as eager ops
(``<case>.foreach_eager.npz``); float32 and bfloat16 parameters
(``<case>.bf16_foreach[_eager].npz``); and the compiled float32 run on the
non-finite gradients of --nonfinite (``<case>.foreach_nonfinite.npz``; the
inputs are nonfinite.inputs.npz).

A fourth output (--nonfinite) repeats the eager runs of four cases with a few
NaN / +inf / -inf gradient entries (NONFINITE) and stores them as
``nonfinite.inputs.npz`` and ``<case>.nonfinite.npz``: how the reference's
ops carry non-finite values (lerp, addcmul, sqrt, clamp, sign of NaN, the
diagnostics' sums) is pinned by its own run.

Usage:  python tests/golden/make_golden.py [--ref /root/reference] [--compiled] [--state-only] [--nonfinite]
                                          [--bf16] [--foreach]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# Tensor list shared by every case: odd sizes (vector body + scalar tail in
# ATen's CPU loops), a row-sparse 2-D grad, an all-zero grad, and a tensor
# whose grad is None on odd steps (its per-tensor step counter lags).
SHAPES = [(37,), (3, 129), (40, 17), (16,), (20, 8), (5,)]
ZERO_GRAD = 3
ROW_SPARSE = 4
NONE_ON_ODD = 5
N_STEPS = 20
CHECKPOINTS = (1, 7, 8, 9, 20)       # t = delta = 8 puts alpha exactly at 0.5
STATE_AT = 8

CASES = {
    # name: (module, class, ctor kwargs, group weight decays)
    "adana": ("adana", "ADana",
              dict(lr=3e-3, delta=8.0, kappa=0.85, weight_decay=0.4, clipsnr=None,
                   wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0)),
    "dana_mk4": ("adana", "ADana",
                 dict(lr=3e-3, delta=8.0, kappa=0.85, weight_decay=0.4, clipsnr=1.0,
                      wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0)),
    "adana_k1_nowd": ("adana", "ADana",
                      dict(lr=1e-3, delta=6.0, kappa=1.0, weight_decay=0.1, clipsnr=None,
                           wd_decaying=False, wd_ts=1.0, gamma_3_factor=0.5)),
    "dana_star": ("dana_star_mk4", "DANA_STAR_MK4",
                  dict(lr=3e-3, delta=8.0, kappa=0.85, weight_decay=0.4, clipsnr=None,
                       wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0)),
    "dana_star_mk4": ("dana_star_mk4", "DANA_STAR_MK4",
                      dict(lr=3e-3, delta=8.0, kappa=0.85, weight_decay=0.4, clipsnr=1.0,
                           wd_decaying=True, wd_ts=10.0, gamma_3_factor=1.0)),
    "dana_star_mk4_k05": ("dana_star_mk4", "DANA_STAR_MK4",
                          dict(lr=2e-3, delta=8.0, kappa=0.5, weight_decay=0.1, clipsnr=2.0,
                               wd_decaying=False, wd_ts=1.0, gamma_3_factor=0.7)),
}
GROUP_WD_SCALE = (1.0, 0.0)          # group 0 keeps weight_decay, group 1 has none
GROUP_OF = (0, 0, 0, 1, 1, 1)        # tensor -> group


def lr_multiplier(k: int) -> float:
    """Warm-up then cosine-like decay; the value used at step k (1-based)."""
    import math
    if k <= 4:
        return k / 4.0
    return 0.1 + 0.9 * 0.5 * (1 + math.cos(math.pi * (k - 4) / (N_STEPS - 4)))


def make_inputs(seed: int = 1234):
    rng = np.random.default_rng(seed)
    p0 = [rng.normal(0.0, 0.02, s).astype(np.float32) for s in SHAPES]
    grads = []
    for k in range(1, N_STEPS + 1):
        gs = []
        for i, s in enumerate(SHAPES):
            g = rng.normal(0.0, 1e-3, s).astype(np.float32)
            if i == ZERO_GRAD:
                g[...] = 0.0
            if i == ROW_SPARSE:
                rows = rng.random(s[0]) < 0.3
                g[~rows, :] = 0.0
            if len(s) == 1 and i not in (ZERO_GRAD,):
                g *= np.float32(0.1)
            gs.append(g)
        grads.append(gs)
    has_grad = np.ones((N_STEPS, len(SHAPES)), dtype=bool)
    has_grad[0::2, NONE_ON_ODD] = False          # steps 1, 3, 5, ... have grad None
    return p0, grads, has_grad


# Non-finite gradient entries for the --nonfinite fixtures: (step, tensor,
# flat index, value).  Steps 3 and 6; tensor NONE_ON_ODD only on even steps.
NONFINITE = [(3, 0, 2, float("nan")), (3, 0, 5, float("inf")), (3, 0, 9, float("-inf")),
             (3, 1, 7, float("inf")), (3, 3, 4, float("nan")),
             (6, 2, 3, float("nan")), (6, 4, 0, float("-inf")), (6, NONE_ON_ODD, 1, float("inf"))]
NONFINITE_CASES = ("adana", "dana_mk4", "dana_star", "dana_star_mk4")


def inject_nonfinite(grads):
    """Copies of the step gradients with the NONFINITE entries written in."""
    out = [[g.copy() for g in gs] for gs in grads]
    for k, i, j, val in NONFINITE:
        out[k - 1][i].reshape(-1)[j] = np.float32(val)
    return out


def load_module(ref: str, name: str):
    path = os.path.join(ref, "src", "optim", name + ".py")
    spec = importlib.util.spec_from_file_location("_ref_" + name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def state_dict_fixture(sd) -> dict:
    """Flatten an optimizer state_dict into npz entries + a JSON schema."""
    import torch

    out, schema = {}, {"state": {}, "param_groups": []}
    for idx, st in sd["state"].items():
        ent = {}
        for k, v in st.items():
            if isinstance(v, torch.Tensor):
                out[f"state.{idx}.{k}"] = v.detach().cpu().numpy().copy()
                ent[k] = {"type": "Tensor", "dtype": str(v.dtype), "shape": list(v.shape)}
            else:
                ent[k] = {"type": type(v).__name__, "value": v}
        schema["state"][str(idx)] = ent
    for g in sd["param_groups"]:
        schema["param_groups"].append({k: (v if not isinstance(v, float) else float(v))
                                       for k, v in g.items()})
    out["schema"] = np.array(json.dumps(schema))
    return out


def _bits(t) -> np.ndarray:
    """A tensor as numpy: float32 values, or the 16-bit patterns of bfloat16."""
    import torch

    t = t.detach().cpu()
    return t.view(torch.int16).numpy().view(np.uint16).copy() if t.dtype == torch.bfloat16 else t.numpy().copy()


def run_case(ref: str, case: str, compiled: bool, p0, grads, has_grad, state_out=None, bf16: bool = False,
             foreach: bool = False):
    import torch

    modname, clsname, kw = CASES[case]
    cls = getattr(load_module(ref, modname), clsname)
    dt = torch.bfloat16 if bf16 else torch.float32
    params = [torch.nn.Parameter(torch.from_numpy(x.copy()).to(dt)) for x in p0]
    groups = []
    for gi, scale in enumerate(GROUP_WD_SCALE):
        groups.append({"params": [p for i, p in enumerate(params) if GROUP_OF[i] == gi],
                       "weight_decay": kw["weight_decay"] * scale})
    opt = cls(groups, **kw, use_foreach=foreach)
    if not compiled:
        opt._get_compiled_fn = lambda shape: opt._update_param_compiled
        opt._foreach_compute_kernel = None      # the foreach path then calls its _impl as eager ops
    peak = kw["lr"]
    out = {}
    diags = np.full((N_STEPS, len(SHAPES), 5), np.nan, dtype=np.float32)
    keys = ("current_alpha", "gradient_norm", "auto_factor_mean", "current_kappa_factor",
            "m_norm")
    for k in range(1, N_STEPS + 1):
        for g in opt.param_groups:
            g["lr"] = peak * lr_multiplier(k)
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grads[k - 1][i].copy()).to(dt) if has_grad[k - 1, i] else None
        opt.step()
        for i, p in enumerate(params):
            st = opt.state[p]
            if st:
                diags[k - 1, i] = [float(st[x]) for x in keys]
        if state_out is not None and k == STATE_AT:
            state_out.update(state_dict_fixture(opt.state_dict()))
        if k in CHECKPOINTS:
            for i, p in enumerate(params):
                st = opt.state[p]
                out[f"p{i}_t{k}"] = _bits(p)
                for name in ("m", "v", "tau"):
                    if name in st:
                        out[f"{name}{i}_t{k}"] = _bits(st[name])
                out[f"step{i}_t{k}"] = np.int64(st.get("step", 0))
    out["diag"] = diags
    out["weighted_step_count"] = np.array([g["weighted_step_count"] for g in opt.param_groups])
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--compiled", action="store_true")
    ap.add_argument("--state-only", action="store_true",
                    help="only (re)write the <case>.state8.npz checkpoint fixtures")
    ap.add_argument("--bf16", action="store_true",
                    help="only write <case>.bf16_eager.npz and <case>.bf16_compiled.npz (bfloat16 parameters)")
    ap.add_argument("--nonfinite", action="store_true",
                    help="only write nonfinite.inputs.npz and <case>.nonfinite.npz (NaN/inf gradient entries)")
    ap.add_argument("--foreach", action="store_true",
                    help="only write the use_foreach=True runs: <case>.foreach[_eager].npz and "
                         "<case>.bf16_foreach[_eager].npz")
    args = ap.parse_args()
    import torch

    torch.set_num_threads(4)
    p0, grads, has_grad = make_inputs()
    inputs = {f"p0_{i}": x for i, x in enumerate(p0)}
    for k in range(N_STEPS):
        for i in range(len(SHAPES)):
            inputs[f"g_{k + 1}_{i}"] = grads[k][i]
    inputs["has_grad"] = has_grad
    meta = {"shapes": SHAPES, "group_of": GROUP_OF, "group_wd_scale": GROUP_WD_SCALE,
            "n_steps": N_STEPS, "checkpoints": CHECKPOINTS,
            "lr_multiplier": [lr_multiplier(k) for k in range(1, N_STEPS + 1)],
            "cases": {c: {"module": m, "class": cl, "kwargs": kw}
                      for c, (m, cl, kw) in CASES.items()},
            "torch": torch.__version__, "cpu_capability": torch.backends.cpu.get_cpu_capability()}
    inputs["meta"] = np.array(json.dumps(meta))
    if args.nonfinite:
        grads_nf = inject_nonfinite(grads)
        assert all(has_grad[k - 1, i] for k, i, _, _ in NONFINITE)
        nf = dict(inputs)
        for k in range(N_STEPS):
            for i in range(len(SHAPES)):
                nf[f"g_{k + 1}_{i}"] = grads_nf[k][i]
        meta_nf = dict(meta, cases={c: meta["cases"][c] for c in NONFINITE_CASES},
                       nonfinite=[[k, i, j, repr(v)] for k, i, j, v in NONFINITE])
        nf["meta"] = np.array(json.dumps(meta_nf))
        np.savez_compressed(os.path.join(HERE, "nonfinite.inputs.npz"), **nf)
        for case in NONFINITE_CASES:
            out = run_case(args.ref, case, False, p0, grads_nf, has_grad)
            np.savez_compressed(os.path.join(HERE, f"{case}.nonfinite.npz"), **out)
            print(f"wrote {case}.nonfinite.npz", flush=True)
        return 0
    if args.foreach:
        grads_nf = inject_nonfinite(grads)
        for case in NONFINITE_CASES:
            out = run_case(args.ref, case, True, p0, grads_nf, has_grad, foreach=True)
            np.savez_compressed(os.path.join(HERE, f"{case}.foreach_nonfinite.npz"), **out)
            print(f"wrote {case}.foreach_nonfinite.npz", flush=True)
        for bf16 in (False, True):
            for mode in ("compiled", "eager"):
                for case in CASES:
                    out = run_case(args.ref, case, mode == "compiled", p0, grads, has_grad, bf16=bf16, foreach=True)
                    name = f"{case}.{'bf16_' if bf16 else ''}foreach{'_eager' if mode == 'eager' else ''}.npz"
                    np.savez_compressed(os.path.join(HERE, name), **out)
                    print(f"wrote {name}", flush=True)
        return 0
    if args.bf16:
        for mode in ("eager", "compiled"):
            for case in CASES:
                out = run_case(args.ref, case, mode == "compiled", p0, grads, has_grad, bf16=True)
                np.savez_compressed(os.path.join(HERE, f"{case}.bf16_{mode}.npz"), **out)
                print(f"wrote {case}.bf16_{mode}.npz", flush=True)
        return 0
    if args.state_only:
        for case in CASES:
            st = {}
            run_case(args.ref, case, False, p0, grads, has_grad, state_out=st)
            np.savez_compressed(os.path.join(HERE, f"{case}.state{STATE_AT}.npz"), **st)
            print(f"wrote {case}.state{STATE_AT}.npz", flush=True)
        return 0
    np.savez_compressed(os.path.join(HERE, "inputs.npz"), **inputs)
    modes = ["eager"] + (["compiled"] if args.compiled else [])
    for mode in modes:
        for case in CASES:
            st = {} if mode == "eager" else None
            out = run_case(args.ref, case, mode == "compiled", p0, grads, has_grad, state_out=st)
            np.savez_compressed(os.path.join(HERE, f"{case}.{mode}.npz"), **out)
            print(f"wrote {case}.{mode}.npz", flush=True)
            if st:
                np.savez_compressed(os.path.join(HERE, f"{case}.state{STATE_AT}.npz"), **st)


if __name__ == "__main__":
    sys.exit(main())
