"""Write golden vectors for Manau (src/optim/manau.py) from the reference itself.

Runs ONLY in the build container (the reference is not available on the GPU
boxes and never travels): it loads src/optim/manau.py from the reference
checkout by file path, drives its own ``step()`` on CPU over a small seeded
GPT-like parameter list (named, so that Manau assigns the embedding and the
1-D parameters to its Dana-Star-MK4 branch and the other 2-D weights to
Muon), and stores inputs and outputs as ``manau.<case>.npz`` next to this
script.

Manau.step() starts with ``torch.cuda.current_device()`` (manau.py:314),
whose value only the distributed all-gather buffers use (:377-389); this
container has no GPU, so the script answers that one call with device 0.
Everything the recorded values depend on is the reference's own code.

Recorded per case: parameters, Dana state (dana_m, dana_v, dana_tau) and
Muon buffers at CHECKPOINTS, every step's Dana diagnostics, the groups'
weighted_step_count, the state_dict schema at STATE_AT and the constructor's
printed parameter-assignment summary.

--nonfinite repeats two cases with NaN / +inf / -inf gradient entries in
Dana-branch tensors (NONFINITE) and writes ``manau.nonfinite.inputs.npz`` and
``manau.<case>.nonfinite.npz``.

Usage:  python tests/golden/make_golden_manau.py [--ref /root/reference] [--nonfinite]
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

# (name, shape, group): names drive Manau's Muon / Dana split (manau.py:178-196)
PARAMS = [
    ("transformer.wte.weight", (97, 24), 1),          # embedding: Dana
    ("transformer.h.0.attn.c_attn.weight", (72, 24), 0),  # 2-D: Muon
    ("transformer.h.0.attn.c_proj.weight", (24, 24), 0),  # 2-D: Muon
    ("transformer.h.0.mlp.c_fc.weight", (40, 24), 0),     # 2-D: Muon (rows > cols)
    ("transformer.h.0.mlp.c_proj.weight", (24, 40), 0),   # 2-D: Muon (rows < cols)
    ("transformer.h.0.ln_1.weight", (24,), 1),        # 1-D: Dana
    ("transformer.h.0.ln_1.bias", (24,), 1),          # 1-D: Dana
    ("transformer.ln_f.weight", (24,), 1),            # 1-D: Dana
    ("lm_head.weight", (97, 24), 1),                  # head: Dana
]
N_STEPS = 12
CHECKPOINTS = (1, 8, 9, 12)                           # delta = 8: alpha crosses 0.5
STATE_AT = 8

CASES = {
    "manau": dict(lr=2e-2, weight_decay=0.1, kappa=0.85, clipsnr=1.0, delta=8.0, wd_decaying=False,
                  weight_time=False, dana_momentum=False),
    "manau_wt": dict(lr=2e-2, weight_decay=0.1, kappa=0.5, clipsnr=2.0, delta=8.0, wd_decaying=True,
                     wd_ts=5.0, weight_time=True, dana_momentum=True),
    "manau_mk4": dict(lr=1e-2, weight_decay=0.0, kappa=0.85, clipsnr=4.0, delta=6.0, mk4A=0.1, mk4B=0.25,
                      wd_decaying=False, weight_time=False, dana_momentum=False),
}
GROUP_WD_SCALE = (1.0, 0.5)


def lr_multiplier(k: int) -> float:
    return min(1.0, k / 3.0) * (1.0 - 0.5 * (k - 1) / N_STEPS)


def make_inputs(seed: int = 4321):
    rng = np.random.default_rng(seed)
    p0 = [rng.normal(0.0, 0.02, s).astype(np.float32) for _, s, _ in PARAMS]
    grads = []
    for _ in range(N_STEPS):
        gs = []
        for i, (name, s, _) in enumerate(PARAMS):
            g = rng.normal(0.0, 1e-3, s).astype(np.float32)
            if name == "transformer.wte.weight":      # row-sparse embedding gradient
                g[rng.random(s[0]) >= 0.3, :] = 0.0
            if name.endswith("ln_1.bias"):              # a few exactly-zero gradient entries
                g[:3] = 0.0
            gs.append(g)
        grads.append(gs)
    return p0, grads


# Non-finite gradient entries for --nonfinite: (step, tensor, flat index,
# value), in Dana-branch tensors (the embedding, a LayerNorm vector, the head).
NONFINITE = [(3, 0, 5, float("nan")), (3, 0, 30, float("inf")), (3, 5, 2, float("-inf")),
             (6, 8, 11, float("nan")), (6, 7, 0, float("inf"))]
NONFINITE_CASES = ("manau", "manau_mk4")


def inject_nonfinite(grads):
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


def schema_of(sd) -> dict:
    import torch

    schema = {"state": {}, "param_groups": []}
    for idx, st in sd["state"].items():
        schema["state"][str(idx)] = {
            k: ({"type": "Tensor", "dtype": str(v.dtype), "shape": list(v.shape)} if isinstance(v, torch.Tensor)
                else {"type": type(v).__name__}) for k, v in st.items()}
    for g in sd["param_groups"]:
        schema["param_groups"].append(sorted(k for k in g if k != "params"))
    return schema


def run_case(ref: str, case: str, p0, grads):
    import torch

    torch.cuda.current_device = lambda: 0            # see the module docstring
    Manau = load_module(ref, "manau").Manau
    kw = CASES[case]
    params = [torch.nn.Parameter(torch.from_numpy(x.copy())) for x in p0]
    groups = []
    for gi, scale in enumerate(GROUP_WD_SCALE):
        idx = [i for i, (_, _, g) in enumerate(PARAMS) if g == gi]
        groups.append({"params": [params[i] for i in idx], "param_names": [PARAMS[i][0] for i in idx],
                       "weight_decay": kw["weight_decay"] * scale})
    import contextlib
    import io

    printed = io.StringIO()
    with contextlib.redirect_stdout(printed):        # the constructor's assignment summary
        opt = Manau(groups, **kw)
    peak = kw["lr"]
    out = {}
    diag_keys = ("current_alpha", "current_alpha_factor", "gradient_norm", "auto_factor_mean", "m_norm")
    diags = np.full((N_STEPS, len(PARAMS), 5), np.nan, dtype=np.float64)
    wsc = np.zeros((N_STEPS, len(groups)), dtype=np.float64)
    for k in range(1, N_STEPS + 1):
        for g in opt.param_groups:
            g["lr"] = peak * lr_multiplier(k)
        for i, p in enumerate(params):
            p.grad = torch.from_numpy(grads[k - 1][i].copy())
        opt.step()
        for i, p in enumerate(params):
            st = opt.state[p]
            if not st.get("use_muon", False):
                diags[k - 1, i] = [float(st[x]) for x in diag_keys]
        wsc[k - 1] = [g["weighted_step_count"] for g in opt.param_groups]
        if k == STATE_AT:
            out["schema"] = np.array(json.dumps(schema_of(opt.state_dict())))
        if k in CHECKPOINTS:
            for i, p in enumerate(params):
                st = opt.state[p]
                out[f"p{i}_t{k}"] = p.detach().numpy().copy()
                for name in ("dana_m", "dana_v", "dana_tau", "muon_buffer"):
                    if name in st:
                        out[f"{name}{i}_t{k}"] = st[name].numpy().copy()
                out[f"step{i}_t{k}"] = np.int64(st.get("step", 0))
    out["diag"] = diags
    out["weighted_step_count"] = wsc
    out["use_muon"] = np.array([bool(opt.state[p].get("use_muon", False)) for p in params])
    out["ctor_stdout"] = np.array(printed.getvalue())
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--nonfinite", action="store_true",
                    help="only write manau.nonfinite.inputs.npz and manau.<case>.nonfinite.npz")
    args = ap.parse_args()
    import torch

    torch.set_num_threads(4)
    p0, grads = make_inputs()
    inputs = {f"p0_{i}": x for i, x in enumerate(p0)}
    for k in range(N_STEPS):
        for i in range(len(PARAMS)):
            inputs[f"g_{k + 1}_{i}"] = grads[k][i]
    meta = {"params": PARAMS, "group_wd_scale": GROUP_WD_SCALE, "n_steps": N_STEPS, "checkpoints": CHECKPOINTS,
            "state_at": STATE_AT, "lr_multiplier": [lr_multiplier(k) for k in range(1, N_STEPS + 1)],
            "cases": CASES, "torch": torch.__version__}
    inputs["meta"] = np.array(json.dumps(meta))
    if args.nonfinite:
        grads = inject_nonfinite(grads)
        for k in range(N_STEPS):
            for i in range(len(PARAMS)):
                inputs[f"g_{k + 1}_{i}"] = grads[k][i]
        meta_nf = dict(meta, cases={c: CASES[c] for c in NONFINITE_CASES},
                       nonfinite=[[k, i, j, repr(v)] for k, i, j, v in NONFINITE])
        inputs["meta"] = np.array(json.dumps(meta_nf))
        np.savez_compressed(os.path.join(HERE, "manau.nonfinite.inputs.npz"), **inputs)
        for case in NONFINITE_CASES:
            out = run_case(args.ref, case, p0, grads)
            np.savez_compressed(os.path.join(HERE, f"manau.{case}.nonfinite.npz"), **out)
            print("wrote", case, "nonfinite")
        return
    np.savez_compressed(os.path.join(HERE, "manau.inputs.npz"), **inputs)
    for case in CASES:
        out = run_case(args.ref, case, p0, grads)
        np.savez_compressed(os.path.join(HERE, f"manau.{case}.npz"), **out)
        print("wrote", case)


if __name__ == "__main__":
    main()
