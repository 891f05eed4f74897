"""Shared test helpers: ulp distances, golden-fixture replay, seeded inputs."""
from __future__ import annotations

import json
import os
import sys
from typing import Dict, List, Optional

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in binary32 ulps (+0 == -0; NaN vs NaN counts as 0)."""
    a = np.ascontiguousarray(a, dtype=np.float32).ravel()
    b = np.ascontiguousarray(b, dtype=np.float32).ravel()

    def ordered(x):
        i = x.view(np.int32).astype(np.int64)
        return np.where(i < 0, -(i & 0x7FFFFFFF), i)

    d = np.abs(ordered(a) - ordered(b))
    both_nan = np.isnan(a) & np.isnan(b)
    d[both_nan] = 0
    return d


def bf16_ulp_diff(a16: np.ndarray, b16: np.ndarray) -> np.ndarray:
    """Distance in bfloat16 ulps between two uint16 bit arrays."""
    def ordered(x):
        i = np.ascontiguousarray(x, dtype=np.uint16).ravel().astype(np.int64)
        return np.where(i >= 0x8000, -(i & 0x7FFF), i)

    return np.abs(ordered(a16) - ordered(b16))


def load_golden_inputs(name: str = "inputs"):
    """Inputs of the golden runs: ``inputs`` (finite gradients) or
    ``nonfinite.inputs`` (the same with NaN / inf entries)."""
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    meta = json.loads(str(z["meta"]))
    shapes = [tuple(s) for s in meta["shapes"]]
    p0 = [z[f"p0_{i}"] for i in range(len(shapes))]
    grads = [[z[f"g_{k}_{i}"] for i in range(len(shapes))]
             for k in range(1, meta["n_steps"] + 1)]
    return meta, p0, grads, z["has_grad"]


def load_golden_case(case: str, mode: str = "eager") -> Optional[Dict[str, np.ndarray]]:
    path = os.path.join(GOLDEN, f"{case}.{mode}.npz")
    if not os.path.exists(path):
        return None
    z = np.load(path)
    return {k: z[k] for k in z.files}


def golden_cases(mode: str = "eager") -> List[str]:
    meta, *_ = load_golden_inputs()
    return [c for c in meta["cases"] if os.path.exists(os.path.join(GOLDEN, f"{c}.{mode}.npz"))]


def is_star_class(cls_name: str) -> bool:
    return cls_name == "DANA_STAR_MK4"


def load_reference_state_dict(case: str, device: str = "cpu"):
    """The reference optimizer's own ``state_dict()`` at step 8 of the golden
    run (tests/golden/<case>.state8.npz), rebuilt as torch objects."""
    import torch

    z = np.load(os.path.join(GOLDEN, f"{case}.state8.npz"))
    schema = json.loads(str(z["schema"]))
    state = {}
    for idx, ent in schema["state"].items():
        st = {}
        for k, spec in ent.items():
            if spec["type"] == "Tensor":
                st[k] = torch.from_numpy(z[f"state.{idx}.{k}"].copy()).to(device)
            else:
                st[k] = spec["value"]
        state[int(idx)] = st
    groups = [dict(g) for g in schema["param_groups"]]
    return {"state": state, "param_groups": groups}, schema


def state_dict_schema(sd) -> dict:
    """Keys, Python types, dtypes and shapes of an optimizer state_dict (the
    form of the fixture schema) and its group entries."""
    import torch

    out = {"state": {}, "param_groups": []}
    for idx, st in sd["state"].items():
        ent = {}
        for k, v in st.items():
            if isinstance(v, torch.Tensor):
                ent[k] = {"type": "Tensor", "dtype": str(v.dtype), "shape": list(v.shape)}
            else:
                ent[k] = {"type": type(v).__name__}
        out["state"][str(idx)] = ent
    for g in sd["param_groups"]:
        out["param_groups"].append(sorted(g.keys()))
    return out
