"""ctypes binding of ``libadana_mta.so`` (C ABI: include/adana_mta.h).

The library is built in-tree by ``adana_amd/csrc/Makefile`` (driven by
``__graft_entry__.build()``).  It links ``libamdhip64.so.7`` by soname, so once
``torch`` has loaded its own HIP runtime the dynamic loader binds the library
to that same runtime and torch's streams and device pointers are valid in it.
A missing library is an error: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libadana_mta.so")

ABI_VERSION = 8
CHUNK_ELEMS = 1024
ALIGN_ELEMS = 4
MAX_CLASSES = 8
FOLD_CHUNKS = 512
DIRECT_CHUNKS = 512

VARIANT_STAR = 0x1
GRAD_BF16 = 0x2
PARAM_BF16 = 0x4
WRITE_GRAD = 0x8
VARIANT_MANAU = 0x10
STATE_BF16 = 0x20
NUMERICS_EAGER = 0x40
FOREACH = 0x80
DESC_VEC_OK = 0x1

# adana_tensor_desc as a numpy record (64 bytes, same field order; the
# gradient pointers are a separate array, adana_plan.grad).
DESC_DTYPE = np.dtype([
    ("param", np.uint64), ("reserved0", np.uint64), ("m", np.uint64), ("v", np.uint64),
    ("tau", np.uint64), ("param_lp", np.uint64), ("numel", np.int64),
    ("sclass", np.int32), ("flags", np.uint32),
])
assert DESC_DTYPE.itemsize == 64


class HParams(ctypes.Structure):
    """adana_hparams."""

    _fields_ = [
        ("peak_lr", ctypes.c_double), ("delta", ctypes.c_double), ("kappa", ctypes.c_double),
        ("epsilon", ctypes.c_double), ("weight_decay", ctypes.c_double),
        ("clipsnr", ctypes.c_double), ("wd_ts", ctypes.c_double),
        ("gamma_3_factor", ctypes.c_double), ("has_clip", ctypes.c_int32),
        ("wd_decaying", ctypes.c_int32), ("eager", ctypes.c_int32), ("foreach", ctypes.c_int32),
    ]


class StepScalars(ctypes.Structure):
    """adana_step_scalars (64 bytes)."""

    _fields_ = [
        ("a", ctypes.c_float), ("oma", ctypes.c_float), ("lerp_coef", ctypes.c_float),
        ("s", ctypes.c_float), ("eps", ctypes.c_float), ("pw", ctypes.c_float),
        ("min_p", ctypes.c_float), ("clip", ctypes.c_float), ("c3", ctypes.c_float),
        ("cg2", ctypes.c_float), ("opw", ctypes.c_float), ("star_exp", ctypes.c_float),
        ("pow_mode", ctypes.c_int32), ("has_clip", ctypes.c_int32),
        ("lerp_small", ctypes.c_int32), ("pow_int", ctypes.c_int32),
    ]


assert ctypes.sizeof(StepScalars) == 64


class ManauHParams(ctypes.Structure):
    """adana_manau_hparams."""

    _fields_ = [
        ("delta", ctypes.c_double), ("kappa", ctypes.c_double), ("mk4A", ctypes.c_double),
        ("mk4B", ctypes.c_double), ("clipsnr", ctypes.c_double), ("epsilon", ctypes.c_double),
        ("weight_decay", ctypes.c_double), ("wd_ts", ctypes.c_double),
        ("wd_decaying", ctypes.c_int32), ("reserved", ctypes.c_int32),
    ]


class ManauScalars(ctypes.Structure):
    """adana_manau_scalars (64 bytes; fills an adana_step_scalars slot)."""

    _fields_ = [
        ("a", ctypes.c_float), ("oma", ctypes.c_float), ("s", ctypes.c_float), ("eps", ctypes.c_float),
        ("min_p", ctypes.c_float), ("clip", ctypes.c_float), ("lr", ctypes.c_float), ("wdf", ctypes.c_float),
        ("e", ctypes.c_float * 3), ("mode", ctypes.c_int32 * 3), ("has_wd", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


assert ctypes.sizeof(ManauScalars) == 64


class Plan(ctypes.Structure):
    """adana_plan: host struct of device pointers."""

    _fields_ = [
        ("desc", ctypes.c_void_p), ("grad", ctypes.c_void_p), ("vstart", ctypes.c_void_p),
        ("chunk_first", ctypes.c_void_p),
        ("fold_first", ctypes.c_void_p), ("n_tensors", ctypes.c_int32),
        ("reserved", ctypes.c_int32), ("n_chunks", ctypes.c_int64), ("n_folds", ctypes.c_int64),
    ]

# Every symbol include/adana_mta.h declares (checked by the CPU test suite).
EXPORTS = (
    "adana_abi_version", "adana_last_error", "adana_step_scalars_init", "adana_manau_scalars_init",
    "adana_plan_layout", "adana_plan_index", "adana_workspace_bytes", "adana_mta_step",
    "adana_mta_step_scaled", "adana_grad_clip_norm", "adana_grad_scale",
    "adana_order_stats_workspace", "adana_order_stats_workspace_compact", "adana_order_stats",
    "adana_mta_step_noalloc",
)
NOALLOC_SCRATCH_BYTES = 64 << 20

_lib = None


class AdanaLibraryError(RuntimeError):
    pass


def _declare(L) -> None:
    P = ctypes.c_void_p
    i32, i64, u32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32
    L.adana_abi_version.argtypes = []
    L.adana_abi_version.restype = ctypes.c_int
    L.adana_last_error.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    L.adana_last_error.restype = ctypes.c_size_t
    L.adana_step_scalars_init.argtypes = [ctypes.POINTER(StepScalars), ctypes.POINTER(HParams),
                                          ctypes.c_double, i64]
    L.adana_step_scalars_init.restype = ctypes.c_int
    L.adana_manau_scalars_init.argtypes = [ctypes.POINTER(ManauScalars), ctypes.POINTER(ManauHParams),
                                           ctypes.c_double, ctypes.c_double, ctypes.c_double]
    L.adana_manau_scalars_init.restype = ctypes.c_int
    L.adana_plan_layout.argtypes = [P, i32, P, P, ctypes.POINTER(i64)]
    L.adana_plan_layout.restype = i64
    L.adana_plan_index.argtypes = [P, i32, i64, P, P]
    L.adana_plan_index.restype = ctypes.c_int
    L.adana_workspace_bytes.argtypes = [ctypes.POINTER(Plan)]
    L.adana_workspace_bytes.restype = ctypes.c_size_t
    L.adana_mta_step.argtypes = [ctypes.POINTER(Plan), P, i32, u32, P, ctypes.c_size_t, P, P]
    L.adana_mta_step.restype = ctypes.c_int
    L.adana_mta_step_noalloc.argtypes = [ctypes.POINTER(Plan), P, i32, u32, P, P]
    L.adana_mta_step_noalloc.restype = ctypes.c_int
    L.adana_mta_step_scaled.argtypes = [ctypes.POINTER(Plan), P, i32, u32, P, P, ctypes.c_size_t, P, P]
    L.adana_mta_step_scaled.restype = ctypes.c_int
    L.adana_grad_clip_norm.argtypes = [ctypes.POINTER(Plan), u32, ctypes.c_double, P, ctypes.c_size_t,
                                       P, P, P]
    L.adana_grad_clip_norm.restype = ctypes.c_int
    L.adana_grad_scale.argtypes = [ctypes.POINTER(Plan), u32, P, P]
    L.adana_grad_scale.restype = ctypes.c_int
    L.adana_order_stats_workspace.argtypes = [i32, i64]
    L.adana_order_stats_workspace.restype = ctypes.c_size_t
    L.adana_order_stats_workspace_compact.argtypes = [P, P, i32]
    L.adana_order_stats_workspace_compact.restype = ctypes.c_size_t
    L.adana_order_stats.argtypes = [P, P, i32, P, P, P, P, ctypes.c_size_t, P]
    L.adana_order_stats.restype = ctypes.c_int


def _hip_runtimes_mapped():
    try:
        with open("/proc/self/maps") as f:
            return sorted({ln.split()[-1] for ln in f if "libamdhip64" in ln})
    except OSError:
        return []


def lib():
    """Load the HIP library (after torch's HIP runtime) or raise."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  -- torch's libamdhip64 must be resident first

    if not os.path.exists(LIB_PATH):
        raise AdanaLibraryError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "or `make -C adana_amd/csrc` (the ADana step has no non-HIP path)")
    L = ctypes.CDLL(LIB_PATH)
    _declare(L)
    v = L.adana_abi_version()
    if v != ABI_VERSION:
        raise AdanaLibraryError(f"libadana_mta ABI {v} != expected {ABI_VERSION}; rebuild")
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise AdanaLibraryError(f"two HIP runtimes are mapped ({runtimes}); the kernel library "
                                "must share torch's")
    _lib = L
    return L


def last_error() -> str:
    L = lib()
    buf = ctypes.create_string_buffer(512)
    L.adana_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise AdanaLibraryError(f"{what} failed (code {rc}): {last_error()}")


def step_scalars(hp: HParams, lr: float, step: int) -> StepScalars:
    sc = StepScalars()
    check(lib().adana_step_scalars_init(ctypes.byref(sc), ctypes.byref(hp), float(lr), int(step)),
          "adana_step_scalars_init")
    return sc


def manau_scalars(hp: ManauHParams, lr: float, step: float, alpha: float) -> ManauScalars:
    sc = ManauScalars()
    check(lib().adana_manau_scalars_init(ctypes.byref(sc), ctypes.byref(hp), float(lr), float(step),
                                         float(alpha)), "adana_manau_scalars_init")
    return sc


def plan_layout(numels: np.ndarray):
    """Return (vstart[int64 n+1], fold_first[int32 n+1], n_chunks, n_folds)."""
    numels = np.ascontiguousarray(numels, dtype=np.int64)
    n = numels.size
    vstart = np.zeros(n + 1, dtype=np.int64)
    fold_first = np.zeros(n + 1, dtype=np.int32)
    n_folds = ctypes.c_int64(0)
    chunks = lib().adana_plan_layout(ctypes.c_void_p(numels.ctypes.data), n,
                                     ctypes.c_void_p(vstart.ctypes.data),
                                     ctypes.c_void_p(fold_first.ctypes.data), ctypes.byref(n_folds))
    if chunks < 0:
        check(int(chunks), "adana_plan_layout")
    return vstart, fold_first, int(chunks), int(n_folds.value)


def workspace_bytes(plan: Plan) -> int:
    return int(lib().adana_workspace_bytes(ctypes.byref(plan)))
