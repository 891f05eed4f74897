"""CPU tests of the product's host side: the C ABI library loads and exports
every symbol include/adana_mta.h declares, its host scalar code agrees bit for
bit with the oracle's independent restatement, the layout is sound, and the
Python classes keep the reference's interface.  No GPU compute is called."""
import ctypes
import inspect
import math
import os
import re

import numpy as np
import pytest
import torch

from helpers import ROOT


def _header_functions():
    text = open(os.path.join(ROOT, "include", "adana_mta.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(adana_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from adana_amd import _lib

    L = _lib.lib()
    declared = _header_functions()
    assert declared, "no functions parsed from the header"
    for name in declared:
        assert hasattr(L, name), f"{name} declared in include/adana_mta.h but not exported"
    assert sorted(_lib.EXPORTS) == declared
    assert L.adana_abi_version() == _lib.ABI_VERSION


def test_single_hip_runtime_mapped():
    from adana_amd import _lib

    _lib.lib()
    assert len(_lib._hip_runtimes_mapped()) <= 1


def _hp(_lib, **kw):
    hp = _lib.HParams()
    hp.peak_lr = kw["peak_lr"]
    hp.delta = kw["delta"]
    hp.kappa = kw["kappa"]
    hp.epsilon = kw["epsilon"]
    hp.weight_decay = kw["weight_decay"]
    hp.has_clip = 0 if kw["clipsnr"] is None else 1
    hp.clipsnr = 0.0 if kw["clipsnr"] is None else kw["clipsnr"]
    hp.wd_ts = kw["wd_ts"]
    hp.gamma_3_factor = kw["gamma_3_factor"]
    hp.wd_decaying = int(kw["wd_decaying"])
    return hp


def _f32bits(x):
    return np.float32(x).view(np.int32)


@pytest.mark.parametrize("kappa", [0.85, 1.0, 0.5, 0.75, 1.5, -1.0, 0.0])
def test_host_scalars_match_oracle_bitwise(oracle_mod, kappa):
    from adana_amd import _lib

    rng = np.random.default_rng(int(abs(kappa) * 100) + 7)
    for trial in range(60):
        kw = dict(peak_lr=float(10 ** rng.uniform(-4, -1)), delta=float(rng.choice([8.0, 6.0, 16.0, 3.5])),
                  kappa=kappa, epsilon=float(rng.choice([1e-8, 1e-6, 1e-10])),
                  weight_decay=float(rng.choice([0.0, 0.4, 0.1, 1.3])),
                  clipsnr=[None, 1.0, 2.0, 0.37][trial % 4],
                  wd_decaying=bool(trial % 2), wd_ts=float(rng.choice([1.0, 10.0, 20.0, 37.5])),
                  gamma_3_factor=float(rng.choice([1.0, 0.5, 0.0, 1.7])))
        lr = kw["peak_lr"] * float(rng.uniform(0.01, 1.0))
        t = int(rng.choice([1, 2, 7, 8, 9, 100, 12345, 2 ** 20 + 3]))
        sc = _lib.step_scalars(_hp(_lib, **kw), lr, t)
        ref = oracle_mod.step_scalars(lr=lr, t=t, **kw)
        for name in ("a", "oma", "s", "eps", "pw", "min_p", "c3", "cg2", "opw", "star_exp"):
            assert _f32bits(getattr(sc, name)) == _f32bits(getattr(ref, name)), (name, kw, lr, t)
        assert sc.pow_mode == ref.pow_mode
        assert sc.has_clip == ref.has_clip
        if ref.has_clip:
            assert _f32bits(sc.clip) == _f32bits(ref.clip)
        # lerp helper fields: ATen's |w| < 0.5 branch and its coefficient
        assert sc.lerp_small == int(abs(float(ref.a)) < 0.5)
        coef = ref.a if sc.lerp_small else np.float32(ref.a) - np.float32(1.0)
        assert _f32bits(sc.lerp_coef) == _f32bits(coef)


@pytest.mark.parametrize("compiled", [True, False], ids=["compiled", "eager"])
@pytest.mark.parametrize("foreach", [1, 2], ids=["fp32_step", "bf16_step"])
@pytest.mark.parametrize("kappa", [0.85, 1.0, 0.5, 1.5])
def test_host_foreach_scalars_match_oracle_bitwise(oracle_mod, kappa, foreach, compiled):
    """adana_step_scalars_init with hparams.foreach (the use_foreach=True
    path) against the oracle's independent restatement (oracle.foreach_scalars),
    bit for bit; c3, cg2 and opw carry gamma_3_factor, lr and the weight-decay
    factor; with bfloat16 parameters the step is rounded to bfloat16 and the
    lerp coefficient comes from alpha rounded to bfloat16."""
    from adana_amd import _lib

    rng = np.random.default_rng(int(kappa * 100) + 31 * foreach + int(compiled))
    for trial in range(40):
        kw = dict(peak_lr=float(10 ** rng.uniform(-4, -1)), delta=float(rng.choice([8.0, 6.0, 7.3, 3.5])),
                  kappa=kappa, epsilon=float(rng.choice([1e-8, 1e-6])),
                  weight_decay=float(rng.choice([0.0, 0.4, 0.1])), clipsnr=[None, 1.0, 2.0, 0.37][trial % 4],
                  wd_decaying=bool(trial % 2), wd_ts=float(rng.choice([1.0, 10.0, 37.5])),
                  gamma_3_factor=float(rng.choice([1.0, 0.5, 0.7])))
        lr = kw["peak_lr"] * float(rng.uniform(0.01, 1.0))
        t = int(rng.choice([1, 2, 7, 8, 9, 100, 257, 12345, 2 ** 20 + 3]))
        hp = _hp(_lib, **kw)
        hp.foreach = foreach
        hp.eager = 0 if compiled else 1
        sc = _lib.step_scalars(hp, lr, t)
        ref = oracle_mod.foreach_scalars(lr=lr, t=t, compiled=compiled, step_bf16=foreach == 2, **kw)
        for name in ("a", "oma", "s", "eps", "pw", "min_p", "star_exp"):
            assert _f32bits(getattr(sc, name)) == _f32bits(getattr(ref, name)), (name, kw, lr, t)
        for name, rname in (("c3", "g3f"), ("cg2", "lr"), ("opw", "wdf")):
            assert _f32bits(getattr(sc, name)) == _f32bits(getattr(ref, rname)), (name, kw, lr, t)
        assert sc.pow_mode == ref.pow_mode and sc.has_clip == ref.has_clip
        aw = oracle_mod.bf16_to_f32(oracle_mod.f32_to_bf16(np.array([ref.a], np.float32)))[0] \
            if foreach == 2 else np.float32(ref.a)
        assert sc.lerp_small == int(abs(float(aw)) < 0.5)
        coef = aw if sc.lerp_small else np.float32(aw) - np.float32(1.0)
        assert _f32bits(sc.lerp_coef) == _f32bits(coef)
    hp.foreach = 3
    with pytest.raises(_lib.AdanaLibraryError, match="foreach"):
        _lib.step_scalars(hp, 1e-3, 1)


def test_host_scalars_reject_bad_input():
    from adana_amd import _lib

    hp = _lib.HParams(peak_lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8)
    with pytest.raises(_lib.AdanaLibraryError, match="step"):
        _lib.step_scalars(hp, 1e-3, 0)
    hp.peak_lr = 0.0
    with pytest.raises(_lib.AdanaLibraryError, match="peak lr"):
        _lib.step_scalars(hp, 1e-3, 1)


def test_plan_layout_properties():
    from adana_amd import _lib

    rng = np.random.default_rng(0)
    numels = np.concatenate([rng.integers(0, 70000, 300), [0, 1, 3, 4, 5, 16384, 16385],
                             [5_000_000, 0, 7, 512 * 1024, 512 * 1024 + 1]])
    vstart, fold_first, chunks, n_folds = _lib.plan_layout(numels)
    C = _lib.CHUNK_ELEMS
    A = _lib.ALIGN_ELEMS
    assert vstart[0] == 0
    assert np.all(vstart % A == 0)
    # each tensor starts at the previous end rounded up to A, moved to the next
    # chunk boundary only when it would otherwise cross that boundary
    end = 0
    for vs, n in zip(vstart[:-1].tolist(), numels.tolist()):
        r = end % C
        want = end + (C - r) if (r and r + n > C) else end
        assert vs == want
        assert vs % C == 0 or vs % C + n <= C                 # no chunk boundary crossed from inside
        end = vs + -(-n // A) * A
    assert vstart[-1] == end
    assert chunks == math.ceil(vstart[-1] / C)
    # (chunk, tensor) segment slots chunk + tensor are distinct
    slots = set()
    for i, (vs, n) in enumerate(zip(vstart[:-1], numels)):
        if n == 0:
            continue
        for b in range(vs // C, (vs + n - 1) // C + 1):
            assert b + i not in slots
            slots.add(b + i)
    assert max(slots) < chunks + len(numels)
    # fold workgroups: ceil(chunks of tensor / FOLD_CHUNKS) for a tensor of more
    # than DIRECT_CHUNKS chunks; none for smaller ones (summed directly)
    for i, (vs, n) in enumerate(zip(vstart[:-1], numels)):
        nch = 0 if n == 0 else (vs + n - 1) // C - vs // C + 1
        want = math.ceil(nch / _lib.FOLD_CHUNKS) if nch > _lib.DIRECT_CHUNKS else 0
        assert fold_first[i + 1] - fold_first[i] == want
    assert fold_first[-1] == n_folds
    assert _lib.plan_layout(np.zeros(0, np.int64))[2] == 0
    # the chunk -> first tensor rule the device index kernel applies
    first = np.searchsorted(vstart[:-1], np.arange(chunks) * C, side="right") - 1
    for c in range(0, chunks, 7):
        i = first[c]
        lo = c * C
        assert vstart[i] <= lo
        assert all(vstart[k] + numels[k] <= lo for k in range(max(0, i - 50), i))


def test_workspace_bytes():
    from adana_amd import _lib

    pl = _lib.Plan(n_tensors=10, n_chunks=100, n_folds=12)
    # chunk partials, then folds, then one arrival counter per tensor, then the
    # bfloat16 pow table (one entry per bf16 value in [1, +inf]), each 256-byte aligned
    folds_at = (110 * 16 + 255) // 256 * 256
    counters_at = (folds_at + 12 * 32 + 255) // 256 * 256
    table_at = (counters_at + 10 * 4 + 255) // 256 * 256
    assert _lib.workspace_bytes(pl) == table_at + (0x7F80 - 0x3F80 + 1) * 2
    # a list without elements launches no step kernel: no table, and nothing at all when empty
    assert _lib.workspace_bytes(_lib.Plan(n_tensors=3, n_chunks=0, n_folds=0)) == 256 + 3 * 4
    assert _lib.workspace_bytes(_lib.Plan(n_tensors=0, n_chunks=0, n_folds=0)) == 0


def test_mta_step_rejects_bad_arguments():
    from adana_amd import _lib

    L = _lib.lib()
    sc = (_lib.StepScalars * 1)()
    scp = ctypes.cast(sc, ctypes.c_void_p)
    assert L.adana_mta_step(None, scp, 1, 0, None, 0, None, None) == -1
    assert "null plan" in _lib.last_error()
    pl = _lib.Plan(n_tensors=-1)
    assert L.adana_mta_step(ctypes.byref(pl), scp, 1, 0, None, 0, None, None) == -1
    assert "bad sizes" in _lib.last_error()
    pl = _lib.Plan(n_tensors=3, n_chunks=1, n_folds=3)
    assert L.adana_mta_step(ctypes.byref(pl), scp, 1, 0, None, 0, None, None) == -1
    assert "null pointer" in _lib.last_error()
    assert L.adana_mta_step(ctypes.byref(pl), scp, 1, 0x100, None, 0, None, None) == -1
    assert "variant flags" in _lib.last_error()
    assert L.adana_mta_step(ctypes.byref(pl), scp, 1, _lib.FOREACH | _lib.VARIANT_MANAU, None, 0, None, None) == -1
    assert "ADANA_FOREACH excludes" in _lib.last_error()
    fake = ctypes.c_void_p(0x1000)
    pl = _lib.Plan(desc=0x1000, vstart=0x1000, chunk_first=0x1000, fold_first=0x1000,
                   n_tensors=3, n_chunks=1, n_folds=3)
    assert L.adana_mta_step(ctypes.byref(pl), scp, 1, 0, fake, 1 << 20, fake, None) == -1
    assert "null pointer" in _lib.last_error()                   # no gradient pointer array
    pl.grad = 0x1000
    assert L.adana_mta_step(ctypes.byref(pl), scp, 0, 0, fake, 1 << 20, fake, None) == -1
    assert "n_classes" in _lib.last_error()
    assert L.adana_mta_step(ctypes.byref(pl), scp, 1, 0, fake, 16, fake, None) == -1
    assert "workspace" in _lib.last_error()
    assert L.adana_mta_step(ctypes.byref(_lib.Plan()), None, 0, 0, None, 0, None, None) == 0
    assert L.adana_plan_index(None, 0, 0, None, None) == 0
    assert L.adana_plan_index(None, 3, 5, None, None) == -1


def test_mta_step_noalloc_rejects_bad_arguments():
    """The allocation-free step checks its arguments, and refuses a list
    whose scratch would not fit the static array, before any device call."""
    from adana_amd import _lib

    L = _lib.lib()
    sc = (_lib.StepScalars * 1)()
    scp = ctypes.cast(sc, ctypes.c_void_p)
    assert L.adana_mta_step_noalloc(None, scp, 1, 0, None, None) == -1
    assert "null plan" in _lib.last_error()
    pl = _lib.Plan(n_tensors=3, n_chunks=1, n_folds=3)
    assert L.adana_mta_step_noalloc(ctypes.byref(pl), scp, 1, 0, None, None) == -1
    assert "null pointer" in _lib.last_error()
    pl = _lib.Plan(desc=0x1000, vstart=0x1000, chunk_first=0x1000, fold_first=0x1000, n_tensors=3,
                   n_chunks=_lib.NOALLOC_SCRATCH_BYTES // 16, n_folds=0)
    assert L.adana_mta_step_noalloc(ctypes.byref(pl), scp, 1, 0, ctypes.c_void_p(0x1000), None) == -3
    assert "static" in _lib.last_error()
    assert L.adana_mta_step_noalloc(ctypes.byref(_lib.Plan()), None, 0, 0, None, None) == 0


# --------------------------------------------------------------------------
# Python interface parity with the reference classes
# --------------------------------------------------------------------------

REF_ADANA_SIG = ["params", "lr", "delta", "kappa", "epsilon", "weight_decay", "clipsnr",
                 "wd_decaying", "wd_ts", "gamma_3_factor", "use_foreach"]     # adana.py:32-45
REF_ADANA_DEFAULTS = dict(lr=1.0, delta=8.0, kappa=1.0, epsilon=1e-8, weight_decay=0.0,
                          clipsnr=None, wd_decaying=False, wd_ts=1.0, gamma_3_factor=1.0,
                          use_foreach=False)
REF_STAR_SIG = ["params", "lr", "delta", "kappa", "mk4A", "mk4B", "epsilon", "weight_decay",
                "clipsnr", "weight_time", "wd_decaying", "wd_ts", "gamma_3_factor",
                "use_foreach"]                                                 # dana_star_mk4.py:10-26
REF_STAR_DEFAULTS = dict(lr=1.0, delta=8.0, kappa=1.0, mk4A=0.0, mk4B=0.0, epsilon=1e-8,
                         weight_decay=0.0, clipsnr=1.0, weight_time=False, wd_decaying=False,
                         wd_ts=1.0, gamma_3_factor=1.0, use_foreach=False)


@pytest.mark.parametrize("which", ["ADana", "DANA_STAR_MK4"])
def test_constructor_matches_reference(which):
    import adana_amd

    cls = getattr(adana_amd, which)
    sig = inspect.signature(cls.__init__)
    positional = [n for n, p in sig.parameters.items()
                  if n != "self" and p.kind == p.POSITIONAL_OR_KEYWORD]
    ref_sig, ref_def = ((REF_ADANA_SIG, REF_ADANA_DEFAULTS) if which == "ADana"
                        else (REF_STAR_SIG, REF_STAR_DEFAULTS))
    assert positional == ref_sig
    for k, v in ref_def.items():
        assert sig.parameters[k].default == v, k
    p = torch.nn.Parameter(torch.zeros(3))
    opt = cls([p], lr=0.01, delta=6.0, epsilon=1e-7, weight_decay=0.2)
    assert set(opt.param_groups[0]) == {"params", "lr", "delta", "epsilon", "weight_decay",
                                        "weighted_step_count"}
    assert opt.param_groups[0]["weighted_step_count"] == 0
    for attr in ("lr", "delta", "kappa", "epsilon", "weight_decay", "clipsnr", "wd_decaying",
                 "wd_ts", "gamma_3_factor", "use_foreach"):
        assert hasattr(opt, attr)


def test_star_asserts_like_reference():
    import adana_amd

    p = torch.nn.Parameter(torch.zeros(3))
    for kw in (dict(mk4A=0.1), dict(mk4B=1.0), dict(weight_time=True)):
        with pytest.raises(AssertionError):
            adana_amd.DANA_STAR_MK4([p], **kw)


def test_cpu_parameters_fail_loudly():
    """No silent CPU fallback: a step on CPU tensors raises."""
    import adana_amd

    p = torch.nn.Parameter(torch.ones(8))
    p.grad = torch.ones(8)
    opt = adana_amd.ADana([p], lr=1e-3)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()


def test_grad_none_is_skipped_without_state():
    import adana_amd

    p = torch.nn.Parameter(torch.ones(8))
    opt = adana_amd.DANA_STAR_MK4([p], lr=1e-3)
    opt.step()
    assert len(opt.state[p]) == 0
    assert opt.param_groups[0]["weighted_step_count"] == 1.0


def test_hoststep_advance_if_same():
    """The C steady-state walk: advances every state's step only when every
    p.grad is the very object recorded at the last step (None included)."""
    from adana_amd import _hoststep

    class P:
        def __init__(self, g):
            self.grad = g

    g1, g2 = object(), object()
    params = [P(g1), P(None), P(g2)]
    states = [{"step": 3}, {"step": 7}]
    assert _hoststep.advance_if_same(params, [g1, None, g2], states) is True
    assert [s["step"] for s in states] == [4, 8]
    params[2].grad = object()                                  # a new gradient object
    assert _hoststep.advance_if_same(params, [g1, None, g2], states) is False
    assert [s["step"] for s in states] == [4, 8]               # untouched
    params[2].grad = g2
    params[1].grad = g1                                        # None -> tensor
    assert _hoststep.advance_if_same(params, [g1, None, g2], states) is False
    assert _hoststep.advance_if_same(params, [g1, g1], states) is False   # length mismatch
    with pytest.raises(KeyError):
        _hoststep.advance_if_same([], [], [{"m": 1}])


def test_hoststep_on_torch_tensors():
    """The same walk on real parameters (read through torch's C++ tensors):
    identity of the gradient tensor, not equality of its values or address;
    tensor subclasses take the generic attribute path.  Step counts stay
    exact and keep their type; bump_versions moves each autograd version
    counter by one, as torch._C._increment_version does."""
    from adana_amd import _hoststep

    class Sub(torch.Tensor):
        pass

    ps = [torch.nn.Parameter(torch.zeros(3)), torch.zeros(4, requires_grad=True), torch.nn.Parameter(torch.zeros(2)),
          torch.zeros(5).as_subclass(Sub).requires_grad_()]
    for p in ps[:2] + ps[3:]:
        p.grad = torch.ones_like(p)
    gs = [p.grad for p in ps]
    assert gs[2] is None and type(gs[3]) is Sub
    states = [{"step": 10 ** 30}, {"step": int("1000")}, {"step": int("1000")}, {"step": 2.5}]
    assert _hoststep.advance_if_same(ps, gs, states) is True
    assert [s["step"] for s in states] == [10 ** 30 + 1, 1001, 1001, 3.5]
    assert type(states[3]["step"]) is float and states[1]["step"] is states[2]["step"]
    ps[0].grad = ps[0].grad.detach()                           # same storage, new tensor
    assert _hoststep.advance_if_same(ps, gs, states) is False
    assert [s["step"] for s in states] == [10 ** 30 + 1, 1001, 1001, 3.5]
    ps[0].grad = gs[0]
    gs[1].add_(1.0)                                            # in place: still the same tensor
    assert _hoststep.advance_if_same(ps, gs, states) is True
    ps[2].grad = torch.zeros(2)                                # None -> tensor
    assert _hoststep.advance_if_same(ps, gs, states) is False
    ps[2].grad = None
    ps[3].grad = torch.ones(5).as_subclass(Sub)               # subclass: generic path sees it
    assert _hoststep.advance_if_same(ps, gs, states) is False
    ps[3].grad = gs[3]
    assert _hoststep.advance_if_same(ps, gs, states) is True
    with pytest.raises(TypeError):
        _hoststep.advance_if_same(ps[:1], gs[:1], [[1]])

    before = [p._version for p in ps]
    _hoststep.bump_versions(ps)
    assert [p._version for p in ps] == [v + 1 for v in before]
    with pytest.raises(TypeError):
        _hoststep.bump_versions([ps[0], 3])
    assert [p._version for p in ps] == [v + 1 for v in before]   # checked before any bump
    with torch.inference_mode():
        t = torch.zeros(2)
    with pytest.raises(RuntimeError, match="inference"):
        _hoststep.bump_versions([t])


def test_stream_probe_library_rejects_bad_arguments():
    """bench.py's stream-rate probes (probes/libadana_probe.so) load and
    refuse malformed launches before touching a device."""
    import ctypes
    import os

    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "probes",
                        "libadana_probe.so")
    lib = ctypes.CDLL(path)
    fn = lib.adana_probe_stream_5r4w
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    five = (ctypes.c_void_p * 5)(*([0x1000] * 5))
    part = 0x9000
    assert fn(None, 1024, part, 4, None) == -1            # no array table
    assert fn(five, 1024, None, 4, None) == -1            # no partials
    assert fn(five, 1000, part, 4, None) == -1            # not a multiple of 1024
    assert fn(five, 0, part, 4, None) == -1               # empty
    assert fn(five, 1024, part, -1, None) == -1           # negative cap
    holes = (ctypes.c_void_p * 5)(0x1000, 0x1000, 0, 0x1000, 0x1000)
    assert fn(holes, 1024, part, 4, None) == -1           # null array
    odd = (ctypes.c_void_p * 5)(0x1000, 0x1004, 0x1000, 0x1000, 0x1000)
    assert fn(odd, 1024, part, 4, None) == -1             # misaligned array
    for name in ("adana_probe_stream_5r0w", "adana_probe_stream_0r4w"):
        f = getattr(lib, name)
        f.argtypes = fn.argtypes
        f.restype = ctypes.c_int
        assert f(odd, 1024, part, 4, None) == -1
        assert f(five, 1000, part, 4, None) == -1
    f4 = lib.adana_probe_stream_4r3w
    f4.argtypes = fn.argtypes
    f4.restype = ctypes.c_int
    assert f4(odd, 1024, part, 4, None) == -1             # misaligned array
    assert f4(five, 1000, part, 4, None) == -1            # not a multiple of 1024
    assert f4(None, 1024, part, 4, None) == -1            # no array table
    cp = lib.adana_probe_copy
    cp.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    cp.restype = ctypes.c_int
    assert cp(0x1000, 0x1000, 1024, part, 0, None) == -1  # same array
    assert cp(0x1000, 0x2000, 1000, part, 0, None) == -1  # not a multiple of 1024
    assert cp(0, 0x2000, 1024, part, 0, None) == -1       # null
    assert cp(0x1000, 0x2000, 1024, None, 0, None) == -1  # no partials
    ms = lib.adana_probe_stream_master
    ms.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    ms.restype = ctypes.c_int
    a, g, mm, v, p16 = 0x1000, 0x2000, 0x3000, 0x4000, 0x5000
    assert ms(a, g, mm, v, p16, 1000, part, 4, None) == -1     # not a multiple of 1024
    assert ms(a, None, mm, v, p16, 1024, part, 4, None) == -1   # null gradient
    assert ms(a + 8, g, mm, v, p16, 1024, part, 4, None) == -1  # fp32 array not 16-byte aligned
    assert ms(a, g + 4, mm, v, p16, 1024, part, 4, None) == -1  # bf16 array not 8-byte aligned
    assert ms(a, g, mm, v, p16, 1024, None, 4, None) == -1      # no partials
    assert ms(a, g, mm, v, p16, 1024, part, -1, None) == -1     # negative cap


def test_flat_params_follow_the_groups():
    """The cached parameter list is checked object for object against the
    groups: a parameter replaced inside a group's list (same list, same
    length) and an added group are both picked up, as the reference's step,
    which re-reads group['params'] every time, would see them."""
    import adana_amd
    from adana_amd import _hoststep

    a, b, c = (torch.nn.Parameter(torch.zeros(3)) for _ in range(3))
    opt = adana_amd.ADana([a, b], lr=1e-3)
    flat, gidx = opt._flat_params()
    assert flat == [a, b] and gidx == [0, 0]
    assert _hoststep.same_params(opt.param_groups, flat)
    opt.param_groups[0]["params"][1] = c                     # in place
    assert not _hoststep.same_params(opt.param_groups, flat)
    flat, _ = opt._flat_params()
    assert flat[1] is c
    d = torch.nn.Parameter(torch.zeros(2))
    opt.add_param_group({"params": [d], "weight_decay": 0.1})
    flat, gidx = opt._flat_params()
    assert flat == [a, c, d] and gidx == [0, 0, 1]
    assert not _hoststep.same_params(opt.param_groups, [a, c])            # shorter cache
    assert not _hoststep.same_params(opt.param_groups, [a, c, d, d])      # longer cache
    with pytest.raises(KeyError):
        _hoststep.same_params([{"lr": 1.0}], [])


def test_hoststep_grads_ptrs_and_steps():
    """grads_of is [p.grad for p in params] plus the None pattern; data_ptrs
    gives each data_ptr() (0 for None); advance_steps increments every
    counter; advance_if_same with parameter pointers refuses a parameter
    whose storage was rebound (p.data = ...)."""
    from adana_amd import _hoststep

    class Sub(torch.Tensor):
        pass

    ps = [torch.nn.Parameter(torch.zeros(3)), torch.nn.Parameter(torch.zeros(2)),
          torch.zeros(4).as_subclass(Sub).requires_grad_()]
    ps[0].grad = torch.ones(3)
    ps[2].grad = torch.ones(4).as_subclass(Sub)
    grads, absent = _hoststep.grads_of(ps)
    assert grads[0] is ps[0].grad and grads[1] is None and grads[2] is ps[2].grad
    assert absent == bytes([0, 1, 0])
    ptrs = np.frombuffer(_hoststep.data_ptrs([ps[0], None, ps[2].grad]), dtype=np.uint64)
    assert ptrs.tolist() == [ps[0].data_ptr(), 0, ps[2].grad.data_ptr()]
    with pytest.raises(AttributeError):                       # not a tensor: no data_ptr()
        _hoststep.data_ptrs(["x"])
    states = [{"step": 1}, {"step": 1}]
    _hoststep.advance_steps(states)
    assert [s["step"] for s in states] == [2, 2]
    pp = _hoststep.data_ptrs(ps)
    assert _hoststep.advance_if_same(ps, grads, states, pp) is True
    assert [s["step"] for s in states] == [3, 3]
    ps[1].data = torch.zeros(2)                                 # storage rebound
    assert _hoststep.advance_if_same(ps, grads, states, pp) is False
    assert [s["step"] for s in states] == [3, 3]
    assert _hoststep.advance_if_same(ps, grads, states, _hoststep.data_ptrs(ps)) is True
    assert _hoststep.advance_if_same(ps, grads, states, b"short") is False
    pp, gp = _hoststep.data_ptrs(ps), _hoststep.data_ptrs(grads)
    assert _hoststep.advance_if_same(ps, grads, states, pp, gp) is True
    grads[0].set_(torch.ones(3))                                # same object, new storage
    assert _hoststep.advance_if_same(ps, grads, states, pp, gp) is False
    assert _hoststep.advance_if_same(ps, grads, states, pp, _hoststep.data_ptrs(grads)) is True


def test_hoststep_grads_match():
    """grads_match accepts dense contiguous gradients of each parameter's
    shape and the expected dtype, and refuses anything else (the optimizer
    then checks pair by pair and raises the precise error)."""
    from adana_amd import _hoststep

    ps = [torch.nn.Parameter(torch.zeros(4, 3)), torch.nn.Parameter(torch.zeros(5))]
    good = [torch.zeros(4, 3), torch.zeros(5)]
    assert _hoststep.grads_match(ps, good, False) is True
    assert _hoststep.grads_match(ps, good, True) is False                       # dtype
    assert _hoststep.grads_match(ps, [torch.zeros(3, 4), good[1]], False) is False   # shape
    assert _hoststep.grads_match(ps, [torch.zeros(3, 4).t(), good[1]], False) is False  # not contiguous
    assert _hoststep.grads_match(ps, [good[0], torch.zeros(5, dtype=torch.float64)], False) is False
    assert _hoststep.grads_match(ps, [good[0], torch.zeros(5).to_sparse()], False) is False
    assert _hoststep.grads_match(ps, [good[0], None], False) is False
    assert _hoststep.grads_match(ps, good[:1], False) is False                   # length
    b = [torch.nn.Parameter(torch.zeros(4, dtype=torch.bfloat16))]
    assert _hoststep.grads_match(b, [torch.zeros(4, dtype=torch.bfloat16)], True) is True


def test_missing_library_fails_loudly(monkeypatch):
    """Without the built HIP library there is no step at all: loading it, and
    constructing an optimizer, raise AdanaLibraryError naming the build
    command (no CPU or eager fallback exists)."""
    import adana_amd
    from adana_amd import _lib

    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libadana_mta.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(_lib.AdanaLibraryError, match="is not built"):
        _lib.lib()
    with pytest.raises(_lib.AdanaLibraryError, match="no non-HIP path"):
        adana_amd.DANA_STAR_MK4([torch.nn.Parameter(torch.zeros(3))], lr=1e-3)


def test_rebound_parameter_of_another_shape_raises():
    """A parameter whose storage is rebound to another shape (``p.data = x``)
    no longer fits its laid-out state: the plan check raises before any
    launch, as the reference's ``m.lerp_(grad, alpha)`` would
    (src/optim/adana.py:101).  The check runs on host tensors only."""
    import adana_amd
    from adana_amd.optim import _LaunchSet

    for cls in (adana_amd.ADana, adana_amd.DANA_STAR_MK4):
        ps = [torch.nn.Parameter(torch.zeros(6)), torch.nn.Parameter(torch.zeros(2, 3))]
        opt = cls(ps, lr=1e-3)
        ls = _LaunchSet(torch.device("cpu"), 0, 0)
        ls.params = ps
        ls.states = [{"m": torch.zeros(6), "v": torch.zeros(6), "tau": torch.zeros(6)},
                     {"m": torch.zeros(2, 3), "v": torch.zeros(2, 3), "tau": torch.zeros(2, 3)}]
        opt._check_state_shapes(ls)                       # shapes agree: no error
        ps[1].data = torch.zeros(3, 2).t()
        opt._check_state_shapes(ls)                       # another layout of the shape: staged
        ps[1].data = torch.zeros(1, 3).expand(2, 3)
        with pytest.raises(NotImplementedError, match="share memory"):
            opt._check_state_shapes(ls)
        ps[1].data = torch.zeros(3, 3)
        with pytest.raises(RuntimeError, match="must match the size"):
            opt._check_state_shapes(ls)


def test_staging_decisions():
    """The descriptor rows of a launch set point at the state's layout: a
    parameter or gradient whose strides differ from its state's is given a
    staging buffer of the state's shape, strides and its own dtype, kept
    (same address) while it still fits; tensors of the state's layout are
    used in place.  Host tensors only (no launch)."""
    import adana_amd
    from adana_amd.optim import _LaunchSet

    big = torch.zeros(12, 40)
    ps = [torch.nn.Parameter(big[:, 5:21]), torch.nn.Parameter(torch.zeros(9, 7).t()),
          torch.nn.Parameter(torch.zeros(50))]
    opt = adana_amd.ADana(ps, lr=1e-3)
    ls = _LaunchSet(torch.device("cpu"), 0, 0)
    ls.params = ps
    ls.states = [{"m": torch.zeros_like(p), "v": torch.zeros_like(p)} for p in ps]
    ls.sclass = [0, 0, 0]
    assert ls.states[0]["m"].is_contiguous() and ls.states[1]["m"].stride() == ps[1].stride()
    ls.grads = [torch.zeros(16, 12).t(), torch.zeros(7, 9), torch.zeros(50)]
    d = opt._desc_rows(ls)
    assert [j for j, _, _ in ls.stage] == [0, 1]
    (_, p0, g0), (_, p1, g1) = ls.stage
    assert p0.is_contiguous() and p0.shape == ps[0].shape and g0.is_contiguous()   # gapped p, transposed g
    assert p1 is None and g1.stride() == ps[1].stride()                            # contiguous g of a permuted p
    g = ls.host_grad                                                               # adana_plan.grad
    assert int(d["param"][0]) == p0.data_ptr() and int(g[0]) == g0.data_ptr()
    assert int(d["param"][1]) == ps[1].data_ptr() and int(g[1]) == g1.data_ptr()
    assert int(d["param"][2]) == ps[2].data_ptr() and int(g[2]) == ls.grads[2].data_ptr()
    assert int(d["reserved0"].max()) == 0
    ls.grads = [torch.zeros(12, 16), torch.zeros(9, 7).t(), torch.zeros(50)]
    opt._desc_rows(ls)
    assert [(j, ps_ is not None, gs is not None) for j, ps_, gs in ls.stage] == [(0, True, False)]
    assert ls.stage[0][1] is p0                                                    # the same buffer


def test_dense_layouts():
    """The layouts the element-wise step runs over in storage order:
    contiguous and permuted tensors, empty tensors of any strides; not
    gapped or overlapping ones."""
    from adana_amd._layout import dense_layout, same_layout

    a = torch.zeros(3, 4)
    assert dense_layout(a) and dense_layout(a.t()) and dense_layout(torch.zeros(2, 3, 4).permute(2, 0, 1))
    assert dense_layout(torch.from_numpy(np.zeros((0,), np.float32)))          # stride 0, no elements
    assert dense_layout(torch.zeros(5, 1, 3)[:, :, :])
    assert not dense_layout(a[:, :2]) and not dense_layout(a.expand(2, 3, 4)) and not dense_layout(a[::2])
    from adana_amd._layout import no_overlap
    assert no_overlap(a) and no_overlap(a.t()) and no_overlap(a[:, :2]) and no_overlap(a[::2])
    assert no_overlap(torch.zeros(20, 30).t()[2:17]) and no_overlap(torch.zeros(3, 1, 4)[:, :, ::3])
    assert not no_overlap(a.expand(2, 3, 4)) and not no_overlap(torch.zeros(4).as_strided((3, 2), (1, 1)))
    assert same_layout(a.t(), torch.ones(3, 4).t())
    assert not same_layout(a.t(), a.t().contiguous())
    assert same_layout(torch.zeros(3, 1), torch.zeros(1, 3).t())               # size-1 dims' strides ignored


def test_deepcopy_and_pickle_keep_the_configuration():
    """torch.optim.Optimizer pickles only defaults, state and param_groups;
    the constructor's instance attributes (self.lr, self.kappa, ...)
    travel too, so a deepcopy or an unpickled optimizer can step, and its
    engine caches start empty.  Host tensors only (no step)."""
    import copy
    import pickle

    import adana_amd

    for cls, kw in ((adana_amd.ADana, dict(kappa=0.7, clipsnr=2.0)),
                    (adana_amd.DANA_STAR_MK4, dict(kappa=0.6, clipsnr=3.0, wd_ts=5.0))):
        opt = cls([torch.nn.Parameter(torch.zeros(3))], lr=2e-3, fresh_diagnostics=False, **kw)
        for other in (copy.deepcopy(opt), pickle.loads(pickle.dumps(opt))):
            for k, v in vars(opt).items():
                if not k.startswith("_"):
                    assert k in vars(other), (cls.__name__, k)
                    if k not in ("state", "param_groups", "defaults"):   # torch's __setstate__ adds to defaults
                        assert getattr(other, k) == v, (cls.__name__, k)
            assert other._sets is None and other._fast is False and other._diag_loc == {}
            assert other.param_groups[0]["params"][0] is not opt.param_groups[0]["params"][0]


def test_bind_diag_entries():
    """_hoststep.bind_diag binds states[j][key] to a 0-d tensor over element
    5 * j + col of the buffer, each with a 4-byte storage of its own that
    keeps the buffer alive; a column outside [0, 5), a buffer shorter than 5
    per state, and non-dict states are refused."""
    from adana_amd import _hoststep

    buf = torch.arange(10, dtype=torch.float32)
    states = [{}, {}]
    _hoststep.bind_diag(buf, states, [(0, "a"), (4, "e")])
    assert [float(s[k]) for s in states for k in ("a", "e")] == [0.0, 4.0, 5.0, 9.0]
    t = states[1]["e"]
    assert t.dim() == 0 and t.untyped_storage().nbytes() == 4 and t.data_ptr() == buf.data_ptr() + 4 * 9
    buf[9] = 42.0
    del buf
    assert float(t) == 42.0
    with pytest.raises(ValueError, match="column"):
        _hoststep.bind_diag(torch.zeros(10), [{}, {}], [(5, "x")])
    with pytest.raises(ValueError, match="too small"):
        _hoststep.bind_diag(torch.zeros(9), [{}, {}], [(0, "x")])
    with pytest.raises(TypeError, match="dicts"):
        _hoststep.bind_diag(torch.zeros(10), [{}, 3], [(0, "x")])


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
def test_scalar_fill_in_place(numerics):
    """The launch fills its scalar classes in place (adana_step_scalars_init
    into the set's array, hyper-parameters cached per group and rebuilt when
    one changes): the same bits as the one-off scalars, per class, for the
    group's current lr and the class's step.  Host only (no launch)."""
    import adana_amd
    from adana_amd import _lib
    from adana_amd.optim import _LaunchSet

    ps = [torch.nn.Parameter(torch.zeros(4)) for _ in range(3)]
    opt = adana_amd.DANA_STAR_MK4([{"params": ps[:2]}, {"params": ps[2:], "weight_decay": 0.3, "lr": 2e-3}],
                                  lr=1e-3, kappa=0.85, wd_decaying=True, wd_ts=7.0, numerics=numerics)
    ls = _LaunchSet(torch.device("cpu"), 0, 0)
    ls.sc_arr = (_lib.StepScalars * _lib.MAX_CLASSES)()
    classes = [(0, 3), (1, 3), (0, 5)]
    for wd in (0.3, 0.5):                       # a changed group value reaches the scalars
        opt.param_groups[1]["weight_decay"] = wd
        assert opt._fill_scalars(ls, classes) == 3
        for k, (gi, t) in enumerate(classes):
            want = _lib.step_scalars(opt._hparams(opt.param_groups[gi]), opt.param_groups[gi]["lr"], t)
            assert bytes(ls.sc_arr[k]) == bytes(want), (wd, k)


def test_foreach_builds_on_every_state_kind():
    """use_foreach=True builds with either numerics on float32, bfloat16 and
    master-weight parameters, and the choice is the constructor's (it
    travels with a deep copy)."""
    import copy

    import adana_amd

    for dt, master in ((torch.float32, False), (torch.bfloat16, False), (torch.bfloat16, True)):
        for numerics in ("compiled", "eager"):
            p = torch.nn.Parameter(torch.zeros(16, dtype=dt))
            opt = adana_amd.DANA_STAR_MK4([p], lr=1e-3, use_foreach=True, numerics=numerics, master_weights=master)
            assert opt._foreach and opt.use_foreach
            assert copy.deepcopy(opt)._foreach
    assert not adana_amd.ADana([torch.nn.Parameter(torch.zeros(4))], lr=1e-3)._foreach
