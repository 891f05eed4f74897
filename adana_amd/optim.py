"""Drop-in ``ADana`` and ``DANA_STAR_MK4`` whose ``step()`` runs one HIP kernel.

Reference: mlexpos/adana ``src/optim/adana.py`` (ADana: ``clipsnr=None`` is
ADana, a float is Dana-MK4) and ``src/optim/dana_star_mk4.py`` (Dana-Star /
Dana-Star-MK4).  Constructor arguments, defaults, ``param_groups`` keys,
instance attributes and per-parameter state keys are the reference's:

    state[p] = {'step': int, 'm': T, 'v': T, ['tau': T,]
                'current_alpha', 'gradient_norm', 'auto_factor_mean',
                'current_kappa_factor', 'm_norm'}        (0-d tensors of p's dtype)

T has p's shape, dtype and, as zeros_like gives them, strides: p's own for a
contiguous or permuted p, contiguous for a p with gaps (a slice such as
``w[:, :k]``).  The kernel pairs elements by their offset in the state's
layout; a parameter or gradient of another layout is copied into a staging
buffer of that layout before the launch and (the parameter) back after it,
on the same stream.  Since T has p's dtype, bfloat16 parameters keep
bfloat16 m, v and tau, as in the reference.

Numerics.  The reference always steps through torch.compile
(src/optim/adana.py:72-79, 210-216; src/optim/dana_star_mk4.py:88-96, 275),
and that is what the kernel reproduces by default (``numerics="compiled"``):
Inductor's forms of lerp_ and addcmul_ (every product and sum rounded on its
own), binary32 arithmetic throughout, and for bfloat16 state a rounding to
bfloat16 only where m, v, tau and p are stored.  ``numerics="eager"``
(keyword-only, an extension) reproduces the same update run as ATen eager
ops instead: lerp_ and addcmul_ as single-rounded fused multiply-adds and, on
bfloat16 state, every op rounded to bfloat16.

``use_foreach=True`` (the reference's constructor argument) selects the
reference's foreach path (src/optim/adana.py:229-370,
src/optim/dana_star_mk4.py:298-536), whose kernel its constructor compiles:
the same update in other op forms (no addcmul, ATen's lerp, tau_reg as a
maximum, mfac = nt * (|m| / tau_reg), g2 and g3 scaled last, weight decay as
p + p * wdf) with its own scalars (alpha as a binary32 quotient, the step in
the parameters' dtype).  The step is still one launch.  As in the
reference, the choice is made at construction; ``numerics="eager"`` with it
is the same path's kernel run as eager ops.

What differs is how a step executes.  The reference loops over tensors in
Python, makes six 0-d device tensors per tensor and calls a torch.compile'd
update per tensor (src/optim/adana.py:184-225).  Here the host computes the
per-step scalars once per (group, step) class in C, and a single
multi-tensor HIP kernel (adana_amd/csrc/adana_mta.hip) updates every tensor
and writes all diagnostics into one device buffer.  The per-tensor host work
(gradient checks and pointers, step counters, version counters) is one C++
pass (adana_amd/_hoststep.StepTable); only gradient pointers that moved since
the last step are uploaded.

Diagnostics.  The reference binds five new 0-d tensors per parameter every
step (adana.py:221-225), so a diagnostic kept from one step keeps its value.
Here every step writes into the same buffer, over which the state entries
are bound; before a step rewrites it, any entry something else still refers
to (a Python reference, a view, a detach()) is moved to a copy of its own
and the state gets a new tensor.  The check reads each entry's reference
counts, in the same C++ pass as the gradient checks (helper threads on long
lists: 0.03-0.09 ms for 10,000 tensors).  ``fresh_diagnostics=False``
(keyword-only, an extension) turns it off: every entry is then refreshed in
place, and a kept diagnostic follows the buffer.

Gradient clipping (src/optim/base.py:250-257): ``opt.clip_grad_norm_(max_norm)``
(or ``adana_amd.clip_grad_norm_(params, max_norm, optimizer=opt)``) returns
torch.nn.utils.clip_grad_norm_'s total norm and folds the in-place scaling
into the next ``step()`` (adana_amd/clip.py).

Extension (no reference counterpart): ``master_weights=True`` lets bfloat16
parameters keep a float32 master copy (state key ``'master'``) with float32
m/v[/tau] instead; the update runs in float32 on the master and the bf16
parameter is written as RNE(master) in the same pass.
"""
from __future__ import annotations

import ctypes
import operator
import weakref
from typing import Iterable, List, Optional

import numpy as np
import torch
from torch.optim import Optimizer
from torch.optim import optimizer as _torch_optimizer

from . import _hoststep, _lib
from ._layout import dense_layout, no_overlap, same_layout
from .clip import GradPlan, clip_grad_norm_ as _clip_grad_norm

DIAG_KEYS = ("current_alpha", "gradient_norm", "auto_factor_mean",
             "current_kappa_factor", "m_norm")
_GRAD = operator.attrgetter("grad")
_DATA_PTR = torch.Tensor.data_ptr


class _SlabRef:
    """Keeps a slab alive and exposes one region of it to torch.as_tensor."""

    __slots__ = ("buf", "__cuda_array_interface__")


_SLAB_ALIGN = 1024      # elements (4 KB): every state tensor starts a fresh work chunk
_CANARY32 = 0x7FA5A5A5  # a float32 NaN bit pattern around each state slab's tensors
_CANARY16 = 0x7FA5      # the bfloat16 one


def _carve(buf: torch.Tensor, off: int, shape, strides=None) -> torch.Tensor:
    """A tensor of ``shape`` (and element ``strides``; None: contiguous) and
    ``buf``'s dtype (float32 or bfloat16) over ``buf[off:]`` with a storage of
    its own (deepcopy, torch.save and the like see only its bytes); the slab
    lives as long as any tensor carved from it.  bfloat16 has no
    array-interface type code: it is carved as int16 and viewed as bfloat16
    (a view of that private storage)."""
    ref = _SlabRef()
    ref.buf = buf
    bf16 = buf.dtype == torch.bfloat16
    es = buf.element_size()
    ref.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": "<i2" if bf16 else "<f4",
                                    "data": (buf.data_ptr() + es * off, False), "version": 3,
                                    "strides": None if strides is None else tuple(es * x for x in strides)}
    t = torch.as_tensor(ref, device=buf.device)
    return t.view(torch.bfloat16) if bf16 else t


class _LaunchSet:
    """Tensors sharing one kernel instantiation, one device and <= MAX_CLASSES
    scalar classes: one adana_mta_step call per step."""

    def __init__(self, device, flags, class_base):
        self.device = device
        self.flags = flags
        self.class_base = class_base
        self.index: List[int] = []       # positions in the step's (param, grad) list
        self.params: List[torch.Tensor] = []
        self.grads: List[torch.Tensor] = []
        self.states: List[dict] = []
        self.sclass: List[int] = []
        self.host_desc = None
        self.host_grad = None       # numpy uint64: the gradient pointers the device array holds
        self.vstart = None
        self.fold_first = None
        self.n_chunks = 0
        self.n_folds = 0
        self.dev_table = None       # [descriptors | vstart | fold_first]
        self.dev_grad = None        # int64 device array: adana_plan.grad
        self.chunk_first = None
        self.workspace = None
        self.plan = None
        self.diag = None
        self.table = None           # _hoststep.StepTable over the rows (diagnostics; the fast scan)
        self.grad_addr = 0          # host_grad's address (StepTable.scan writes there)
        self.sc_arr = None          # the launch's scalar classes, filled in place every step
        self.args = None            # the launch's constant ctypes arguments
        self.ptr_key = None         # the parameters' data pointers the tables hold
        self.stage = []             # (row, param staging or None, grad staging or None)
        self.stage_bufs = {}        # (row, "p" | "g") -> staging tensor, kept while it fits


class _DanaFamily(Optimizer):
    """Shared engine of ADana and DANA_STAR_MK4 (one code path for both)."""

    _STAR = False
    _VARIANT = 0                                   # adana_mta_step variant flags
    _KEYS = ("m", "v", "tau")                      # state keys of the moments and tau
    _DIAG_COLUMNS = tuple(enumerate(DIAG_KEYS))    # (kernel output column, state key)

    def _engine_init(self, master_weights: bool, fresh_diagnostics: Optional[bool] = None,
                     numerics: str = "compiled") -> None:
        if numerics not in ("compiled", "eager"):
            raise ValueError(f"numerics must be 'compiled' or 'eager', got {numerics!r}")
        self.master_weights = bool(master_weights)
        self.fresh_diagnostics = fresh_diagnostics
        self.numerics = numerics
        # the reference picks its foreach kernel in the constructor (adana.py:63-70)
        self._foreach = bool(getattr(self, "use_foreach", False))
        self._diag_cols = [tuple(c) for c in self._DIAG_COLUMNS]
        self._sets: Optional[List[_LaunchSet]] = None
        self._structure = None
        self._flat = None
        self._fast = False          # one launch set, no staging: step() may take StepTable.scan
        self._classes = None
        self._hp_cache = {}
        self._pending_clip = None
        self._clip_plan_obj = None
        self._diag_loc = {}        # param -> (launch set, row) of its latest plan
        self._diag_epoch = 0       # bumped whenever a plan or the state tensors change
        self._diag_cache = None
        self._slab_guards = []     # (weakref to a state slab, family, base, total, [(offset, numel)])
        _lib.lib()  # fail at construction, not at the first step, without the kernel library

    # -- pickling and deepcopy --------------------------------------------
    # torch.optim.Optimizer pickles only defaults, state and param_groups, so
    # the constructor's instance attributes (self.lr, self.kappa, ...) would
    # be lost and the copy's first step() would fail.  They travel with the
    # rest; the device tables, launch sets and caches are rebuilt by the
    # copy's first step() (its state tensors are its own, not slab views).
    def __getstate__(self):
        # A clip deferred to the next step() must reach the copy too.  With
        # write_back it is applied to the gradients now, as torch's in-place
        # clipping would have left them.  Without write_back the caller's
        # gradients stay unscaled: the coefficient travels with the state and
        # the copy defers the same scaling on its own gradients.
        pend = self._pending_clip
        if pend is not None and pend[3]:
            self.flush_clip()
            pend = None
        state = super().__getstate__()
        state["_config"] = {k: v for k, v in vars(self).items() if not k.startswith("_") and k not in state}
        if pend is not None:
            state["_pending_clip_coef"] = pend[2]
        return state

    def __setstate__(self, state):
        config = state.pop("_config", None)
        coef = state.pop("_pending_clip_coef", None)
        super().__setstate__(state)
        if config is not None:
            self.__dict__.update(config)
            self._engine_init(self.master_weights, self.fresh_diagnostics, getattr(self, "numerics", "compiled"))
        if coef is not None:
            params, _ = self._flat_params()
            own = [g for g in map(_GRAD, params) if g is not None]
            if own:                  # (nn.Parameter's deepcopy drops .grad: nothing to scale then)
                plan = self._clip_plan(own[0].device, own[0].dtype == torch.bfloat16)
                plan.prepare(own)
                self._pending_clip = (own, plan, coef, False)

    # -- state ------------------------------------------------------------
    def _state_families(self, p: torch.Tensor):
        fams = list(self._KEYS[:3 if self._STAR else 2])
        if p.dtype == torch.bfloat16 and self.master_weights:
            fams.append("master")
        return fams

    def _state_dtype(self, p: torch.Tensor) -> torch.dtype:
        """dtype of p's m, v, tau: p's own, as zeros_like(p) gives it
        (src/optim/adana.py:193-194), except float32 in master-weights mode."""
        return torch.float32 if (p.dtype == torch.bfloat16 and self.master_weights) else p.dtype

    def _pack_states(self, items, source) -> None:
        """Allocate the state tensors of the (param, state) pairs ``items``:
        zero m, v[, tau] shaped like p (src/optim/adana.py:191-195;
        src/optim/dana_star_mk4.py:255), float32 (the bf16 extension's moments
        and its master copy, taken from p, too), or copies of ``source``
        (param -> old state).  On the GPU they are laid out family by family:
        all m tensors end to end in one slab, then all v, all tau, each tensor
        4 KB aligned and with a storage of its own (measured 2-3% faster steps
        than one allocation per tensor, interleaved m, v, tau)."""
        by_dev = {}
        for p, st in items:
            dense = (p.device.type == "cuda" and dense_layout(p) and p.dtype in (torch.float32, torch.bfloat16))
            if not dense:   # a layout with gaps (zeros_like(p) is contiguous), or not steppable here
                for fam in self._state_families(p):
                    old = source[p][fam] if source is not None else None
                    if old is not None:
                        st[fam] = old
                    elif fam == "master":
                        st[fam] = p.detach().to(torch.float32)
                    else:
                        st[fam] = torch.zeros_like(p, dtype=self._state_dtype(p))
                continue
            by_dev.setdefault(p.device, []).append((p, st))
        for dev, group in by_dev.items():
            fams = {}
            for p, st in group:
                for fam in self._state_families(p):
                    dt = torch.float32 if fam == "master" else self._state_dtype(p)
                    fams.setdefault((fam, dt), []).append((p, st))
            for (fam, dt), members in fams.items():
                offs, total = [], 0
                for p, _ in members:
                    offs.append(total)
                    total += (p.numel() + _SLAB_ALIGN - 1) // _SLAB_ALIGN * _SLAB_ALIGN
                # headroom so that the first tensor starts on a _SLAB_ALIGN-element boundary
                slab = torch.zeros(total + _SLAB_ALIGN, dtype=dt, device=dev)
                base = (-(slab.data_ptr() // slab.element_size())) % _SLAB_ALIGN
                # canaries before the first tensor and after the last (no kernel writes there)
                bits = slab.view(torch.int16 if dt == torch.bfloat16 else torch.int32)
                canary = _CANARY16 if dt == torch.bfloat16 else _CANARY32
                bits[:base].fill_(canary)
                bits[base + total:].fill_(canary)
                self._slab_guards.append((weakref.ref(slab), fam, base, total,
                                          [(off, p.numel()) for (p, _), off in zip(members, offs)]))
                for (p, st), off in zip(members, offs):
                    # zeros_like(p): p's shape and, for a transposed or permuted p, its strides
                    t = _carve(slab, base + off, p.shape, None if p.is_contiguous() else p.stride())
                    if source is not None:
                        t.copy_(source[p][fam])
                    elif fam == "master":
                        t.copy_(p.detach())
                    st[fam] = t

    def _check_slab_guards(self) -> int:
        """Check the elements of every live state slab that belong to no state
        tensor: the canaries before the first tensor and after the last still
        hold their bit pattern, and the padding between tensors is still zero.
        Returns the number of slabs checked; raises RuntimeError naming the
        first element that changed (a kernel wrote outside its tensors)."""
        checked = 0
        for ref, fam, base, total, members in self._slab_guards:
            slab = ref()
            if slab is None:
                continue
            bits = slab.view(torch.int16 if slab.dtype == torch.bfloat16 else torch.int32)
            canary = _CANARY16 if slab.dtype == torch.bfloat16 else _CANARY32
            spans = [(0, base, canary), (base + total, bits.numel(), canary)]
            ends = [off + n for off, n in members]
            starts = [off for off, _ in members[1:]] + [total]
            spans += [(base + e, base + s, 0) for e, s in zip(ends, starts) if s > e]
            for lo, hi, want in spans:
                if hi > lo:
                    bad = (bits[lo:hi] != want).nonzero()
                    if bad.numel():
                        raise RuntimeError(f"{type(self).__name__}: state slab {fam!r} element "
                                           f"{lo + int(bad[0])} outside every tensor was overwritten")
            checked += 1
        return checked

    def invalidate_plan(self) -> None:
        """Forget cached device tables and tensor lists (call after swapping a
        state tensor by hand; new gradients, rebound parameter storage and
        parameters replaced in a group's list are followed by step())."""
        self._sets = None
        self._structure = None
        self._flat = None
        self._fast = False
        self._diag_epoch += 1

    def load_state_dict(self, state_dict) -> None:
        """torch's load_state_dict (checkpoints of the reference optimizers load
        as they are: src/optim/utils.py:283-361 saves ``opt.state_dict()``).  In
        master-weights mode the moments of bf16 parameters are kept float32, and
        a checkpoint without a ``'master'`` entry (the reference keeps none)
        starts the master copy from the bf16 parameter."""
        super().load_state_dict(state_dict)
        if self.master_weights:
            # torch casts floating state to the parameter dtype on load; the
            # master copy and the moments of bf16 parameters stay float32.
            saved = state_dict["state"]
            order = [p for g in self.param_groups for p in g["params"]]
            saved_ids = [i for g in state_dict["param_groups"] for i in g["params"]]
            for pid, p in zip(saved_ids, order):
                if pid in saved and p.dtype == torch.bfloat16:
                    st = self.state[p]
                    for k in ("master", "m", "v", "tau"):
                        if k in saved[pid]:
                            st[k] = saved[pid][k].to(device=p.device, dtype=torch.float32)
                    if "m" in st and "master" not in st:
                        st["master"] = p.detach().to(torch.float32)
        # lay the loaded moments out in slabs, as a fresh run has them
        items, source = [], {}
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p) if p in self.state else None
                if st and all(k in st for k in self._state_families(p)):
                    source[p] = {k: st[k] for k in self._state_families(p)}
                    items.append((p, st))
        self._pack_states(items, source)
        self.invalidate_plan()

    # -- gradient clipping -------------------------------------------------
    def clip_grad_norm_(self, max_norm: float, norm_type: float = 2.0,
                        error_if_nonfinite: bool = False, foreach: Optional[bool] = None, *,
                        write_back: bool = True) -> torch.Tensor:
        """torch.nn.utils.clip_grad_norm_ over this optimizer's parameters, with
        the scaling fused into the next step() (adana_amd/clip.py)."""
        params, _ = self._flat_params()
        return _clip_grad_norm(params, max_norm, norm_type, error_if_nonfinite, foreach,
                               optimizer=self, write_back=write_back)

    def flush_clip(self) -> None:
        """Apply a pending clip scaling to the gradients now (in place)."""
        pend = self._pending_clip
        if pend is not None:
            self._pending_clip = None
            pend[1].scale(pend[2])

    def zero_grad(self, set_to_none: bool = True) -> None:
        self._pending_clip = None          # the clipped gradients are being discarded
        super().zero_grad(set_to_none=set_to_none)

    def _clip_plan(self, device, bf16: bool) -> GradPlan:
        plan = self._clip_plan_obj
        if plan is None or plan.device != device or plan.bf16 != bf16:
            plan = self._clip_plan_obj = GradPlan(device, bf16)
        return plan

    def _arm_clip(self, grads, plan, clip, write_back: bool) -> bool:
        """Defer clip scaling to the next step() if ``grads`` are exactly the
        gradients that step will consume; False leaves the scaling to the caller."""
        params, _ = self._flat_params()
        own = [g for g in map(_GRAD, params) if g is not None]
        if len(own) != len(grads):
            return False
        ids = set(map(id, grads))
        if not all(id(g) in ids for g in own):
            return False
        self._pending_clip = (own, plan, clip, bool(write_back))
        return True

    # -- plan -------------------------------------------------------------
    def _validate(self, p: torch.Tensor, g: torch.Tensor) -> int:
        """Return the kernel variant flags of one (param, grad) pair or raise."""
        if p.device.type != "cuda":
            raise RuntimeError(f"{type(self).__name__}: parameters must live on a ROCm GPU "
                               f"(got {p.device}); the step has no CPU path")
        if g.is_sparse:
            raise RuntimeError(f"{type(self).__name__} does not support sparse gradients")
        if g.device != p.device or g.shape != p.shape:
            raise RuntimeError(f"{type(self).__name__}: grad must match its parameter's "
                               f"device and shape ({g.device}/{tuple(g.shape)} vs "
                               f"{p.device}/{tuple(p.shape)})")
        if not no_overlap(p):
            # the reference's in-place ops on such a parameter raise (an
            # expanded one) or race; the update is written back element by element
            raise NotImplementedError(f"{type(self).__name__}: parameters whose elements may share memory "
                                      f"(strides {tuple(p.stride())}) are not supported")
        flags = (self._VARIANT | (_lib.NUMERICS_EAGER if self.numerics == "eager" else 0)
                 | (_lib.FOREACH if self._foreach else 0))
        if p.dtype == torch.float32:
            if g.dtype != torch.float32:
                raise RuntimeError(f"{type(self).__name__}: float32 parameter with {g.dtype} "
                                   "gradient (expected float32)")
        elif p.dtype == torch.bfloat16:
            if g.dtype != torch.bfloat16:
                raise RuntimeError(f"{type(self).__name__}: bfloat16 parameter with {g.dtype} "
                                   "gradient (expected bfloat16)")
            # master_weights: float32 master and moments (extension); otherwise the
            # reference's own bfloat16 path, m, v, tau bfloat16 as zeros_like(p) makes them
            flags |= _lib.GRAD_BF16 | (_lib.PARAM_BF16 if self.master_weights else _lib.STATE_BF16)
        else:
            raise NotImplementedError(f"{type(self).__name__}: parameter dtype {p.dtype}")
        return flags

    def _desc_rows(self, ls: _LaunchSet) -> np.ndarray:
        """Descriptor rows of the launch set, and its gradient pointers in
        ``ls.host_grad`` (the gradient's staging buffer where it has one).
        The descriptor's vector-path flag covers the pointers other than the
        gradient's, whose alignment the kernel checks itself."""
        n = len(ls.params)
        d = np.zeros(n, dtype=_lib.DESC_DTYPE)
        gptr = np.zeros(n, dtype=np.uint64)
        km, kv, kt = self._KEYS
        stage = []
        vec = 8 if ls.flags & _lib.STATE_BF16 else 16       # 4 elements of the state dtype
        for j, (p, g, st) in enumerate(zip(ls.params, ls.grads, ls.states)):
            # The kernel pairs elements by storage offset, in the layout of the
            # state (zeros_like(p): p's strides for a contiguous or permuted p,
            # contiguous for one with gaps).  A parameter or gradient of
            # another layout is staged through a buffer of the state's layout.
            m = st[km]
            ps = None if same_layout(p, m) else self._staging(ls, j, "p", p, m)
            gs = None if same_layout(g, m) else self._staging(ls, j, "g", g, m)
            if ps is not None or gs is not None:
                stage.append((j, ps, gs))
            pt = p if ps is None else ps
            master = st.get("master")
            param_ptr = master.data_ptr() if master is not None else pt.data_ptr()
            lp_ptr = pt.data_ptr() if master is not None else 0
            tau_ptr = st[kt].data_ptr() if self._STAR else 0
            gptr[j] = (g if gs is None else gs).data_ptr()
            m_ptr, v_ptr = st[km].data_ptr(), st[kv].data_ptr()
            ok = (param_ptr % vec == 0 and m_ptr % vec == 0 and v_ptr % vec == 0
                  and tau_ptr % vec == 0 and lp_ptr % 8 == 0)
            d[j] = (param_ptr, 0, m_ptr, v_ptr, tau_ptr, lp_ptr, p.numel(), ls.sclass[j],
                    _lib.DESC_VEC_OK if ok else 0)
        ls.host_grad = gptr
        ls.grad_addr = gptr.ctypes.data
        ls.stage = stage
        return d

    @staticmethod
    def _staging(ls: _LaunchSet, j: int, kind: str, x: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
        """The staging buffer of row j's parameter or gradient: x's dtype in
        ``like``'s shape and layout, kept across steps (its address is in the
        device descriptors) while that still fits."""
        key = (j, kind)
        buf = ls.stage_bufs.get(key)
        if buf is None or buf.dtype != x.dtype or not same_layout(buf, like) or buf.device != like.device:
            buf = ls.stage_bufs[key] = torch.empty_strided(like.shape, like.stride(), dtype=x.dtype,
                                                           device=like.device)
        return buf

    def _upload(self, ls: _LaunchSet) -> None:
        """Copy [descriptors | vstart | fold_first] and the gradient pointers
        to the device (async, pinned) and point the plan at them."""
        table = np.concatenate([ls.host_desc.view(np.uint8), ls.vstart.view(np.uint8),
                                ls.fold_first.view(np.uint8)])
        host = torch.from_numpy(table).pin_memory()
        n = len(ls.params)
        if ls.dev_table is None or ls.dev_table.numel() != host.numel():
            ls.dev_table = torch.empty(host.numel(), dtype=torch.uint8, device=ls.device)
        if ls.dev_grad is None or ls.dev_grad.numel() != max(n, 1):
            ls.dev_grad = torch.zeros(max(n, 1), dtype=torch.int64, device=ls.device)
        ls.dev_table.copy_(host, non_blocking=True)
        if n:
            ls.dev_grad.copy_(torch.from_numpy(ls.host_grad.view(np.int64)).pin_memory(), non_blocking=True)
        base = ls.dev_table.data_ptr()
        if ls.plan is None:
            ls.plan = _lib.Plan()
        ls.plan.desc = base
        ls.plan.grad = ls.dev_grad.data_ptr()
        ls.plan.vstart = base + 64 * n
        ls.plan.fold_first = base + 64 * n + 8 * (n + 1)
        ls.plan.n_tensors = n
        ls.plan.n_chunks = ls.n_chunks
        ls.plan.n_folds = ls.n_folds

    @staticmethod
    def _upload_grads(ls: _LaunchSet, lo: int, hi: int) -> None:
        """Copy gradient pointers [lo, hi) of ls.host_grad to the device (async,
        pinned; stream-ordered before the launch that reads them)."""
        host = torch.from_numpy(ls.host_grad[lo:hi].view(np.int64)).pin_memory()
        ls.dev_grad[lo:hi].copy_(host, non_blocking=True)

    def _build(self, params, grads, states, sclass, flags_list, inactive=None) -> List[_LaunchSet]:
        """Lay out the launch sets of this step's (param, grad, state) rows.
        ``inactive``: the optimizer's other parameters (no gradient now);
        given, and with a single launch set that stages nothing, step() may
        take the one-pass StepTable.scan from the next step on."""
        sets = {}
        for i, (p, g, st, c, fl) in enumerate(zip(params, grads, states, sclass, flags_list)):
            key = (p.device, fl, c // _lib.MAX_CLASSES)
            ls = sets.get(key)
            if ls is None:
                ls = sets[key] = _LaunchSet(p.device, fl, (c // _lib.MAX_CLASSES) * _lib.MAX_CLASSES)
            ls.index.append(i)
            ls.params.append(p)
            ls.grads.append(g)
            ls.states.append(st)
            ls.sclass.append(c - ls.class_base)
        out = list(sets.values())
        fast = (inactive is not None and len(out) == 1
                and all(type(t) in (torch.Tensor, torch.nn.Parameter) for t in params)
                and all(type(t) in (torch.Tensor, torch.nn.Parameter) for t in inactive))
        for ls in out:
            self._check_state_shapes(ls)
            numels = np.fromiter((p.numel() for p in ls.params), dtype=np.int64, count=len(ls.params))
            ls.vstart, ls.fold_first, ls.n_chunks, ls.n_folds = _lib.plan_layout(numels)
            ls.host_desc = self._desc_rows(ls)
            ls.ptr_key = _hoststep.data_ptrs(ls.params)
            fast = fast and not ls.stage
            with torch.cuda.device(ls.device):
                self._upload(ls)
                n = len(ls.params)
                ls.chunk_first = torch.empty(max(ls.n_chunks, 1), dtype=torch.int32, device=ls.device)
                stream = torch.cuda.current_stream(ls.device).cuda_stream
                _lib.check(_lib.lib().adana_plan_index(
                    ctypes.c_void_p(ls.plan.vstart), n, ls.n_chunks,
                    ctypes.c_void_p(ls.chunk_first.data_ptr()), ctypes.c_void_p(stream)),
                    "adana_plan_index")
                ls.plan.chunk_first = ls.chunk_first.data_ptr()
                ls.workspace = torch.empty(max(_lib.workspace_bytes(ls.plan), 1), dtype=torch.uint8,
                                           device=ls.device)
                # the reference's bfloat16 path keeps bfloat16 diagnostics
                ls.diag = torch.full((len(ls.params), 5), float("nan"), device=ls.device,
                                     dtype=torch.bfloat16 if ls.flags & _lib.STATE_BF16 else torch.float32)
            ls.sc_arr = (_lib.StepScalars * _lib.MAX_CLASSES)()
            ls.args = (ctypes.byref(ls.plan), ctypes.cast(ls.sc_arr, ctypes.c_void_p),
                       ctypes.c_void_p(ls.workspace.data_ptr()), ls.workspace.numel(),
                       ctypes.c_void_p(ls.diag.data_ptr()))
            # The rows' table: its scan is the fast path of the next steps (a
            # single launch set only), and it keeps the diagnostics bound as
            # 0-d tensors over the kernel's output rows, each with a storage of
            # its own (a deepcopy of one parameter's state, as DynamicsLogger
            # takes, src/logger/logger.py:93, copies its own bytes only).
            ls.table = _hoststep.step_table(ls.params, ls.states, list(inactive) if fast else [],
                                            bool(ls.flags & _lib.GRAD_BF16))
            ls.table.diag_bind(ls.diag, self._diag_cols)
            for j, p in enumerate(ls.params):
                self._diag_loc[p] = (ls, j)
        self._fast = fast
        self._diag_epoch += 1
        return out

    # -- diagnostics read-out ---------------------------------------------
    def diagnostics_host(self):
        """Every parameter's five diagnostics (DIAG_KEYS order) as float32 rows
        of a numpy array, in param_groups order, skipping parameters without
        them: one asynchronous device-to-host copy per diagnostics buffer and
        one synchronisation, instead of one ``.item()`` per value.  Returns
        (params, values[n, 5]).  Where each parameter's row lives is cached
        until a plan or the state tensors change (call ``invalidate_plan()``
        after replacing state tensors by hand)."""
        all_params, _ = self._flat_params()
        key = (self._diag_epoch, self._flat[0])
        cache = self._diag_cache
        col0, mark = self._DIAG_COLUMNS[0]
        if cache is None or cache[0] != key:
            params, by_buf, loose = [], {}, []
            for p in all_params:
                st = self.state.get(p) if p in self.state else None
                if not st or mark not in st:
                    continue
                loc = self._diag_loc.get(p)
                if loc is not None and st[mark].data_ptr() != (loc[0].diag.data_ptr()
                                                               + loc[0].diag.element_size() * (5 * loc[1] + col0)):
                    loc = None                     # state tensors replaced (e.g. load_state_dict)
                if loc is None:
                    loose.append((len(params), st))
                else:
                    ent = by_buf.setdefault(id(loc[0]), (loc[0], [], []))
                    ent[1].append(loc[1])
                    ent[2].append(len(params))
                params.append(p)
            bufs = [(ls, np.asarray(rows, np.int64), np.asarray(pos, np.int64))
                    for ls, rows, pos in by_buf.values()]
            cache = self._diag_cache = (key, params, bufs, loose)
        _, params, bufs, loose = cache
        host = []
        for ls, _, _ in bufs:                      # each launch set's latest buffer
            h = torch.empty(ls.diag.shape, dtype=ls.diag.dtype, pin_memory=True)
            h.copy_(ls.diag, non_blocking=True)
            host.append(h)
        for dev in {ls.diag.device for ls, _, _ in bufs}:
            torch.cuda.current_stream(dev).synchronize()
        out = np.empty((len(params), 5), dtype=np.float32)
        for (ls, rows, pos), h in zip(bufs, host):
            out[pos] = (h.float() if h.dtype == torch.bfloat16 else h).numpy()[rows]
        for pos, st in loose:                      # loaded, not yet stepped: read one by one
            out[pos] = np.nan
            for col, k in self._DIAG_COLUMNS:
                out[pos, col] = float(st[k])
        return params, out

    # -- step -------------------------------------------------------------
    def _hparams(self, group, foreach: int = 0) -> "_lib.HParams":
        """adana_hparams of a group; ``foreach``: 0, or the foreach path's
        scalars for float32 (1) or bfloat16 (2) state."""
        hp = _lib.HParams()
        hp.peak_lr = self.lr
        hp.delta = group["delta"]
        hp.kappa = self.kappa
        hp.epsilon = group["epsilon"]
        hp.weight_decay = group["weight_decay"]
        hp.has_clip = 0 if self.clipsnr is None else 1
        hp.clipsnr = 0.0 if self.clipsnr is None else float(self.clipsnr)
        hp.wd_ts = self.wd_ts
        hp.gamma_3_factor = self.gamma_3_factor
        hp.wd_decaying = 1 if self.wd_decaying else 0
        hp.eager = 1 if self.numerics == "eager" else 0
        hp.foreach = foreach
        return hp

    def _flat_params(self):
        """All parameters in group order, with their group index (cached; the
        cache is checked object for object against the groups every call, so
        added groups and parameters replaced in place are picked up)."""
        sig = tuple((id(g["params"]), len(g["params"])) for g in self.param_groups)
        if (self._flat is None or self._flat[0] != sig
                or not _hoststep.same_params(self.param_groups, self._flat[1])):
            params, gidx = [], []
            for gi, group in enumerate(self.param_groups):
                params.extend(group["params"])
                gidx.extend([gi] * len(group["params"]))
            self._flat = (sig, params, gidx)
            self._fast = False
        return self._flat[1], self._flat[2]

    def _group_hparams(self, gi: int, foreach: int = 0) -> "_lib.HParams":
        """Group gi's hyper-parameters for the scalar code, rebuilt only when a
        value they are made of changed."""
        g = self.param_groups[gi]
        key = (g["delta"], g["epsilon"], g["weight_decay"], self.lr, self.kappa, self.clipsnr, self.wd_ts,
               self.gamma_3_factor, self.wd_decaying, self.numerics)
        ent = self._hp_cache.get((gi, foreach))
        if ent is None or ent[0] != key:
            ent = self._hp_cache[(gi, foreach)] = (key, self._hparams(g, foreach))
        return ent[1]

    def _fill_scalars(self, ls: _LaunchSet, classes) -> int:
        """Write the launch set's scalar classes (adana_step_scalars_init, per
        (group, step) class, at the group's current lr) into ls.sc_arr;
        return their count."""
        L = _lib.lib()
        n_cls = min(_lib.MAX_CLASSES, len(classes) - ls.class_base)
        # the foreach path's step tensor has the parameters' dtype (adana.py:258)
        fe = (2 if ls.flags & _lib.STATE_BF16 else 1) if self._foreach else 0
        for k in range(n_cls):
            gi, t = classes[ls.class_base + k]
            _lib.check(L.adana_step_scalars_init(ctypes.byref(ls.sc_arr[k]),
                                                 ctypes.byref(self._group_hparams(gi, fe)),
                                                 float(self.param_groups[gi]["lr"]), int(t)),
                       "adana_step_scalars_init")
        return n_cls

    def step(self, closure=None):
        """One optimizer step (src/optim/adana.py:155-227); returns the
        closure's loss.  Runs under no_grad, with the closure under
        enable_grad.  Step pre/post hooks (per optimizer and global) and the
        profiler's ``Optimizer.step#...`` range behave as for any
        torch.optim.Optimizer: with a hook registered or a profiler running
        the call goes through torch's own step wrapper; otherwise it skips
        that wrapper's per-call machinery (about 10 us of host time)."""
        if (self._optimizer_step_pre_hooks or self._optimizer_step_post_hooks
                or _torch_optimizer._global_optimizer_pre_hooks or _torch_optimizer._global_optimizer_post_hooks
                or torch._C._autograd._profiler_enabled()):
            return self._step_hooked(closure)
        prev = torch.is_grad_enabled()
        torch._C._set_grad_enabled(False)
        try:
            loss = self._step(closure)
        finally:
            torch._C._set_grad_enabled(prev)
        self._optimizer_step_code()
        return loss

    # torch.optim.Optimizer wraps a subclass's step() unless it is marked as
    # hooked; this one dispatches to the wrapped form itself when needed.
    step.hooked = True

    def _step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()

        for group in self.param_groups:
            # src/optim/adana.py:163-167: g2 = g3 = lr, sf = lr / self.lr
            group["weighted_step_count"] += group["lr"] / self.lr
        all_params, gidx = self._flat_params()
        if self._fast:
            # One launch set that stages nothing: one C++ pass checks that every
            # row still has a gradient of its parameter's layout and that no
            # other parameter gained one, gathers the gradient pointers, does
            # every ``state['step'] += 1`` (adana.py:197) and bumps the
            # parameters' versions; only pointers that moved are uploaded.
            # With the diagnostics' check on, the same pass classifies the
            # bound diagnostics (helper threads on long plans).
            ls = self._sets[0]
            checked = self._diag_checked()
            span = ls.table.scan(ls.grad_addr, checked)
            if span is not None:
                self._classes = [(gi, t + 1) for gi, t in self._classes]
                if span[1] > span[0]:
                    self._upload_grads(ls, span[0], span[1])
                if checked and span[2] is not None:
                    self._diag_rehome(ls, span[2], span[3])
                    return self._launch(None, None, self._classes, loss, diag_done=True)
                return self._launch(None, None, self._classes, loss)
        # The general path: the reference's walk (adana.py:184-197) in Python.
        params, grads, states, keys, inactive = [], [], [], [], []
        fresh = []
        rows = []
        need = ("m", "v", "tau") if self._STAR else ("m", "v")
        for p, gi in zip(all_params, gidx):
            g = p.grad
            if g is None:                                                    # adana.py:186
                inactive.append(p)
                continue
            st = self.state[p]
            if len(st) != 0:
                # a state without its moments or step counter fails as the
                # reference's ``m, v = state['m'], state['v']`` and
                # ``state['step'] += 1`` do (adana.py:193-197), here before any
                # counter moves
                for k in need + ("step",):
                    if k not in st:
                        raise KeyError(k)
            rows.append((p, g, st, gi))
        for p, g, st, gi in rows:
            if len(st) == 0:                                                 # adana.py:191-195
                fresh.append((p, st))
                st["step"] = 0
            st["step"] += 1                                                  # adana.py:197
            params.append(p)
            grads.append(g)
            states.append(st)
            keys.append((gi, st["step"]))
        if fresh:
            self._pack_states(fresh, None)
        if not params:
            self._fast = False
            return loss
        # (group, step) scalar classes
        cls_index = {}
        sclass = []
        for k in keys:
            c = cls_index.get(k)
            if c is None:
                c = cls_index[k] = len(cls_index)
            sclass.append(c)
        classes = list(cls_index)
        structure = (tuple(map(id, params)), tuple(sclass), tuple(map(id, inactive)))
        if self._sets is None or structure != self._structure:
            flags = [self._validate(p, g) for p, g in zip(params, grads)]
            self._sets = self._build(params, grads, states, sclass, flags, inactive)
            self._structure = structure
        else:
            for ls in self._sets:
                ls.grads = grads if len(self._sets) == 1 else [grads[i] for i in ls.index]
                self._refresh_ptrs(ls)
        self._classes = classes
        return self._launch(params, grads, classes, loss)

    _step_hooked = Optimizer.profile_hook_step(torch.no_grad()(_step))

    def _diag_checked(self) -> bool:
        """Whether this step checks the bound diagnostics before rewriting them
        in place (always, unless fresh_diagnostics=False)."""
        return self.fresh_diagnostics is not False

    def _diag_guard(self, ls: _LaunchSet) -> None:
        """Before a step rewrites ls.diag in place: every bound diagnostic that
        something else still refers to keeps its value in a copy of its own
        (taken on the launch's stream, ahead of the launch), and the state
        gets a new 0-d tensor over the buffer, as the reference binds new
        tensors every step (src/optim/adana.py:221-225)."""
        held, lost = ls.table.diag_check()
        self._diag_rehome(ls, held, lost)

    def _diag_rehome(self, ls: _LaunchSet, held, lost) -> None:
        """Give the held diagnostics (flat indices from StepTable.diag_check or
        .scan) copies of their values, on the launch's stream ahead of the
        launch, and bind new 0-d tensors over the buffer for the held and lost
        ones."""
        if not held and not lost:
            return
        copy = ls.diag.new_empty(0)
        if held:
            nc = len(self._diag_cols)
            flat = [(k // nc) * 5 + self._diag_cols[k % nc][0] for k in held]
            copy = ls.diag.view(-1).index_select(0, torch.tensor(flat, dtype=torch.int64, device=ls.device))
        ls.table.diag_rehome(held, copy, lost, ls.diag)

    def _launch(self, params, grads, classes, loss, diag_done: bool = False):
        """One adana_mta_step (or adana_mta_step_scaled) per launch set.
        ``params``/``grads``: the step's rows from the general path (their
        versions are bumped here), or None after StepTable.scan (which bumped
        them).  ``diag_done``: the scan has already guarded the diagnostics."""
        # a clip armed by clip_grad_norm_(..., optimizer=self) on exactly these
        # gradients is applied inside the kernel; otherwise it is applied now
        gscale, wflag = None, 0
        pend = self._pending_clip
        if pend is not None:
            own, _, clip, write_back = pend
            if grads is None:
                same = self._sets[0].table.grads_are(own)
            else:
                same = len(own) == len(grads) and all(map(operator.is_, grads, own))
            if same and all(ls.device == clip.device for ls in self._sets):
                self._pending_clip = None
                gscale = clip.data_ptr() + 4
                wflag = _lib.WRITE_GRAD if write_back else 0
            else:
                self.flush_clip()

        L = _lib.lib()
        checked = self._diag_checked() and not diag_done
        cur = torch.cuda.current_device()
        for ls in self._sets:
            n_cls = self._fill_scalars(ls, classes)
            if ls.device.index == cur:
                self._launch_set(L, ls, n_cls, gscale, wflag, checked)
            else:
                with torch.cuda.device(ls.device):
                    self._launch_set(L, ls, n_cls, gscale, wflag, checked)
        if params is not None:
            _hoststep.bump_versions(params)                # p was updated in place
        if wflag:
            _hoststep.bump_versions(pend[0])
        return loss

    def _launch_set(self, L, ls: _LaunchSet, n_cls: int, gscale, wflag: int, checked: bool) -> None:
        """One launch set's staging copies, diagnostics guard and step launch,
        with ls.device current, on torch's current stream."""
        stream = ctypes.c_void_p(torch._C._cuda_getCurrentRawStream(ls.device.index))
        plan, sc, ws, ws_bytes, diag = ls.args
        if checked:
            self._diag_guard(ls)
        for j, ps, gs in ls.stage:       # into the state's layout (same stream)
            if ps is not None and not ls.flags & _lib.PARAM_BF16:   # the master is read instead
                ps.copy_(ls.params[j])
            if gs is not None:
                gs.copy_(ls.grads[j])
        if gscale is None:
            rc = L.adana_mta_step(plan, sc, n_cls, ls.flags, ws, ws_bytes, diag, stream)
            if rc:
                _lib.check(rc, "adana_mta_step")
        else:
            _lib.check(L.adana_mta_step_scaled(plan, sc, n_cls, ls.flags | wflag, ctypes.c_void_p(gscale),
                                               ws, ws_bytes, diag, stream), "adana_mta_step_scaled")
        for j, ps, gs in ls.stage:       # and back
            if ps is not None:
                ls.params[j].copy_(ps)
            if gs is not None and wflag:
                ls.grads[j].copy_(gs)

    def _check_state_shapes(self, ls: _LaunchSet) -> None:
        """A parameter whose storage was rebound (``p.data = x``) must keep the
        shape of its state: the laid-out plan, the workspace and the state
        slabs are sized by it.  The reference fails the same way, in
        ``m.lerp_(grad, alpha)`` (src/optim/adana.py:101).  (A new layout of
        the same shape is staged like any other.)"""
        km = self._KEYS[0]
        for p, st in zip(ls.params, ls.states):
            m = st[km]
            if p.shape != m.shape:
                a, b = tuple(m.shape), tuple(p.shape)
                raise RuntimeError(f"{type(self).__name__}: parameter of shape {b} has optimizer state "
                                   f"of shape {a}: the size of tensor a ({a}) must match the size of "
                                   f"tensor b ({b})")
            if not no_overlap(p):
                raise NotImplementedError(f"{type(self).__name__}: parameters whose elements may share memory "
                                          f"(strides {tuple(p.stride())}) are not supported")

    def _refresh_ptrs(self, ls: _LaunchSet) -> None:
        """Re-point the launch set's tables at this step's gradients and the
        parameters' current storage (the general path; re-uploaded only where
        an address moved: new gradient tensors, or ``p.data`` rebound)."""
        pkey = _hoststep.data_ptrs(ls.params)
        gptr = np.frombuffer(_hoststep.data_ptrs(ls.grads), dtype=np.uint64)
        bf16 = bool(ls.flags & _lib.GRAD_BF16)
        if pkey == ls.ptr_key and not ls.stage and _hoststep.grads_match(ls.params, ls.grads, bf16):
            # only gradients may have moved, each a dense tensor of its
            # parameter's layout and the set's dtype: re-point those
            moved = np.flatnonzero(gptr != ls.host_grad)
            if moved.size:
                ls.host_grad[:] = gptr
                with torch.cuda.device(ls.device):
                    self._upload_grads(ls, int(moved[0]), int(moved[-1]) + 1)
                ls.table.forget()
            return
        if pkey != ls.ptr_key:
            self._check_state_shapes(ls)
        for p, g in zip(ls.params, ls.grads):
            if self._validate(p, g) != ls.flags:
                raise RuntimeError(f"{type(self).__name__}: gradient dtype changed")
        ls.host_desc = self._desc_rows(ls)
        with torch.cuda.device(ls.device):
            self._upload(ls)
        if pkey != ls.ptr_key or ls.stage:
            # the rows' storage moved (or is staged): the fast scan's table is
            # rebuilt from the next general step's plan
            self._structure = None
            self._fast = False
        ls.ptr_key = pkey
        ls.table.forget()


class ADana(_DanaFamily):
    """ADana (``clipsnr=None``) and Dana-MK4 (``clipsnr=float``).

    Same constructor, defaults, group keys and state keys as
    src/optim/adana.py:32-70.  ``use_foreach=True`` gives the reference's
    foreach path's numerics (see the module docstring).  Keyword-only
    extensions (see the module
    docstring): ``numerics`` ("compiled", the reference's default
    torch.compile path, or "eager"), ``master_weights`` for bfloat16
    parameters and ``fresh_diagnostics`` for the diagnostics' check.
    """

    _STAR = False

    def __init__(self, params: Iterable[torch.Tensor], lr: float = 1.0, delta: float = 8.0,
                 kappa: float = 1.0, epsilon: float = 1e-8, weight_decay: float = 0.0,
                 clipsnr: float = None, wd_decaying: bool = False, wd_ts: float = 1.0,
                 gamma_3_factor: float = 1.0, use_foreach: bool = False, *,
                 master_weights: bool = False, fresh_diagnostics: Optional[bool] = None,
                 numerics: str = "compiled"):
        defaults = dict(lr=lr, delta=delta, epsilon=epsilon, weight_decay=weight_decay,
                        weighted_step_count=0)
        self.lr = lr
        self.delta = delta
        self.kappa = kappa
        self.epsilon = epsilon
        self.weight_decay = weight_decay
        self.clipsnr = clipsnr
        self.wd_decaying = wd_decaying
        self.wd_ts = wd_ts
        self.gamma_3_factor = gamma_3_factor
        self.use_foreach = use_foreach
        super().__init__(params, defaults)
        self._engine_init(master_weights, fresh_diagnostics, numerics)


class DANA_STAR_MK4(_DanaFamily):
    """Dana-Star (``clipsnr=None``) and Dana-Star-MK4 (``clipsnr=float``).

    Same constructor (including the mk4A / mk4B / weight_time assertions),
    defaults, group keys and state keys as src/optim/dana_star_mk4.py:10-86;
    the same keyword-only extensions as ADana.
    """

    _STAR = True
    _VARIANT = _lib.VARIANT_STAR

    def __init__(self, params: Iterable[torch.Tensor], lr: float = 1.0, delta: float = 8.0,
                 kappa: float = 1.0, mk4A: float = 0.0, mk4B: float = 0.0,
                 epsilon: float = 1e-8, weight_decay: float = 0.0, clipsnr: float = 1.0,
                 weight_time: bool = False, wd_decaying: bool = False, wd_ts: float = 1.0,
                 gamma_3_factor: float = 1.0, use_foreach: bool = False, *,
                 master_weights: bool = False, fresh_diagnostics: Optional[bool] = None,
                 numerics: str = "compiled"):
        assert mk4A == 0.0, f"mk4A must be 0.0, got {mk4A}"
        assert mk4B == 0.0, f"mk4B must be 0.0, got {mk4B}"
        assert weight_time == False, f"weight_time must be False, got {weight_time}"  # noqa: E712
        defaults = dict(lr=lr, delta=delta, epsilon=epsilon, weight_decay=weight_decay,
                        weighted_step_count=0)
        self.lr = lr
        self.delta = delta
        self.kappa = kappa
        self.mk4A = 0.0
        self.mk4B = 0.0
        self.clipsnr = clipsnr
        self.epsilon = epsilon
        self.weight_decay = weight_decay
        self.weight_time = False
        self.wd_decaying = wd_decaying
        self.wd_ts = wd_ts
        self.gamma_3_factor = gamma_3_factor
        self.use_foreach = use_foreach
        super().__init__(params, defaults)
        self._engine_init(master_weights, fresh_diagnostics, numerics)
