"""adana_mta_step_noalloc (scratch in the library's static device array)
against adana_mta_step (scratch in a caller workspace), through the C ABI:
calls in a row on the same device, each later one over a different list,
each bit for bit equal to the workspace entry point (p, m, v, tau and the
five diagnostics): float32 lists in both numerics, a list of more than 256
combine folds (its second combine launch), bfloat16 state with the eager
path's pow table (placed in the scratch) and in the compiled numerics, the
foreach path on float32 and bfloat16 state; and a list too large for the
static scratch is refused before any launch."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


class _List:
    """One tensor list with its device tables, in two identical copies of
    p / m / v / tau (one per entry point) and shared gradients.  ``bf16``:
    bfloat16 parameters, state and gradients (ADANA_STATE_BF16)."""

    def __init__(self, sizes, star, seed, bf16=False, eager=False, foreach=False):
        from adana_amd import _lib

        self.sizes = sizes
        self.star = star
        self.bf16 = bf16
        self.eager = eager
        self.foreach = foreach
        self.dt = torch.bfloat16 if bf16 else torch.float32
        self.gen = torch.Generator(device="cuda")
        self.gen.manual_seed(seed)
        p0 = [(torch.randn(n, device="cuda", generator=self.gen) * 0.02).to(self.dt) for n in sizes]
        self.copies = []
        for _ in range(2):
            c = {"p": [x.clone() for x in p0], "m": [torch.zeros_like(x) for x in p0],
                 "v": [torch.zeros_like(x) for x in p0], "tau": [torch.zeros_like(x) for x in p0]}
            self.copies.append(c)
        del p0
        self.g = [torch.empty(n, device="cuda", dtype=self.dt) for n in sizes]
        n = len(sizes)
        vstart, fold_first, self.n_chunks, self.n_folds = _lib.plan_layout(np.array(sizes, np.int64))
        self.plans, self.tables, self.chunk_first = [], [], []
        self.gtab = torch.tensor([x.data_ptr() for x in self.g], dtype=torch.int64, device="cuda")
        L = _lib.lib()
        stream = torch.cuda.current_stream().cuda_stream
        for c in self.copies:
            desc = np.zeros(n, _lib.DESC_DTYPE)
            for i in range(n):
                desc[i] = (c["p"][i].data_ptr(), 0, c["m"][i].data_ptr(), c["v"][i].data_ptr(),
                           c["tau"][i].data_ptr() if star else 0, 0, sizes[i], 0, _lib.DESC_VEC_OK)
            table = torch.from_numpy(np.concatenate([desc.view(np.uint8), vstart.view(np.uint8),
                                                     fold_first.view(np.uint8)])).cuda()
            plan = _lib.Plan(desc=table.data_ptr(), grad=self.gtab.data_ptr(), vstart=table.data_ptr() + 64 * n,
                             fold_first=table.data_ptr() + 64 * n + 8 * (n + 1), n_tensors=n,
                             n_chunks=self.n_chunks, n_folds=self.n_folds)
            cf = torch.empty(max(self.n_chunks, 1), dtype=torch.int32, device="cuda")
            _lib.check(L.adana_plan_index(ctypes.c_void_p(plan.vstart), n, self.n_chunks,
                                          ctypes.c_void_p(cf.data_ptr()), ctypes.c_void_p(stream)), "plan_index")
            plan.chunk_first = cf.data_ptr()
            self.plans.append(plan)
            self.tables.append(table)
            self.chunk_first.append(cf)
        self.diag = [torch.full((5 * n,), float("nan"), device="cuda", dtype=self.dt) for _ in range(2)]
        self.ws = torch.empty(_lib.workspace_bytes(self.plans[0]), dtype=torch.uint8, device="cuda")
        assert _lib.workspace_bytes(self.plans[0]) <= _lib.NOALLOC_SCRATCH_BYTES

    def step(self, t):
        from adana_amd import _lib

        L = _lib.lib()
        for gi, n in zip(self.g, self.sizes):
            gi.copy_(torch.randn(n, device="cuda", generator=self.gen) * 1e-3)
        hp = _lib.HParams(peak_lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=0.4, clipsnr=2.0,
                          wd_ts=10.0, gamma_3_factor=0.7, has_clip=1, wd_decaying=1, eager=int(self.eager),
                          foreach=(2 if self.bf16 else 1) if self.foreach else 0)
        sc = (_lib.StepScalars * 1)(_lib.step_scalars(hp, 1e-3, t))
        flags = ((_lib.VARIANT_STAR if self.star else 0) | (_lib.NUMERICS_EAGER if self.eager else 0)
                 | (_lib.FOREACH if self.foreach else 0))
        if self.bf16:
            flags |= _lib.GRAD_BF16 | _lib.STATE_BF16
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.adana_mta_step(ctypes.byref(self.plans[0]), ctypes.cast(sc, ctypes.c_void_p), 1, flags,
                                    ctypes.c_void_p(self.ws.data_ptr()), self.ws.numel(),
                                    ctypes.c_void_p(self.diag[0].data_ptr()), stream), "adana_mta_step")
        _lib.check(L.adana_mta_step_noalloc(ctypes.byref(self.plans[1]), ctypes.cast(sc, ctypes.c_void_p), 1,
                                            flags, ctypes.c_void_p(self.diag[1].data_ptr()), stream),
                   "adana_mta_step_noalloc")
        torch.cuda.synchronize()

    def assert_equal(self, where):
        a, b = self.copies
        keys = ("p", "m", "v") + (("tau",) if self.star else ())
        iv = torch.int16 if self.bf16 else torch.int32
        for key in keys:
            for i in range(len(self.sizes)):
                assert torch.equal(a[key][i].view(iv), b[key][i].view(iv)), (where, key, i)
        assert torch.equal(self.diag[0].view(iv), self.diag[1].view(iv)), (where, self.diag[0], self.diag[1])


def test_noalloc_matches_workspace_entry_point():
    print("case: adana_mta_step_noalloc vs adana_mta_step, Dana-Star list of 10.1M elements", flush=True)
    big = _List([1 << 20, 3, 70_000, 9_000_000, 5], star=True, seed=11)
    for t in (1, 2):
        big.step(t)
        big.assert_equal(f"big t={t}")
    print("case: adana_mta_step_noalloc second call, smaller ADana list, eager numerics", flush=True)
    small = _List([5000, 17, 1024], star=False, seed=12, eager=True)
    for t in (1, 2):
        small.step(t)
        small.assert_equal(f"small t={t}")
    print("case: adana_mta_step_noalloc, 2,000 small Dana-Star tensors (shared chunks, direct combine)",
          flush=True)
    sizes = np.exp(np.random.default_rng(13).uniform(0, np.log(5000), 2000)).astype(np.int64).tolist()
    many = _List(sizes, star=True, seed=13)
    for t in (1, 2):
        many.step(t)
        many.assert_equal(f"many t={t}")


def test_noalloc_two_launch_combine():
    """A tensor of more than 256 combine folds (257 * 512 chunks) takes the
    combine's second launch, its folds in the static scratch."""
    print("case: adana_mta_step_noalloc, one tensor of 257 folds (134.8M elements), Dana-Star", flush=True)
    n = 257 * 512 * 1024 - 100
    big = _List([n, 7], star=True, seed=21)
    assert big.n_folds > 256
    for t in (1, 2):
        big.step(t)
        big.assert_equal(f"257 folds t={t}")
    del big
    torch.cuda.empty_cache()


@pytest.mark.parametrize("eager", [True, False], ids=["eager_pow_table", "compiled"])
def test_noalloc_bf16_state(eager):
    """bfloat16 state: the eager path's pow table, filled first in the
    scratch, and the compiled path, against the workspace entry point."""
    print("case: adana_mta_step_noalloc, bf16 state Dana-Star, eager", eager, flush=True)
    lst = _List([70_000, 3, 1 << 20, 4099], star=True, seed=31, bf16=True, eager=eager)
    for t in range(1, 13):                      # tau * t passes 1: the pow sees arguments above 1
        lst.step(t)
        lst.assert_equal(f"bf16 t={t}")


@pytest.mark.parametrize("kind", ["fp32", "bf16_compiled", "bf16_eager"])
def test_noalloc_foreach(kind):
    """The foreach path (ADANA_FOREACH, scalars with hparams.foreach) through
    both entry points: float32, and bfloat16 state compiled and eager (its
    pow table in the scratch)."""
    bf16 = kind != "fp32"
    print("case: adana_mta_step_noalloc, foreach path,", kind, flush=True)
    lst = _List([70_000, 3, 1 << 20, 4099], star=True, seed=41, bf16=bf16, eager=kind == "bf16_eager",
                foreach=True)
    for t in range(1, 11):
        lst.step(t)
        lst.assert_equal(f"foreach {kind} t={t}")


def test_noalloc_replayed_from_a_captured_graph():
    """adana_mta_step_noalloc captured once into a HIP graph (torch.cuda.graph),
    then replayed four times, each replay after the gradients were refilled
    outside the graph and with eager work and synchronisations between
    replays: every replay equals an eager adana_mta_step call with the same
    scalars on the other copy, bit for bit (p, m, v, tau, diagnostics).  The
    captured launches are the main kernel and the combine; no memset node is
    recorded (the main kernel clears the arrival counters itself)."""
    from adana_amd import _lib

    print("case: adana_mta_step_noalloc captured in a HIP graph, 4 replays", flush=True)
    L = _lib.lib()
    lst = _List([1 << 20, 3, 70_000, 4099, 5], star=True, seed=51)
    hp = _lib.HParams(peak_lr=1e-3, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=0.4, clipsnr=2.0,
                      wd_ts=10.0, gamma_3_factor=0.7, has_clip=1, wd_decaying=1)
    flags = _lib.VARIANT_STAR

    def scalars(t):
        return (_lib.StepScalars * 1)(_lib.step_scalars(hp, 1e-3, t))

    def call_ws(sc):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.adana_mta_step(ctypes.byref(lst.plans[0]), ctypes.cast(sc, ctypes.c_void_p), 1, flags,
                                    ctypes.c_void_p(lst.ws.data_ptr()), lst.ws.numel(),
                                    ctypes.c_void_p(lst.diag[0].data_ptr()), s), "adana_mta_step")

    def call_noalloc(sc):
        s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        _lib.check(L.adana_mta_step_noalloc(ctypes.byref(lst.plans[1]), ctypes.cast(sc, ctypes.c_void_p), 1,
                                            flags, ctypes.c_void_p(lst.diag[1].data_ptr()), s),
                   "adana_mta_step_noalloc")

    def refill():
        for gi, n in zip(lst.g, lst.sizes):
            gi.copy_(torch.randn(n, device="cuda", generator=lst.gen) * 1e-3)

    # an eager step on both copies first (the scratch's device address is looked up there)
    refill()
    sc1 = scalars(1)
    call_ws(sc1)
    call_noalloc(sc1)
    torch.cuda.synchronize()
    lst.assert_equal("eager t=1")
    sc2 = scalars(2)                 # the graph keeps these scalars: every replay is a step at t = 2
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call_noalloc(sc2)
    torch.cuda.synchronize()
    lst.assert_equal("after capture (nothing ran)")
    for k in range(4):
        refill()
        torch.cuda.synchronize()
        graph.replay()
        call_ws(sc2)
        torch.cuda.synchronize()
        lst.assert_equal(f"replay {k}")
        torch.empty(1 << 20, device="cuda").normal_()     # unrelated eager work between replays
        torch.cuda.synchronize()
    del graph


def test_noalloc_rejects_lists_beyond_its_scratch():
    """A list needing more scratch than the static array gets
    ADANA_E_UNSUPPORTED and a message, before any device work (the plan's
    device pointers are never read)."""
    from adana_amd import _lib

    L = _lib.lib()
    print("case: adana_mta_step_noalloc refuses an oversized list", flush=True)
    chunks = _lib.NOALLOC_SCRATCH_BYTES // 16 + 1
    plan = _lib.Plan(desc=16, grad=16, vstart=16, fold_first=16, chunk_first=16, n_tensors=1, n_chunks=chunks,
                     n_folds=0)
    hp = _lib.HParams(peak_lr=1e-3, delta=8.0, kappa=1.0, epsilon=1e-8)
    sc = (_lib.StepScalars * 1)(_lib.step_scalars(hp, 1e-3, 1))
    rc = L.adana_mta_step_noalloc(ctypes.byref(plan), ctypes.cast(sc, ctypes.c_void_p), 1, 0,
                                  ctypes.c_void_p(16), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == -3
    assert "static" in _lib.last_error()
