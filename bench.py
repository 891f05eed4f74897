#!/usr/bin/env python3
"""Benchmark of the ADana-family optimizer step on one MI355X.

A "step" is one ``optimizer.step()`` over the workload's whole parameter list
with parameters, gradients and state already resident in HBM.  The default
workload is the north-star: Dana-Star-MK4, fp32 params and state, on the
2,645,527,040-parameter list of BASELINE config 4's geometry (d_model 2560,
32 layers, MLP 4x, vocab 50304, tied embedding).  Other workloads (c1..c5)
are the remaining BASELINE configs; north_star_clip adds the training loop's
gradient-norm clipping before every step (src/optim/base.py:250-257, max_norm
0.5 as scripts/launch.sh:47) through the optimizer's fused clip, including the
loop's ``grad_norm.item()``.  Two workloads time the step's consumers instead
of the step: tau_stats (TauStatsCollector's tau order statistics over the
north-star state, src/optim/tau_stats_collector.py:131-160) and diag_readout
(log_optimizer_schedules over C5's 10,000 tensors, src/optim/utils.py:532).
manau runs Manau (src/optim/manau.py) on the north-star model and reports its
Dana-Star-MK4 branch (the HIP kernel) beside the whole step.

Prints ONE JSON line.  ``value`` is the whole-step throughput in algorithmic
HBM GB/s (bytes the update must move per element x elements / wall-clock ms
per step, host work included).  ``roofline.achieved`` uses the device time of
the step's kernels, measured with HIP events recorded on the stream they are
launched on.  ``cpu_baseline`` times the reference's step restated as torch eager ops over
CPU tensors (oracle/torch_ref.py, the reference's per-tensor loop) on the
host's cores on a bounded sample of the same workload, with the same update
under torch.compile (the reference's default, Inductor's C++ code) and the C
oracle (OpenMP) beside it.
"""
from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "optimizer step ms + achieved HBM GB/s (% of peak) at 2.62B params, 1 GPU"
HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20          # MI355X Infinity Cache (memory-side last-level cache)

# Launcher conventions (reference scripts/launch.sh:36-40,188-223,309-312):
# kappa 0.85, delta 8, omega 4, clipsnr 2.0, weight_decay = omega / wd_ts,
# wd_ts = iterations / 10, wd_decaying.
def _hp(iterations, clipsnr=2.0, peak_lr=1e-3):
    wd_ts = iterations / 10.0
    return dict(lr=peak_lr, delta=8.0, kappa=0.85, epsilon=1e-8, weight_decay=4.0 / wd_ts,
                clipsnr=clipsnr, wd_decaying=True, wd_ts=wd_ts)


def gpt_shapes(vocab, d, layers, mlp=4, ln_bias=False):
    """(decay, no_decay) parameter shapes of a tied-embedding GPT, grouped the
    way src/models/base.py:503-561 groups them (Linear weights decay; the
    embedding and LayerNorm vectors do not)."""
    decay, nodecay = [], [(vocab, d)]
    for _ in range(layers):
        decay += [(3 * d, d), (d, d), (mlp * d, d), (d, mlp * d)]
        nodecay += [(d,), (d,)] * (2 if ln_bias else 1)
    nodecay += [(d,)] * (2 if ln_bias else 1)
    return decay, nodecay


STEP_WORKLOADS = ("north_star", "north_star_clip", "north_star_bf16", "c1", "c2", "c3", "c4", "c5")


def workload(name):
    """Return a dict describing one BASELINE workload."""
    if name == "c1":
        return dict(name=name, optimizer="ADana", star=False, groups=[[(1024, 4096)]],
                    group_wd=[1.0], hp=_hp(100, clipsnr=None), master=False, schedule=None,
                    grad_note="dense N(0,1e-3)")
    if name == "c2":
        decay, nodecay = gpt_shapes(50304, 512, 8, ln_bias=True)
        return dict(name=name, optimizer="Dana-MK4", star=False, groups=[decay, nodecay],
                    group_wd=[1.0, 0.0], hp=_hp(200, peak_lr=3e-3), master=False,
                    schedule="cos_inf", grad_note="N(0,1e-3); 1-D grads x0.1")
    if name == "c3":
        decay, nodecay = gpt_shapes(50304, 2048, 24)
        return dict(name=name, optimizer="Dana-Star-MK4", star=True, groups=[decay, nodecay],
                    group_wd=[1.0, 0.0], hp=_hp(500), master=False, schedule=None,
                    grad_note="N(0,1e-3); embedding rows nonzero w.p. 0.1")
    if name == "north_star_clip":
        w = workload("north_star")
        w.update(name=name, clip=0.5, grad_note=w["grad_note"] + "; clip_grad_norm_(0.5) each step")
        return w
    if name == "north_star_bf16":
        # the reference's own bfloat16 path: bfloat16 parameters and gradients make m, v, tau
        # bfloat16 (zeros_like(p)) and every op rounds to bfloat16
        w = workload("north_star")
        w.update(name=name, state_bf16=True, grad_note="bf16 N(0,1e-3); embedding rows nonzero w.p. 0.1")
        return w
    if name in ("c4", "north_star"):
        decay, nodecay = gpt_shapes(50304, 2560, 32)
        if name == "c4":
            return dict(name=name, optimizer="ADana", star=False, groups=[decay, nodecay],
                        group_wd=[1.0, 0.0], hp=_hp(100, clipsnr=None), master=True,
                        schedule=None, grad_note="bf16 N(0,1e-3)")
        return dict(name=name, optimizer="Dana-Star-MK4", star=True, groups=[decay, nodecay],
                    group_wd=[1.0, 0.0], hp=_hp(100), master=False, schedule=None,
                    grad_note="N(0,1e-3); embedding rows nonzero w.p. 0.1")
    if name == "c5":
        rng = np.random.default_rng(5)
        sizes = np.floor(np.exp(rng.uniform(math.log(64), math.log(65536), 10000))).astype(int)
        # Default warm-up 40 steps: with the same gradients every step the state settles
        # over the first ~35 steps, during which the power manager lowers the shader clock
        # (1.65-1.8 GHz against 2.2-2.35) and this VALU-heavy list runs 10-20% slower; with
        # new gradients every step, as in training, those steps run at the settled rate.
        return dict(name=name, optimizer="Dana-Star-MK4", star=True,
                    groups=[[(int(n),) for n in sizes]], group_wd=[1.0], hp=_hp(200),
                    master=False, schedule=None, grad_note="N(0,1e-3); 5% of tensors all-zero",
                    default_warmup=40,
                    warmup_note="40 warm-up steps: with the same synthetic gradients every step, steps "
                                "5-35 run at a lowered shader clock that steps with new gradients do not see")
    raise SystemExit(f"unknown workload {name}")


def bytes_per_elem(w):
    if w.get("state_bf16"):
        return 18 if w["star"] else 14        # p, g, m, v (+tau) read, p, m, v (+tau) written, 2 B each
    if w["master"]:
        b = 28 + (8 if w["star"] else 0)      # master 4+4, g 2, m/v 16, p_bf16 2 (+tau 8)
    else:
        b = 36 if w["star"] else 28
    if w.get("clip"):
        b += 2 * (2 if w["master"] else 4)    # norm pass reads g, the step writes clipped g back
    return b


def cpu_model() -> str:
    """The host CPU's model name (first 'model name' of /proc/cpuinfo), and
    the cores this process may use."""
    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{name}; {len(os.sched_getaffinity(0))} cores available"


def cos_inf_schedule(n_iterations, n_warmup, div_factor, final_div_factor, n_inf):
    """The lr factor of the reference's ``cos_inf`` scheduler
    (src/optim/schedule.py:70-98), restated: a linear warm-up from
    1/div_factor to 1 over n_warmup steps, a cosine down to
    1/(div_factor * final_div_factor) at n_iterations - n_inf, constant after.
    src/main.py:411-423 applies it through torch.optim.lr_scheduler.LambdaLR,
    so optimizer step k (0-based) runs at peak * factor(k)."""
    final = 1.0 / div_factor / final_div_factor
    n_anneal = n_iterations - n_inf

    def factor(step):
        if step < n_warmup:
            return step / n_warmup + (1 - step / n_warmup) / div_factor
        if step < n_anneal:
            t = (step - n_warmup) / (n_anneal - n_warmup)
            return final + 0.5 * (1.0 - final) * (1 + np.cos(np.pi * t))
        return final

    return factor


# C2's scheduler: --scheduler cos_inf with 200 iterations, warm-up 200 / 50 = 4 steps,
# div_factor 1e2, final_div_factor 1e-1 and no constant tail (scripts/launch.sh:176,311)
C2_SCHEDULE = dict(n_iterations=200, n_warmup=4, div_factor=1e2, final_div_factor=1e-1, n_inf=0)


def build_gpu(w, seed=0, foreach=False):
    import torch
    import adana_amd

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    pdtype = torch.bfloat16 if (w["master"] or w.get("state_bf16")) else torch.float32
    groups, params = [], []
    zero_rng = np.random.default_rng(seed + 1)
    # Every parameter first, then every gradient: the order in which a model's
    # constructor and then its backward pass allocate them.
    for gi, shapes in enumerate(w["groups"]):
        ps = []
        for s in shapes:
            p = torch.empty(s, dtype=torch.float32, device=dev).normal_(0.0, 0.02, generator=gen)
            ps.append(torch.nn.Parameter(p.to(pdtype)))
        params += ps
        groups.append(dict(params=ps, weight_decay=w["hp"]["weight_decay"] * w["group_wd"][gi]))
    for gi, shapes in enumerate(w["groups"]):
        for ti, (s, p) in enumerate(zip(shapes, groups[gi]["params"])):
            g = torch.empty(s, dtype=torch.float32, device=dev).normal_(0.0, 1e-3, generator=gen)
            if w["name"] == "c2" and len(s) == 1:
                g.mul_(0.1)
            if w["name"] in ("c3", "north_star", "north_star_clip", "north_star_bf16") and gi == 1 and ti == 0:
                rows = torch.rand(s[0], device=dev, generator=gen) < 0.1     # row-sparse embedding grad
                g.mul_(rows[:, None].to(g.dtype))
            if w["name"] == "c5" and zero_rng.random() < 0.05:
                g.zero_()
            p.grad = g.to(pdtype)
    cls = adana_amd.DANA_STAR_MK4 if w["star"] else adana_amd.ADana
    opt = cls(groups, master_weights=w["master"], use_foreach=foreach, **w["hp"])
    return opt, params


def _sample_shapes(w, max_elems):
    """The workload's first tensors (flattened), up to max_elems elements in
    all, the last one cut short if needed."""
    out, total = [], 0
    for s in (s for shapes in w["groups"] for s in shapes):
        n = min(int(np.prod(s)), max_elems - total)
        if n <= 0:
            break
        out.append(n)
        total += n
    return out, total


def cpu_threads() -> int:
    """Host threads for the CPU baselines: the process's CPU affinity, capped
    by OMP_NUM_THREADS when it is set (the GPU box sets it to its CPU share)."""
    cores = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    return max(cores, 1)


def cpu_baseline(w, target_s=10.0, max_elems=1 << 25):
    """The reference's CPU step, timed on the host's cores on a bounded sample
    of the workload (its first tensors, up to max_elems elements): the step
    restated as torch ops over CPU tensors with the reference's per-tensor
    loop (oracle/torch_ref.py: src/optim/adana.py:162-225,
    src/optim/dana_star_mk4.py:215-294; bit-identical to the reference's own
    eager run, tests/test_torch_restatement.py), torch.set_num_threads over
    the cores, timed twice: as eager ops, and with the update under
    torch.compile as the reference runs it by default (compiled_leg).
    ``value`` is the compiled rate, or the eager one where the compiled leg
    is not timed.  Beside them, the C oracle (oracle/adana_oracle.c, OpenMP)
    on the same sample.  bf16-master workloads time the float32 master
    update; the bf16-state workload (the reference's own bfloat16 path) runs
    all three on bfloat16 tensors."""
    import torch

    from oracle import oracle as O
    from oracle.torch_ref import TorchRefGroup, TorchRefOptimizer

    cores = cpu_threads()
    sizes, total = _sample_shapes(w, max_elems)
    all_elems = sum(int(np.prod(s)) for shapes in w["groups"] for s in shapes)
    hp = w["hp"]
    rng = np.random.default_rng(3)
    ps = [rng.normal(0, 0.02, n).astype(np.float32) for n in sizes]
    gs = [rng.normal(0, 1e-3, n).astype(np.float32) for n in sizes]
    frac = total / all_elems
    bpe = bytes_per_elem(w)

    def timed(step):
        step()                                    # warm-up: first touch of the state
        reps, t0 = 0, time.perf_counter()
        while True:
            step()
            reps += 1
            el = time.perf_counter() - t0
            if el >= target_s or reps >= 50:
                return el / reps, reps

    s16 = bool(w.get("state_bf16"))
    tdt = torch.bfloat16 if s16 else torch.float32
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    tp = [torch.from_numpy(x.copy()).to(tdt) for x in ps]
    tg = [[torch.from_numpy(x).to(tdt) for x in gs]]
    ref = TorchRefOptimizer(groups=[TorchRefGroup(params=tp, lr=hp["lr"], delta=hp["delta"], epsilon=hp["epsilon"],
                                                  weight_decay=hp["weight_decay"])],
                            star=w["star"], peak_lr=hp["lr"], kappa=hp["kappa"], clipsnr=hp["clipsnr"],
                            wd_decaying=hp["wd_decaying"], wd_ts=hp["wd_ts"])
    per_t, reps_t = timed(lambda: ref.step(tg))
    del tp, ref
    compiled = compiled_leg(w, ps, tg, total, bpe, timed, cores)
    torch.set_num_threads(prev)
    del tg

    threads = O.set_threads(cores)
    cps = [O.f32_to_bf16(x) for x in ps] if s16 else [x.copy() for x in ps]
    cgs = [O.f32_to_bf16(x) for x in gs] if s16 else gs
    opt = O.OracleOptimizer(groups=[O.OracleGroup(params=cps, lr=hp["lr"], delta=hp["delta"],
                                                  epsilon=hp["epsilon"], weight_decay=hp["weight_decay"])],
                            star=w["star"], peak_lr=hp["lr"], kappa=hp["kappa"], clipsnr=hp["clipsnr"],
                            wd_decaying=hp["wd_decaying"], wd_ts=hp["wd_ts"], bf16=s16)
    per_c, reps_c = timed(lambda: opt.step([cgs]))
    sample = (f"{total} of the workload's {all_elems} elements ({100 * frac:.2f}%): its first {len(sizes)} tensors, "
              f"{'bf16 parameters and state' if s16 else 'fp32'}")
    eager = {"value": round(total * bpe / per_t / 1e9, 3), "unit": "GB/s", "cores": cores,
             "ms_per_step_sample": round(per_t * 1e3, 3),
             "sample": f"same sample, oracle/torch_ref.py (the reference's step() as torch eager ops, per-tensor "
                       f"loop) with torch.set_num_threads({cores}); {reps_t} timed steps after 1 warm-up"}
    c_oracle = {"value": round(total * bpe / per_c / 1e9, 3), "unit": "GB/s", "cores": threads,
                "ms_per_step_sample": round(per_c * 1e3, 3),
                "sample": f"same sample, oracle/adana_oracle.c with {threads} OpenMP threads, {reps_c} timed steps"}
    head = compiled if compiled.get("value") is not None else eager
    path = "compiled" if head is compiled else "eager"
    how = ("the reference's update under torch.compile (its default path), one wrapper per shape" if head is compiled
           else f"the reference's step() as torch eager ops ({compiled['reason']})")
    return {"value": head["value"], "unit": "GB/s", "cores": cores, "kind": "port", "path": path,
            "cpu_model": cpu_model(),
            "sample": f"{sample}; {how}, oracle/torch_ref.py's per-tensor loop, torch.set_num_threads({cores}) "
                      f"(the process's CPU affinity, capped by OMP_NUM_THREADS); "
                      f"{head['ms_per_step_sample']:.1f} ms/step",
            "sample_fraction": round(frac, 5), "ms_per_step_sample": head["ms_per_step_sample"],
            "compiled": compiled, "eager": eager, "c_oracle": c_oracle}


def compiled_leg(w, ps, tg, total, bpe, timed, cores, max_shapes=8):
    """The reference's default CPU path on the same sample: the per-tensor
    update compiled by torch.compile(dynamic=False, fullgraph=False) with one
    wrapper per tensor shape (src/optim/adana.py:72-79,
    src/optim/dana_star_mk4.py:88-96), Inductor's C++ code on the host's
    cores.  Compilation happens in the warm-up step and is reported apart.
    Samples with more than ``max_shapes`` distinct shapes are not timed:
    every wrapper recompiles the same function, and past torch._dynamo's
    recompile limit (8) the reference's loop runs the eager ops, which the
    eager leg already times."""
    import torch

    from oracle.torch_ref import TorchRefGroup, TorchRefOptimizer, update

    shapes = sorted({x.shape for x in ps})
    if len(shapes) > max_shapes:
        return {"value": None, "reason": f"{len(shapes)} distinct shapes in the sample: past torch._dynamo's "
                                         f"recompile limit the reference's loop runs its eager ops"}
    hp = w["hp"]
    tdt = tg[0][0].dtype
    print(f"[bench] compiling the reference's update with torch.compile for {len(shapes)} shapes",
          file=sys.stderr, flush=True)
    import torch._inductor.config as inductor_config

    # compile in this process: no compile-worker subprocesses started from a
    # process that holds the GPU
    inductor_config.compile_threads = 1
    try:
        wrappers = {}

        def update_fn(p):
            fn = wrappers.get(p.shape)
            if fn is None:
                fn = wrappers[p.shape] = torch.compile(update, dynamic=False, fullgraph=False)
            return fn

        tp = [torch.from_numpy(x.copy()).to(tdt) for x in ps]
        ref = TorchRefOptimizer(groups=[TorchRefGroup(params=tp, lr=hp["lr"], delta=hp["delta"],
                                                      epsilon=hp["epsilon"], weight_decay=hp["weight_decay"])],
                                star=w["star"], peak_lr=hp["lr"], kappa=hp["kappa"], clipsnr=hp["clipsnr"],
                                wd_decaying=hp["wd_decaying"], wd_ts=hp["wd_ts"])
        t0 = time.perf_counter()
        ref.step(tg, update_fn=update_fn)                  # compiles every shape
        compile_s = time.perf_counter() - t0
        per, reps = timed(lambda: ref.step(tg, update_fn=update_fn))
    except Exception as e:                                 # no host compiler, Inductor error
        return {"value": None, "reason": f"torch.compile failed: {type(e).__name__}: {str(e)[:200]}"}
    return {"value": round(total * bpe / per / 1e9, 3), "unit": "GB/s", "cores": cores,
            "ms_per_step_sample": round(per * 1e3, 3), "compile_s": round(compile_s, 1),
            "sample": f"same sample, oracle/torch_ref.py's update under torch.compile(dynamic=False, "
                      f"fullgraph=False), one wrapper per shape (Inductor C++ on {cores} threads); "
                      f"{reps} timed steps after the compiling step"}


def copy_probe(steps):
    """Plain device-to-device copy of a known size (1 GiB read + 1 GiB written
    per launch): the calibration for the HBM FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = (1 << 30) // 4
    a = torch.ones(n, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        b.copy_(a)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"copy_probe_bytes_read": 1 << 30, "copy_probe_bytes_written": 1 << 30,
                      "ms_per_copy": round(ms, 4), "GBps": round(2 * (1 << 30) / ms / 1e6, 1)}))
    return 0


def master_ceiling(n_elems, reps=5):
    """The HBM rate of the bf16-master ADana step's access pattern without its
    arithmetic (stream_probe.hip's stream_master_kernel: fp32 master, m, v and
    bf16 gradient read; fp32 master, m, v and bf16 parameter written; 28 bytes
    per element), the better of 4 and 5 resident workgroups per CU."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "probes", "libadana_probe.so"))
    fn = lib.adana_probe_stream_master
    fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    n = n_elems // 1024 * 1024
    f32 = [torch.zeros(n, device="cuda:0") for _ in range(3)]
    b16 = [torch.zeros(n, dtype=torch.bfloat16, device="cuda:0") for _ in range(2)]
    partials = torch.empty(n // 1024 * 4, device="cuda:0")
    stream = torch.cuda.current_stream()
    best = None
    for cap in (4, 5):
        def run():
            rc = fn(ctypes.c_void_p(f32[0].data_ptr()), ctypes.c_void_p(b16[0].data_ptr()),
                    ctypes.c_void_p(f32[1].data_ptr()), ctypes.c_void_p(f32[2].data_ptr()),
                    ctypes.c_void_p(b16[1].data_ptr()), n, ctypes.c_void_p(partials.data_ptr()), cap,
                    ctypes.c_void_p(stream.cuda_stream))
            if rc != 0:
                raise RuntimeError(f"adana_probe_stream_master failed ({rc})")
        run()
        torch.cuda.synchronize()
        ms = launch_ms(run, reps, stream)
        gbs = 28 * n / (ms * 1e-3) / 1e9
        if best is None or gbs > best[0]:
            best = (gbs, cap, ms)
    del f32, b16, partials
    torch.cuda.empty_cache()
    return {"achieved": round(best[0], 2), "frac": round(best[0] / HBM_PEAK_GBS, 4), "wgs_per_cu": best[1],
            "ms": round(best[2], 4),
            "probe": f"fp32 master, m, v and bf16 gradient of {n} elements read, master, m, v written back "
                     f"in place and the bf16 parameter written, one 16-byte partial per 1024-element chunk: "
                     f"the bf16-master step's access pattern without its arithmetic (stream_probe.hip), "
                     f"mean of {reps} back-to-back launches"}


def stream_ceiling(n_elems, reps=5, star=True):
    """The HBM rate of the step's access pattern without its arithmetic:
    5 fp32 arrays read and 4 written back in place (Dana-Star: p, g, m, v,
    tau), or 4 read and 3 written back (fp32 ADana: p, g, m, v), with the step
    kernel's tiles, load/store policies and residency cap
    (probes/stream_probe.hip), at the workload's element count; the
    better of 3 and 4 resident workgroups per CU.  Also a STREAM copy of the
    same element count in the same style (the better of uncapped and 6)."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "probes", "libadana_probe.so"))
    fn = lib.adana_probe_stream_5r4w if star else lib.adana_probe_stream_4r3w
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    n_read, n_write = (5, 4) if star else (4, 3)
    bpe = 4 * (n_read + n_write)
    n = n_elems // 1024 * 1024
    arrays = [torch.zeros(n, device="cuda:0") for _ in range(5)]
    partials = torch.empty(n // 1024 * 4, device="cuda:0")
    ptrs = (ctypes.c_void_p * 5)(*[a.data_ptr() for a in arrays])
    stream = torch.cuda.current_stream()
    best = None
    for cap in (3, 4):
        def run():
            rc = fn(ptrs, n, ctypes.c_void_p(partials.data_ptr()), cap, ctypes.c_void_p(stream.cuda_stream))
            if rc != 0:
                raise RuntimeError(f"adana_probe_stream_5r4w failed ({rc})")
        run()
        torch.cuda.synchronize()
        ms = launch_ms(run, reps, stream)
        gbs = bpe * n / (ms * 1e-3) / 1e9
        if best is None or gbs > best[0]:
            best = (gbs, cap, ms)
    mix = {"achieved": round(best[0], 2), "frac": round(best[0] / HBM_PEAK_GBS, 4), "wgs_per_cu": best[1],
           "ms": round(best[2], 4),
           "probe": f"{n_read} fp32 arrays of {n} elements read, {n_write} written back in place, one 16-byte "
                    f"partial per 1024-element chunk: the step kernel's access pattern without its arithmetic "
                    f"(stream_probe.hip), mean of {reps} back-to-back launches"}
    # STREAM copy (arrays[1] -> arrays[0]) in the same style, the better of uncapped and 6 per CU
    cp = lib.adana_probe_copy
    cp.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                   ctypes.c_void_p]
    cp.restype = ctypes.c_int
    best_copy = None
    for cap in (0, 6):
        def run_copy():
            rc = cp(ctypes.c_void_p(arrays[0].data_ptr()), ctypes.c_void_p(arrays[1].data_ptr()), n,
                    ctypes.c_void_p(partials.data_ptr()), cap, ctypes.c_void_p(stream.cuda_stream))
            if rc != 0:
                raise RuntimeError(f"adana_probe_copy failed ({rc})")
        run_copy()
        torch.cuda.synchronize()
        ms = launch_ms(run_copy, reps, stream)
        gbs = 8 * n / (ms * 1e-3) / 1e9
        if best_copy is None or gbs > best_copy[0]:
            best_copy = (gbs, cap)
    del arrays, partials
    torch.cuda.empty_cache()
    copy = {"achieved": round(best_copy[0], 2), "frac": round(best_copy[0] / HBM_PEAK_GBS, 4),
            "wgs_per_cu": best_copy[1], "probe": f"STREAM copy of {n} fp32 elements, same access style"}
    return mix, copy


def settle_gc():
    """Run Python's cyclic garbage collector once and freeze what survives,
    before a workload's warm-up steps.  A full collection over the setup's
    objects (~270K after importing torch and building the north-star state)
    takes ~70 ms; one that came due inside a timed loop would measure the
    bench's setup, not the step.  Collecting before the warm-up rather than
    right before the timed loop leaves the warm-up steps to bring the GPU's
    clock back up after the pause."""
    gc.collect()
    gc.freeze()


def launch_ms(run, reps, stream):
    """Mean device time of ``reps`` back-to-back calls of ``run`` (after one
    untimed call), from events at the two ends only: an event between two
    launches leaves the GPU idle for a few microseconds, which would count
    against a short probe."""
    import torch

    run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        run()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def same_cap_probe(run_step, w, n_elems, n_tensors, reps=5, rounds=3):
    """The step and its access pattern without the arithmetic at the step's
    own residency cap, timed alternately in one process (``rounds`` rounds of
    ``reps`` back-to-back steps, then ``reps`` back-to-back probe launches):
    the probe is probes/stream_probe.hip's 5-in/4-out (Dana-Star), 4-in/3-out
    (ADana) or bf16-master kernel, and the cap is the one the step's launch
    takes (4 resident workgroups per CU on grids of at least 64 chunks per
    CU, none on smaller grids or for Dana-Star's pow instance on lists of
    small tensors).  Returns None for workloads without a probe (bfloat16
    state)."""
    import ctypes

    import torch

    if w.get("state_bf16"):
        return None
    n = n_elems // 1024 * 1024
    n_chunks = n // 1024
    small = n_chunks < 64 * n_tensors
    general_pow = w["star"] and 0.0 < 1.0 - w["hp"]["kappa"] < 1.0
    cap = 0 if (n_chunks < 64 * 256 or (general_pow and small)) else 4
    lib = ctypes.CDLL(os.path.join(ROOT, "probes", "libadana_probe.so"))
    stream = torch.cuda.current_stream()
    partials = torch.empty(n_chunks * 4, device="cuda:0")
    if w["master"]:
        fn = lib.adana_probe_stream_master
        fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        fn.restype = ctypes.c_int
        f32 = [torch.zeros(n, device="cuda:0") for _ in range(3)]
        b16 = [torch.zeros(n, dtype=torch.bfloat16, device="cuda:0") for _ in range(2)]
        bpe = 28
        args = [ctypes.c_void_p(f32[0].data_ptr()), ctypes.c_void_p(b16[0].data_ptr()),
                ctypes.c_void_p(f32[1].data_ptr()), ctypes.c_void_p(f32[2].data_ptr()),
                ctypes.c_void_p(b16[1].data_ptr()), n, ctypes.c_void_p(partials.data_ptr()), cap,
                ctypes.c_void_p(stream.cuda_stream)]
        keep = (f32, b16)
        what = "bf16-master pattern (28 B/element)"
    else:
        fn = lib.adana_probe_stream_5r4w if w["star"] else lib.adana_probe_stream_4r3w
        fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        fn.restype = ctypes.c_int
        arrays = [torch.zeros(n, device="cuda:0") for _ in range(5 if w["star"] else 4)]
        ptrs = (ctypes.c_void_p * 5)(*([a.data_ptr() for a in arrays] + [0] * (5 - len(arrays))))
        bpe = 36 if w["star"] else 28
        args = [ptrs, n, ctypes.c_void_p(partials.data_ptr()), cap, ctypes.c_void_p(stream.cuda_stream)]
        keep = (arrays, ptrs)
        what = ("5 fp32 arrays read, 4 written back" if w["star"] else "4 fp32 arrays read, 3 written back")

    def run_probe():
        if fn(*args) != 0:
            raise RuntimeError("stream probe launch failed")

    steps, probes = [], []
    for _ in range(rounds):
        steps.append(launch_ms(run_step, reps, stream))
        probes.append(launch_ms(run_probe, reps, stream))
    del keep, partials
    torch.cuda.empty_cache()
    step_ms, probe_ms = float(np.median(steps)), float(np.median(probes))
    probe_gbs = bpe * n / (probe_ms * 1e-3) / 1e9
    return {"wgs_per_cu": cap, "probe_ms": round(probe_ms, 4), "probe_achieved": round(probe_gbs, 2),
            "probe_frac": round(probe_gbs / HBM_PEAK_GBS, 4), "step_ms": round(step_ms, 4),
            "step_over_probe": round(probe_ms / step_ms, 4),
            "note": f"the step's access pattern without its arithmetic ({what}, stream_probe.hip) at the "
                    f"step's own residency cap ({cap or 'none'} workgroups per CU), timed alternately with the "
                    f"step in this process: {rounds} rounds of {reps} back-to-back launches each, medians; "
                    f"step_over_probe = probe ms / step ms (the step's rate as a fraction of the probe's)"}


def stream_sweep(args):
    """The memory system's ceiling for the north-star step's access pattern.

    The step streams 5 fp32 arrays in and 4 back out (36 B per element) over
    2.65e9 elements.  This workload times that pattern without arithmetic
    (probes/stream_probe.hip) in every launch shape tried, on arrays of the
    north-star size, in a fixed launch order so that a ``rocprofv3 --pmc``
    run over the same command can attribute every dispatch:
      * one-shot workgroups (the step's shape) at 1..8 resident workgroups per
        CU and uncapped;
      * the same five arrays read only and four written only, and a copy;
      * then (after the separate arrays are freed) the one-shot shape at the
        step's cap of 4 with the five arrays placed in one allocation,
        ``k * (n + 4 Mi)`` floats plus ``k * skew`` bytes from its start
        (array k = 0..4): the rate's dependence on the arrays' relative
        placement, which the caller's allocator decides for p and g.
    Each configuration is launched 1 + reps times (one warm-up), in two
    rounds; the JSON line lists the launch order and each configuration's
    best median.  ``value`` is the best 5-read/4-write rate over separately
    allocated arrays (the placement leg is reported beside it)."""
    import ctypes

    import torch

    lib = ctypes.CDLL(os.path.join(ROOT, "probes", "libadana_probe.so"))
    P, I64, INT = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    for name in ("adana_probe_stream_5r4w", "adana_probe_stream_5r0w", "adana_probe_stream_0r4w"):
        getattr(lib, name).argtypes = [P, I64, P, INT, P]
        getattr(lib, name).restype = INT
    lib.adana_probe_copy.argtypes = [P, P, I64, P, INT, P]
    lib.adana_probe_copy.restype = INT
    n = 2645527040 // 1024 * 1024
    arrays = [torch.zeros(n, device="cuda:0") for _ in range(5)]
    partials = torch.empty(n // 1024 * 4, device="cuda:0")
    ptrs = (ctypes.c_void_p * 5)(*[a.data_ptr() for a in arrays])
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    part = ctypes.c_void_p(partials.data_ptr())
    a0, a1 = ctypes.c_void_p(arrays[0].data_ptr()), ctypes.c_void_p(arrays[1].data_ptr())
    cfgs = []                                   # (name, bytes per launch, launch)
    for cap in (1, 2, 3, 4, 5, 6, 7, 8, 0):
        cfgs.append((f"5r4w one-shot cap {cap or 'none'}", 36 * n,
                     lambda cap=cap: lib.adana_probe_stream_5r4w(ptrs, n, part, cap, st)))
    for cap in (3, 4, 0):
        cfgs.append((f"5r0w read-only cap {cap or 'none'}", 20 * n,
                     lambda cap=cap: lib.adana_probe_stream_5r0w(ptrs, n, part, cap, st)))
    for cap in (3, 4, 0):
        cfgs.append((f"0r4w write-only cap {cap or 'none'}", 16 * n,
                     lambda cap=cap: lib.adana_probe_stream_0r4w(ptrs, n, part, cap, st)))
    for cap in (4, 0):
        cfgs.append((f"1r1w copy cap {cap or 'none'}", 8 * n,
                     lambda cap=cap: lib.adana_probe_copy(a0, a1, n, part, cap, st)))
    reps = max(2, args.steps)
    best = {}
    order = []

    def one(rnd, name, nbytes, fn):
        print(f"[bench] stream_sweep round {rnd}: {name}", file=sys.stderr, flush=True)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        if fn() != 0:
            raise RuntimeError(f"probe launch failed: {name}")
        stream = torch.cuda.current_stream()
        for k in range(reps):
            ev[k].record(stream)
            if fn() != 0:
                raise RuntimeError(f"probe launch failed: {name}")
        ev[-1].record(stream)
        torch.cuda.synchronize()
        order.append([name, 1 + reps])
        ms = float(np.median([ev[k].elapsed_time(ev[k + 1]) for k in range(reps)]))
        tbs = nbytes / (ms * 1e-3) / 1e12
        if name not in best or tbs > best[name]["TB/s"]:
            best[name] = {"TB/s": round(tbs, 3), "ms": round(ms, 3), "frac": round(tbs * 1e3 / HBM_PEAK_GBS, 4)}

    def sweep(cfgs):
        for rnd in range(2):
            for name, nbytes, fn in cfgs:
                one(rnd, name, nbytes, fn)

    sweep(cfgs)
    # placement leg: one allocation, array k at k * (n + 4 Mi) floats + k * skew bytes
    del arrays, ptrs, a0, a1, cfgs
    torch.cuda.empty_cache()
    slot = n + (4 << 20)
    buf = torch.zeros(5 * slot, device="cuda:0")
    place = []
    for skew in (0, 4096, 8192, 1 << 20, (2 << 20) + 8192):
        pp = (ctypes.c_void_p * 5)(*[buf.data_ptr() + 4 * k * slot + k * skew for k in range(5)])
        place.append((f"placement: one allocation, skew {skew} B per array, cap 4", 36 * n,
                      lambda pp=pp: lib.adana_probe_stream_5r4w(pp, n, part, 4, st)))
    sweep(place)
    del buf
    top = max((v["TB/s"], k) for k, v in best.items() if k.startswith("5r4w"))
    print(json.dumps({"metric": "5-read/4-write stream ceiling at the north-star size (TB/s)", "value": top[0],
                      "unit": "TB/s", "n_gpus": 1, "steps": reps, "warmup": 1, "ms_per_step": best[top[1]]["ms"],
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                      "data": "synthetic (zeros)",
                      "config": {"workload": "stream_sweep", "elements": n, "best": top[1]},
                      "configs": best, "launch_order": order}), flush=True)
    return 0


def consumer_bench(args):
    """Time a consumer of the optimizer state on the GPU against the
    reference's host path on a bounded sample."""
    import torch
    import adana_amd
    from adana_amd.tau_stats import order_stat_indices

    tau = args.workload in ("tau_stats", "tau_stats_spread")
    w = workload("north_star" if tau else "c5")
    print(f"[bench] {args.workload}: building {w['name']} state on cuda:0", file=sys.stderr, flush=True)
    opt, params = build_gpu(w)
    for _ in range(3):
        opt.step()
    torch.cuda.synchronize()
    plain = None
    if tau:
        taus = [opt.state[p]["tau"] for p in params]
        n_elems = sum(t.numel() for t in taus)
        if args.workload == "tau_stats_spread":
            # After 3 steps with the same gradients nearly every tau sits in one narrow
            # cluster.  A run's tau is spread over (0, 1): Beta(2, 5) draws here
            # (X / (X + Y), X ~ Gamma(2), Y ~ Gamma(5), each -log of a product of uniforms).
            gen = torch.Generator(device="cuda:0")
            gen.manual_seed(7)
            for t in taus:
                u = lambda: torch.rand(t.shape, device="cuda:0", generator=gen)  # noqa: E731
                x = -torch.log(u() * u())
                y = -torch.log(u() * u() * u() * u() * u())
                t.copy_(x / (x + y))
            torch.cuda.synchronize()
        run = lambda: adana_amd.extract_tau_statistics(opt)       # noqa: E731
        unit_bytes = 4 * n_elems                                  # tau scanned once per pass
        from adana_amd import tau_stats as T
        flat = [T._contiguous(t) for t in taus]
        plan = T._batch_plan(tuple(f.numel() for f in flat))[:3]

        def plain(compact):                                       # the selection alone, either way
            T._select(flat, *plan, compact=compact)
    else:
        name = "dana-star-mk4"
        run = lambda: adana_amd.log_optimizer_schedules(opt, name)  # noqa: E731
        n_elems = len(params)
        unit_bytes = 20 * n_elems                                 # five fp32 diagnostics each
    settle_gc()
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    select_ms = None
    if plain is not None:
        # the device selection alone (no result dictionaries), with and without
        # compaction, interleaved call by call
        t = {True: [], False: []}
        for rep in range(args.steps + 1):
            for c in (True, False):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                plain(c)
                torch.cuda.synchronize()
                if rep:
                    t[c].append((time.perf_counter() - t0) * 1e3)
        select_ms = {"compaction": round(float(np.median(t[True])), 4),
                     "no_compaction": round(float(np.median(t[False])), 4),
                     "note": "median over the steps of the device selection alone (adana_order_stats), "
                             "interleaved; compaction is the default"}
    # the reference's host path, timed on a bounded sample
    if tau:
        sample = [t for t in taus][:4]                            # first four tensors of the list
        ns = sum(t.numel() for t in sample)
        c0 = time.perf_counter()
        for t in sample:
            x = t.detach().cpu().flatten().numpy()                # tau_stats_collector.py:151
            srt = np.sort(x)                                      # :355
            idx = order_stat_indices(x.size)
            _ = srt[idx], srt[(x.size - 1) - idx]
        cpu_ms = (time.perf_counter() - c0) * 1e3
        cpu = {"value": round(ns / (cpu_ms * 1e-3) / 1e9, 4), "unit": "Gelem/s", "cores": 1,
               "kind": "port", "cpu_model": cpu_model(),
               "sample": f"first 4 tau tensors ({ns} elements): tau.cpu(), np.sort, order-statistic picks as "
                         f"src/optim/tau_stats_collector.py:131-160, {cpu_ms:.0f} ms"}
        value = n_elems / (ms * 1e-3) / 1e9
        metric = ("tau order statistics over the north-star state (elements/s)" if args.workload == "tau_stats"
                  else "tau order statistics over north-star-sized tau, Beta(2, 5) values (elements/s)")
        unit = "Gelem/s"
    else:
        c0 = time.perf_counter()
        vals = []
        for group in opt.param_groups:                            # src/optim/utils.py:572-596
            for p in group["params"]:
                st = opt.state[p]
                for k in ("current_alpha", "current_kappa_factor", "auto_factor_mean", "m_norm"):
                    vals.append(st[k].item())
        cpu_ms = (time.perf_counter() - c0) * 1e3
        cpu = {"value": round(n_elems / (cpu_ms * 1e-3), 1), "unit": "tensors/s", "cores": 1,
               "kind": "port", "cpu_model": cpu_model(),
               "sample": f"all {n_elems} tensors, value by value (.item() per diagnostic) as "
                         f"src/optim/utils.py:572-596, {cpu_ms:.1f} ms"}
        value = n_elems / (ms * 1e-3)
        metric, unit = "log_optimizer_schedules over 10,000 tensors (tensors/s)", "tensors/s"
    print(json.dumps({"metric": metric, "value": round(value, 4), "unit": unit, "n_gpus": 1,
                      "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
                      "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
                      "data": "synthetic",
                      "config": {"workload": args.workload, "state_of": w["name"], "elements": n_elems,
                                 "bytes_read_once": unit_bytes,
                                 **({"tau": "Beta(2, 5) draws over the state's tau tensors"}
                                    if args.workload == "tau_stats_spread" else {})},
                      **({"select_ms": select_ms} if select_ms is not None else {}),
                      "cpu_baseline": cpu}), flush=True)
    return 0


def manau_model(seed=0, grad_seed=None):
    """The north-star model's parameter list as Manau takes it (named groups:
    the 2-D Linear weights with weight decay 0.1; the tied embedding and the
    LayerNorm weights without), on cuda:0, with N(0, 1e-3) gradients
    (embedding rows nonzero w.p. 0.1), and Manau's hyper-parameters."""
    import torch

    d, layers, vocab = 2560, 32, 50304
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    decay, nodecay = [], [("transformer.wte.weight", (vocab, d))]
    for l in range(layers):
        decay += [(f"transformer.h.{l}.attn.c_attn.weight", (3 * d, d)),
                  (f"transformer.h.{l}.attn.c_proj.weight", (d, d)),
                  (f"transformer.h.{l}.mlp.c_fc.weight", (4 * d, d)),
                  (f"transformer.h.{l}.mlp.c_proj.weight", (d, 4 * d))]
        nodecay += [(f"transformer.h.{l}.ln_1.weight", (d,)), (f"transformer.h.{l}.ln_2.weight", (d,))]
    nodecay += [("transformer.ln_f.weight", (d,))]
    groups, params = [], []
    for named, wd in ((decay, 0.1), (nodecay, 0.0)):
        ps = [torch.nn.Parameter(torch.empty(s, device=dev).normal_(0, 0.02, generator=gen)) for _, s in named]
        groups.append({"params": ps, "param_names": [n for n, _ in named], "weight_decay": wd})
        params += ps
    manau_grads(params, groups[1]["params"][0], gen if grad_seed is None else grad_seed)
    hp = dict(lr=2e-2, kappa=0.85, clipsnr=2.0, delta=8.0, wd_decaying=True, wd_ts=10.0)
    return groups, params, hp


def manau_grads(params, emb, gen):
    """N(0, 1e-3) gradients for every parameter, the embedding's rows nonzero
    with probability 0.1 (``gen``: a cuda generator or an integer seed)."""
    import torch

    if isinstance(gen, int):
        seed, gen = gen, torch.Generator(device="cuda:0")
        gen.manual_seed(seed)
    for p in params:
        p.grad = torch.empty_like(p).normal_(0, 1e-3, generator=gen)
    rows = (torch.rand((emb.shape[0], 1), device=emb.device, generator=gen) < 0.1).float()
    emb.grad.mul_(rows)                                          # row-sparse embedding gradient


def manau_bench(args):
    """Manau (src/optim/manau.py) on the north-star model: Muon for the 2-D
    Linear weights, the HIP Dana-Star-MK4 branch for the tied embedding and
    the 1-D LayerNorm weights.  ``value`` is the Dana branch's algorithmic
    GB/s (36 B per element, HIP events around its launches); the whole Manau
    step, bfloat16 Newton-Schulz included, is reported beside it."""
    import contextlib
    import io

    import torch

    import adana_amd

    groups, params, hp = manau_model()
    with contextlib.redirect_stdout(io.StringIO()):
        opt = adana_amd.Manau(groups, **hp)
    dana = [p for p in params if not opt.state[p]["use_muon"]]
    n_dana = sum(p.numel() for p in dana)
    n_muon = sum(p.numel() for p in params) - n_dana
    print(f"[bench] manau: {n_muon} Muon + {n_dana} Dana params", file=sys.stderr, flush=True)
    settle_gc()
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()

    def timed(fn, k):                                            # events at the loop's two ends only
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(k):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / k, e0.elapsed_time(e1) / k

    full_wall, full_dev = timed(opt.step, args.steps)
    dana_wall, dana_dev = timed(opt._dana_step, args.steps)    # the branch alone, as step() runs it last
    algo = 36 * n_dana
    achieved = algo / (dana_dev * 1e-3) / 1e9
    result = {
        "metric": "Manau Dana-Star-MK4 branch step, achieved HBM GB/s (north-star model's embedding + 1-D params)",
        "value": round(algo / (dana_wall * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(dana_wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "manau", "optimizer": "Manau", "dana_params": n_dana, "muon_params": n_muon,
                   "bytes_per_elem": 36, "hyperparams": hp, "grads": "N(0,1e-3); embedding rows nonzero w.p. 0.1"},
        "kernel_ms_per_step": round(dana_dev, 4),
        "full_manau_step_ms": round(full_wall, 3),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "mta_step_kernel (Manau variant) + combine_kernel"},
    }
    del opt, params, groups
    torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        from oracle import oracle as O

        threads = O.set_threads(cpu_threads())
        rng = np.random.default_rng(3)
        n = 1 << 25
        arrs = [rng.normal(0, 0.02, n).astype(np.float32), rng.normal(0, 1e-3, n).astype(np.float32)]
        m, v, tau = (np.zeros(n, np.float32) for _ in range(3))
        sc = O.manau_scalars(lr=2e-2, step=5, alpha=8 / 13, kappa=0.85, mk4A=0.0, mk4B=0.0, clipsnr=2.0,
                             epsilon=1e-8, weight_decay=0.0, wd_decaying=True, wd_ts=10.0)
        O.manau_element_step(arrs[0], arrs[1], m, v, tau, sc)
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < args.cpu_seconds:
            O.manau_element_step(arrs[0], arrs[1], m, v, tau, sc)
            reps += 1
        per = (time.perf_counter() - t0) / reps
        result["cpu_baseline"] = {"value": round(36 * n / per / 1e9, 3), "unit": "GB/s", "cores": threads,
                                  "kind": "port", "cpu_model": cpu_model(),
                                  "sample": f"{n} elements, {reps} steps of oracle/adana_oracle.c's Manau branch "
                                            f"with {threads} OpenMP threads, {per * 1e3:.1f} ms/step"}
    print(json.dumps(result), flush=True)
    return 0


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warm-up steps (default 3; 40 for c5)")
    ap.add_argument("--workload", default="north_star",
                    choices=["north_star", "north_star_clip", "north_star_bf16", "c1", "c2", "c3", "c4", "c5",
                             "copy_probe", "tau_stats", "tau_stats_spread", "diag_readout", "manau",
                             "stream_sweep"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ceiling-probe", action="store_true",
                    help="skip the 5-read/4-write stream probe reported as roofline.mix_ceiling")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--foreach", action="store_true",
                    help="step with use_foreach=True (the reference's foreach path's numerics)")
    args = ap.parse_args()
    if args.warmup is None:
        args.warmup = workload(args.workload).get("default_warmup", 3) if args.workload in STEP_WORKLOADS else 3
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build's step is single-GPU "
              f"(--gpus {args.gpus} requested); the update is element-wise, so each rank would run it on "
              f"its own shard", file=sys.stderr)
        return 2

    import __graft_entry__
    import torch

    __graft_entry__.ensure_built()      # a fresh checkout has no built libraries
    gc.freeze()                         # the imports' objects: later collections skip them
    if args.workload == "copy_probe":
        return copy_probe(args.steps)
    if args.workload in ("tau_stats", "tau_stats_spread", "diag_readout"):
        return consumer_bench(args)
    if args.workload == "manau":
        return manau_bench(args)
    if args.workload == "stream_sweep":
        return stream_sweep(args)
    w = workload(args.workload)
    print(f"[bench] workload {w['name']} ({w['optimizer']}): building on cuda:0", file=sys.stderr,
          flush=True)
    opt, params = build_gpu(w, foreach=args.foreach)
    n_elems = sum(p.numel() for p in params)
    bpe = bytes_per_elem(w)
    algo_bytes = n_elems * bpe
    grad_norms = []
    sched = None
    if w["schedule"] == "cos_inf":
        # src/main.py:411-423: LambdaLR sets group['lr'] = peak * factor(k) after step k
        sched = torch.optim.lr_scheduler.LambdaLR(opt, cos_inf_schedule(**C2_SCHEDULE))

    def one_step(_k):
        if w.get("clip"):
            grad_norms.append(opt.clip_grad_norm_(w["clip"]).item())   # src/optim/base.py:250-257
        opt.step()
        if sched is not None:
            sched.step()

    settle_gc()
    torch.cuda.synchronize()
    for k in range(args.warmup):
        one_step(k)
    torch.cuda.synchronize()
    print(f"[bench] warm-up done ({args.warmup} steps); timing {args.steps}", file=sys.stderr,
          flush=True)
    stream = torch.cuda.current_stream()
    # The timed loop holds events at its two ends only: an event recorded between
    # steps leaves the GPU idle for ~3 us (C1 0.0282 -> 0.0249 ms per step without
    # them), which is the harness's cost, not the step's.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for k in range(args.steps):
        one_step(args.warmup + k)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    kern_ms = e0.elapsed_time(e1) / args.steps
    # the per-step spread, from the next steps bracketed one by one (markers included)
    events = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    for k in range(args.steps):
        events[k].record(stream)
        one_step(args.warmup + args.steps + k)
    events[-1].record(stream)
    torch.cuda.synchronize()
    dev_ms = [events[k].elapsed_time(events[k + 1]) for k in range(args.steps)]
    achieved = algo_bytes / (kern_ms * 1e-3) / 1e9
    value = algo_bytes / (ms_per_step * 1e-3) / 1e9

    host = None
    if not w.get("clip"):
        # Host time of opt.step() alone (its launches are asynchronous), three ways:
        #  * same_grads: the same gradient tensors every step;
        #  * reference_loop: the reference's training loop (src/optim/base.py:250-289):
        #    zero_grad(set_to_none=True), a backward pass that gives every parameter a
        #    new gradient tensor (autograd allocates it from the caching allocator; the
        #    loss sum((p * w).sum()) makes that gradient w, the workload's gradient),
        #    then a host synchronisation (the loop's grad_norm.item()) before step();
        #  * moved_every_step: every gradient replaced by a tensor at another address
        #    before each step (the worst case for re-pointing).
        cur = [p.grad for p in params]
        alt = [g.clone() for g in cur]

        def backward():
            with torch.enable_grad():
                loss = torch.stack([(p * g).sum() for p, g in zip(params, cur)]).sum()
            loss.backward()

        def host_ms(mode, k0):
            t = []
            for k in range(args.steps):
                if mode == "moved_every_step":
                    for p, g in zip(params, alt if k % 2 == 0 else cur):
                        p.grad = g
                elif mode == "reference_loop":
                    opt.zero_grad(set_to_none=True)
                    backward()
                    torch.cuda.synchronize()
                h0 = time.perf_counter()
                one_step(k0 + k)
                t.append((time.perf_counter() - h0) * 1e3)
            torch.cuda.synchronize()
            return round(float(np.median(t)), 4)

        k0 = args.warmup + 2 * args.steps
        host = {mode: host_ms(mode, k0 + i * args.steps)
                for i, mode in enumerate(("same_grads", "reference_loop", "moved_every_step"))}
        host["note"] = ("median host time of opt.step() alone (launches are asynchronous): same_grads, the same "
                        "gradient tensors every step; reference_loop, zero_grad(set_to_none=True), a backward pass "
                        "that gives every parameter a new gradient tensor, and a host synchronisation before each "
                        "step, as src/optim/base.py:250-289 runs it; moved_every_step, every p.grad replaced "
                        "by a tensor at another address before each step")
        for p, g in zip(params, cur):
            p.grad = g
        del alt, cur

    same_cap = None
    if not args.no_ceiling_probe and not w.get("clip"):
        print("[bench] timing the step and its access pattern at the step's residency cap, alternately",
              file=sys.stderr, flush=True)
        k_sc = [args.warmup + 5 * args.steps]

        def run_step():
            one_step(k_sc[0])
            k_sc[0] += 1

        same_cap = same_cap_probe(run_step, w, n_elems, len(params))

    cold = None
    if algo_bytes < MALL_BYTES:
        # the step's working set fits in the 256 MB MALL (Infinity Cache) and stays there between
        # back-to-back steps: also time each step after evicting it with a 1 GiB write
        flush = torch.empty(1 << 28, device="cuda:0")
        cold_ms = []
        for k in range(args.steps):
            flush.fill_(float(k))
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            one_step(args.warmup + 4 * args.steps + k)
            e1.record(stream)
            torch.cuda.synchronize()
            cold_ms.append(e0.elapsed_time(e1))
        del flush
        cms = float(np.mean(cold_ms))
        cold = {"kernel_ms_per_step": round(cms, 4), "achieved": round(algo_bytes / (cms * 1e-3) / 1e9, 2),
                "frac": round(algo_bytes / (cms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "note": "MALL evicted before each step by writing a 1 GiB buffer; events bracket the step only"}

    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{w['name']}.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    result = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16+f32" if w["master"] else ("bf16" if w.get("state_bf16") else "f32"), "data": "synthetic",
        "config": {"workload": w["name"], "optimizer": w["optimizer"], "params": n_elems,
                   "tensors": len(params), "bytes_per_elem": bpe,
                   "algorithmic_bytes_per_step": algo_bytes, "grads": w["grad_note"],
                   "hyperparams": w["hp"], "master_weights": w["master"],
                   "numerics": ("compiled, use_foreach=True (the reference's foreach kernel under torch.compile)"
                                if args.foreach else "compiled (the reference's default torch.compile path)"),
                   "parallelism": "single GPU",
                   **({"warmup_note": w["warmup_note"]} if "warmup_note" in w else {}),
                   **({"lr_schedule": dict(C2_SCHEDULE, kind="cos_inf (src/optim/schedule.py:70-98)",
                                           via="torch.optim.lr_scheduler.LambdaLR")} if sched else {}),
                   **({"grad_clip": w["clip"], "first_grad_norm": grad_norms[0]} if w.get("clip") else {})},
        "kernel_ms_per_step": round(kern_ms, 4),
        **({"host_step_ms": host} if host else {}),
        **({"mall_cold": cold} if cold else {}),
        "kernel_ms_p90": round(float(np.percentile(dev_ms, 90)), 4),
        "timing_note": "value and ms_per_step: wall time of the timed loop (Python's garbage collector run and "
                       "the setup's objects frozen before the warm-up); kernel_ms_per_step: events at the loop's "
                       "two ends only; kernel_ms_p90: the next steps with an event between every two",
        "params_per_s": round(n_elems / (ms_per_step * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "kernel": ("grad_sumsq_kernel + sumsq_fold_kernel + clip_finalize_kernel + "
                                "mta_step_kernel + combine_kernel (HIP events at the two ends of the timed steps)"
                                if w.get("clip") else
                                "mta_step_kernel + combine_kernel (HIP events at the two ends of the timed steps)")},
    }
    del opt, params
    torch.cuda.empty_cache()
    if same_cap is not None:
        result["roofline"]["same_cap_probe"] = same_cap
    if bpe in (28, 36) and not w["master"] and not args.no_ceiling_probe:
        # the same access pattern without the arithmetic: what the memory system allows this mix
        print("[bench] timing the stream probe of the step's access pattern", file=sys.stderr, flush=True)
        ceiling, copy = stream_ceiling(n_elems, star=bpe == 36)
        result["roofline"]["mix_ceiling"] = ceiling
        result["roofline"]["frac_of_mix_ceiling"] = round(achieved / ceiling["achieved"], 4)
        result["roofline"]["stream_copy"] = copy
        result["roofline"]["frac_of_stream_copy"] = round(achieved / copy["achieved"], 4)
    if bpe == 28 and w["master"] and not w.get("clip") and not args.no_ceiling_probe:
        print("[bench] timing the bf16-master stream probe", file=sys.stderr, flush=True)
        ceiling = master_ceiling(n_elems)
        result["roofline"]["mix_ceiling"] = ceiling
        result["roofline"]["frac_of_mix_ceiling"] = round(achieved / ceiling["achieved"], 4)
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle baseline", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(w, target_s=args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
