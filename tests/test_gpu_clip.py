"""GPU parity of gradient-norm clipping: ``adana_amd.clip_grad_norm_`` (the
norm pass + in-place scaling kernels) and its step-fused form
(``opt.clip_grad_norm_`` then ``opt.step()``), against the oracle's
restatement of torch.nn.utils.clip_grad_norm_ with norm_type 2
(oracle.clip_norms / clip_coef / clip_scale, pinned to torch's own CPU
function in tests/test_clip_cpu.py).  The reference's loop clips every step
before opt.step() (src/optim/base.py:250-257).

Bars (stated per assertion):
  * total norm: within 2e-6 relative of the oracle's binary64 value and of
    torch's clip_grad_norm_ run on a copy of the gradients on the GPU (torch
    reduces in binary32, so neither is bit-defined); bfloat16 totals within
    one bfloat16 ulp;
  * the coefficient and every clipped gradient: bit-exact against the
    oracle's torch-order formula evaluated on the GPU's total;
  * a fused step: the unclipped step's bars (tests/test_gpu_parity.py)
    against the oracle stepping on the clipped gradients.
"""
import ctypes

import numpy as np
import pytest
import torch

from helpers import ulp_diff
from test_gpu_parity import DEV, Pair, _gpt_list, _normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]


def _bits(t):
    return t.detach().float().cpu().numpy().view(np.uint32)


def _mixed_list(rng, bf16):
    """Matrices, vectors, sizes that are not multiples of 4, an empty tensor
    and an unaligned view (element-wise path)."""
    shapes = [(257, 96), (96,), (1,), (2,), (3,), (5,), (7,), (0,), (1000, 33), (4096,)]
    dt = torch.bfloat16 if bf16 else torch.float32
    params, grads = [], []
    for s in shapes:
        params.append(torch.nn.Parameter(torch.zeros(s, dtype=dt, device=DEV)))
        grads.append(torch.from_numpy(_normal(rng, s, 1e-2)).to(DEV, dt))
    base = torch.from_numpy(_normal(rng, (1 + 999,), 1e-2)).to(DEV, dt)
    params.append(torch.nn.Parameter(torch.zeros(999, dtype=dt, device=DEV)))
    grads.append(base[1:])                                   # 2- or 4-byte offset view
    for p, g in zip(params, grads):
        p.grad = g
    return params


def _check_total(total, grads_np, bf16, O, torch_total=None):
    t = float(total.float().item())
    _, ot = O.clip_norms(grads_np, bf16)
    if bf16:
        assert abs(t - float(ot)) <= float(np.spacing(np.float32(ot))) * 65536, (t, ot)
    else:
        assert abs(t - float(ot)) <= 2e-6 * abs(float(ot)), (t, ot)
        if torch_total is not None:
            tt = float(torch_total.float().item())
            assert abs(t - tt) <= 2e-6 * abs(tt), (t, tt)
    return np.float32(t)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("max_norm", [0.5, 1e3])
def test_clip_standalone(oracle_mod, bf16, max_norm):
    """clip_grad_norm_ without an optimizer: norm pass + in-place scale pass."""
    import adana_amd

    print("case: standalone clip bf16", bf16, "max_norm", max_norm, flush=True)
    O = oracle_mod
    rng = np.random.default_rng(11)
    params = _mixed_list(rng, bf16)
    orig = [p.grad.float().cpu().numpy().copy() for p in params]
    clones = [torch.nn.Parameter(p.detach().clone()) for p in params]
    for c, p in zip(clones, params):
        c.grad = p.grad.clone()
    torch_total = torch.nn.utils.clip_grad_norm_(clones, max_norm)
    total = adana_amd.clip_grad_norm_(params, max_norm)
    torch.cuda.synchronize()
    assert total.dtype == (torch.bfloat16 if bf16 else torch.float32)
    assert total.device == params[0].device and total.dim() == 0
    t = _check_total(total, orig, bf16, O, torch_total)
    coef = O.clip_coef(t, max_norm, bf16)
    if max_norm == 1e3:
        assert coef == np.float32(1.0)
    else:
        assert coef < np.float32(1.0)
    for i, (p, g) in enumerate(zip(params, orig)):
        exp = O.clip_scale(g, coef, bf16)
        d = ulp_diff(p.grad.float().cpu().numpy(), exp)
        assert d.size == 0 or d.max() == 0, f"tensor {i}: clipped grad differs by {d.max()} ulp"


def test_clip_edge_values(oracle_mod):
    """All-zero gradients (coefficient 1), NaN and inf gradients (torch
    propagates them), error_if_nonfinite, empty and gradient-less lists."""
    import adana_amd

    print("case: clip edge values", flush=True)
    ps = [torch.nn.Parameter(torch.zeros(n, device=DEV)) for n in (10, 33)]
    for p in ps:
        p.grad = torch.zeros_like(p)
    total = adana_amd.clip_grad_norm_(ps, 0.5)
    assert float(total) == 0.0
    assert all(torch.count_nonzero(p.grad).item() == 0 for p in ps)

    for bad in (float("nan"), float("inf")):
        ps = [torch.nn.Parameter(torch.zeros(n, device=DEV)) for n in (10, 33)]
        for i, p in enumerate(ps):
            p.grad = torch.full_like(p, 1e-3 * (i + 1))
        ps[1].grad[5] = bad
        clones = [torch.nn.Parameter(p.detach().clone()) for p in ps]
        for c, p in zip(clones, ps):
            c.grad = p.grad.clone()
        tt = torch.nn.utils.clip_grad_norm_(clones, 0.5)
        total = adana_amd.clip_grad_norm_(ps, 0.5)
        assert np.array_equal(np.float32(float(total)), np.float32(float(tt)), equal_nan=True)
        for c, p in zip(clones, ps):
            np.testing.assert_array_equal(p.grad.cpu().numpy(), c.grad.cpu().numpy())
        ps[1].grad[5] = bad
        with pytest.raises(RuntimeError, match="non-finite"):
            adana_amd.clip_grad_norm_(ps, 0.5, error_if_nonfinite=True)

    assert float(adana_amd.clip_grad_norm_([], 1.0)) == 0.0
    assert float(adana_amd.clip_grad_norm_([torch.nn.Parameter(torch.ones(3, device=DEV))], 1.0)) == 0.0


def _clipped_pair_step(pair, O, grads, max_norm, write_back=True, bf16=False):
    """Set grads, clip through the optimizer (fused), step both sides."""
    for tp, gs in zip(pair.gpu_params, grads):
        for p, g in zip(tp, gs):
            if bf16:
                p.grad = torch.from_numpy(g.view(np.int16).copy()).view(torch.bfloat16).to(DEV)
            else:
                p.grad = torch.from_numpy(g.copy()).to(DEV)
    pair.prev = [[x.copy() for x in cp] for cp in pair.cpu_params]
    flat = [O.bf16_to_f32(g).reshape(g.shape) if bf16 else g for gs in grads for g in gs]
    total = pair.opt.clip_grad_norm_(max_norm, write_back=write_back)
    t = _check_total(total, flat, bf16, O)
    coef = O.clip_coef(t, max_norm, bf16)
    if bf16:
        scaled = [[O.f32_to_bf16(O.clip_scale(O.bf16_to_f32(g), coef, True)).reshape(g.shape) for g in gs]
                  for gs in grads]
    else:
        scaled = [[O.clip_scale(g, coef) for g in gs] for gs in grads]
    before = [[p.grad.clone() for p in tp] for tp in pair.gpu_params]
    pair.opt.step()
    pair.oracle.step(scaled)
    torch.cuda.synchronize()
    for tp, sg, bg in zip(pair.gpu_params, scaled, before):
        for p, s, b in zip(tp, sg, bg):
            got = p.grad.cpu()
            if write_back:
                exp = (torch.from_numpy(s.view(np.int16).copy()).view(torch.bfloat16) if bf16
                       else torch.from_numpy(s))
                assert torch.equal(got.view(torch.int16) if bf16 else got,
                                   exp.view(torch.int16) if bf16 else exp), "written-back grad"
            else:
                assert torch.equal(got, b.cpu()), "grad must stay unscaled without write_back"
    return coef


@pytest.mark.parametrize("star", [False, True])
@pytest.mark.parametrize("write_back", [True, False])
def test_clip_fused_step(oracle_mod, star, write_back):
    """opt.clip_grad_norm_(0.5) + opt.step() on a GPT-shaped list with two
    groups: the step consumes the clipped gradients inside its kernel."""
    print("case: fused clip star", star, "write_back", write_back, flush=True)
    O = oracle_mod
    rng = np.random.default_rng(21)
    decay, nodecay = _gpt_list(rng, vocab=503, d=64, layers=2)
    pair = Pair(O, star, [(decay, {"weight_decay": 0.2}), (nodecay, {"weight_decay": 0.0})],
                lr=3e-3, delta=8.0, kappa=0.85, clipsnr=2.0, wd_decaying=True, wd_ts=20.0)
    clipped = 0
    for k in range(6):
        std = 1e-1 if k % 2 == 0 else 1e-4          # alternate clipping / not clipping
        gl = [[_normal(rng, x.shape, std) for x in ps] for ps in (decay, nodecay)]
        coef = _clipped_pair_step(pair, O, gl, 0.5, write_back)
        clipped += int(coef < 1)
        pair.compare(where=f"k={k}")
    assert clipped == 3


def test_clip_fused_bf16_master(oracle_mod):
    """C4-style bf16 params + fp32 master with bf16 gradients: the norm,
    coefficient and products are rounded to bfloat16 as torch does."""
    print("case: fused clip bf16 master", flush=True)
    O = oracle_mod
    rng = np.random.default_rng(23)
    ps = [O.f32_to_bf16(_normal(rng, s, 0.02)).reshape(s) for s in ((300, 64), (64,), (17,))]
    pair = Pair(O, False, [(ps, {})], master=True, lr=1e-3, delta=8.0, kappa=0.85,
                weight_decay=0.1, wd_decaying=True, wd_ts=10.0)
    for k in range(4):
        gl = [[O.f32_to_bf16(_normal(rng, x.shape, 3e-2)).reshape(x.shape) for x in ps]]
        coef = _clipped_pair_step(pair, O, gl, 0.5, True, bf16=True)
        assert coef < 1
        pair.compare(where=f"k={k}")


def test_clip_twice_then_step(oracle_mod):
    """A second clip before step() sees the first clip's scaling (as with
    torch's in-place clipping): the pending scale is applied first."""
    import adana_amd

    print("case: clip twice", flush=True)
    rng = np.random.default_rng(31)
    ps = [torch.nn.Parameter(torch.from_numpy(_normal(rng, s, 0.02)).to(DEV)) for s in ((64, 64), (64,))]
    opt = adana_amd.ADana(ps, lr=1e-3, kappa=0.85)
    clones = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    for p, c in zip(ps, clones):
        p.grad = torch.from_numpy(_normal(rng, p.shape, 1.0)).to(DEV)
        c.grad = p.grad.clone()
    t1 = opt.clip_grad_norm_(1.0)
    t2 = opt.clip_grad_norm_(0.25)
    r1 = torch.nn.utils.clip_grad_norm_(clones, 1.0)
    r2 = torch.nn.utils.clip_grad_norm_(clones, 0.25)
    for a, b in ((t1, r1), (t2, r2)):
        assert abs(float(a) - float(b)) <= 2e-6 * float(b)
    assert float(t2) <= 1.0 + 1e-5
    opt.flush_clip()
    for p, c in zip(ps, clones):
        np.testing.assert_allclose(p.grad.cpu().numpy(), c.grad.cpu().numpy(), rtol=1e-6, atol=0)


def test_clip_not_owned_scales_in_place_at_once(oracle_mod):
    """Parameters the optimizer does not step (or a subset) are scaled at
    once, by the HIP grad_scale_kernel, instead of deferred into the step;
    zero_grad drops a pending scale."""
    import adana_amd

    print("case: clip of parameters the optimizer does not own", flush=True)
    rng = np.random.default_rng(41)
    ps = [torch.nn.Parameter(torch.from_numpy(_normal(rng, (128,), 0.02)).to(DEV)) for _ in range(3)]
    opt = adana_amd.ADana(ps[:2], lr=1e-3)
    for p in ps:
        p.grad = torch.full_like(p, 1.0)
    before = ps[0].grad.clone()
    adana_amd.clip_grad_norm_(ps, 0.5, optimizer=opt)      # ps[2] is not the optimizer's
    assert not torch.equal(ps[0].grad, before)              # already scaled
    assert opt._pending_clip is None
    for p in ps:
        p.grad = torch.full_like(p, 1.0)
    opt.clip_grad_norm_(0.5)
    assert opt._pending_clip is not None
    opt.zero_grad(set_to_none=False)
    assert opt._pending_clip is None
    assert all(torch.count_nonzero(p.grad).item() == 0 for p in ps[:2])


def test_c_abi_clip_empty_list():
    """adana_grad_clip_norm on an empty plan writes total 0 and coefficient 1."""
    from adana_amd import _lib

    L = _lib.lib()
    out = torch.full((2,), -1.0, device=DEV)
    plan = _lib.Plan()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(L.adana_grad_clip_norm(ctypes.byref(plan), 0, 0.5, None, 0, None,
                                      ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(stream)),
               "adana_grad_clip_norm")
    torch.cuda.synchronize()
    assert out.tolist() == [0.0, 1.0]


@pytest.mark.parametrize("write_back", [True, False])
def test_deepcopy_with_pending_clip(write_back):
    """copy.deepcopy of an optimizer with a clip deferred to its next step():
    with write_back the original's gradients are scaled then (what torch's
    in-place clipping leaves); without it the original's gradients stay
    unscaled and the copy defers the same scaling.  Either way the original
    and the copy then take bit-identical steps on the clipped gradients.
    (Plain tensors as parameters: nn.Parameter's deepcopy drops .grad.)"""
    import copy

    import adana_amd

    print("case: deepcopy with a pending clip, write_back", write_back, flush=True)
    rng = np.random.default_rng(51)
    ps = [torch.from_numpy(_normal(rng, s, 0.02)).to(DEV).requires_grad_() for s in ((96, 64), (64,), (5,))]
    for p in ps:
        p.grad = torch.from_numpy(_normal(rng, p.shape, 1.0)).to(DEV)
    opt = adana_amd.DANA_STAR_MK4(ps, lr=1e-3, kappa=0.85, clipsnr=2.0)
    twin = [p.detach().clone().requires_grad_() for p in ps]
    for t, p in zip(twin, ps):
        t.grad = p.grad.clone()
    ref = adana_amd.DANA_STAR_MK4(twin, lr=1e-3, kappa=0.85, clipsnr=2.0)
    ref.clip_grad_norm_(0.5, write_back=write_back)
    ref.step()                                   # the fused path, on a twin that is never copied
    unscaled = [p.grad.clone() for p in ps]
    opt.clip_grad_norm_(0.5, write_back=write_back)
    cp = copy.deepcopy(opt)
    assert (opt._pending_clip is None) == write_back
    for p, g in zip(ps, unscaled):
        assert torch.equal(p.grad, g) != write_back      # scaled now only with write_back
    opt.step()
    cp.step()
    torch.cuda.synchronize()
    cps = [p for g in cp.param_groups for p in g["params"]]
    for a, b, c in zip(ps, cps, twin):
        assert torch.equal(a.detach(), c.detach()), "original vs never-copied twin"
        assert torch.equal(b.detach(), c.detach()), "copy vs never-copied twin"
    for a, c in zip(ps, twin):
        assert torch.equal(a.grad, c.grad)
    if not write_back:
        for b, g in zip(cps, unscaled):
            assert torch.equal(b.grad, g), "the copy's gradients stay unscaled too"
