"""CPU checks of gradient-norm clipping.

The oracle's restatement of torch.nn.utils.clip_grad_norm_ (norm_type 2;
called by the reference at src/optim/base.py:250-257 through
src/distributed/backend.py:33-35) is pinned against torch's own CPU function
-- the third-party code the reference calls -- and against closed forms.  The
product's host-side argument handling is checked without a GPU.
"""
import math

import numpy as np
import pytest
import torch

f32 = np.float32


def _torch_clip(grads_np, max_norm, bf16):
    dt = torch.bfloat16 if bf16 else torch.float32
    ps = [torch.nn.Parameter(torch.zeros(g.shape, dtype=dt)) for g in grads_np]
    for p, g in zip(ps, grads_np):
        p.grad = torch.from_numpy(g.copy()).to(dt)
    tot = torch.nn.utils.clip_grad_norm_(ps, max_norm)
    return tot, [p.grad.float().numpy() for p in ps]


@pytest.mark.parametrize("bf16", [False, True])
def test_oracle_clip_matches_torch(oracle_mod, bf16):
    """Coefficient and clipped gradients bit-exact given torch's total norm;
    the oracle's total within 2e-7 (binary32) / equal (bfloat16) of torch's."""
    O = oracle_mod
    rng = np.random.default_rng(7 + bf16)
    for trial in range(150):
        n = int(rng.integers(1, 6))
        shapes = [tuple(int(x) for x in rng.integers(0, 50, size=int(rng.integers(1, 3)))) for _ in range(n)]
        scale = 10.0 ** rng.uniform(-4, 2)
        gs = [rng.normal(0, scale, s).astype(f32) for s in shapes]
        if bf16:
            gs = [O.bf16_to_f32(O.f32_to_bf16(g)).reshape(g.shape) for g in gs]
        max_norm = float(rng.choice([0.5, 1.0, 1e-3, 1e3, 3.7]))
        tot, clipped = _torch_clip(gs, max_norm, bf16)
        assert tot.dtype == (torch.bfloat16 if bf16 else torch.float32)
        t = f32(tot.float().item())
        _, ot = O.clip_norms(gs, bf16)
        if bf16:
            assert abs(float(ot) - float(t)) <= float(np.spacing(t)) * 65536, (trial, ot, t)
        else:
            assert abs(float(ot) - float(t)) <= 2e-7 * max(float(t), 1e-30), (trial, ot, t)
        coef = O.clip_coef(t, max_norm, bf16)
        for g, c in zip(gs, clipped):
            exp = O.clip_scale(g, coef, bf16)
            assert np.array_equal(exp.view(np.uint32), c.view(np.uint32)), (trial, coef)


def test_oracle_clip_closed_forms(oracle_mod):
    """||(3, 4)|| = 5 and the norm of the norms (3, 4) is 5; coefficient is
    reciprocal(5 + 1e-6) * max_norm in binary32, clamped at 1; zero, NaN and
    infinite totals."""
    O = oracle_mod
    norms, total = O.clip_norms([np.array([3.0, 4.0], f32)])
    assert norms[0] == f32(5.0) and total == f32(5.0)
    norms, total = O.clip_norms([np.array([3.0], f32), np.array([-4.0], f32), np.zeros(0, f32)])
    assert [float(x) for x in norms] == [3.0, 4.0, 0.0] and total == f32(5.0)
    den = f32(5.0) + f32(1e-6)
    assert den == f32(5.0000010)
    assert O.clip_coef(f32(5.0), 1.0) == (f32(1.0) / den) * f32(1.0)
    assert O.clip_coef(f32(5.0), 0.5) == (f32(1.0) / den) * f32(0.5)
    assert O.clip_coef(f32(5.0), 100.0) == f32(1.0)
    assert O.clip_coef(f32(0.0), 1e-3) == f32(1.0)               # 1e-3 / 1e-6 > 1
    assert math.isnan(O.clip_coef(f32("nan"), 1.0))
    assert O.clip_coef(f32("inf"), 1.0) == f32(0.0)
    # bfloat16: every op rounds to bfloat16 (5 + 1e-6 -> 5; 1/5 -> 0.2001953125)
    assert O.clip_coef(f32(5.0), 1.0, bf16=True) == f32(0.2001953125)
    # the clipped gradient is g * coef in binary32 (bf16: then rounded)
    g = np.array([1.0, -3.0, 0.1], f32)
    assert np.array_equal(O.clip_scale(g, f32(0.5)), g * f32(0.5))


def test_clip_host_argument_errors():
    """No GPU needed: CPU tensors, norm types other than 2, empty lists."""
    import adana_amd

    p = torch.nn.Parameter(torch.zeros(4))
    p.grad = torch.ones(4)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        adana_amd.clip_grad_norm_([p], 1.0)
    with pytest.raises(NotImplementedError, match="norm_type"):
        adana_amd.clip_grad_norm_([p], 1.0, norm_type=1.0)
    t = adana_amd.clip_grad_norm_([], 1.0)
    assert t.dim() == 0 and float(t) == 0.0
    q = torch.nn.Parameter(torch.zeros(4))
    assert float(adana_amd.clip_grad_norm_(q, 1.0)) == 0.0        # a single tensor, no grad
