"""The step kernel's two-group launches (128-thread workgroups, two groups of four
elements per thread; launch_main in adana_amd/csrc/adana_mta.hip picks them on
grids of at least 64 chunks per CU: lists of 16,384 chunks and more on a
256-CU MI355X, up to 2^18 chunks for float32 state, any size for bfloat16
state), against the oracle on every element: float32 and bf16-master lists of
~20M elements in both numerics, and the reference's bfloat16 state, whose
compiled instance issues both groups' loads first (one of its tensors a view
2 bytes into a buffer, so that its groups take the element-wise path).  Same bars as
tests/test_gpu_parity.py and tests/test_gpu_bf16.py."""
import numpy as np
import pytest
import torch

from test_gpu_bf16 import _bits, _check, _diag_close, _to_gpu16
from test_gpu_parity import STAR_HARD_CASES, Pair, _normal

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

DEV = "cuda:0"
SIZES = [9_000_000, 6_000_003, 5_000_001, 1027]     # 19,540 chunks
HP = dict(lr=1e-3, delta=8.0, kappa=0.85, weight_decay=0.1, clipsnr=2.0, wd_decaying=True, wd_ts=10.0)


def _grid_is_two_group():
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    chunks = sum((n + 1023) // 1024 for n in SIZES)
    return chunks >= 64 * cus and chunks <= (1 << 18)


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("master", [False, True], ids=["fp32", "master"])
@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
def test_two_group_grid_fp32_and_master(oracle_mod, star, master, numerics):
    if not _grid_is_two_group():
        pytest.skip("this device's CU count puts the list outside the two-group range")
    O = oracle_mod
    print(f"case: two-group grid star {star} master {master} {numerics} sizes {SIZES}", flush=True)
    rng = np.random.default_rng(31)

    def param(n):
        x = _normal(rng, (n,), 0.02)
        return O.f32_to_bf16(x) if master else x

    pair = Pair(O, star, [([param(n) for n in SIZES], {})], master=master, numerics=numerics, **HP)
    for k in range(2):
        grads = []
        for n in SIZES:
            g = _normal(rng, (n,), 1e-3)
            grads.append(O.f32_to_bf16(g) if master else g)
        pair.step([grads])
        pair.compare(where=f"two-group k={k}")
    assert pair.opt._check_slab_guards() >= 1


@pytest.mark.parametrize("numerics", ["compiled", "eager"])
@pytest.mark.parametrize("star", [False, True], ids=["adana", "star"])
def test_two_group_grid_bf16_state(oracle_mod, star, numerics):
    import adana_amd

    O = oracle_mod
    print(f"case: two-group grid bf16 state star {star} {numerics} sizes {SIZES}", flush=True)
    rng = np.random.default_rng(32)
    host = [O.f32_to_bf16(rng.normal(0, 0.02, n).astype(np.float32)) for n in SIZES]
    gpu = []
    flat = torch.empty(SIZES[1] + 1, dtype=torch.bfloat16, device=DEV)
    for i, h in enumerate(host):
        if i == 1:                              # 2 bytes in: not 8-byte aligned, the element-wise path
            v = flat[1:]
            v.copy_(_to_gpu16(h))
            gpu.append(torch.nn.Parameter(v))
        else:
            gpu.append(torch.nn.Parameter(_to_gpu16(h)))
    cls = adana_amd.DANA_STAR_MK4 if star else adana_amd.ADana
    opt = cls(gpu, numerics=numerics, **HP)
    orc = O.OracleOptimizer(groups=[O.OracleGroup(params=host, lr=HP["lr"], weight_decay=HP["weight_decay"])],
                            star=star, peak_lr=HP["lr"], kappa=HP["kappa"], clipsnr=HP["clipsnr"],
                            wd_decaying=True, wd_ts=HP["wd_ts"], bf16=True, numerics=numerics)
    for t in range(1, 3):
        g16 = [O.f32_to_bf16(rng.normal(0, 1e-3, n).astype(np.float32)) for n in SIZES]
        for p, g in zip(gpu, g16):
            p.grad = _to_gpu16(g)
        opt.step()
        orc.step([g16])
        torch.cuda.synchronize()
        for i, p in enumerate(gpu):
            st, ost = opt.state[p], orc.state[id(host[i])]
            tag = f"two-group bf16 star {star} {numerics} t={t} tensor {i} (n={SIZES[i]})"
            for key in ("m", "v", "tau") if star else ("m", "v"):
                _check(_bits(st[key]), ost[key], f"{tag} {key}")
            got = _bits(p)
            _check(got, host[i], f"{tag} p", STAR_HARD_CASES if star else 0)
            host[i][...] = got.reshape(host[i].shape)
            _diag_close([float(st[key]) for key in O.DIAG_KEYS], [float(ost[key]) for key in O.DIAG_KEYS], tag)
    assert opt._check_slab_guards() >= 1
