"""bench.py's host-side contract, on the CPU: the workloads' sizes and
layouts (the benchmarked configurations: the 2.62B north-star list and C1-C5),
the algorithmic bytes per element the roofline uses, the warm-up defaults,
the lr schedule, and the refusal of more than one GPU (before anything
touches a GPU)."""
import math
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _elements(w):
    return sum(math.prod(s) for shapes in w["groups"] for s in shapes)


def _tensors(w):
    return sum(len(shapes) for shapes in w["groups"])


def test_workload_sizes():
    """The north star and C4 are the 2.62B-param list (d_model 2560, 32
    layers, MLP 4x, vocab 50304, tied; 194 tensors); C3 the d_model 2048,
    24-layer one; C2 the ~51M GPT list with LayerNorm biases; C1 one 4M
    tensor; C5 10,000 log-uniform tensors in [64, 65536]."""
    ns = bench.workload("north_star")
    assert _elements(ns) == 2_645_527_040 and _tensors(ns) == 194
    assert _elements(bench.workload("c4")) == 2_645_527_040
    assert _elements(bench.workload("north_star_bf16")) == 2_645_527_040
    assert _elements(bench.workload("c3")) == 1_311_082_496
    c2 = bench.workload("c2")
    assert _elements(c2) == 50_938_880 and _tensors(c2) == 67
    assert _elements(bench.workload("c1")) == 4 * 1024 * 1024
    c5 = bench.workload("c5")
    sizes = [math.prod(s) for s in c5["groups"][0]]
    assert len(sizes) == 10_000 and min(sizes) >= 64 and max(sizes) <= 65536
    assert _elements(c5) == 94_406_322


def test_variants_and_bytes_per_element():
    """Optimizer variant, precision and the roofline's algorithmic bytes per
    element of every step workload."""
    want = {
        "north_star": ("Dana-Star-MK4", 36), "north_star_clip": ("Dana-Star-MK4", 44),
        "north_star_bf16": ("Dana-Star-MK4", 18), "c1": ("ADana", 28), "c2": ("Dana-MK4", 28),
        "c3": ("Dana-Star-MK4", 36), "c4": ("ADana", 28), "c5": ("Dana-Star-MK4", 36),
    }
    assert set(want) == set(bench.STEP_WORKLOADS)
    for name, (opt, bpe) in want.items():
        w = bench.workload(name)
        assert w["optimizer"] == opt, name
        assert bench.bytes_per_elem(w) == bpe, name
    assert bench.workload("c4")["master"] and not bench.workload("north_star")["master"]
    assert bench.workload("north_star_bf16").get("state_bf16")


def test_default_warmups():
    """C5 warms up 40 steps (its fixed synthetic gradients lower the clock for
    ~35 steps), and says why in its line; every other workload 3."""
    for name in bench.STEP_WORKLOADS:
        w = bench.workload(name)
        if name == "c5":
            assert w["default_warmup"] == 40 and "warm-up" in w["warmup_note"]
        else:
            assert w.get("default_warmup", 3) == 3, name


def test_cos_inf_schedule():
    """C2's lr factor is the reference's cos_inf (src/optim/schedule.py:88-96:
    step/n_warmup + (1 - step/n_warmup)/div_factor while warming up, then
    final + (1 - final)(1 + cos(pi t))/2 with final = 1/div/final_div = 0.1),
    pinned here by values worked out from that formula by hand."""
    f = bench.cos_inf_schedule(**bench.C2_SCHEDULE)
    assert bench.C2_SCHEDULE == dict(n_iterations=200, n_warmup=4, div_factor=1e2, final_div_factor=1e-1,
                                     n_inf=0)
    assert f(0) == pytest.approx(0.01, rel=1e-15)            # 0 + 1/100
    assert f(1) == pytest.approx(0.2575, rel=1e-15)          # 1/4 + (3/4)/100
    assert f(2) == pytest.approx(0.505, rel=1e-15)
    assert f(3) == pytest.approx(0.7525, rel=1e-15)
    assert f(4) == pytest.approx(1.0, rel=1e-15)             # t = 0: 0.1 + 0.9
    assert f(102) == pytest.approx(0.55, rel=1e-12)          # t = 1/2: 0.1 + 0.45
    assert f(199) == pytest.approx(0.1 + 0.45 * (1 - math.cos(math.pi / 196)), rel=1e-12)
    assert f(200) == pytest.approx(0.1, rel=1e-15) and f(500) == f(200)
    assert all(f(k) < f(k + 1) for k in range(4)) and all(f(k) > f(k + 1) for k in range(4, 200))


def test_c2_lr_through_lambdalr():
    """The bench drives C2's lr through torch.optim.lr_scheduler.LambdaLR as
    src/main.py:411-423 does: step k runs at peak * factor(k), group['lr']
    set at construction (k = 0) and after every step."""
    import torch

    p = torch.nn.Parameter(torch.zeros(1))
    opt = torch.optim.SGD([p], lr=3e-3)
    f = bench.cos_inf_schedule(**bench.C2_SCHEDULE)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, f)
    seen = []
    for _ in range(8):
        seen.append(opt.param_groups[0]["lr"])
        opt.step()
        sched.step()
    assert seen == [3e-3 * f(k) for k in range(8)]


def test_more_than_one_gpu_is_refused(capsys, monkeypatch):
    """`bench.py --gpus N` with N > 1 exits with status 2 and a message, before
    it imports torch's GPU side or the library."""
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "2"])
    assert bench.main() == 2
    assert "measures one GPU" in capsys.readouterr().err
