"""The binary64-core pow the Dana-Star kernel uses (adana_amd/csrc/adana_pow.h)
agrees bit for bit with the oracle's fp32(pow(double x, double y)) -- the C
library's pow -- over the kernel's domain x >= 1, for the exponents
fp32(1 - kappa) of typical and edge kappas."""
import os
import subprocess

import pytest

from helpers import ROOT


def test_pow_core_matches_libm(tmp_path):
    exe = tmp_path / "pow_harness"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(ROOT, "tests", "pow_harness.cpp"), "-lm"], check=True)
    kappas = [0.85, 0.75, 0.8, 0.9, 0.95, 0.6, 0.0, 1.3, -0.5, 0.999]
    ys = [repr(1.0 - k) for k in kappas]
    out = subprocess.run([str(exe), "300000"] + ys, check=True, capture_output=True, text=True)
    mism, total = map(int, out.stdout.split()[-2:])
    assert total == 300000 * len(ys)
    assert mism == 0, out.stdout
