"""The binary64-core pow of the Dana-Star kernel (adana_amd/csrc/adana_pow.h)
against the oracle's fp32(pow(double x, double y)) -- the C library's pow --
over the kernel's domain x >= 1, for the exponents fp32(1 - kappa) of typical
and edge kappas.  The guarded entry point (any exponent) must agree bit for
bit; the unguarded one the kernel uses for 0 < y < 1 may differ only where x**y
lies within ~2^-51 of a binary32 half-way point (measured rate ~5e-9)."""
import os
import subprocess

from helpers import ROOT


def test_pow_core_matches_libm(tmp_path):
    exe = tmp_path / "pow_harness"
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(ROOT, "tests", "pow_harness.cpp"), "-lm"], check=True)
    kappas = [0.85, 0.75, 0.8, 0.9, 0.95, 0.6, 0.0, 1.3, -0.5, 0.999]
    ys = [repr(1.0 - k) for k in kappas]
    per = 300000
    out = subprocess.run([str(exe), str(per)] + ys, check=True, capture_output=True, text=True)
    mism, mism_unit, total = map(int, out.stdout.split()[-3:])
    assert total == per * len(ys)
    assert mism == 0, out.stdout
    assert mism_unit <= 1, out.stdout
