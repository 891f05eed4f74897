"""Exhaustive checks, on the GPU, that the shortened division and square root
of adana_amd/csrc/adana_fastmath.h return exactly what the IEEE sequences do
over the input ranges the Dana-Star kernel feeds them, and that the bfloat16
path's rounding, division and square root agree with round-to-nearest-even
of the IEEE results on every input."""
import ctypes
import os
import struct

import pytest
import torch

from helpers import ROOT

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a ROCm GPU")]

LIB = os.path.join(ROOT, "tests", "libadana_mathcheck.so")


def _bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def _run(which, lo, hi):
    import adana_amd._lib  # noqa: F401  (torch's HIP runtime first)

    L = ctypes.CDLL(LIB)
    L.adana_mathcheck.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p,
                                  ctypes.c_void_p]
    out = torch.tensor([0, 2 ** 63 - 1], dtype=torch.int64, device="cuda:0")
    rc = L.adana_mathcheck(which, lo, hi, ctypes.c_void_p(out.data_ptr()),
                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    return int(out[0]), int(out[1])


def test_div_core_exhaustive_on_tau_range():
    """p_estimate = ct / (1 - ct) for every binary32 ct in [+0, 0.5]."""
    print("case: div_core exhaustive [0, 0.5]", flush=True)
    bad, first = _run(0, 0, _bits(0.5))
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}"


def test_sqrt_normal_exhaustive():
    """sqrt for every binary32 in [2^-96, +inf] (tau_reg lies in [2^-24, 1];
    sqrt_f32 sends the second moment there when it is at least 2^-96)."""
    print("case: sqrt_normal exhaustive [2^-96, inf]", flush=True)
    bad, first = _run(1, _bits(2.0 ** -96), 0x7F800000)
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}"


def test_bf16_conversion_is_rne_on_every_binary32():
    """gfx950's conversion instruction (v_cvt_pk_bf16_f32) over all 2^32
    binary32 patterns: round-to-nearest-even, NaN -> (bits >> 16) | 0x40; the
    integer form bf16_round_int (the launch's bf16 scalars) gives the same bits."""
    print("case: bf16 conversion exhaustive", flush=True)
    bad, first = _run(2, 0, 0xFFFFFFFF)
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}"


def test_div_bf16_exhaustive_over_all_pairs():
    """bf16(div_bf16(a, b)) == bf16(a / b) for all 2^32 pairs of bfloat16 a, b
    (zeros, subnormals, infinities and NaNs included)."""
    print("case: div_bf16 exhaustive", flush=True)
    bad, first = _run(3, 0, 0xFFFFFFFF)
    assert bad == 0, f"{bad} mismatches, first pair {first:#010x}"


def test_sqrt_bf16_exhaustive():
    """bf16(sqrt_bf16(x)) == bf16(sqrtf(x)) for all 65,536 bfloat16 x."""
    print("case: sqrt_bf16 exhaustive", flush=True)
    bad, first = _run(4, 0, 0xFFFF)
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}"


def test_sqrt_f32_exhaustive():
    """sqrt_f32(x) == sqrtf(x) bit for bit on all 2^32 binary32 patterns."""
    print("case: sqrt_f32 exhaustive", flush=True)
    bad, first = _run(5, 0, 0xFFFFFFFF)
    assert bad == 0, f"{bad} mismatches, first pattern {first:#010x}"
