// adana_fastmath.h -- correctly rounded binary32 division and square root for
// operand ranges on which the full IEEE sequences' range scaling and
// special-case fixups are identities.  Same results, fewer instructions.
// tests/gpu_mathcheck.hip checks both exhaustively over the ranges the
// optimizer kernel uses them on.
#ifndef ADANA_FASTMATH_H
#define ADANA_FASTMATH_H

#include <hip/hip_runtime.h>

namespace adana {

// Correctly rounded a / b for operands on which the IEEE division sequence's
// range scaling (v_div_scale) and special-case fixup (v_div_fixup) are
// identities: b normal in [0.5, 1], and a either normal or b == 1.  This is the
// same refinement chain the full sequence runs (reciprocal, one Newton step,
// two remainder corrections), so the result is bit-identical to a / b there.
__device__ __forceinline__ float div_core(float a, float b) {
    float y = __builtin_amdgcn_rcpf(b);
    const float e = __builtin_fmaf(-b, y, 1.0f);
    y = __builtin_fmaf(e, y, y);
    float q = a * y;
    float r = __builtin_fmaf(-b, q, a);
    q = __builtin_fmaf(r, y, q);
    r = __builtin_fmaf(-b, q, a);
    return __builtin_fmaf(r, y, q);
}

// Correctly rounded sqrt for x >= 2^-96 (or NaN): the hardware square root
// followed by the neighbour test of the full IEEE sequence, without its
// small-input scaling and zero/inf/negative fixups (identities there).
__device__ __forceinline__ float sqrt_normal(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sm = __uint_as_float(__float_as_uint(s) - 1u);
    const float sp = __uint_as_float(__float_as_uint(s) + 1u);
    const float rm = __builtin_fmaf(-sm, s, x);
    const float rp = __builtin_fmaf(-sp, s, x);
    float o = rm <= 0.0f ? sm : s;
    o = rp > 0.0f ? sp : o;
    return o;
}

}  // namespace adana

#endif  // ADANA_FASTMATH_H
