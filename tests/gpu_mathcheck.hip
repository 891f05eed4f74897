// Exhaustive GPU checks of adana_amd/csrc/adana_fastmath.h against the
// compiler's IEEE division and square root (test infrastructure, built into
// tests/libadana_mathcheck.so by __graft_entry__.build()).
//   which = 0: div_core(a, 1 - a) vs a / (1 - a) for the binary32 patterns
//              [lo, hi] (the Dana-Star p_estimate division, a = clamped tau)
//   which = 1: sqrt_normal(x) vs sqrtf(x) for the patterns [lo, hi]
// out[0] counts mismatching patterns, out[1] holds the smallest one.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../adana_amd/csrc/adana_fastmath.h"

__global__ void check_kernel(int which, uint32_t lo, uint64_t count, unsigned long long *out) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const uint32_t bits = lo + static_cast<uint32_t>(i);
        const float x = __uint_as_float(bits);
        float got, ref;
        if (which == 0) {
            got = adana::div_core(x, 1.0f - x);
            ref = x / (1.0f - x);
        } else {
            got = adana::sqrt_normal(x);
            ref = sqrtf(x);
        }
        const bool same = __float_as_uint(got) == __float_as_uint(ref) || (got != got && ref != ref);
        if (!same) {
            atomicAdd(&out[0], 1ull);
            atomicMin(&out[1], static_cast<unsigned long long>(bits));
        }
    }
}

extern "C" int adana_mathcheck(int which, uint32_t lo, uint32_t hi, unsigned long long *d_out,
                               void *stream) {
    if (hi < lo || (which != 0 && which != 1) || !d_out) return -1;
    const uint64_t count = static_cast<uint64_t>(hi) - lo + 1;
    hipLaunchKernelGGL(check_kernel, dim3(8192), dim3(256), 0, static_cast<hipStream_t>(stream), which, lo,
                       count, d_out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
