// Exhaustive GPU checks of adana_amd/csrc/adana_fastmath.h against the
// compiler's IEEE division and square root (test infrastructure, built into
// tests/libadana_mathcheck.so by __graft_entry__.build()).
//   which = 0: div_core(a, 1 - a) vs a / (1 - a) for the binary32 patterns
//              [lo, hi] (the Dana-Star p_estimate division, a = clamped tau)
//   which = 1: sqrt_normal(x) vs sqrtf(x) for the patterns [lo, hi]
//   which = 2: bf16_bits(x) (the conversion instruction) vs round-to-nearest-
//              even in integer arithmetic, NaN -> (bits >> 16) | 0x40, for the
//              binary32 patterns [lo, hi]; bf16_round(x), bf16_pack2(x, x)
//              and bf16_round_int(x) hold the same bits
//   which = 3: bf16_round(div_bf16(a, b)) vs bf16_round(a / b) for the pairs
//              pattern = (a's bfloat16 bits << 16) | b's bits in [lo, hi]
//   which = 4: bf16_round(sqrt_bf16(x)) vs bf16_round(sqrtf(x)) for the
//              bfloat16 patterns [lo, hi] (hi <= 0xffff)
//   which = 5: sqrt_f32(x) vs sqrtf(x) for the binary32 patterns [lo, hi]
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
        } else if (which == 1) {
            got = adana::sqrt_normal(x);
            ref = sqrtf(x);
        } else if (which == 2) {
            const uint32_t h = adana::bf16_bits(x);
            const uint32_t hr = __float_as_uint(adana::bf16_round(x));          // (0, x) pair form
            const uint32_t hp = adana::bf16_pack2(x, x);                        // packed pair form
            const uint32_t hi = __float_as_uint(adana::bf16_round_int(x));      // integer form
            if (hr != (h << 16) || hp != (h | (h << 16)) || hi != hr) {
                atomicAdd(&out[0], 1ull);
                atomicMin(&out[1], static_cast<unsigned long long>(bits));
                continue;
            }
            uint32_t r;
            if ((bits & 0x7fffffffu) > 0x7f800000u) {
                r = (bits >> 16) | 0x40u;
            } else {
                r = (bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16;
            }
            got = __uint_as_float(h);                  // compared bit for bit, never as floats
            ref = __uint_as_float(r);
        } else if (which == 3) {
            const float a = __uint_as_float(bits & 0xffff0000u), b = __uint_as_float(bits << 16);
            got = adana::bf16_round(adana::div_bf16(a, b));
            ref = adana::bf16_round(a / b);
        } else if (which == 4) {
            const float v = __uint_as_float(bits << 16);
            got = adana::bf16_round(adana::sqrt_bf16(v));
            ref = adana::bf16_round(sqrtf(v));
        } else {
            got = adana::sqrt_f32(x);
            ref = sqrtf(x);
        }
        const bool same = __float_as_uint(got) == __float_as_uint(ref) ||
                          (which != 2 && got != got && ref != ref);
        if (!same) {
            atomicAdd(&out[0], 1ull);
            atomicMin(&out[1], static_cast<unsigned long long>(bits));
        }
    }
}

extern "C" int adana_mathcheck(int which, uint32_t lo, uint32_t hi, unsigned long long *d_out,
                               void *stream) {
    if (hi < lo || which < 0 || which > 5 || (which == 4 && hi > 0xffffu) || !d_out) return -1;
    const uint64_t count = static_cast<uint64_t>(hi) - lo + 1;
    hipLaunchKernelGGL(check_kernel, dim3(8192), dim3(256), 0, static_cast<hipStream_t>(stream), which, lo,
                       count, d_out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
