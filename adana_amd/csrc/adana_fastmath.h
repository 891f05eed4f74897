// adana_fastmath.h -- correctly rounded binary32 division and square root for
// operand ranges on which the full IEEE sequences' range scaling and
// special-case fixups are identities, and the bfloat16 path's rounding,
// division and square root.  Same results, fewer instructions.
// tests/gpu_mathcheck.hip checks each exhaustively: the binary32 ones over the
// ranges the optimizer kernel uses them on, the bfloat16 ones over every
// bfloat16 input (every pair for the division) and the rounding over every
// binary32 input.
#ifndef ADANA_FASTMATH_H
#define ADANA_FASTMATH_H

#include <hip/hip_runtime.h>

namespace adana {

// v_cmp_class_f32 masks.
constexpr int kClassZero = (1 << 5) | (1 << 6);
constexpr int kClassNormal = (1 << 3) | (1 << 8);
constexpr int kClassPosNormal = 1 << 8;

// x, as a new value the compiler cannot compute before the branch that holds
// this (one v_mov in that branch): keeps an IEEE sequence in its rare arm
// instead of being run for every element and selected.
__device__ __forceinline__ float opaque(float x) {
    float y;
    asm volatile("v_mov_b32 %0, %1" : "=v"(y) : "v"(x));
    return y;
}

// A class mask for v_cmp_class_f32, held in an SGPR.  With a constant mask the
// compiler picks the VOPC form, whose mask operand must be a VGPR, and writes
// the literal into a VGPR before every test (gfx9's VOP3 encodings take no
// literal); from an SGPR the VOP3 form reads it directly, one VALU instruction
// per test instead of two.
__device__ __forceinline__ int class_mask(int m) {
    int r;
    asm("s_mov_b32 %0, %1" : "=s"(r) : "i"(m));
    return r;
}

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

// Correctly rounded sqrt for every binary32 x: sqrt_normal on [2^-96, +inf]
// and for +-0 (about 8 instructions against the IEEE sequence's 20), the IEEE
// sequence for small nonzero and negative inputs and NaNs, behind a real
// branch.  Zeros stay on the fast path: a second moment that never saw a
// nonzero gradient (zero rows of an embedding) is 0 for whole waves.
__device__ __forceinline__ float sqrt_f32(float x) {
    float s = sqrt_normal(x);
    if (__builtin_expect(!(x >= 0x1p-96f || x == 0.0f), 0)) s = __builtin_sqrtf(opaque(x));
    return s;
}

// ---------------------------------------------------------------------------
// bfloat16 rounding and the bfloat16 path's division and square root.
// ---------------------------------------------------------------------------

// Round to nearest even; a NaN stays a quiet NaN ((bits >> 16) | 0x40): gfx950's
// v_cvt_pk_bf16_f32, which rounds two binary32 values into the two halves of
// one register.  bf16_round converts the pair (0, f): the low half is then
// zero and the high half bf16(f), so the register is already the rounded
// value as a binary32 -- one instruction, no shift.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned short bf16_bits(float f) {
    return __builtin_bit_cast(unsigned short, static_cast<__bf16>(f));
}
__device__ __forceinline__ float bf16_round(float f) {
    const f32x2_t v = {0.0f, f};
    return __builtin_bit_cast(float, __builtin_convertvector(v, bf16x2_t));
}
// The same rounding in integer arithmetic, for host code and for values
// that are the same for every lane (the launch's scalars, rounded once on
// the host): round to nearest even, a NaN quieted as above.
__host__ __device__ inline float bf16_round_int(float f) {
    const unsigned int u = __builtin_bit_cast(unsigned int, f);
    const unsigned int r = (u & 0x7fffffffu) > 0x7f800000u ? (u | 0x00400000u) : u + 0x7fffu + ((u >> 16) & 1u);
    return __builtin_bit_cast(float, r & 0xffff0000u);
}
// bf16(lo) | bf16(hi) << 16: two values' bits in one 32-bit word.
__device__ __forceinline__ unsigned int bf16_pack2(float lo, float hi) {
    const f32x2_t v = {lo, hi};
    return __builtin_bit_cast(unsigned int, __builtin_convertvector(v, bf16x2_t));
}

// a / b for bfloat16 values a and b: a binary32 value that rounds to the same
// bfloat16 as the correctly rounded binary32 quotient.  Why the hardware
// reciprocal is enough: with a = A 2^i and b = B 2^j (A, B at most 8
// significant bits), a quotient equal to a bfloat16 midpoint M 2^k (M odd, 9
// bits) would need A = M B, more than 8 bits; so a normal quotient lies at
// least 2^k / 255 > 2^7 binary32 ulps from every midpoint, and a * rcp(b)
// (within 2 ulps) rounds like it.  A zero product with a normal reciprocal is
// a zero numerator or a quotient below 2^-149, which the IEEE quotient rounds
// to a bfloat16 zero of the same sign.  Anything else (a subnormal, infinite
// or NaN quotient or reciprocal) takes the IEEE sequence.
__device__ __forceinline__ float div_bf16(float a, float b) {
    const float y = __builtin_amdgcn_rcpf(b);
    float q = a * y;
    const bool fast = __builtin_amdgcn_classf(q, class_mask(kClassNormal | kClassZero)) &&
                      __builtin_amdgcn_classf(y, class_mask(kClassNormal));
    if (__builtin_expect(!fast, 0)) q = opaque(a) / b;
    return q;
}

// sqrt(x) for a bfloat16 value x: a binary32 value that rounds to the same
// bfloat16 as the correctly rounded square root.  sqrt(x) = M 2^k (M odd, 9
// bits) would need x = M^2 2^2k, 17 significant bits; so sqrt(x) lies at least
// 2^5 binary32 ulps from every bfloat16 midpoint and the hardware square root
// (within 1 ulp) rounds like the exact one.  Zeros give themselves; other
// inputs (subnormals, negatives, infinities) and NaNs take the IEEE sequence.
__device__ __forceinline__ float sqrt_bf16(float x) {
    float s = __builtin_amdgcn_sqrtf(x);
    if (__builtin_expect(!__builtin_amdgcn_classf(x, class_mask(kClassPosNormal | kClassZero)), 0))
        s = __builtin_sqrtf(opaque(x));
    return s;
}

}  // namespace adana

#endif  // ADANA_FASTMATH_H
