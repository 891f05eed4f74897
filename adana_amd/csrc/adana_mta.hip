// adana_mta.hip -- gfx950 multi-tensor kernels of the ADana-family optimizer
// step and the C ABI declared in include/adana_mta.h.
//
// Reference (mlexpos/adana): ADana._update_param_compiled
// (src/optim/adana.py:81-153) and DANA_STAR_MK4._update_param_compiled
// (src/optim/dana_star_mk4.py:105-205), run there once per tensor under
// torch.compile.  Here one launch covers the whole tensor list:
//
//   * the list is laid end to end in a virtual index space (each tensor
//     starting at a multiple of 4 elements) cut into ADANA_CHUNK_ELEMS-element
//     chunks; one 256-thread workgroup owns one chunk, which may span several
//     small tensors or be one slice of a large one;
//   * each workgroup streams p, g, m, v (and tau) once with 16-byte loads,
//     applies the update element by element and writes p, m, v (tau) once;
//   * the four per-tensor sums behind the diagnostics are reduced per
//     (chunk, tensor) segment with DPP wave reductions and an LDS combine,
//     written to partials[chunk + tensor], and combined per tensor in binary64
//     by a fold kernel and a one-wave-per-tensor finalize kernel
//     (deterministic, no atomics).
//
// Element arithmetic follows the reference's op order with every op one
// correctly rounded binary32 operation (built with -ffp-contract=off), in one
// of the reference's two numerics: its default torch.compile path (Inductor's
// decompositions of lerp_ and addcmul_, products and sums rounded one by one,
// bfloat16 state rounded only where it is stored), or, with
// ADANA_NUMERICS_EAGER, its ATen ops (lerp_ and addcmul_ as single-rounded
// FMAs; bfloat16 state rounded after every op).
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "adana_mta.h"
#include "adana_internal.h"
#include "adana_fastmath.h"
#include "adana_pow.h"

namespace {
thread_local char g_err[512] = "";
}  // namespace

int adana_set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

namespace {

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kChunk = ADANA_CHUNK_ELEMS;
static_assert(kChunk == 4 * kBlock, "auxiliary kernels use 256-thread workgroups");
static_assert(ADANA_ALIGN_ELEMS % 4 == 0, "tensors start on vector boundaries");
static_assert(sizeof(adana_tensor_desc) == 64, "descriptor layout");
static_assert(sizeof(adana_step_scalars) == 64, "scalar layout");
static_assert(sizeof(adana_manau_scalars) == sizeof(adana_step_scalars), "Manau scalars share the slot");

// A class's binary32 scalars as the bfloat16 ops see them (the reference's
// bfloat16 path, ADANA_STATE_BF16).  Computed once per launch on the host
// (ScalarPack::c16) and by pow16_fill_kernel; bf16_round_int is the
// conversion instruction's rounding in integer arithmetic.
struct Scalars16 {
    float a16, lerp_coef16, eps16, pw16, min_p16, clip16, c3_16, cg2_16, e16;
    int32_t lerp_small16;
};
__host__ __device__ inline Scalars16 scalars16(const adana_step_scalars &sc) {
    Scalars16 q;
    q.a16 = adana::bf16_round_int(sc.a);
    q.lerp_small16 = fabsf(q.a16) < 0.5f;
    q.lerp_coef16 = q.lerp_small16 ? q.a16 : q.a16 - 1.0f;
    q.eps16 = adana::bf16_round_int(sc.eps);
    q.pw16 = adana::bf16_round_int(sc.pw);
    q.min_p16 = adana::bf16_round_int(sc.min_p);
    q.clip16 = adana::bf16_round_int(sc.clip);
    q.c3_16 = adana::bf16_round_int(sc.c3);
    q.cg2_16 = adana::bf16_round_int(sc.cg2);
    q.e16 = adana::bf16_round_int(sc.star_exp);
    return q;
}

struct ScalarPack {
    adana_step_scalars c[ADANA_MAX_CLASSES];
    const float *gscale;          // device pointer to the clip coefficient, or NULL
    int32_t write_grad;           // store the scaled gradient back (ADANA_WRITE_GRAD)
    int32_t reserved;
    const unsigned short *pow16;  // POW_TABLE16: the launch's pow table in the workspace
    Scalars16 c16[ADANA_MAX_CLASSES];   // ADANA_STATE_BF16: scalars16(c[k])
};

// ---------------------------------------------------------------------------
// Element math
// ---------------------------------------------------------------------------

__device__ __forceinline__ float sign_f(float x) {  // torch.sign: 0 for +-0, NaN
    return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
}
// torch.clamp(x, max=c), torch.clamp(x, min=c), torch.relu: NaN propagates.
// gfx950's IEEE 754-2019 minimum / maximum (v_minimum3_f32, v_maximum3_f32),
// one instruction each.  They order -0 below +0, where the compare-and-select
// forms return x; that differs only for zeros of opposite sign, which the step
// never meets with a visible effect: the bounds are 0.5, 1 and the SNR clip
// applied to a non-negative factor, and relu's result is added to min_p > 0.
__device__ __forceinline__ float clamp_max(float x, float c) { return __builtin_elementwise_minimum(x, c); }
__device__ __forceinline__ float clamp_min(float x, float c) { return __builtin_elementwise_maximum(x, c); }
__device__ __forceinline__ float relu_f(float x) { return __builtin_elementwise_maximum(x, 0.0f); }

__device__ __forceinline__ float bf16_to_f32(unsigned short h) {
    return __uint_as_float(static_cast<unsigned int>(h) << 16);
}
// Round to nearest even (NaN stays a quiet NaN): gfx950's conversion instruction.
__device__ __forceinline__ unsigned short f32_to_bf16(float f) { return adana::bf16_bits(f); }
__device__ __forceinline__ float bf16_round(float f) { return adana::bf16_round(f); }

// x ** k for an integer k (|k| < 32), as Inductor's pow lowering expands it
// (torch/_inductor/lowering.py, pow_recursive): for k < 0 the powers of
// 1 / x; x ** 2j = (x ** j) ** 2 and x ** (2j + 1) = (x ** j) ** 2 * x, i.e.
// left-to-right binary powering, every product rounded.  k == 0 gives 1.
__host__ __device__ inline float pow_int_f32(float x, int k) {
    if (k < 0) {
        x = 1.0f / x;
        k = -k;
    }
    if (k == 0) return 1.0f;
    int top = 0;
    while ((k >> (top + 1)) != 0) ++top;
    float r = x;
    for (int b = top - 1; b >= 0; --b) {
        r = r * r;
        if ((k >> b) & 1) r = r * x;
    }
    return r;
}

// clip_grad_norm_'s in-place product (torch/nn/utils/clip_grad.py,
// _clip_grads_with_norm_: torch._foreach_mul_(grads, clip_coef_clamped)):
// g * coef in binary32, rounded to bfloat16 for bfloat16 gradients.
template <bool GBF16>
__device__ __forceinline__ float scale_grad(float g, float s) {
    const float x = g * s;
    return GBF16 ? bf16_round(x) : x;
}

// x ** e with ATen's exponent specialisations (pow(Tensor, Scalar)).  POWK
// selects the code at compile time: POW_GENERAL (0 < e < 1, i.e. 0 < kappa
// < 1) evaluates in binary64 and rounds once (adana_pow.h); POW_ONE (kappa
// == 1) is exactly 1; POW_SPECIAL dispatches on the remaining ATen
// specialisations, with any other exponent through the slow-path-guarded pow.
enum PowKind { POW_GENERAL = 0, POW_ONE = 1, POW_SPECIAL = 2,
               // Manau's Dana-Star-MK4 branch with mk4A = mk4B = 0 (its other two
               // powers are then a copy and a one), by the kind of its 1 - kappa
               // exponent; POW_MANAU_MK4: any exponents, chosen per class at run time
               POW_MANAU_GENERAL = 3, POW_MANAU_ONE = 4, POW_MANAU_SPECIAL = 5, POW_MANAU_MK4 = 6,
               // bfloat16 state with one general exponent for the launch: the pow of
               // every possible input read from a table the launch fills first
               POW_TABLE16 = 7 };
constexpr bool is_manau(int powk) { return powk >= POW_MANAU_GENERAL && powk <= POW_MANAU_MK4; }
constexpr bool pow_tables(int powk) { return powk == POW_GENERAL || powk == POW_MANAU_GENERAL; }

// The pow's tables as the kernel reads them: POW_GENERAL instances copy them
// into LDS at the start of each workgroup (3 KB), so the per-lane table reads
// are LDS reads rather than gathers on the vector-memory path that carries
// the step's streaming loads and stores.
struct PowTab {
    const adana::LogPair *log;
    const double *exp2j;
    const unsigned short *pow16;   // POW_TABLE16 only
};

template <int POWK>
__device__ __forceinline__ float pow_aten(float x, const adana_step_scalars &sc, const PowTab &tab) {
    if constexpr (POWK == POW_GENERAL) {
        return adana::pow_f32_unit_exp_tab(x, sc.star_exp, tab.log, tab.exp2j);
    } else if constexpr (POWK == POW_ONE) {
        return 1.0f;
    } else {
        switch (sc.pow_mode) {
        case ADANA_POW_ONE: return 1.0f;
        case ADANA_POW_IDENTITY: return x;
        case ADANA_POW_SQRT: return adana::sqrt_f32(x);
        case ADANA_POW_RSQRT: return 1.0f / adana::sqrt_f32(x);
        case ADANA_POW_RECIP: return 1.0f / x;
        case ADANA_POW_SQUARE: return x * x;
        case ADANA_POW_CUBE: return (x * x) * x;
        case ADANA_POW_INVSQ: return 1.0f / (x * x);
        case ADANA_POW_INT: return pow_int_f32(x, sc.pow_int);
        default: return adana::pow_f32_via_f64(x, sc.star_exp);
        }
    }
}

// Which of the reference's forms of the update an instance computes:
//  NUM_COMPILED  the per-tensor update under torch.compile (the default);
//  NUM_EAGER     the same update as ATen's eager ops (ADANA_NUMERICS_EAGER);
//  NUM_FOREACH   the use_foreach=True path's kernel (ADANA_FOREACH), float32
//                state, compiled or eager (the two differ only in host
//                scalars);
//  NUM_FOREACH16 the same path on bfloat16 state under torch.compile: ATen's
//                lerp rounds m and tau to bfloat16 (its coefficient comes
//                from alpha rounded to bfloat16, set by the host), the tau
//                update is read rounded, the rest is binary32, and the
//                averaged alpha factor and mfac are the bfloat16 tensors;
//  NUM_FOREACH_EAGER16 that path's eager ops on bfloat16 state, every op
//                rounded to bfloat16 (update_n16).
enum Numerics { NUM_COMPILED = 0, NUM_EAGER = 1, NUM_FOREACH = 2, NUM_FOREACH16 = 3, NUM_FOREACH_EAGER16 = 4 };
constexpr bool is_foreach(int num) { return num >= NUM_FOREACH; }
// bfloat16 state with every op rounded to bfloat16 (the eager ATen forms)
constexpr bool rounds_every_op(int num) { return num == NUM_EAGER || num == NUM_FOREACH_EAGER16; }

// m.lerp_(grad, alpha) with w = alpha, c = (|w| < 0.5 ? w : w - 1) (w - 1 is
// precomputed, exact) and b = (|w| < 0.5 ? self : end).  ATen (eager, and
// the foreach path's lerp in both modes) computes fma(c, end - self, b);
// Inductor's decomposition (torch._refs.lerp, the per-tensor compiled path)
// computes c * (end - self) + b, product and sum rounded separately.
template <int NUM>
__device__ __forceinline__ float lerp_op(float self, float end, const adana_step_scalars &sc) {
    if constexpr (NUM == NUM_COMPILED) {
        return sc.lerp_coef * (end - self) + (sc.lerp_small ? self : end);
    } else {
        const float r = __builtin_fmaf(sc.lerp_coef, end - self, sc.lerp_small ? self : end);
        return NUM == NUM_FOREACH16 ? bf16_round(r) : r;
    }
}
// v.mul_(1 - alpha).addcmul_(grad, grad, value=alpha): ATen's addcmul_ is
// fma(alpha * g, g, v * (1 - alpha)); Inductor computes v * (1 - alpha) +
// (g * g) * alpha, and so does the foreach path (mul_, mul, mul, add_).
template <int NUM>
__device__ __forceinline__ float ema2_op(float v, float g, const adana_step_scalars &sc) {
    if constexpr (NUM == NUM_EAGER) return __builtin_fmaf(sc.a * g, g, v * sc.oma);
    else return v * sc.oma + (g * g) * sc.a;
}
// The foreach path's alpha factor and mfac as the diagnostics average them:
// the bfloat16 tensors its kernel returns on bfloat16 state.
template <int NUM>
__device__ __forceinline__ float diag_val(float x) { return NUM == NUM_FOREACH16 ? bf16_round(x) : x; }

__device__ __forceinline__ void accumulate(float (&acc)[4], float af, float g, float mfac, float m) {
    acc[0] += af;
    acc[1] += g * g;
    acc[2] += mfac;
    acc[3] += m * m;
}

// The end of the foreach path's update (src/optim/adana.py:345-368,
// src/optim/dana_star_mk4.py:497-528): g3 = (inner * gamma_3_factor) * lr,
// g2 = (g * nt) * lr, p + neg(g2 + g3), then p + p * wdf.  (The per-tensor
// scalar fields c3, cg2 and opw carry gamma_3_factor, lr and wdf here.)
__device__ __forceinline__ float foreach_p(float p, float g, float inner, float nt, const adana_step_scalars &sc) {
    const float g3t = (inner * sc.c3) * sc.cg2;
    const float g2t = (g * nt) * sc.cg2;
    const float pn = p - (g2t + g3t);
    return pn + pn * sc.opw;
}

// ADana / Dana-MK4, one element: src/optim/adana.py:101-143; foreach path
// :316-368.
template <int NUM>
__device__ __forceinline__ float adana_elem(float p, float g, float &m, float &v,
                                            const adana_step_scalars &sc, float (&acc)[4]) {
    const float mn = lerp_op<NUM>(m, g, sc);                     // :101
    const float vn = ema2_op<NUM>(v, g, sc);                     // :104 mul_, addcmul_
    const float se = adana::sqrt_f32(vn) + sc.eps;               // :107
    const float nt = 1.0f / se;                                  // :110
    const float mfac = fabsf(mn) * nt;                           // :111, :115
    float af = sc.pw * mfac;                                     // :119 / :123
    if (sc.has_clip) af = clamp_max(af, sc.clip);
    const float inner = sign_f(mn) * af + mn * nt;               // :126
    float pn;
    if constexpr (is_foreach(NUM)) {
        pn = foreach_p(p, g, inner, nt, sc);                     // :349-368
    } else {
        const float g3t = sc.c3 * inner;
        const float g2t = (sc.cg2 * g) * nt;                     // :129
        pn = p + (g2t + g3t);                                    // :132-135
        pn = pn * sc.opw;                                        // :143
    }
    m = mn;
    v = vn;
    accumulate(acc, diag_val<NUM>(af), g, diag_val<NUM>(mfac), mn);
    return pn;
}

// Dana-Star / Dana-Star-MK4, split around the per-element pow so that the
// kernel can evaluate four pows together and share their rare slow path.
struct StarMid {
    float m, v, se, tau, tr, et;
};

// src/optim/dana_star_mk4.py:137-159; foreach path :425-463
template <int NUM>
__device__ __forceinline__ StarMid star_phase_a(float g, float m, float v, float tau,
                                                const adana_step_scalars &sc) {
    StarMid o;
    o.m = lerp_op<NUM>(m, g, sc);                                // :137
    o.v = ema2_op<NUM>(v, g, sc);                                // :140
    const float sv = adana::sqrt_f32(o.v);
    o.se = sv + sc.eps;                                          // :143
    const float ag = fabsf(g);                                   // :147
    float tu;
    if constexpr (is_foreach(NUM)) {
        tu = ag / ((ag + sv) + sc.eps);                          // :429-436
        if constexpr (NUM == NUM_FOREACH16) tu = bf16_round(tu);   // lerp_'s operand, stored
    } else {
        tu = ag / (ag + o.se);                                   // :148
    }
    o.tau = lerp_op<NUM>(tau, tu, sc);                           // :149
    const float ct = clamp_max(o.tau, 0.5f);                     // :152
    // ct in [0, 0.5]: 1 - ct is in [0.5, 1], and exactly 1 when ct < 2^-25
    const float pe = adana::div_core(ct, 1.0f - ct);                    // :153
    if constexpr (is_foreach(NUM)) {
        o.tr = clamp_min(pe, sc.min_p);                          // :457 maximum(p_estimate, min_p)
    } else {
        o.tr = sc.min_p + relu_f(pe - sc.min_p);                 // :154-156
    }
    o.et = clamp_min(o.tau * sc.s, 1.0f);                        // :159 / :461-463
    return o;
}

// src/optim/dana_star_mk4.py:163-195, given pw = effective_time ** (1 - kappa);
// foreach path :468-528
template <int NUM>
__device__ __forceinline__ float star_phase_b(float p, float g, const StarMid &a, float pw,
                                              const adana_step_scalars &sc, float (&acc)[4]) {
    // tau_reg >= 1/(1+t) >= 2^-24 (t < 2^24): far above sqrt's scaling range
    const float nt = adana::sqrt_normal(a.tr) / a.se;                   // :163-164
    const float mnt = fabsf(a.m) * nt;                           // :165
    float mfac;
    if constexpr (is_foreach(NUM)) mfac = nt * (fabsf(a.m) / a.tr);     // :474-476
    else mfac = mnt / a.tr;                                      // :167
    float af = pw * mfac;                                        // :170 / :174
    if (sc.has_clip) af = clamp_max(af, sc.clip);
    // sign(m) * (tau_reg * af + |m| * nt); the foreach path's
    // (tau_reg * sign(m)) * af + m * nt (:490-497) rounds to the same value
    const float inner = sign_f(a.m) * (a.tr * af + mnt);         // :177
    float pn;
    if constexpr (is_foreach(NUM)) {
        pn = foreach_p(p, g, inner, nt, sc);                     // :499-528
    } else {
        const float g3t = sc.c3 * inner;
        const float g2t = (sc.cg2 * g) * nt;                     // :180
        pn = p + (g2t + g3t);                                    // :183-186
        pn = pn * sc.opw;                                        // :195
    }
    accumulate(acc, diag_val<NUM>(af), g, diag_val<NUM>(mfac), a.m);
    return pn;
}

// ---------------------------------------------------------------------------
// The reference's own bfloat16 path (ADANA_STATE_BF16): bfloat16 parameters
// make m, v and tau bfloat16 too (zeros_like(p), src/optim/adana.py:191-195;
// src/optim/dana_star_mk4.py:251-255).  Compiled (the default), Inductor
// loads them as binary32, runs the binary32 update above and rounds the four
// stored results to bfloat16: thread_elems does exactly that.  Eager
// (ADANA_NUMERICS_EAGER), every tensor op rounds its binary32 result to
// bfloat16, as ATen's kernels do on bfloat16 tensors (below).  How each op
// meets its float32 0-d and Python-scalar operands (probed op by op against
// torch 2.10 and pinned by the reference's own bfloat16 run):
//   * lerp_'s float32 0-d weight is rounded to bfloat16 first;
//   * mul / div with the 0-d tensor second (v.mul_(1 - a), tau * step,
//     p.mul_(1 + wd)) use its binary32 value; with the 0-d tensor first
//     ((-g2) * grad, (-g3)*gf * x, pow * mfac, min_p + x) or in add / sub
//     (add_(epsilon), pe - min_p) it is rounded to bfloat16;
//   * addcmul_(g, g, value=a) = fma(a * g, g, v), a unrounded;
//   * Dana-Star's pow(et, 1 - kappa) takes the exponent rounded to bfloat16;
//   * clamp(x, max=c) compares with c rounded to bfloat16.
// Divisions and square roots of bfloat16 values use adana::div_bf16 and
// adana::sqrt_bf16, whose results round to the same bfloat16 as the IEEE ones.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float rb(float x) { return bf16_round(x); }

// POW_TABLE16: one entry per bfloat16 value in [1, +inf] (bits 0x3F80 .. 0x7F80).
constexpr unsigned int kPow16Entries = 0x7F80u - 0x3F80u + 1u;


// src/optim/adana.py:101-143 on bfloat16 tensors
__device__ __forceinline__ float adana_elem16(float p, float g, float &m, float &v, const adana_step_scalars &sc,
                                              const Scalars16 &q, float (&acc)[4]) {
    const float mn = rb(__builtin_fmaf(q.lerp_coef16, g - m, q.lerp_small16 ? m : g));   // :101
    float vn = rb(v * sc.oma);                                                          // :104 mul_
    vn = rb(__builtin_fmaf(sc.a * g, g, vn));                                           //      addcmul_
    const float se = rb(rb(adana::sqrt_bf16(vn)) + q.eps16);                            // :107
    const float nt = rb(adana::div_bf16(1.0f, se));                                     // :110
    const float mfac = rb(fabsf(mn) * nt);                                              // :111, :115
    float af = rb(q.pw16 * mfac);                                                       // :119 / :123
    if (sc.has_clip) af = clamp_max(af, q.clip16);
    const float inner = rb(sign_f(mn) * af + rb(mn * nt));                              // :126
    const float g3t = rb(q.c3_16 * inner);
    const float g2t = rb(rb(q.cg2_16 * g) * nt);                                        // :129
    float pn = rb(p + rb(g2t + g3t));                                                   // :132-135
    pn = pn * sc.opw;           // :143, rounded to bfloat16 by the store (the same RNE)
    m = mn;
    v = vn;
    accumulate(acc, af, g, mfac, mn);
    return pn;
}

// src/optim/dana_star_mk4.py:137-159 on bfloat16 tensors
__device__ __forceinline__ StarMid star16_phase_a(float g, float m, float v, float tau, const adana_step_scalars &sc,
                                                  const Scalars16 &q) {
    StarMid o;
    o.m = rb(__builtin_fmaf(q.lerp_coef16, g - m, q.lerp_small16 ? m : g));            // :137
    o.v = rb(v * sc.oma);                                                               // :140
    o.v = rb(__builtin_fmaf(sc.a * g, g, o.v));
    o.se = rb(rb(adana::sqrt_bf16(o.v)) + q.eps16);                                     // :143
    const float ag = fabsf(g);                                                          // :147
    const float tu = rb(adana::div_bf16(ag, rb(ag + o.se)));                            // :148
    o.tau = rb(__builtin_fmaf(q.lerp_coef16, tu - tau, q.lerp_small16 ? tau : tu));     // :149
    const float ct = clamp_max(o.tau, 0.5f);                                            // :152
    const float pe = rb(adana::div_bf16(ct, rb(1.0f - ct)));                            // :153
    o.tr = rb(q.min_p16 + relu_f(rb(pe - q.min_p16)));                                  // :154-156
    o.et = clamp_min(rb(o.tau * sc.s), 1.0f);                                           // :159
    return o;
}

// src/optim/dana_star_mk4.py:163-195 on bfloat16 tensors, given pw = et ** e16
__device__ __forceinline__ float star16_phase_b(float p, float g, const StarMid &a, float pw,
                                                const adana_step_scalars &sc, const Scalars16 &q, float (&acc)[4]) {
    const float nt = rb(adana::div_bf16(rb(adana::sqrt_bf16(a.tr)), a.se));             // :163-164
    const float mnt = rb(fabsf(a.m) * nt);                                              // :165
    const float mfac = rb(adana::div_bf16(mnt, a.tr));                                  // :167
    float af = rb(pw * mfac);                                                           // :170 / :174
    if (sc.has_clip) af = clamp_max(af, q.clip16);
    const float inner = sign_f(a.m) * rb(rb(a.tr * af) + mnt);                          // :177
    const float g3t = rb(q.c3_16 * inner);
    const float g2t = rb(rb(q.cg2_16 * g) * nt);                                        // :180
    float pn = rb(p + rb(g2t + g3t));                                                   // :183-186
    pn = pn * sc.opw;           // :195, rounded to bfloat16 by the store (the same RNE)
    accumulate(acc, af, g, mfac, a.m);
    return pn;
}

// et ** e16 rounded to bfloat16 (ATen's pow(Tensor, Scalar) on bfloat16:
// exponent rounded to bfloat16, specialisations chosen on the binary64
// exponent, the result rounded to binary32 and then to bfloat16).
template <int POWK>
__device__ __forceinline__ float pow16(float x, const adana_step_scalars &sc, const Scalars16 &q, const PowTab &tab) {
    if constexpr (POWK == POW_TABLE16) {
        // x = max(bf16(tau * t), 1) is a bfloat16 value in [1, +inf] or a NaN:
        // entry (bits >> 16) - 0x3F80 of the table pow16_fill_kernel wrote
        // with the POW_GENERAL code below, so the same bits.  A NaN gives
        // itself, quieted, as that code does.
        // Branch-free (the load reads entry 0 for a NaN), so a thread's
        // lookups are in flight together.
        const unsigned int idx = (__float_as_uint(x) >> 16) - 0x3F80u;
        const bool in = idx < kPow16Entries;
        const float t = bf16_to_f32(tab.pow16[in ? idx : 0u]);
        return in ? t : rb(x);
    } else if constexpr (POWK == POW_GENERAL) {
        return rb(adana::pow_f32_unit_exp_tab(x, q.e16, tab.log, tab.exp2j));
    } else if constexpr (POWK == POW_ONE) {
        return 1.0f;
    } else {
        switch (sc.pow_mode) {
        case ADANA_POW_ONE: return 1.0f;
        case ADANA_POW_IDENTITY: return x;
        case ADANA_POW_SQRT: return rb(adana::sqrt_bf16(x));
        case ADANA_POW_RSQRT: return rb(1.0f / adana::sqrt_f32(x));
        case ADANA_POW_RECIP: return rb(adana::div_bf16(1.0f, x));
        case ADANA_POW_SQUARE: return rb(x * x);
        case ADANA_POW_CUBE: return rb((x * x) * x);
        case ADANA_POW_INVSQ: return rb(1.0f / (x * x));
        default: return rb(adana::pow_f32_via_f64(x, q.e16));
        }
    }
}

// The POW_TABLE16 table of a launch whose classes share one general exponent
// (sc: any of them): entry k = pow16 of the bfloat16 value with bits
// 0x3F80 + k, by the POW_GENERAL code, stored as bfloat16 bits.
__global__ __launch_bounds__(256) void pow16_fill_kernel(unsigned short *__restrict__ tab, adana_step_scalars sc) {
    const unsigned int k = blockIdx.x * 256u + threadIdx.x;
    if (k >= kPow16Entries) return;
    const Scalars16 q = scalars16(sc);
    const float x = bf16_to_f32(static_cast<unsigned short>(0x3F80u + k));
    tab[k] = f32_to_bf16(pow16<POW_GENERAL>(x, sc, q, PowTab{adana::kLog, adana::kExp2J, nullptr}));
}

// The foreach path's eager ops on bfloat16 state (src/optim/adana.py:316-368,
// src/optim/dana_star_mk4.py:425-528, torch.compile off): every op rounded to
// bfloat16 with the operand rules above, and two of the foreach ops' own: the
// in-place _foreach_mul_ by gamma_3_factor takes it rounded to bfloat16
// (q.c3_16; the out-of-place products do not round their Python scalars),
// and the epsilon added, in place or not, is rounded too (q.eps16).  The
// float32 0-d factors second in a product (1 - alpha, alpha, lr, wdf) keep
// their binary32 values.  The host passes min_p, ADana's power and wdf as the
// reference's 0-d results (bfloat16 step, foreach_scalars).
__device__ __forceinline__ float adana_elem16fe(float p, float g, float &m, float &v, const adana_step_scalars &sc,
                                                const Scalars16 &q, float (&acc)[4]) {
    const float mn = rb(__builtin_fmaf(q.lerp_coef16, g - m, q.lerp_small16 ? m : g));   // _foreach_lerp_
    float vn = rb(v * sc.oma);                                                          // _foreach_mul_
    vn = rb(vn + rb(rb(g * g) * sc.a));                                                 // mul, mul, add_
    const float nt = rb(adana::div_bf16(1.0f, rb(rb(adana::sqrt_bf16(vn)) + q.eps16)));   // sqrt, add, recip
    const float mfac = rb(fabsf(mn) * nt);
    float af = rb(sc.pw * mfac);                                                        // pow (0-d), mul
    if (sc.has_clip) af = clamp_max(af, q.clip16);
    const float inner = rb(rb(rb(sign_f(mn) * af) + rb(mn * nt)) * q.c3_16);           // ..., mul_(gamma)
    const float upd = rb(rb(inner * sc.cg2) + rb(rb(g * nt) * sc.cg2));                // mul(g3), g2, add
    float pn = rb(p - upd);                                                             // neg_, add_
    pn = pn + rb(pn * sc.opw);  // mul, add_ (rounded to bfloat16 by the store)
    m = mn;
    v = vn;
    accumulate(acc, af, g, mfac, mn);
    return pn;
}

__device__ __forceinline__ StarMid star16fe_phase_a(float g, float m, float v, float tau, const adana_step_scalars &sc,
                                                    const Scalars16 &q) {
    StarMid o;
    o.m = rb(__builtin_fmaf(q.lerp_coef16, g - m, q.lerp_small16 ? m : g));            // _foreach_lerp_
    o.v = rb(v * sc.oma);                                                               // _foreach_mul_
    o.v = rb(o.v + rb(rb(g * g) * sc.a));                                               // mul, mul, add_
    const float sv = rb(adana::sqrt_bf16(o.v));
    o.se = rb(sv + q.eps16);                                                            // norm_den
    const float ag = fabsf(g);
    const float tu = rb(adana::div_bf16(ag, rb(rb(ag + sv) + q.eps16)));                // add, add_, div
    o.tau = rb(__builtin_fmaf(q.lerp_coef16, tu - tau, q.lerp_small16 ? tau : tu));    // _foreach_lerp_
    const float ct = clamp_max(o.tau, 0.5f);
    const float pe = rb(adana::div_bf16(ct, rb(1.0f - ct)));                            // neg, add_, div
    o.tr = clamp_min(pe, sc.min_p);                                                     // maximum
    o.et = clamp_min(rb(o.tau * sc.s), 1.0f);                                           // mul, maximum
    return o;
}

__device__ __forceinline__ float star16fe_phase_b(float p, float g, const StarMid &a, float pw,
                                                  const adana_step_scalars &sc, const Scalars16 &q, float (&acc)[4]) {
    const float nt = rb(adana::div_bf16(rb(adana::sqrt_bf16(a.tr)), a.se));             // sqrt, div
    const float mfac = rb(nt * rb(adana::div_bf16(fabsf(a.m), a.tr)));                 // abs, div, mul
    float af = rb(pw * mfac);                                                           // pow, mul
    if (sc.has_clip) af = clamp_max(af, q.clip16);
    const float g3i = rb(rb(rb(a.tr * sign_f(a.m)) * af) + rb(a.m * nt));
    const float upd = rb(rb(rb(g3i * q.c3_16) * sc.cg2) + rb(rb(g * nt) * sc.cg2));    // mul_(gamma), g3, g2
    float pn = rb(p - upd);                                                             // neg_, add_
    pn = pn + rb(pn * sc.opw);  // mul, add_ (rounded to bfloat16 by the store)
    accumulate(acc, af, g, mfac, a.m);
    return pn;
}

template <bool STAR, int POWK, int N, bool FE = false>
__device__ __forceinline__ void update_n16(float (&P)[N], const float (&G)[N], float (&M)[N], float (&V)[N],
                                           float (&T)[N], const adana_step_scalars &sc, const Scalars16 &q,
                                           const PowTab &tab, float (&acc)[4]) {
    if constexpr (!STAR) {
#pragma unroll
        for (int k = 0; k < N; ++k)
            P[k] = FE ? adana_elem16fe(P[k], G[k], M[k], V[k], sc, q, acc) : adana_elem16(P[k], G[k], M[k], V[k], sc, q, acc);
    } else {
        StarMid a[N];
#pragma unroll
        for (int k = 0; k < N; ++k)
            a[k] = FE ? star16fe_phase_a(G[k], M[k], V[k], T[k], sc, q) : star16_phase_a(G[k], M[k], V[k], T[k], sc, q);
        float pw[N];
#pragma unroll
        for (int k = 0; k < N; ++k) pw[k] = pow16<POWK>(a[k].et, sc, q, tab);
#pragma unroll
        for (int k = 0; k < N; ++k) {
            P[k] = FE ? star16fe_phase_b(P[k], G[k], a[k], pw[k], sc, q, acc)
                      : star16_phase_b(P[k], G[k], a[k], pw[k], sc, q, acc);
            M[k] = a[k].m;
            V[k] = a[k].v;
            T[k] = a[k].tau;
        }
    }
}

// ---------------------------------------------------------------------------
// Manau's eager Dana-Star-MK4 branch (src/optim/manau.py:556-613).  Same state
// as Dana-Star, different op order: multiply-then-add moments (ATen's
// add_(x, alpha=a) is one fused multiply-add), (|g| + sqrt v) + eps in the
// tau update, torch.maximum for tau_reg and the effective time, weight decay
// applied to p before the update, and two more per-element powers for
// general mk4A / mk4B.
// ---------------------------------------------------------------------------
__device__ __forceinline__ adana_manau_scalars as_manau(const adana_step_scalars &sc) {
    adana_manau_scalars m;
    __builtin_memcpy(&m, &sc, sizeof m);
    return m;
}

// torch.maximum: NaN if either operand is NaN, else the larger (the first of equals)
__device__ __forceinline__ float maximum_f(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    return a < b ? b : a;
}

// x ** e with ATen's pow(Tensor, Scalar) specialisations (mode chosen on the
// binary64 exponent; e is its binary32 rounding), any other exponent through
// the slow-path-guarded binary64 pow.
__device__ __forceinline__ float pow_by_mode(float x, float e, int mode) {
    switch (mode) {
    case ADANA_POW_ONE: return 1.0f;
    case ADANA_POW_IDENTITY: return x;
    case ADANA_POW_SQRT: return adana::sqrt_f32(x);
    case ADANA_POW_RSQRT: return 1.0f / adana::sqrt_f32(x);
    case ADANA_POW_RECIP: return 1.0f / x;
    case ADANA_POW_SQUARE: return x * x;
    case ADANA_POW_CUBE: return (x * x) * x;
    case ADANA_POW_INVSQ: return 1.0f / (x * x);
    default: return adana::pow_f32_via_f64(x, e);
    }
}

template <int POWK>
__device__ __forceinline__ float manau_elem(float p, float g, float &m, float &v, float &tau,
                                            const adana_manau_scalars &sc, const PowTab &tab, float (&acc)[4]) {
    const float mn = __builtin_fmaf(g, sc.a, m * sc.oma);            // :567 mul_(1-a).add_(g, alpha=a)
    const float vn = __builtin_fmaf(sc.a * g, g, v * sc.oma);        // :569 mul_(1-a).addcmul_(g, g, value=a)
    const float ag = fabsf(g);
    const float sv = adana::sqrt_f32(vn);
    const float tu = ag / ((ag + sv) + sc.eps);                      // :572, _tau_updater :292-299
    const float tn = __builtin_fmaf(tu, sc.a, tau * sc.oma);         // :573
    const float ct = clamp_max(tn, 0.5f);                            // _tau_reg :277-282
    const float pe = ct / (1.0f - ct);
    const float tr = maximum_f(pe, sc.min_p);
    const float et = maximum_f(tn * sc.s, 1.0f);                     // _effective_time :288-290
    const float nt = adana::sqrt_f32(tr) / (sv + sc.eps);            // _norm_term :301-310
    const float mfac = (nt * fabsf(mn)) / tr;                        // :583
    float af;                                                        // :584-589
    if constexpr (POWK == POW_MANAU_MK4) {
        af = (pow_by_mode(et, sc.e[0], sc.mode[0]) * pow_by_mode(mfac, sc.e[1], sc.mode[1])) *
             pow_by_mode(nt, sc.e[2], sc.mode[2]);
    } else {                                  // mfac ** 1 is mfac; nt ** 0 is 1, and x * 1 == x
        float p0;
        if constexpr (POWK == POW_MANAU_GENERAL) {
            p0 = adana::pow_f32_unit_exp_tab(et, sc.e[0], tab.log, tab.exp2j);
        } else if constexpr (POWK == POW_MANAU_ONE) {
            p0 = 1.0f;
        } else {
            p0 = pow_by_mode(et, sc.e[0], sc.mode[0]);
        }
        af = p0 * mfac;
    }
    af = clamp_max(af, sc.clip);
    const float i1 = (tr * sign_f(mn)) * af;                         // :590-593 (1.0 * m is m)
    const float g3t = sc.lr * (i1 + mn * nt);
    const float g2t = (sc.lr * g) * nt;                              // :600
    const float u = -(g2t + g3t);                                    // :603
    float pn = sc.has_wd ? p * sc.wdf : p;                           // :606-610
    pn = pn + u;                                                     // :613
    m = mn;
    v = vn;
    tau = tn;
    accumulate(acc, af, g, mfac, mn);                                // :595-598
    return pn;
}

// One element of either variant (the element-wise tail path).
template <bool STAR, int POWK, int NUM>
__device__ __forceinline__ float update_elem(float p, float g, float &m, float &v, float &tau,
                                             const adana_step_scalars &sc, const PowTab &tab, float (&acc)[4]) {
    if constexpr (is_manau(POWK)) {
        return manau_elem<POWK>(p, g, m, v, tau, as_manau(sc), tab, acc);
    } else if constexpr (!STAR) {
        return adana_elem<NUM>(p, g, m, v, sc, acc);
    } else {
        const StarMid a = star_phase_a<NUM>(g, m, v, tau, sc);
        const float pn = star_phase_b<NUM>(p, g, a, pow_aten<POWK>(a.et, sc, tab), sc, acc);
        m = a.m;
        v = a.v;
        tau = a.tau;
        return pn;
    }
}

// N consecutive elements of one thread (the vector path).  Dana-Star runs
// phase A for all N, then the N pows, then phase B.
template <bool STAR, int POWK, int NUM, int N>
__device__ __forceinline__ void update_n(float (&P)[N], const float (&G)[N], float (&M)[N], float (&V)[N],
                                         float (&T)[N], const adana_step_scalars &sc, const PowTab &tab,
                                         float (&acc)[4]) {
    if constexpr (is_manau(POWK)) {
        const adana_manau_scalars ms = as_manau(sc);
#pragma unroll
        for (int k = 0; k < N; ++k) P[k] = manau_elem<POWK>(P[k], G[k], M[k], V[k], T[k], ms, tab, acc);
    } else if constexpr (!STAR) {
#pragma unroll
        for (int k = 0; k < N; ++k) P[k] = adana_elem<NUM>(P[k], G[k], M[k], V[k], sc, acc);
    } else {
        StarMid a[N];
#pragma unroll
        for (int k = 0; k < N; ++k) a[k] = star_phase_a<NUM>(G[k], M[k], V[k], T[k], sc);
        float pw[N];
#pragma unroll
        for (int k = 0; k < N; ++k) pw[k] = pow_aten<POWK>(a[k].et, sc, tab);
#pragma unroll
        for (int k = 0; k < N; ++k) {
            P[k] = star_phase_b<NUM>(P[k], G[k], a[k], pw[k], sc, acc);
            M[k] = a[k].m;
            V[k] = a[k].v;
            T[k] = a[k].tau;
        }
    }
}

// ---------------------------------------------------------------------------
// Wave reduction: the sum over a wave's 64 lanes, left in lane 63.  GFX9 DPP
// lane moves fused into the adds (no LDS round trips): quad_perm xor 1 and
// xor 2, row_half_mirror and row_mirror (swap the halves of 8- and 16-lane
// groups whose lanes already agree), then row_bcast:15 and row_bcast:31
// fold rows 0-2 into row 3.  Fixed order: deterministic.
// ---------------------------------------------------------------------------
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false);
    return v + __int_as_float(t);
}
__device__ __forceinline__ void wave_sum4_to_lane63(float (&a)[4]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = dpp_add<0xB1, 0xF>(a[k]);   // quad_perm(1,0,3,2)
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = dpp_add<0x4E, 0xF>(a[k]);   // quad_perm(2,3,0,1)
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = dpp_add<0x141, 0xF>(a[k]);  // row_half_mirror
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = dpp_add<0x140, 0xF>(a[k]);  // row_mirror
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = dpp_add<0x142, 0xA>(a[k]);  // row_bcast:15 into rows 1, 3
#pragma unroll
    for (int k = 0; k < 4; ++k) a[k] = dpp_add<0x143, 0xC>(a[k]);  // row_bcast:31 into rows 2, 3
}

// ---------------------------------------------------------------------------
// Memory access: global (not flat) 16-byte vectors, non-temporal for the
// streamed arrays (each byte is touched once per step).
// ---------------------------------------------------------------------------

#define GLOBAL_AS __attribute__((address_space(1)))
template <int N>
struct VecT;
template <>
struct VecT<4> {
    typedef float F __attribute__((ext_vector_type(4)));
    typedef unsigned int H __attribute__((ext_vector_type(2)));  // 4 bf16
};
template <>
struct VecT<2> {
    typedef float F __attribute__((ext_vector_type(2)));
    typedef unsigned int H;                                       // 2 bf16
};

template <int N>
__device__ __forceinline__ void ld_n(const float *p, float (&o)[N]) {
    const typename VecT<N>::F v = __builtin_nontemporal_load((const GLOBAL_AS typename VecT<N>::F *)(p));
#pragma unroll
    for (int k = 0; k < N; ++k) o[k] = v[k];
}
template <int N>
__device__ __forceinline__ void st_n(float *p, const float (&x)[N]) {
    typename VecT<N>::F v;
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = x[k];
    __builtin_nontemporal_store(v, (GLOBAL_AS typename VecT<N>::F *)(p));
}
// N bfloat16 values <-> their bits packed two per 32-bit word
template <int N>
__device__ __forceinline__ void ld_bf16_n(const void *p, float (&o)[N]) {
    const typename VecT<N>::H h = __builtin_nontemporal_load((const GLOBAL_AS typename VecT<N>::H *)(p));
    if constexpr (N == 2) {
        o[0] = __uint_as_float(h << 16);
        o[1] = __uint_as_float(h & 0xffff0000u);
    } else {
#pragma unroll
        for (int k = 0; k < N / 2; ++k) {
            o[2 * k] = __uint_as_float(h[k] << 16);
            o[2 * k + 1] = __uint_as_float(h[k] & 0xffff0000u);
        }
    }
}
template <int N>
__device__ __forceinline__ void st_bf16_n(void *p, const float (&x)[N]) {
    typename VecT<N>::H h;
    if constexpr (N == 2) {
        h = adana::bf16_pack2(x[0], x[1]);
    } else {
#pragma unroll
        for (int k = 0; k < N / 2; ++k) h[k] = adana::bf16_pack2(x[2 * k], x[2 * k + 1]);
    }
    __builtin_nontemporal_store(h, (GLOBAL_AS typename VecT<N>::H *)(p));
}

// The vector path's fp32 stores of p, m, v, tau go out as buffer stores
// with the system-scope + non-temporal policy (sc1 nt): the data is not
// re-read by this step, and on MI355X this lets the write stream through the
// caches 1-2% faster than a non-temporal global store (same-process A/B on
// 2.65B params).  The resource's base is the segment's first element, so a
// lane's byte offset is below 4 KB.
typedef unsigned int U32x4 __attribute__((ext_vector_type(4)));
constexpr int kStorePolicy = 16 | 2;   // sc1 | nt
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float *base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void st4_stream(const float *seg_base, int byte_off, const float (&x)[4]) {
    U32x4 u;
#pragma unroll
    for (int k = 0; k < 4; ++k) u[k] = __float_as_uint(x[k]);
    __builtin_amdgcn_raw_buffer_store_b128(u, buffer_rsrc(seg_base), byte_off, 0, kStorePolicy);
}

template <bool GBF16, int N>
__device__ __forceinline__ void load_grad_n(const void *g, int64_t off, float (&o)[N]) {
    if constexpr (GBF16) ld_bf16_n<N>(static_cast<const unsigned short *>(g) + off, o);
    else ld_n<N>(static_cast<const float *>(g) + off, o);
}
// The vector path's alignment of a gradient: 16 bytes for float32, 8 for bfloat16.
template <bool GBF16>
__device__ __forceinline__ bool grad_vec_aligned(const void *g) {
    return (reinterpret_cast<uintptr_t>(g) & (GBF16 ? 7u : 15u)) == 0;
}
template <bool GBF16>
__device__ __forceinline__ float load_grad1(const void *g, int64_t off) {
    if constexpr (GBF16) return bf16_to_f32(static_cast<const unsigned short *>(g)[off]);
    else return static_cast<const float *>(g)[off];
}
// Gradient write-back (only with ADANA_WRITE_GRAD: the caller's gradient
// buffers are writable then).
template <bool GBF16, int N>
__device__ __forceinline__ void store_grad_n(const void *g, int64_t off, const float (&x)[N]) {
    if constexpr (GBF16) st_bf16_n<N>(const_cast<unsigned short *>(static_cast<const unsigned short *>(g)) + off, x);
    else st_n<N>(const_cast<float *>(static_cast<const float *>(g)) + off, x);
}
template <bool GBF16>
__device__ __forceinline__ void store_grad1(const void *g, int64_t off, float x) {
    if constexpr (GBF16) const_cast<unsigned short *>(static_cast<const unsigned short *>(g))[off] = f32_to_bf16(x);
    else const_cast<float *>(static_cast<const float *>(g))[off] = x;
}

// ---------------------------------------------------------------------------
// Main multi-tensor kernel: one 1024-element chunk per workgroup, GROUPS
// groups of VEC = 4 consecutive elements (one 16-byte vector per array) per
// thread: 256 threads with one group, 128 with two (launch_main picks).  Each
// group is one load -> update -> store pass; waves exit right after their
// last stores.
//
// A chunk inside one tensor (every chunk of a large tensor but its ends) is
// one uniform segment.  A chunk shared by several tensors (small tensors
// packed together, or a tensor's tail and the next one's head) is still one
// pass: each thread finds its own tensor by a binary search over the chunk's
// tensors, all threads load and store at once, and only the per-tensor
// partial sums are then reduced segment by segment.
// ---------------------------------------------------------------------------

// Parameter modes of the step (ADANA_PARAM_BF16 / ADANA_STATE_BF16):
//   PM_F32    float32 parameter and state;
//   PM_MASTER float32 master copy and state, bfloat16 parameter = RNE(master);
//   PM_BF16   the reference's bfloat16 path: parameter, m, v, tau bfloat16,
//             every op rounded to bfloat16 (update_n16).
enum ParamMode { PM_F32 = 0, PM_MASTER = 1, PM_BF16 = 2 };

// One thread's elements of tensor d from element `off` on (`left` of them
// remain in the tensor; VEC at most are processed), with their diagnostics
// terms added to acc.  UNIFORM: every thread of the workgroup works on this
// tensor and the chunk's part of it starts at element seg0, so the fp32
// stores go out as buffer stores from that uniform base.
template <bool STAR, bool GBF16, int PM, int POWK, int NUM, int VEC, bool UNIFORM>
__device__ __forceinline__ void thread_elems(const adana_tensor_desc &d, const void *grad, int64_t off, int64_t left,
                                             int64_t seg0, const ScalarPack &pack, float gs, const PowTab &tab,
                                             float (&acc)[4]) {
    const adana_step_scalars &sc = pack.c[d.sclass];
    const bool scaled = pack.gscale != nullptr;                    // uniform
    const int cnt = left < VEC ? static_cast<int>(left) : VEC;
    // the descriptor's flag covers every pointer but the gradient's
    const bool vec_ok = (d.flags & ADANA_DESC_VEC_OK) && grad_vec_aligned<GBF16>(grad);
    if constexpr (PM == PM_BF16 && !rounds_every_op(NUM)) {
        // the compiled paths on bfloat16 state: binary32 throughout (but for
        // the foreach path's lerps), the four stored results rounded to
        // bfloat16 (round to nearest even)
        unsigned short *pp = static_cast<unsigned short *>(d.param) + off;
        unsigned short *mp = reinterpret_cast<unsigned short *>(d.m) + off;
        unsigned short *vp = reinterpret_cast<unsigned short *>(d.v) + off;
        unsigned short *tp = STAR ? reinterpret_cast<unsigned short *>(d.tau) + off : nullptr;
        if (cnt == VEC && vec_ok) {
            float P[VEC], G[VEC], M[VEC], V[VEC], T[VEC];
            ld_bf16_n<VEC>(pp, P);
            load_grad_n<true, VEC>(grad, off, G);
            ld_bf16_n<VEC>(mp, M);
            ld_bf16_n<VEC>(vp, V);
            if constexpr (STAR) {
                ld_bf16_n<VEC>(tp, T);
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) T[k] = 0.0f;
            }
            if (scaled) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) G[k] = scale_grad<true>(G[k], gs);
                if (pack.write_grad) store_grad_n<true, VEC>(grad, off, G);
            }
            update_n<STAR, POWK, NUM, VEC>(P, G, M, V, T, sc, tab, acc);
            st_bf16_n<VEC>(pp, P);
            st_bf16_n<VEC>(mp, M);
            st_bf16_n<VEC>(vp, V);
            if constexpr (STAR) st_bf16_n<VEC>(tp, T);
        } else {
            for (int e = 0; e < cnt; ++e) {
                float mm = bf16_to_f32(mp[e]), vv = bf16_to_f32(vp[e]), tt = STAR ? bf16_to_f32(tp[e]) : 0.0f;
                float g = load_grad1<true>(grad, off + e);
                if (scaled) {
                    g = scale_grad<true>(g, gs);
                    if (pack.write_grad) store_grad1<true>(grad, off + e, g);
                }
                const float o = update_elem<STAR, POWK, NUM>(bf16_to_f32(pp[e]), g, mm, vv, tt, sc, tab, acc);
                pp[e] = f32_to_bf16(o);
                mp[e] = f32_to_bf16(mm);
                vp[e] = f32_to_bf16(vv);
                if constexpr (STAR) tp[e] = f32_to_bf16(tt);
            }
        }
        return;
    }
    if constexpr (PM == PM_BF16) {
        const Scalars16 &q = pack.c16[d.sclass];
        unsigned short *pp = static_cast<unsigned short *>(d.param) + off;
        unsigned short *mp = reinterpret_cast<unsigned short *>(d.m) + off;
        unsigned short *vp = reinterpret_cast<unsigned short *>(d.v) + off;
        unsigned short *tp = STAR ? reinterpret_cast<unsigned short *>(d.tau) + off : nullptr;
        if (cnt == VEC && vec_ok) {
            float P[VEC], G[VEC], M[VEC], V[VEC], T[VEC];
            ld_bf16_n<VEC>(pp, P);
            load_grad_n<true, VEC>(grad, off, G);
            ld_bf16_n<VEC>(mp, M);
            ld_bf16_n<VEC>(vp, V);
            if constexpr (STAR) {
                ld_bf16_n<VEC>(tp, T);
            } else {
#pragma unroll
                for (int k = 0; k < VEC; ++k) T[k] = 0.0f;
            }
            if (scaled) {
#pragma unroll
                for (int k = 0; k < VEC; ++k) G[k] = scale_grad<true>(G[k], gs);
                if (pack.write_grad) store_grad_n<true, VEC>(grad, off, G);
            }
            update_n16<STAR, POWK, VEC, NUM == NUM_FOREACH_EAGER16>(P, G, M, V, T, sc, q, tab, acc);
            st_bf16_n<VEC>(pp, P);
            st_bf16_n<VEC>(mp, M);
            st_bf16_n<VEC>(vp, V);
            if constexpr (STAR) st_bf16_n<VEC>(tp, T);
        } else {
            for (int e = 0; e < cnt; ++e) {
                float P[1] = {bf16_to_f32(pp[e])}, M[1] = {bf16_to_f32(mp[e])}, V[1] = {bf16_to_f32(vp[e])};
                float T[1] = {STAR ? bf16_to_f32(tp[e]) : 0.0f};
                float G[1] = {load_grad1<true>(grad, off + e)};
                if (scaled) {
                    G[0] = scale_grad<true>(G[0], gs);
                    if (pack.write_grad) store_grad1<true>(grad, off + e, G[0]);
                }
                update_n16<STAR, POWK, 1, NUM == NUM_FOREACH_EAGER16>(P, G, M, V, T, sc, q, tab, acc);
                pp[e] = f32_to_bf16(P[0]);
                mp[e] = f32_to_bf16(M[0]);
                vp[e] = f32_to_bf16(V[0]);
                if constexpr (STAR) tp[e] = f32_to_bf16(T[0]);
            }
        }
        return;
    }
    float *pp = static_cast<float *>(d.param) + off;
    float *mp = d.m + off;
    float *vp = d.v + off;
    float *tp = STAR ? d.tau + off : nullptr;
    if (cnt == VEC && vec_ok) {
        float P[VEC], G[VEC], M[VEC], V[VEC], T[VEC];
        ld_n<VEC>(pp, P);
        load_grad_n<GBF16, VEC>(grad, off, G);
        ld_n<VEC>(mp, M);
        ld_n<VEC>(vp, V);
        if constexpr (STAR) {
            ld_n<VEC>(tp, T);
        } else {
#pragma unroll
            for (int k = 0; k < VEC; ++k) T[k] = 0.0f;
        }
        if (scaled) {
#pragma unroll
            for (int k = 0; k < VEC; ++k) G[k] = scale_grad<GBF16>(G[k], gs);
            if (pack.write_grad) store_grad_n<GBF16, VEC>(grad, off, G);
        }
        update_n<STAR, POWK, NUM, VEC>(P, G, M, V, T, sc, tab, acc);
        if constexpr (UNIFORM && VEC == 4) {
            const int byte_off = static_cast<int>((off - seg0) * 4);
            st4_stream(static_cast<float *>(d.param) + seg0, byte_off, P);
            st4_stream(d.m + seg0, byte_off, M);
            st4_stream(d.v + seg0, byte_off, V);
            if constexpr (STAR) st4_stream(d.tau + seg0, byte_off, T);
        } else {
            st_n<VEC>(pp, P);
            st_n<VEC>(mp, M);
            st_n<VEC>(vp, V);
            if constexpr (STAR) st_n<VEC>(tp, T);
        }
        if constexpr (PM == PM_MASTER) st_bf16_n<VEC>(static_cast<unsigned short *>(d.param_lp) + off, P);
    } else {
        // unaligned tensor, or the last (< VEC) elements of a tensor
        for (int e = 0; e < cnt; ++e) {
            float mm = mp[e], vv = vp[e], tt = STAR ? tp[e] : 0.0f;
            float g = load_grad1<GBF16>(grad, off + e);
            if (scaled) {
                g = scale_grad<GBF16>(g, gs);
                if (pack.write_grad) store_grad1<GBF16>(grad, off + e, g);
            }
            const float o = update_elem<STAR, POWK, NUM>(pp[e], g, mm, vv, tt, sc, tab, acc);
            pp[e] = o;
            mp[e] = mm;
            vp[e] = vv;
            if constexpr (STAR) tp[e] = tt;
            if constexpr (PM == PM_MASTER) static_cast<unsigned short *>(d.param_lp)[off + e] = f32_to_bf16(o);
        }
    }
}

// The GROUPS groups of one thread in a chunk that lies inside tensor d, group
// k at element off + k * span, when every group is a whole aligned vector:
// all groups' loads are issued before the first group's arithmetic, so a
// wave's second group is in flight while it computes the first.  Returns
// false (nothing done) otherwise; the caller then runs thread_elems per group,
// each group's loads after the previous group's stores.  Only the compiled
// bfloat16-state instances take it: they are bound by arithmetic and gain
// from the overlap (Dana-Star at 2.65B params: 11.16 -> 10.78 ms), while the
// float32 ones, bound by HBM, lose to the extra loads in flight (north-star
// 15.02 -> 16.37 ms, C2 0.239 -> 0.266 ms; same-box A/B).
template <bool STAR, bool GBF16, int PM, int POWK, int NUM, int VEC, int GROUPS>
__device__ __forceinline__ bool thread_groups_uniform(const adana_tensor_desc &d, const void *grad, int64_t off,
                                                      int64_t left, int64_t seg0, int span, const ScalarPack &pack,
                                                      float gs, const PowTab &tab, float (&acc)[4]) {
    static_assert(VEC == 4, "grouped path: 16-byte vectors");
    if constexpr (PM != PM_BF16 || rounds_every_op(NUM) || GROUPS == 1) {
        return false;
    } else {
        const bool vec_ok = (d.flags & ADANA_DESC_VEC_OK) && grad_vec_aligned<GBF16>(grad);
        if (!vec_ok || left < static_cast<int64_t>(GROUPS - 1) * span + VEC) return false;
        const adana_step_scalars &sc = pack.c[d.sclass];
        float P[GROUPS][VEC], G[GROUPS][VEC], M[GROUPS][VEC], V[GROUPS][VEC], T[GROUPS][VEC];
#pragma unroll
        for (int k = 0; k < GROUPS; ++k) {
            const int64_t o = off + static_cast<int64_t>(k) * span;
            if constexpr (PM == PM_BF16) {
                ld_bf16_n<VEC>(static_cast<unsigned short *>(d.param) + o, P[k]);
                ld_bf16_n<VEC>(reinterpret_cast<unsigned short *>(d.m) + o, M[k]);
                ld_bf16_n<VEC>(reinterpret_cast<unsigned short *>(d.v) + o, V[k]);
                if constexpr (STAR) ld_bf16_n<VEC>(reinterpret_cast<unsigned short *>(d.tau) + o, T[k]);
            } else {
                ld_n<VEC>(static_cast<float *>(d.param) + o, P[k]);
                ld_n<VEC>(d.m + o, M[k]);
                ld_n<VEC>(d.v + o, V[k]);
                if constexpr (STAR) ld_n<VEC>(d.tau + o, T[k]);
            }
            load_grad_n<GBF16, VEC>(grad, o, G[k]);
            if constexpr (!STAR) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) T[k][e] = 0.0f;
            }
        }
        if (pack.gscale != nullptr) {
#pragma unroll
            for (int k = 0; k < GROUPS; ++k) {
#pragma unroll
                for (int e = 0; e < VEC; ++e) G[k][e] = scale_grad<GBF16>(G[k][e], gs);
                if (pack.write_grad) store_grad_n<GBF16, VEC>(grad, off + static_cast<int64_t>(k) * span, G[k]);
            }
        }
#pragma unroll
        for (int k = 0; k < GROUPS; ++k) {
            const int64_t o = off + static_cast<int64_t>(k) * span;
            update_n<STAR, POWK, NUM, VEC>(P[k], G[k], M[k], V[k], T[k], sc, tab, acc);
            if constexpr (PM == PM_BF16) {
                st_bf16_n<VEC>(static_cast<unsigned short *>(d.param) + o, P[k]);
                st_bf16_n<VEC>(reinterpret_cast<unsigned short *>(d.m) + o, M[k]);
                st_bf16_n<VEC>(reinterpret_cast<unsigned short *>(d.v) + o, V[k]);
                if constexpr (STAR) st_bf16_n<VEC>(reinterpret_cast<unsigned short *>(d.tau) + o, T[k]);
            } else {
                const int byte_off = static_cast<int>((o - seg0) * 4);
                st4_stream(static_cast<float *>(d.param) + seg0, byte_off, P[k]);
                st4_stream(d.m + seg0, byte_off, M[k]);
                st4_stream(d.v + seg0, byte_off, V[k]);
                if constexpr (STAR) st4_stream(d.tau + seg0, byte_off, T[k]);
                if constexpr (PM == PM_MASTER) st_bf16_n<VEC>(static_cast<unsigned short *>(d.param_lp) + o, P[k]);
            }
        }
        return true;
    }
}

// The workgroup's sums of acc, stored by thread 0 as one float4: a wave
// reduction, then a fixed-order combine of the waves in LDS.  The LDS slot
// alternates between calls (par), so no barrier is needed after thread 0 has
// read it.
template <int kW>
__device__ __forceinline__ void block_partial(float (&acc)[4], float (*red)[kW][4], int &par, float4 *dst) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    wave_sum4_to_lane63(acc);
    if (lane == 63) {
#pragma unroll
        for (int k = 0; k < 4; ++k) red[par][wave][k] = acc[k];
    }
    __syncthreads();
    if (tid == 0) {
        float4 q = make_float4(red[par][0][0], red[par][0][1], red[par][0][2], red[par][0][3]);
#pragma unroll
        for (int w = 1; w < kW; ++w) {
            q.x += red[par][w][0];
            q.y += red[par][w][1];
            q.z += red[par][w][2];
            q.w += red[par][w][3];
        }
        *dst = q;
    }
    par ^= 1;
}

template <bool STAR, bool GBF16, int PM, int POWK, int NUM, int VEC, int GROUPS>
__global__ __launch_bounds__(kChunk / (VEC * GROUPS)) void mta_step_kernel(
        const adana_tensor_desc *__restrict__ desc, const void *const *__restrict__ gradp,
        const int64_t *__restrict__ vstart, const int32_t *__restrict__ chunk_first, int32_t n, ScalarPack pack,
        float *__restrict__ partials, int32_t *__restrict__ counters) {
    // GROUPS groups of VEC consecutive elements per thread, group k at element
    // k * kSpan of the chunk: each group's loads and stores stay coalesced,
    // and the per-chunk work (descriptor loads, table copy, reduction) is
    // shared by GROUPS * VEC elements per thread.
    constexpr int kThreads = kChunk / (VEC * GROUPS);
    constexpr int kSpan = kThreads * VEC;
    constexpr int kW = kThreads / 64;
    __shared__ float red[2][kW][4];
    int par = 0;
    const int tid = threadIdx.x;
    const int64_t chunk = blockIdx.x;
    const int64_t lo = chunk * kChunk;
    const int64_t hi = lo + kChunk;
    const int64_t mine = lo + VEC * tid;   // virtual index of this thread's first group
    float4 *part4 = reinterpret_cast<float4 *>(partials);
    // the combine kernel's per-tensor arrival counters start at zero
    for (int64_t k = chunk * kThreads + tid; k < n; k += static_cast<int64_t>(gridDim.x) * kThreads) counters[k] = 0;
    // A compiler-only barrier (no instruction).  Measured, not derived: with
    // it the compiler loads the gradient scale with a vector load and orders
    // the ADana instances' arithmetic differently, and in a same-process A/B
    // the 51M-param Dana-MK4 list stepped 3.5-4% faster and the bf16-master
    // ADana list 1.3% faster; the Dana-Star lists did not move.
    asm volatile("" ::: "memory");
    const float gs = pack.gscale != nullptr ? *pack.gscale : 1.0f;
    PowTab tab{adana::kLog, adana::kExp2J, pack.pow16};
    // Dana-Star's binary64 pow reads its tables from LDS.  The 3 KB are 192
    // 16-byte words (kLog, then kExp2J), kTabPer per thread; the loads are
    // issued here and the words written to LDS only after the chunk's
    // descriptor loads below are issued, so the two round trips overlap.
    // (Writing them after the streaming loads instead, with the barrier
    // between those loads and the arithmetic, cost the 10,000-tensor list 8%.)
    constexpr bool kTab = STAR && pow_tables(POWK);
    constexpr int kTabWords = 192;
    constexpr int kTabPer = (kTabWords + kThreads - 1) / kThreads;
    static_assert(sizeof(adana::kLog) == 128 * 16 && sizeof(adana::kExp2J) == 64 * 16, "table layout");
    static_assert(kTabPer <= 2, "at most two table words per thread");
    __shared__ uint4 s_tab[kTab ? kTabWords : 1];
    // two named words, not an array: a private array here is placed in LDS
    uint4 tab_w0{}, tab_w1{};
    auto table_word = [](int w) {
        return w < 128 ? reinterpret_cast<const uint4 *>(adana::kLog)[w]
                       : reinterpret_cast<const uint4 *>(adana::kExp2J)[w - 128];
    };
    if constexpr (kTab) {
        if (tid < kTabWords) tab_w0 = table_word(tid);
        if constexpr (kTabPer > 1) {
            if (tid + kThreads < kTabWords) tab_w1 = table_word(tid + kThreads);
        }
        tab = PowTab{reinterpret_cast<const adana::LogPair *>(s_tab), reinterpret_cast<const double *>(s_tab + 128),
                     nullptr};
    }

    const int i0 = chunk_first[chunk];
    const int64_t vs0 = vstart[i0];
    const adana_tensor_desc d0 = desc[i0];
    const void *g0 = gradp[i0];
    // both bounds at once (no short circuit), so that the descriptor's numel
    // is fetched with the rest of it rather than after a branch
    const bool inside = (vs0 <= lo) & (vs0 + d0.numel >= hi);
    if constexpr (kTab) {
        if (tid < kTabWords) s_tab[tid] = tab_w0;
        if constexpr (kTabPer > 1) {
            if (tid + kThreads < kTabWords) s_tab[tid + kThreads] = tab_w1;
        }
        __syncthreads();
    }
    if (inside) {
        // the whole chunk lies in tensor i0
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (!thread_groups_uniform<STAR, GBF16, PM, POWK, NUM, VEC, GROUPS>(
                d0, g0, mine - vs0, vs0 + d0.numel - mine, lo - vs0, kSpan, pack, gs, tab, acc)) {
#pragma unroll
            for (int k = 0; k < GROUPS; ++k) {
                const int64_t m = mine + k * kSpan;
                thread_elems<STAR, GBF16, PM, POWK, NUM, VEC, true>(d0, g0, m - vs0, vs0 + d0.numel - m, lo - vs0,
                                                                         pack, gs, tab, acc);
            }
        }
        block_partial<kW>(acc, red, par, part4 + chunk + i0);
        return;
    }
    // Shared chunk: its tensors are i0 .. i1 (chunk_first of the next chunk is
    // the first tensor reaching it, which may also reach into this one).
    const int i1 = (chunk + 1 < static_cast<int64_t>(gridDim.x)) ? chunk_first[chunk + 1] : n - 1;
    int own[GROUPS];
    float acc[GROUPS][4];
#pragma unroll
    for (int k = 0; k < GROUPS; ++k) {
        const int64_t m = mine + k * kSpan;
        int l = i0, r = i1;                  // this group's tensor: the last i with vstart[i] <= m
        while (l < r) {
            const int mid = (l + r + 1) >> 1;
            if (vstart[mid] <= m) l = mid; else r = mid - 1;
        }
        own[k] = l;
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[k][c] = 0.0f;
        const adana_tensor_desc d = desc[l];
        const int64_t vs = vstart[l];
        if (m >= vs && m < vs + d.numel)
            thread_elems<STAR, GBF16, PM, POWK, NUM, VEC, false>(d, gradp[l], m - vs, vs + d.numel - m, 0, pack,
                                                                      gs, tab, acc[k]);
    }
    // one (chunk, tensor) partial per tensor overlapping the chunk, in order
    for (int j = i0; j <= i1; ++j) {
        const int64_t vs = vstart[j];
        if (vs >= hi) break;
        if (vs + desc[j].numel <= lo) continue;                    // uniform across the block
        float a[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) a[c] = (own[0] == j) ? acc[0][c] : 0.0f;
#pragma unroll
        for (int k = 1; k < GROUPS; ++k) {
#pragma unroll
            for (int c = 0; c < 4; ++c) a[c] += (own[k] == j) ? acc[k][c] : 0.0f;
        }
        block_partial<kW>(a, red, par, part4 + chunk + j);
    }
}

// chunk -> first tensor whose virtual range reaches the chunk: the last i with
// vstart[i] <= chunk start (empty tensors share their successor's start).
__global__ __launch_bounds__(kBlock) void chunk_index_kernel(const int64_t *__restrict__ vstart, int32_t n,
                                                             int64_t n_chunks,
                                                             int32_t *__restrict__ chunk_first) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c >= n_chunks) return;
    const int64_t lo = c * kChunk;
    int l = 0, r = n - 1;
    while (l < r) {
        const int mid = (l + r + 1) >> 1;
        if (vstart[mid] <= lo) l = mid; else r = mid - 1;
    }
    chunk_first[c] = l;
}

// Diagnostics combine, stage 1: fold workgroup j reduces up to
// ADANA_FOLD_CHUNKS consecutive (chunk, tensor) partials of one tensor in
// binary64, in a fixed order, to folds[j].  fold_first[i] is tensor i's first
// fold workgroup.
constexpr int kFold = ADANA_FOLD_CHUNKS;
constexpr int kFoldPerThread = kFold / kBlock;
static_assert(kFold % kBlock == 0, "fold workgroups cover whole thread rows");
static_assert(kFold <= ADANA_DIRECT_CHUNKS, "a folded tensor (more than ADANA_DIRECT_CHUNKS chunks) has two folds or more");

// Chunk range [lo, hi] of fold j, tensor i's (fold_first[i] <= j < fold_first[i + 1]).
__device__ __forceinline__ void fold_range(int64_t j, int f0, int64_t b0, int64_t b1, int64_t &lo, int64_t &hi) {
    lo = b0 + (j - f0) * kFold;
    hi = (lo + kFold - 1 < b1) ? lo + kFold - 1 : b1;
}

__device__ __forceinline__ void block_sum4(double &s0, double &s1, double &s2, double &s3,
                                           double (*red)[4]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        s0 += __shfl_xor(s0, o, 64);
        s1 += __shfl_xor(s1, o, 64);
        s2 += __shfl_xor(s2, o, 64);
        s3 += __shfl_xor(s3, o, 64);
    }
    if (lane == 0) { red[wave][0] = s0; red[wave][1] = s1; red[wave][2] = s2; red[wave][3] = s3; }
    __syncthreads();
    s0 = ((red[0][0] + red[1][0]) + red[2][0]) + red[3][0];
    s1 = ((red[0][1] + red[1][1]) + red[2][1]) + red[3][1];
    s2 = ((red[0][2] + red[1][2]) + red[2][2]) + red[3][2];
    s3 = ((red[0][3] + red[1][3]) + red[2][3]) + red[3][3];
}

// The five diagnostics of tensor i from its four binary64 sums
// (src/optim/adana.py:146-151, :221-225): float32, or with bf16 (the
// reference's bfloat16 path, whose diagnostics are bfloat16 0-d tensors)
// each value rounded to bfloat16 and the kappa factor the rounded quotient
// of the two rounded means, stored as bfloat16.
__device__ __forceinline__ void write_diag(void *diag, int bf16, int i, double n, double s0, double s1, double s2,
                                           double s3) {
    float o[5];
    o[0] = static_cast<float>(s0 / n);                   // alpha_factor.mean()
    o[1] = static_cast<float>(sqrt(s1));                 // grad.norm()
    o[2] = static_cast<float>(s2 / n);                   // mfac.mean()
    o[4] = static_cast<float>(sqrt(s3));                 // m.norm()
    if (bf16) {
        unsigned short *h = static_cast<unsigned short *>(diag) + 5 * static_cast<int64_t>(i);
        for (int k = 0; k < 5; ++k) o[k] = bf16_round(o[k]);
        o[3] = bf16_round(o[0] / o[2]);                  // current_alpha / auto_factor_mean
        for (int k = 0; k < 5; ++k) h[k] = f32_to_bf16(o[k]);
        return;
    }
    o[3] = o[0] / o[2];
    float *f = static_cast<float *>(diag) + 5 * static_cast<int64_t>(i);
    for (int k = 0; k < 5; ++k) f[k] = o[k];
}

// Diagnostics combine, after the main kernel.
//  * Workgroups [0, n_folds) are fold workgroups: fold j reduces up to
//    ADANA_FOLD_CHUNKS consecutive chunk partials of one tensor of more than
//    ADANA_DIRECT_CHUNKS chunks, in binary64 and a fixed order, to folds[j].
//    A tensor with a single fold (at most ADANA_FOLD_CHUNKS chunks) is
//    finalized by that workgroup.  For more, with kCombineFenced, the last
//    of a tensor's folds to finish (an arrival
//    counter per tensor, zeroed by the main kernel; agent-scope release and
//    acquire, so the folds written on other XCDs are visible) sums the
//    tensor's folds in index order and writes its diagnostics: one launch.
//    With kCombineFoldOnly the fold workgroups only store their folds, and a
//    second launch (kCombineFinalizeFolded) sums them.
//  * The workgroups after them take four tensors each, one wave per tensor:
//    in the first launch the tensors of at most ADANA_DIRECT_CHUNKS chunks,
//    summing their chunk partials directly in binary64; in the
//    kCombineFinalizeFolded launch (no fold workgroups) the folded tensors.
// Every sum has a fixed order whichever workgroup finishes last, so the
// diagnostics are deterministic.  The fenced single launch suits lists with
// few folds; each fold workgroup's release is an L2 write-back of its XCD on
// gfx950, so lists with many folds take the second launch instead
// (kFencedFoldsMax).
enum CombineMode { kCombineFenced = 0, kCombineFoldOnly = 1, kCombineFinalizeFolded = 2 };
constexpr int64_t kFencedFoldsMax = 256;

// One wave: tensor i's diagnostics from its folds, summed in index order.
__device__ __forceinline__ void finalize_folds(const double4 *__restrict__ folds, int f0, int f1, int lane,
                                               void *diag, int diag_bf16, int i, int64_t numel) {
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    for (int f = f0 + lane; f < f1; f += 64) {
        const double4 t = folds[f];
        s0 += t.x; s1 += t.y; s2 += t.z; s3 += t.w;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        s0 += __shfl_xor(s0, o, 64);
        s1 += __shfl_xor(s1, o, 64);
        s2 += __shfl_xor(s2, o, 64);
        s3 += __shfl_xor(s3, o, 64);
    }
    if (lane == 0) write_diag(diag, diag_bf16, i, static_cast<double>(numel), s0, s1, s2, s3);
}
__global__ __launch_bounds__(kBlock) void combine_kernel(const adana_tensor_desc *__restrict__ desc,
                                                         const int64_t *__restrict__ vstart,
                                                         const int32_t *__restrict__ fold_first, int32_t n,
                                                         int32_t n_folds, const float *__restrict__ partials,
                                                         double4 *__restrict__ folds, int32_t *__restrict__ counters,
                                                         void *__restrict__ diag, int diag_bf16, int mode) {
    __shared__ double red[kWaves][4];
    __shared__ int is_last;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t b = blockIdx.x;
    const float4 *p4 = reinterpret_cast<const float4 *>(partials);
    if (b < n_folds) {
        const int64_t j = b;
        int l = 0, r = n - 1;                   // last tensor with fold_first[i] <= j
        while (l < r) {
            const int mid = (l + r + 1) >> 1;
            if (fold_first[mid] <= j) l = mid; else r = mid - 1;
        }
        const int i = l;
        const int64_t vs = vstart[i], numel = desc[i].numel;
        const int64_t b0 = vs / kChunk, b1 = (vs + numel - 1) / kChunk;
        const int f0 = fold_first[i], f1 = fold_first[i + 1];
        int64_t lo, hi;
        fold_range(j, f0, b0, b1, lo, hi);
        float4 q[kFoldPerThread];
#pragma unroll
        for (int u = 0; u < kFoldPerThread; ++u) {
            const int64_t c = lo + u * kBlock + threadIdx.x;
            q[u] = (c <= hi) ? p4[c + i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
#pragma unroll
        for (int u = 0; u < kFoldPerThread; ++u) {
            s0 += q[u].x; s1 += q[u].y; s2 += q[u].z; s3 += q[u].w;
        }
        block_sum4(s0, s1, s2, s3, red);
        if (mode != kCombineFenced) {
            if (threadIdx.x == 0) folds[j] = make_double4(s0, s1, s2, s3);
            return;
        }
        if (threadIdx.x == 0) {
            folds[j] = make_double4(s0, s1, s2, s3);
            // Every arrival releases its fold; only the last one acquires (the
            // increments form one release sequence, so the acquire fence after
            // reading the final count sees every fold).  On gfx950 an
            // agent-scope acquire invalidates the XCD's L2: paid once per
            // tensor, not once per fold workgroup.
            const int prev = __hip_atomic_fetch_add(&counters[i], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            is_last = (prev == f1 - f0 - 1);
            if (is_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
        if (!is_last || wave != 0) return;
        finalize_folds(folds, f0, f1, lane, diag, diag_bf16, i, numel);
        return;
    }
    const int i = static_cast<int>((b - n_folds) * kWaves + wave);
    if (i >= n) return;                                                   // whole wave
    const int nf = fold_first[i + 1] - fold_first[i];
    if (mode == kCombineFinalizeFolded) {
        if (nf > 0) finalize_folds(folds, fold_first[i], fold_first[i + 1], lane, diag, diag_bf16, i, desc[i].numel);
        return;
    }
    if (nf > 0) return;
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    const int64_t numel = desc[i].numel;
    if (numel > 0) {
        const int64_t b0 = vstart[i] / kChunk, b1 = (vstart[i] + numel - 1) / kChunk;
#pragma unroll 8
        for (int64_t c = b0 + lane; c <= b1; c += 64) {
            const float4 q = p4[c + i];
            s0 += q.x; s1 += q.y; s2 += q.z; s3 += q.w;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        s0 += __shfl_xor(s0, o, 64);
        s1 += __shfl_xor(s1, o, 64);
        s2 += __shfl_xor(s2, o, 64);
        s3 += __shfl_xor(s3, o, 64);
    }
    if (lane == 0) write_diag(diag, diag_bf16, i, static_cast<double>(numel), s0, s1, s2, s3);
}

// ---------------------------------------------------------------------------
// Gradient-norm clipping: torch.nn.utils.clip_grad_norm_(params, max_norm)
// as the reference's training loop calls it before every step
// (src/optim/base.py:250-257, src/distributed/backend.py:33-35).  Torch runs
// a per-tensor norm pass, a norm of the norms, and a read-modify-write pass
// over every gradient.  Here: one read-only pass for the sums of squares, the
// same two-stage combine as the diagnostics, and a one-workgroup finalize
// that writes the total norm and the clip coefficient to device memory; the
// optimizer kernel then multiplies by the coefficient as it loads the
// gradient (or grad_scale_kernel does it in place for a caller without one).
// ---------------------------------------------------------------------------

// Sum of squares per (chunk, tensor) segment in binary64 (each square of a
// binary32 value is exact in binary64), written to partials[chunk + tensor].x.
// One workgroup covers kSumsqChunks consecutive chunks.  When they all lie in
// one tensor with aligned vectors (every chunk of a large tensor but its
// ends), each thread issues its kSumsqChunks 16-byte loads at once and the
// per-chunk sums are reduced together; otherwise the chunks are walked one by
// one, segment by segment.  Either way each chunk's partial is the same
// fixed-order sum of its own elements.
constexpr int kSumsqChunks = 4;

template <bool GBF16>
__device__ __forceinline__ void sumsq_chunk(const adana_tensor_desc *__restrict__ desc,
                                              const void *const *__restrict__ gradp,
                                              const int64_t *__restrict__ vstart, int first, int32_t n,
                                              int64_t chunk, double2 *__restrict__ partials, double (*red)[kWaves]) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t lo = chunk * kChunk, hi = lo + kChunk;
    const int64_t mine = lo + 4 * tid;
    for (int i = first; i < n; ++i) {
        const int64_t vs = vstart[i];
        if (vs >= hi) break;
        const int64_t ve = vs + desc[i].numel;
        if (ve <= lo) continue;
        const void *grad = gradp[i];
        double acc = 0.0;
        if (mine >= vs && mine < ve) {
            const int64_t off = mine - vs;
            const int cnt = (ve - mine) < 4 ? static_cast<int>(ve - mine) : 4;
            if (cnt == 4 && grad_vec_aligned<GBF16>(grad)) {
                float G[4];
                load_grad_n<GBF16, 4>(grad, off, G);
#pragma unroll
                for (int k = 0; k < 4; ++k) acc += static_cast<double>(G[k]) * static_cast<double>(G[k]);
            } else {
                for (int e = 0; e < cnt; ++e) {
                    const double g = load_grad1<GBF16>(grad, off + e);
                    acc += g * g;
                }
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) red[0][wave] = acc;
        __syncthreads();
        if (tid == 0) partials[chunk + i] = make_double2(((red[0][0] + red[0][1]) + red[0][2]) + red[0][3], 0.0);
        __syncthreads();
    }
}

template <bool GBF16>
__global__ __launch_bounds__(kBlock) void grad_sumsq_kernel(const adana_tensor_desc *__restrict__ desc,
                                                            const void *const *__restrict__ gradp,
                                                            const int64_t *__restrict__ vstart,
                                                            const int32_t *__restrict__ chunk_first,
                                                            int32_t n, int64_t n_chunks,
                                                            double2 *__restrict__ partials) {
    constexpr int K = kSumsqChunks;
    __shared__ double red[K][kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x) * K;
    const int64_t nc = (n_chunks - c0) < K ? n_chunks - c0 : K;
    const int i0 = chunk_first[c0];
    const int64_t vs = vstart[i0];
    const int64_t numel0 = desc[i0].numel;
    const void *g0 = gradp[i0];
    if (nc == K && vs <= c0 * kChunk && vs + numel0 >= (c0 + K) * kChunk && grad_vec_aligned<GBF16>(g0)) {
        const int64_t off0 = c0 * kChunk + 4 * tid - vs;
        float G[K][4];
#pragma unroll
        for (int c = 0; c < K; ++c) load_grad_n<GBF16, 4>(g0, off0 + c * kChunk, G[c]);
        double acc[K];
#pragma unroll
        for (int c = 0; c < K; ++c) {
            acc[c] = 0.0;
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[c] += static_cast<double>(G[c][k]) * static_cast<double>(G[c][k]);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
            for (int c = 0; c < K; ++c) acc[c] += __shfl_xor(acc[c], o, 64);
        }
        if (lane == 0) {
#pragma unroll
            for (int c = 0; c < K; ++c) red[c][wave] = acc[c];
        }
        __syncthreads();
        if (tid < K)
            partials[c0 + tid + i0] = make_double2(((red[tid][0] + red[tid][1]) + red[tid][2]) + red[tid][3], 0.0);
        return;
    }
    for (int c = 0; c < nc; ++c) sumsq_chunk<GBF16>(desc, gradp, vstart, chunk_first[c0 + c], n, c0 + c, partials, red);
}

// Stage 1 of the norm combine: like the fold workgroups of combine_kernel, for one
// binary64 sum.
__global__ __launch_bounds__(kBlock) void sumsq_fold_kernel(const adana_tensor_desc *__restrict__ desc,
                                                            const int64_t *__restrict__ vstart,
                                                            const int32_t *__restrict__ fold_first, int32_t n,
                                                            const double2 *__restrict__ partials,
                                                            double *__restrict__ folds) {
    __shared__ double red[kWaves];
    const int64_t j = blockIdx.x;
    int l = 0, r = n - 1;
    while (l < r) {
        const int mid = (l + r + 1) >> 1;
        if (fold_first[mid] <= j) l = mid; else r = mid - 1;
    }
    const int i = l;
    const int64_t vs = vstart[i], numel = desc[i].numel;
    const int64_t b0 = vs / kChunk, b1 = (vs + numel - 1) / kChunk;
    int64_t lo, hi;
    fold_range(j, fold_first[i], b0, b1, lo, hi);
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < kFoldPerThread; ++u) {
        const int64_t b = lo + u * kBlock + threadIdx.x;
        if (b <= hi) s += partials[b + i].x;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) folds[j] = ((red[0] + red[1]) + red[2]) + red[3];
}

// Stage 2, one workgroup: per-tensor norms (torch._foreach_norm, in the
// gradient's dtype), the norm of the norms (torch.linalg.vector_norm of their
// stack) and the clip coefficient, in torch's order and dtype:
//   clip_coef = reciprocal(total + 1e-6) * max_norm   (float / Tensor is
//               Tensor.__rtruediv__ = reciprocal() * other)
//   clip_coef_clamped = clamp(clip_coef, max=1.0)     (NaN stays NaN)
// Each op rounds to the gradient dtype (bfloat16 gradients give bfloat16
// norms and coefficient).  clip[0] = total norm, clip[1] = coefficient.
constexpr int kClipThreads = 1024;
// One wave per tensor (tensors w, w + 16, ... for wave w) sums the tensor's
// folds, or its chunk partials directly when it has no folds.
template <bool GBF16>
__global__ __launch_bounds__(kClipThreads) void clip_finalize_kernel(const adana_tensor_desc *__restrict__ desc,
                                                                     const int64_t *__restrict__ vstart,
                                                                     const int32_t *__restrict__ fold_first,
                                                                     int32_t n, const double2 *__restrict__ partials,
                                                                     const double *__restrict__ folds,
                                                                     float max_norm, float *__restrict__ norms,
                                                                     float *__restrict__ clip) {
    constexpr int kClipWaves = kClipThreads / 64;
    __shared__ double red[kClipWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double tot = 0.0;                                    // lane 0: this wave's tensors, in order
    for (int i = wave; i < n; i += kClipWaves) {
        double s = 0.0;
        const int64_t numel = desc[i].numel;
        if (fold_first[i + 1] > fold_first[i]) {
            for (int f = fold_first[i] + lane; f < fold_first[i + 1]; f += 64) s += folds[f];
        } else if (numel > 0) {
            const int64_t b0 = vstart[i] / kChunk, b1 = (vstart[i] + numel - 1) / kChunk;
#pragma unroll 8
            for (int64_t b = b0 + lane; b <= b1; b += 64) s += partials[b + i].x;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
        float nrm = static_cast<float>(sqrt(s));
        if (GBF16) nrm = bf16_round(nrm);
        if (lane == 0) {
            if (norms) norms[i] = nrm;
            tot += static_cast<double>(nrm) * static_cast<double>(nrm);
        }
    }
    if (lane == 0) red[wave] = tot;
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
        for (int w = 0; w < kClipWaves; ++w) t += red[w];
        float total = static_cast<float>(sqrt(t));
        if (GBF16) total = bf16_round(total);
        float den = total + 1e-6f;
        if (GBF16) den = bf16_round(den);
        float rc = 1.0f / den;
        if (GBF16) rc = bf16_round(rc);
        float coef = rc * max_norm;
        if (GBF16) coef = bf16_round(coef);
        coef = coef > 1.0f ? 1.0f : coef;
        clip[0] = total;
        clip[1] = coef;
    }
}

// In-place g *= coef over a gradient list (clip_grad_norm_ without a fused
// optimizer step).
template <bool GBF16>
__global__ __launch_bounds__(kBlock) void grad_scale_kernel(const adana_tensor_desc *__restrict__ desc,
                                                            const void *const *__restrict__ gradp,
                                                            const int64_t *__restrict__ vstart,
                                                            const int32_t *__restrict__ chunk_first,
                                                            int32_t n, const float *__restrict__ scale) {
    const int64_t chunk = blockIdx.x;
    const int64_t lo = chunk * kChunk, hi = lo + kChunk;
    const int64_t mine = lo + 4 * threadIdx.x;
    const float s = *scale;
    for (int i = chunk_first[chunk]; i < n; ++i) {
        const int64_t vs = vstart[i];
        if (vs >= hi) break;
        const int64_t ve = vs + desc[i].numel;
        if (ve <= lo || mine < vs || mine >= ve) continue;
        const void *grad = gradp[i];
        const int64_t off = mine - vs;
        const int cnt = (ve - mine) < 4 ? static_cast<int>(ve - mine) : 4;
        if (cnt == 4 && grad_vec_aligned<GBF16>(grad)) {
            float G[4];
            load_grad_n<GBF16, 4>(grad, off, G);
#pragma unroll
            for (int k = 0; k < 4; ++k) G[k] = scale_grad<GBF16>(G[k], s);
            store_grad_n<GBF16, 4>(grad, off, G);
        } else {
            for (int e = 0; e < cnt; ++e)
                store_grad1<GBF16>(grad, off + e, scale_grad<GBF16>(load_grad1<GBF16>(grad, off + e), s));
        }
    }
}

// Workspace layout: chunk partials (float4 per (chunk, tensor) slot), then the
// folds (double4 each), then the combine's arrival counters (int32 per
// tensor), then the bfloat16 pow table (POW_TABLE16 launches), each part
// 256-byte aligned.
size_t partials_bytes(const adana_plan &pl) {
    return static_cast<size_t>(pl.n_chunks + pl.n_tensors) * 16;
}
size_t folds_offset(const adana_plan &pl) { return (partials_bytes(pl) + 255) / 256 * 256; }
size_t counters_offset(const adana_plan &pl) {
    return (folds_offset(pl) + static_cast<size_t>(pl.n_folds) * 32 + 255) / 256 * 256;
}
size_t pow16_offset(const adana_plan &pl) {
    return (counters_offset(pl) + static_cast<size_t>(pl.n_tensors) * 4 + 255) / 256 * 256;
}
size_t workspace_bytes(const adana_plan &pl) {
    if (pl.n_chunks == 0) return counters_offset(pl) + static_cast<size_t>(pl.n_tensors) * 4;   // no launch needs the table
    return pow16_offset(pl) + static_cast<size_t>(kPow16Entries) * 2;
}

// Residency cap.  The step reaches the highest HBM throughput with 4
// workgroups per CU rather than the 7-8 its registers allow: fewer concurrent
// streams contend less in the memory system (measured on MI355X at 2.65B
// params, uncapped -> capped: ADana fp32 13.1 -> 12.1 ms, Dana-Star kappa=1
// 17.1 -> 16.1 ms, Dana-Star with the pow, tables in LDS, 16.6 -> 16.3 ms;
// same-process sweep of caps 3/4/5/6: bf16 params with fp32 master 11.78 /
// 11.84 / 12.20 / 12.66 ms, north-star 16.19 / 15.57 / 15.86 / 16.17 ms, C3
// 8.19 / 8.07 / 8.14 / 8.32 ms, C2 0.245 / 0.239 / 0.244 / 0.245 ms).  The exception is
// the pow instance on lists of small tensors (`small_tensors`: fewer than 64
// chunks per tensor on average), whose workgroups spend a larger share of
// their time in per-segment work (tensor lookup, reductions, partial stores)
// and in the pow: it runs best at its register limit (Dana-Star over 10,000
// tensors of 64-65536 elements: 0.715 ms capped, 0.666 ms uncapped; the same
// list at kappa = 1 prefers the cap, 0.658 against 0.748 ms).  bfloat16
// state (PM_BF16) moves half the bytes per workgroup and runs best uncapped:
// Dana-Star at 2.65B params with the per-element pow, 14.25 ms at 4,
// 12.84-12.86 ms at 5, 6, 8 and uncapped (its registers allow 5); with the
// pow table (59 VGPRs), 12.25 / 10.82 / 10.29 / 10.04 ms at 4 / 5 / 6 / 7 and
// 10.00 ms uncapped.  The cap is imposed with dynamic
// LDS the kernel does not touch.
template <bool STAR, int PM, int POWK>
constexpr int residency_cap(bool small_tensors) {
    if (PM == PM_BF16 || (STAR && pow_tables(POWK) && small_tensors)) return 0;
    return 4;
}

// Dynamic LDS bytes that, beside the kernel's `static_lds` bytes, leave room
// for exactly `wgs` workgroups per CU on the current device (0: no cap, or
// the device's LDS size is unavailable): each workgroup then holds 256 bytes
// less than a 1/wgs share, so `wgs` fit and `wgs + 1` do not.  Grids of fewer
// than 64 chunks per CU stay uncapped: there the cap only adds dispatch
// rounds.
struct DeviceLds {
    int per_cu = 0, per_block = 0, cus = 0;
};
// The current device's LDS sizes and CU count (zeros if unavailable), read once per device.
DeviceLds device_lds() {
    static DeviceLds cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return DeviceLds{};
    DeviceLds &c = cache[dev];
    if (c.per_cu <= 0) {
        int cu = 0, blk = 0, n_cu = 0;
        if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
            hipDeviceGetAttribute(&blk, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return DeviceLds{};
        c.per_block = blk;
        c.cus = n_cu;
        c.per_cu = cu;
    }
    return c;
}

// Whether a grid of n_chunks workgroups holds at least `per_cu` of them per CU.
bool grid_fills(int64_t n_chunks, int per_cu) {
    const DeviceLds d = device_lds();
    return d.cus > 0 && n_chunks >= static_cast<int64_t>(per_cu) * d.cus;
}

size_t lds_for_cap(int wgs, int64_t n_chunks, size_t static_lds) {
    if (wgs <= 0) return 0;
    const DeviceLds d = device_lds();
    if (d.per_cu <= 0 || !grid_fills(n_chunks, 64)) return 0;
    const size_t per_cu = static_cast<size_t>(d.per_cu);
    if (per_cu < 32 * 1024) return 0;
    const size_t share = per_cu / static_cast<size_t>(wgs);
    if (share <= static_lds + 256 || share <= 256 * static_cast<size_t>(wgs + 1)) return 0;
    const size_t l = share - 256 - static_lds;
    return l <= static_cast<size_t>(d.per_block) ? l : 0;
}

// The launch's device arrays and workspace pointers.
struct LaunchArgs {
    int64_t n_chunks;
    hipStream_t st;
    const adana_tensor_desc *desc;
    const void *const *grad;
    const int64_t *vstart;
    const int32_t *chunk_first;
    int32_t n;
    float *partials;
    int32_t *counters;
};

template <bool STAR, bool GBF16, int PM, int POWK, int NUM, int GROUPS>
void launch_groups(const LaunchArgs &a, const ScalarPack &pack, bool small_tensors) {
    constexpr int kVec = 4;
    constexpr int kThreads = kChunk / (kVec * GROUPS);
    // the cap counts 256-thread workgroups' worth of waves per CU
    const int cap = residency_cap<STAR, PM, POWK>(small_tensors) * (256 / kThreads);
    // the kernel's static LDS: its reduction slots and, for the pow instances, the tables' copy
    constexpr size_t kStaticLds = 2 * (kThreads / 64) * 4 * sizeof(float) +
                                  ((STAR && pow_tables(POWK)) ? 192 * 16 : 16);
    const size_t lds = lds_for_cap(cap, a.n_chunks, kStaticLds);
    hipLaunchKernelGGL((mta_step_kernel<STAR, GBF16, PM, POWK, NUM, kVec, GROUPS>),
                       dim3(static_cast<unsigned>(a.n_chunks)), dim3(kThreads), static_cast<unsigned>(lds), a.st,
                       a.desc, a.grad, a.vstart, a.chunk_first, a.n, pack, a.partials, a.counters);
}

// Two groups of four elements per thread (128-thread workgroups, the chunk's
// fixed work shared by eight elements) where that is a steady gain:
//  * bfloat16 state, bound by arithmetic: north-star list 11.45 -> 10.78 ms
//    (with the loads first), every box and run;
//  * grids of 64 chunks per CU up to kTwoGroupMaxChunks: C2 0.246 -> 0.239 ms.
// One group (256 threads) elsewhere: on smaller grids, which need the threads
// (C1, 4,096 chunks: 0.0259 -> 0.0278 ms with two); on the pow instance over
// lists of small tensors (C5 0.591 -> 0.597); and on large float32 lists,
// where two groups swing with the box's state: 2-3.5% faster on a settled
// box (north-star 15.57 -> 15.02, C3 7.80 -> 7.55, C4 11.93 -> 11.59 ms),
// 2-6% slower in its first minutes (north-star 15.54 -> 16.26 ms, in one
// process on the same tensors; on that box 15.22 -> 14.99 ms ten minutes
// later), while one group stays within 15.2-15.9 ms throughout.
constexpr int64_t kTwoGroupMaxChunks = 1 << 18;
template <bool STAR, bool GBF16, int PM, int POWK, int NUM>
void launch_main(const LaunchArgs &a, const ScalarPack &pack) {
    const bool small_tensors = a.n_chunks < 64 * static_cast<int64_t>(a.n);
    const bool two = grid_fills(a.n_chunks, 64) && !(STAR && pow_tables(POWK) && small_tensors) &&
                     (PM == PM_BF16 || a.n_chunks <= kTwoGroupMaxChunks);
    if (two) launch_groups<STAR, GBF16, PM, POWK, NUM, 2>(a, pack, small_tensors);
    else launch_groups<STAR, GBF16, PM, POWK, NUM, 1>(a, pack, small_tensors);
}

template <bool STAR, bool GBF16, int PM, int NUM>
void launch_pow(int powk, const LaunchArgs &a, const ScalarPack &pack) {
    if constexpr (!STAR) {
        // ADana's (1 + t) ** (1 - kappa) is a host scalar: no per-element pow
        launch_main<false, GBF16, PM, POW_ONE, NUM>(a, pack);
    } else if (powk == POW_GENERAL) {
        launch_main<true, GBF16, PM, POW_GENERAL, NUM>(a, pack);
    } else if (powk == POW_ONE) {
        launch_main<true, GBF16, PM, POW_ONE, NUM>(a, pack);
    } else if (powk == POW_SPECIAL) {
        launch_main<true, GBF16, PM, POW_SPECIAL, NUM>(a, pack);
    } else if constexpr (PM == PM_BF16 && rounds_every_op(NUM)) {
        if (powk == POW_TABLE16) launch_main<true, GBF16, PM, POW_TABLE16, NUM>(a, pack);
    } else if constexpr (!GBF16 && PM == PM_F32 && NUM == NUM_EAGER) {  // Manau's branch: float32, its own op order
        if (powk == POW_MANAU_GENERAL) {
            launch_main<true, false, PM_F32, POW_MANAU_GENERAL, NUM_EAGER>(a, pack);
        } else if (powk == POW_MANAU_ONE) {
            launch_main<true, false, PM_F32, POW_MANAU_ONE, NUM_EAGER>(a, pack);
        } else if (powk == POW_MANAU_SPECIAL) {
            launch_main<true, false, PM_F32, POW_MANAU_SPECIAL, NUM_EAGER>(a, pack);
        } else {
            launch_main<true, false, PM_F32, POW_MANAU_MK4, NUM_EAGER>(a, pack);
        }
    }
}

// The launch's numerics (num: NUM_COMPILED, NUM_EAGER, or NUM_FOREACH for
// the foreach path, whose instance depends on the state's kind: float32
// state, or bfloat16 state compiled or eager).
template <bool STAR, bool GBF16, int PM>
void launch_num(int num, bool eager, int powk, const LaunchArgs &a, const ScalarPack &pack) {
    if (num == NUM_EAGER) {
        launch_pow<STAR, GBF16, PM, NUM_EAGER>(powk, a, pack);
    } else if (num == NUM_COMPILED) {
        launch_pow<STAR, GBF16, PM, NUM_COMPILED>(powk, a, pack);
    } else if constexpr (PM == PM_BF16) {
        if (eager) launch_pow<STAR, GBF16, PM, NUM_FOREACH_EAGER16>(powk, a, pack);
        else launch_pow<STAR, GBF16, PM, NUM_FOREACH16>(powk, a, pack);
    } else {
        launch_pow<STAR, GBF16, PM, NUM_FOREACH>(powk, a, pack);
    }
}

// ---------------------------------------------------------------------------
// Host scalar code
// ---------------------------------------------------------------------------

int pow_mode_of(double e) {
    if (e == 0.0) return ADANA_POW_ONE;
    if (e == 1.0) return ADANA_POW_IDENTITY;
    if (e == 0.5) return ADANA_POW_SQRT;
    if (e == -0.5) return ADANA_POW_RSQRT;
    if (e == -1.0) return ADANA_POW_RECIP;
    if (e == 2.0) return ADANA_POW_SQUARE;
    if (e == 3.0) return ADANA_POW_CUBE;
    if (e == -2.0) return ADANA_POW_INVSQ;
    return ADANA_POW_GENERAL;
}

// Inductor's pow lowering (torch/_inductor/lowering.py, pow): an exponent
// equal to an integer k becomes pow(x, k) -- 1 for k == 0, a copy for k == 1,
// and for any other |k| < 32 the products of pow_recursive (pow_int_f32);
// 0.5 becomes sqrt; anything else stays a pow with the exponent rounded to
// binary32 (-0.5 included).  *k receives the integer exponent.
int pow_mode_compiled(double e, int32_t *k) {
    *k = 0;
    if (e == 0.0) return ADANA_POW_ONE;
    if (e == 1.0) return ADANA_POW_IDENTITY;
    if (e == 0.5) return ADANA_POW_SQRT;
    if (e == std::floor(e) && std::fabs(e) < 32.0) {
        *k = static_cast<int32_t>(e);
        return ADANA_POW_INT;
    }
    return ADANA_POW_GENERAL;
}

// ADana's (1 + step) ** (1 - kappa) on a 0-d float32 tensor under
// torch.compile: Inductor's CPU code evaluates a general exponent as
// std::pow(float, float), the exponent rounded to binary32.
float pow0d_compiled(float x, double e) {
    int32_t k;
    switch (pow_mode_compiled(e, &k)) {
    case ADANA_POW_ONE: return 1.0f;
    case ADANA_POW_IDENTITY: return x;
    case ADANA_POW_SQRT: return std::sqrt(x);
    case ADANA_POW_INT: return pow_int_f32(x, k);
    default: return std::pow(x, static_cast<float>(e));
    }
}

// ATen pow(Tensor, Scalar) on a 0-d float tensor: specialisations as above,
// otherwise std::pow(float, double) evaluated in binary64.
float pow0d(float x, double e) {
    switch (pow_mode_of(e)) {
    case ADANA_POW_ONE: return 1.0f;
    case ADANA_POW_IDENTITY: return x;
    case ADANA_POW_SQRT: return std::sqrt(x);
    case ADANA_POW_RSQRT: return 1.0f / std::sqrt(x);
    case ADANA_POW_RECIP: return 1.0f / x;
    case ADANA_POW_SQUARE: return x * x;
    case ADANA_POW_CUBE: return (x * x) * x;
    case ADANA_POW_INVSQ: return 1.0f / (x * x);
    default: return static_cast<float>(std::pow(static_cast<double>(x), e));
    }
}

// The foreach path's scalars (hp->foreach; src/optim/adana.py:171-176,
// :245-262 and the 0-d tensor ops of _foreach_compute_kernel_impl, :316-365;
// src/optim/dana_star_mk4.py:229-236, :327-340, :455-456, :520-528): the
// step tensor has the parameters' dtype (foreach == 2: bfloat16, rounded to
// nearest even), alpha is the binary32 quotient of the binary32 delta and
// that step, and every 0-d op is binary32.  c3, cg2 and opw carry
// gamma_3_factor, lr and the weight-decay factor wdf.
int foreach_scalars(adana_step_scalars *out, const adana_hparams *hp, double lr, int64_t step) {
    float s = static_cast<float>(step);
    if (hp->foreach == 2) s = adana::bf16_round_int(s);
    const float sf = static_cast<float>(lr / hp->peak_lr);      // :165, :174
    const float d = static_cast<float>(hp->delta);               // :175
    const float a = d / (d + s);                                 // :259
    const float one_p_s = s + 1.0f;                              // :336 / dana_star_mk4.py:455
    memset(out, 0, sizeof *out);
    out->a = a;
    out->oma = 1.0f - a;                                         // :317-318 neg, add_(1.0)
    // ATen's lerp on the state's dtype: a bfloat16 lerp takes its weight
    // rounded to bfloat16
    const float aw = hp->foreach == 2 ? adana::bf16_round_int(a) : a;
    out->lerp_small = std::fabs(aw) < 0.5f ? 1 : 0;
    out->lerp_coef = out->lerp_small ? aw : aw - 1.0f;
    out->s = s;
    out->eps = static_cast<float>(hp->epsilon);
    out->pw = hp->eager ? pow0d(one_p_s, 1.0 - hp->kappa) : pow0d_compiled(one_p_s, 1.0 - hp->kappa);   // :339
    out->min_p = 1.0f / one_p_s;                                 // dana_star_mk4.py:456
    out->has_clip = hp->has_clip ? 1 : 0;
    out->clip = hp->has_clip ? static_cast<float>(hp->clipsnr) : INFINITY;
    out->c3 = static_cast<float>(hp->gamma_3_factor);            // :350
    out->cg2 = static_cast<float>(lr);                           // :172-173 g2, g3
    const float nws = (-static_cast<float>(hp->weight_decay)) * sf;   // :360 / :363
    out->opw = hp->wd_decaying ? (1.0f / (s / static_cast<float>(hp->wd_ts) + 1.0f)) * nws : nws;  // :357-365
    if (hp->foreach == 2 && hp->eager) {
        // eager 0-d ops on the bfloat16 step tensor, each rounded to bfloat16;
        // the pow's exponent rounded to bfloat16; wdf the float32 product of
        // the bfloat16 decay and the float32 (-wd) * sf, or without decay
        // that factor as bfloat16 (.to(p.dtype), :364)
        const auto rb = [](float x) { return adana::bf16_round_int(x); };
        const float ops = rb(s + 1.0f);
        out->min_p = rb(1.0f / ops);
        out->pw = rb(pow0d(ops, static_cast<double>(rb(static_cast<float>(1.0 - hp->kappa)))));
        out->opw = hp->wd_decaying ? rb(1.0f / rb(rb(s / static_cast<float>(hp->wd_ts)) + 1.0f)) * nws : rb(nws);
    }
    out->star_exp = static_cast<float>(1.0 - hp->kappa);         // dana_star_mk4.py:480
    if (hp->eager) {
        out->pow_mode = pow_mode_of(1.0 - hp->kappa);
    } else {
        int32_t k;
        out->pow_mode = pow_mode_compiled(1.0 - hp->kappa, &k);
        out->pow_int = k;
    }
    return ADANA_OK;
}

}  // namespace

extern "C" {

int adana_abi_version(void) { return ADANA_ABI_VERSION; }

size_t adana_last_error(char *buf, size_t len) {
    const size_t n = strlen(g_err);
    if (buf && len) {
        const size_t c = n < len - 1 ? n : len - 1;
        memcpy(buf, g_err, c);
        buf[c] = '\0';
    }
    return n;
}

int adana_step_scalars_init(adana_step_scalars *out, const adana_hparams *hp, double lr,
                            int64_t step) {
    if (!out || !hp) return adana_set_error(ADANA_E_INVALID, "adana_step_scalars_init: null pointer");
    if (step < 1) return adana_set_error(ADANA_E_INVALID, "adana_step_scalars_init: step %lld < 1",
                                 static_cast<long long>(step));
    if (!(hp->peak_lr != 0.0))
        return adana_set_error(ADANA_E_INVALID, "adana_step_scalars_init: peak lr must be nonzero");
    if (hp->foreach < 0 || hp->foreach > 2)
        return adana_set_error(ADANA_E_INVALID, "adana_step_scalars_init: foreach=%d outside [0, 2]", hp->foreach);
    if (hp->foreach) return foreach_scalars(out, hp, lr, step);
    // Host doubles (src/optim/adana.py:163-165, :200), rounded to binary32 the
    // way torch.tensor(x, dtype=float32) does (:203-208).
    const float sf = static_cast<float>(lr / hp->peak_lr);
    const float g = static_cast<float>(lr);
    const float wd = static_cast<float>(hp->weight_decay);
    const float a = static_cast<float>(hp->delta / (hp->delta + static_cast<double>(step)));
    const float s = static_cast<float>(step);
    const float one_p_s = 1.0f + s;
    memset(out, 0, sizeof *out);
    out->a = a;
    out->oma = 1.0f - a;
    out->lerp_small = std::fabs(a) < 0.5f ? 1 : 0;
    out->lerp_coef = out->lerp_small ? a : a - 1.0f;
    out->s = s;
    out->eps = static_cast<float>(hp->epsilon);
    out->pw = hp->eager ? pow0d(one_p_s, 1.0 - hp->kappa) : pow0d_compiled(one_p_s, 1.0 - hp->kappa);
    out->min_p = 1.0f / one_p_s;
    out->has_clip = hp->has_clip ? 1 : 0;
    out->clip = hp->has_clip ? static_cast<float>(hp->clipsnr) : INFINITY;
    out->c3 = (-g) * static_cast<float>(hp->gamma_3_factor);
    out->cg2 = -g;
    float wdf;
    if (hp->wd_decaying) {
        const float q = s / static_cast<float>(hp->wd_ts);
        wdf = ((-wd) / (1.0f + q)) * sf;
    } else {
        wdf = (-wd) * sf;
    }
    out->opw = 1.0f + wdf;
    out->star_exp = static_cast<float>(1.0 - hp->kappa);
    if (hp->eager) {
        out->pow_mode = pow_mode_of(1.0 - hp->kappa);
    } else {
        int32_t k;
        out->pow_mode = pow_mode_compiled(1.0 - hp->kappa, &k);
        out->pow_int = k;
    }
    return ADANA_OK;
}

int adana_manau_scalars_init(adana_manau_scalars *out, const adana_manau_hparams *hp, double lr, double step,
                             double alpha) {
    if (!out || !hp) return adana_set_error(ADANA_E_INVALID, "adana_manau_scalars_init: null pointer");
    if (!(step >= 0.0)) return adana_set_error(ADANA_E_INVALID, "adana_manau_scalars_init: step %g < 0", step);
    // Python floats (src/optim/manau.py:539-555) rounded to binary32 where
    // they meet float32 tensors: as tensor-scalar operands (mul_, add_,
    // addcmul_, clamp, lr * tensor, tau * step) and full_like (min_p).
    memset(out, 0, sizeof *out);
    out->a = static_cast<float>(alpha);
    out->oma = static_cast<float>(1.0 - alpha);                  // :567 mul_(1 - alpha)
    out->s = static_cast<float>(step);                           // :289 tau * step
    out->eps = static_cast<float>(hp->epsilon);
    out->min_p = static_cast<float>(1.0 / (1.0 + step));        // :281 full_like(tau, 1/(1+step))
    out->clip = static_cast<float>(hp->clipsnr);
    out->lr = static_cast<float>(lr);
    const double wdf = hp->wd_decaying ? 1.0 - hp->weight_decay / (1.0 + step / hp->wd_ts) * lr
                                       : 1.0 - hp->weight_decay * lr;            // :606-610
    out->wdf = static_cast<float>(wdf);
    out->has_wd = hp->weight_decay != 0.0 ? 1 : 0;
    const double ex[3] = {1.0 - hp->kappa, 2.0 * hp->mk4B + 1.0, 2.0 * (-hp->mk4A - hp->mk4B)};   // :585-587
    for (int k = 0; k < 3; ++k) {
        out->e[k] = static_cast<float>(ex[k]);
        out->mode[k] = pow_mode_of(ex[k]);
    }
    return ADANA_OK;
}

int64_t adana_plan_layout(const int64_t *numel, int32_t n, int64_t *vstart,
                          int32_t *fold_first, int64_t *n_folds) {
    if (n < 0 || !vstart || !fold_first || !n_folds || (n > 0 && !numel))
        return adana_set_error(ADANA_E_INVALID, "adana_plan_layout: bad arguments");
    int64_t off = 0, folds = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (numel[i] < 0) return adana_set_error(ADANA_E_INVALID, "adana_plan_layout: numel[%d] < 0", i);
        // A tensor that would cross a chunk boundary from inside a chunk
        // starts at the next boundary instead, so that a large tensor's head
        // or tail does not share a chunk: a shared chunk costs a tensor lookup
        // per thread and one partial reduction per tensor (C5's 10,000-tensor
        // list, same process: 0.684 ms without this rule, 0.597 ms with it).
        // Small tensors still pack together inside one chunk.
        const int64_t r = off % kChunk;
        if (r != 0 && r + numel[i] > kChunk) off += kChunk - r;
        vstart[i] = off;
        fold_first[i] = static_cast<int32_t>(folds);
        if (numel[i] > 0) {
            const int64_t chunks_i = (off + numel[i] - 1) / kChunk - off / kChunk + 1;
            if (chunks_i > ADANA_DIRECT_CHUNKS) folds += (chunks_i + kFold - 1) / kFold;
        }
        off += (numel[i] + ADANA_ALIGN_ELEMS - 1) / ADANA_ALIGN_ELEMS * ADANA_ALIGN_ELEMS;
        if (folds > 0x7fffffffLL) return adana_set_error(ADANA_E_UNSUPPORTED, "adana_plan_layout: list too large");
    }
    vstart[n] = off;
    fold_first[n] = static_cast<int32_t>(folds);
    *n_folds = folds;
    const int64_t chunks = (off + kChunk - 1) / kChunk;
    if (chunks > 0x7fffffffLL) return adana_set_error(ADANA_E_UNSUPPORTED, "adana_plan_layout: list too large");
    return chunks;
}

int adana_plan_index(const int64_t *d_vstart, int32_t n_tensors, int64_t n_chunks,
                     int32_t *d_chunk_first, void *stream) {
    if (n_tensors < 0 || n_chunks < 0 || n_chunks > 0x7fffffffLL)
        return adana_set_error(ADANA_E_INVALID, "adana_plan_index: bad sizes");
    if (n_chunks == 0) return ADANA_OK;
    if (n_tensors == 0 || !d_vstart || !d_chunk_first)
        return adana_set_error(ADANA_E_INVALID, "adana_plan_index: null pointer or no tensors");
    const unsigned blocks = static_cast<unsigned>((n_chunks + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(chunk_index_kernel, dim3(blocks), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), d_vstart, n_tensors, n_chunks, d_chunk_first);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return adana_set_error(ADANA_E_HIP, "adana_plan_index: launch failed: %s", hipGetErrorString(err));
    return ADANA_OK;
}

size_t adana_workspace_bytes(const adana_plan *plan) {
    return plan ? workspace_bytes(*plan) : 0;
}

}  // extern "C"

namespace {

// Plan checks shared by the entry points; return ADANA_OK or an error code.
int check_plan(const adana_plan *plan, const char *fn) {
    if (!plan) return adana_set_error(ADANA_E_INVALID, "%s: null plan", fn);
    const adana_plan &pl = *plan;
    if (pl.n_tensors < 0 || pl.n_chunks < 0 || pl.n_chunks > 0x7fffffffLL || pl.n_folds < 0 ||
        pl.n_folds > 0x7fffffffLL)
        return adana_set_error(ADANA_E_INVALID, "%s: bad sizes (n_tensors=%d, n_chunks=%lld)", fn, pl.n_tensors,
                       static_cast<long long>(pl.n_chunks));
    return ADANA_OK;
}
int check_plan_arrays(const adana_plan &pl, const char *fn) {
    if (pl.n_tensors > 0 &&
        (!pl.desc || !pl.grad || !pl.vstart || !pl.fold_first || (pl.n_chunks > 0 && !pl.chunk_first)))
        return adana_set_error(ADANA_E_INVALID, "%s: null pointer in the plan arrays", fn);
    return ADANA_OK;
}

int launch_status(const char *fn, const char *what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return adana_set_error(ADANA_E_HIP, "%s: %s launch failed: %s", fn, what, hipGetErrorString(err));
    return ADANA_OK;
}

int step_impl(const char *fn, const adana_plan *plan, const adana_step_scalars *h_scalars, int32_t n_classes,
              uint32_t variant_flags, const float *d_grad_scale, void *d_workspace, size_t ws_bytes,
              float *d_diag, void *stream) {
    if (int rc = check_plan(plan, fn)) return rc;
    const adana_plan &pl = *plan;
    const uint32_t allowed = ADANA_VARIANT_STAR | ADANA_GRAD_BF16 | ADANA_PARAM_BF16 | ADANA_VARIANT_MANAU |
                             ADANA_STATE_BF16 | ADANA_NUMERICS_EAGER | ADANA_FOREACH |
                             (d_grad_scale ? ADANA_WRITE_GRAD : 0u);
    if (variant_flags & ~allowed)
        return adana_set_error(ADANA_E_INVALID, "%s: unknown variant flags 0x%x", fn, variant_flags);
    const bool manau = variant_flags & ADANA_VARIANT_MANAU;
    if (manau && (variant_flags & (ADANA_GRAD_BF16 | ADANA_PARAM_BF16 | ADANA_STATE_BF16)))
        return adana_set_error(ADANA_E_INVALID, "%s: ADANA_VARIANT_MANAU is float32 only", fn);
    const bool s16 = variant_flags & ADANA_STATE_BF16;
    if (s16 && (!(variant_flags & ADANA_GRAD_BF16) || (variant_flags & ADANA_PARAM_BF16)))
        return adana_set_error(ADANA_E_INVALID, "%s: ADANA_STATE_BF16 needs ADANA_GRAD_BF16 and excludes "
                               "ADANA_PARAM_BF16", fn);
    const bool foreach = variant_flags & ADANA_FOREACH;
    if (foreach && manau)
        return adana_set_error(ADANA_E_INVALID, "%s: ADANA_FOREACH excludes ADANA_VARIANT_MANAU", fn);
    if (int rc = check_plan_arrays(pl, fn)) return rc;
    if (pl.n_tensors == 0) return ADANA_OK;
    if (!d_workspace || !d_diag || !h_scalars)
        return adana_set_error(ADANA_E_INVALID, "%s: null pointer argument", fn);
    if (n_classes < 1 || n_classes > ADANA_MAX_CLASSES)
        return adana_set_error(ADANA_E_INVALID, "%s: n_classes=%d outside [1, %d]", fn, n_classes, ADANA_MAX_CLASSES);
    if (ws_bytes < workspace_bytes(pl))
        return adana_set_error(ADANA_E_INVALID, "%s: workspace of %zu bytes < %zu needed", fn, ws_bytes,
                       workspace_bytes(pl));
    ScalarPack pack;
    memset(&pack, 0, sizeof pack);
    memcpy(pack.c, h_scalars, sizeof(adana_step_scalars) * static_cast<size_t>(n_classes));
    pack.gscale = d_grad_scale;
    pack.write_grad = (variant_flags & ADANA_WRITE_GRAD) ? 1 : 0;
    const bool eager = variant_flags & ADANA_NUMERICS_EAGER;
    if (s16 && eager)
        for (int k = 0; k < n_classes; ++k) pack.c16[k] = scalars16(pack.c[k]);
    hipStream_t st = static_cast<hipStream_t>(stream);
    float *partials = static_cast<float *>(d_workspace);
    double4 *folds = reinterpret_cast<double4 *>(static_cast<char *>(d_workspace) + folds_offset(pl));
    int32_t *counters = reinterpret_cast<int32_t *>(static_cast<char *>(d_workspace) + counters_offset(pl));
    const bool star = variant_flags & ADANA_VARIANT_STAR;
    const bool gb = variant_flags & ADANA_GRAD_BF16;
    const bool pb = variant_flags & ADANA_PARAM_BF16;
    const int32_t n = pl.n_tensors;
    if (pl.n_chunks > 0) {
        // one pow code path per launch: all classes must agree on it
        bool all_one = true, all_general = true, mk4_trivial = true;
        for (int c = 0; c < n_classes; ++c) {
            int mode;
            float e;
            if (manau) {
                adana_manau_scalars ms;
                memcpy(&ms, &h_scalars[c], sizeof ms);
                mode = ms.mode[0];
                e = ms.e[0];
                mk4_trivial = mk4_trivial && ms.mode[1] == ADANA_POW_IDENTITY && ms.mode[2] == ADANA_POW_ONE;
            } else {
                mode = h_scalars[c].pow_mode;
                e = h_scalars[c].star_exp;
            }
            all_one = all_one && mode == ADANA_POW_ONE;
            all_general = all_general && mode == ADANA_POW_GENERAL && e > 0.0f && e < 1.0f;
        }
        int powk = all_general ? POW_GENERAL : (all_one ? POW_ONE : POW_SPECIAL);
        if (manau) powk = mk4_trivial ? powk + POW_MANAU_GENERAL : POW_MANAU_MK4;
        if (s16 && eager && star && powk == POW_GENERAL) {
            // bfloat16 state, every op rounded: the pow's input is a bfloat16
            // value; with one exponent for every class, fill the launch's pow
            // table first (16,385 entries, stream-ordered before the step)
            bool same_exp = true;
            for (int c = 1; c < n_classes; ++c) same_exp = same_exp && h_scalars[c].star_exp == h_scalars[0].star_exp;
            if (same_exp) {
                unsigned short *tab = reinterpret_cast<unsigned short *>(static_cast<char *>(d_workspace) +
                                                                          pow16_offset(pl));
                hipLaunchKernelGGL(pow16_fill_kernel, dim3((kPow16Entries + 255) / 256), dim3(256), 0, st, tab,
                                   h_scalars[0]);
                if (int rc = launch_status(fn, "pow table")) return rc;
                pack.pow16 = tab;
                powk = POW_TABLE16;
            }
        }
        const LaunchArgs la{pl.n_chunks, st, pl.desc, pl.grad, pl.vstart, pl.chunk_first, n, partials, counters};
        const int num = foreach ? NUM_FOREACH : ((eager || manau) ? NUM_EAGER : NUM_COMPILED);
#define ADANA_LAUNCH(S, G, P) launch_num<S, G, P>(num, eager, powk, la, pack)
        if (star || manau) {
            if (s16) ADANA_LAUNCH(true, true, PM_BF16);
            else if (gb) { if (pb) ADANA_LAUNCH(true, true, PM_MASTER); else ADANA_LAUNCH(true, true, PM_F32); }
            else         { if (pb) ADANA_LAUNCH(true, false, PM_MASTER); else ADANA_LAUNCH(true, false, PM_F32); }
        } else {
            if (s16) ADANA_LAUNCH(false, true, PM_BF16);
            else if (gb) { if (pb) ADANA_LAUNCH(false, true, PM_MASTER); else ADANA_LAUNCH(false, true, PM_F32); }
            else         { if (pb) ADANA_LAUNCH(false, false, PM_MASTER); else ADANA_LAUNCH(false, false, PM_F32); }
        }
#undef ADANA_LAUNCH
        if (int rc = launch_status(fn, "main")) return rc;
    }
    const int64_t tensor_wgs = (n + kWaves - 1) / kWaves;
    const bool fenced = pl.n_folds <= kFencedFoldsMax;
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(pl.n_folds + tensor_wgs)), dim3(kBlock), 0, st,
                       pl.desc, pl.vstart, pl.fold_first, n, static_cast<int32_t>(pl.n_folds), partials, folds,
                       counters, static_cast<void *>(d_diag), s16 ? 1 : 0,
                       fenced ? kCombineFenced : kCombineFoldOnly);
    if (int rc = launch_status(fn, "combine")) return rc;
    if (fenced) return ADANA_OK;
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>(tensor_wgs)), dim3(kBlock), 0, st, pl.desc,
                       pl.vstart, pl.fold_first, n, 0, partials, folds, counters, static_cast<void *>(d_diag),
                       s16 ? 1 : 0, static_cast<int>(kCombineFinalizeFolded));
    return launch_status(fn, "combine (finalize)");
}

}  // namespace

extern "C" {

int adana_mta_step(const adana_plan *plan, const adana_step_scalars *h_scalars, int32_t n_classes,
                   uint32_t variant_flags, void *d_workspace, size_t ws_bytes, float *d_diag,
                   void *stream) {
    return step_impl("adana_mta_step", plan, h_scalars, n_classes, variant_flags, nullptr, d_workspace,
                     ws_bytes, d_diag, stream);
}

int adana_mta_step_scaled(const adana_plan *plan, const adana_step_scalars *h_scalars, int32_t n_classes,
                          uint32_t variant_flags, const float *d_grad_scale, void *d_workspace,
                          size_t ws_bytes, float *d_diag, void *stream) {
    if (!d_grad_scale) return adana_set_error(ADANA_E_INVALID, "adana_mta_step_scaled: null gradient scale");
    return step_impl("adana_mta_step_scaled", plan, h_scalars, n_classes, variant_flags, d_grad_scale,
                     d_workspace, ws_bytes, d_diag, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free step: the chunk partials and folds live in a file-scope
// device array (each GPU the library runs on holds its own copy until the
// process ends) instead of a caller workspace.  Host code never uses the
// array's name as an address: the per-device address comes from
// hipGetSymbolAddress, once per device, on the entry point's first call on
// that device.  Every call on one GPU shares that GPU's array; the step
// writes every slot it reads, so nothing needs clearing, but calls that
// overlap on one GPU (two streams, two threads) race on it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char scratch[ADANA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void *> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's copy of `scratch`.
int scratch_address(void **out, const char *fn) {
    int dev = -1;
    hipError_t err = hipGetDevice(&dev);
    if (err != hipSuccess) return adana_set_error(ADANA_E_HIP, "%s: hipGetDevice: %s", fn, hipGetErrorString(err));
    if (dev < 0 || dev >= kMaxDevices) return adana_set_error(ADANA_E_UNSUPPORTED, "%s: device %d", fn, dev);
    void *p = g_scratch[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch[dev].load(std::memory_order_relaxed);
        if (!p) {
            err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (err != hipSuccess || !p)
                return adana_set_error(ADANA_E_HIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                                       hipGetErrorString(err));
            g_scratch[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return ADANA_OK;
}

}  // namespace

extern "C" {

int adana_mta_step_noalloc(const adana_plan *plan, const adana_step_scalars *h_scalars, int32_t n_classes,
                           uint32_t variant_flags, float *d_diag, void *stream) {
    const char *fn = "adana_mta_step_noalloc";
    if (int rc = check_plan(plan, fn)) return rc;
    const size_t need = workspace_bytes(*plan);
    if (need > static_cast<size_t>(ADANA_NOALLOC_SCRATCH_BYTES))
        return adana_set_error(ADANA_E_UNSUPPORTED,
                               "%s: the list needs %zu bytes of scratch (16 per chunk and tensor, 32 per fold), "
                               "more than the library's static %zu bytes; call adana_mta_step with a workspace",
                               fn, need, static_cast<size_t>(ADANA_NOALLOC_SCRATCH_BYTES));
    if (int rc = check_plan_arrays(*plan, fn)) return rc;
    if (plan->n_tensors == 0) return ADANA_OK;
    if (!d_diag || !h_scalars) return adana_set_error(ADANA_E_INVALID, "%s: null pointer argument", fn);
    void *ws = nullptr;
    if (int rc = scratch_address(&ws, fn)) return rc;
    return step_impl(fn, plan, h_scalars, n_classes, variant_flags, nullptr, ws,
                     static_cast<size_t>(ADANA_NOALLOC_SCRATCH_BYTES), d_diag, stream);
}

int adana_grad_clip_norm(const adana_plan *plan, uint32_t grad_flags, double max_norm, void *d_workspace,
                         size_t ws_bytes, float *d_norms, float *d_clip, void *stream) {
    const char *fn = "adana_grad_clip_norm";
    if (int rc = check_plan(plan, fn)) return rc;
    const adana_plan &pl = *plan;
    if (grad_flags & ~ADANA_GRAD_BF16) return adana_set_error(ADANA_E_INVALID, "%s: unknown flags 0x%x", fn, grad_flags);
    if (int rc = check_plan_arrays(pl, fn)) return rc;
    if (!d_clip) return adana_set_error(ADANA_E_INVALID, "%s: null clip output", fn);
    if (pl.n_tensors > 0 && !d_workspace) return adana_set_error(ADANA_E_INVALID, "%s: null workspace", fn);
    if (ws_bytes < workspace_bytes(pl))
        return adana_set_error(ADANA_E_INVALID, "%s: workspace of %zu bytes < %zu needed", fn, ws_bytes,
                       workspace_bytes(pl));
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool gb = grad_flags & ADANA_GRAD_BF16;
    double2 *partials = static_cast<double2 *>(d_workspace);
    double *folds = reinterpret_cast<double *>(static_cast<char *>(d_workspace) + folds_offset(pl));
    const int32_t n = pl.n_tensors;
    if (pl.n_chunks > 0) {
        const dim3 grid(static_cast<unsigned>((pl.n_chunks + kSumsqChunks - 1) / kSumsqChunks));
        if (gb) hipLaunchKernelGGL(grad_sumsq_kernel<true>, grid, dim3(kBlock), 0, st, pl.desc, pl.grad,
                                   pl.vstart, pl.chunk_first, n, pl.n_chunks, partials);
        else hipLaunchKernelGGL(grad_sumsq_kernel<false>, grid, dim3(kBlock), 0, st, pl.desc, pl.grad,
                                pl.vstart, pl.chunk_first, n, pl.n_chunks, partials);
        if (int rc = launch_status(fn, "sum of squares")) return rc;
    }
    if (pl.n_folds > 0) {
        hipLaunchKernelGGL(sumsq_fold_kernel, dim3(static_cast<unsigned>(pl.n_folds)), dim3(kBlock), 0, st,
                           pl.desc, pl.vstart, pl.fold_first, n, partials, folds);
        if (int rc = launch_status(fn, "fold")) return rc;
    }
    // torch casts the Python float max_norm to the coefficient's binary32 opmath
    const float mn = static_cast<float>(max_norm);
    if (gb) hipLaunchKernelGGL(clip_finalize_kernel<true>, dim3(1), dim3(kClipThreads), 0, st, pl.desc, pl.vstart,
                               pl.fold_first, n, partials, folds, mn, d_norms, d_clip);
    else hipLaunchKernelGGL(clip_finalize_kernel<false>, dim3(1), dim3(kClipThreads), 0, st, pl.desc, pl.vstart,
                            pl.fold_first, n, partials, folds, mn, d_norms, d_clip);
    return launch_status(fn, "finalize");
}

int adana_grad_scale(const adana_plan *plan, uint32_t grad_flags, const float *d_scale, void *stream) {
    const char *fn = "adana_grad_scale";
    if (int rc = check_plan(plan, fn)) return rc;
    const adana_plan &pl = *plan;
    if (grad_flags & ~ADANA_GRAD_BF16) return adana_set_error(ADANA_E_INVALID, "%s: unknown flags 0x%x", fn, grad_flags);
    if (int rc = check_plan_arrays(pl, fn)) return rc;
    if (!d_scale) return adana_set_error(ADANA_E_INVALID, "%s: null scale", fn);
    if (pl.n_tensors == 0 || pl.n_chunks == 0) return ADANA_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(pl.n_chunks));
    if (grad_flags & ADANA_GRAD_BF16)
        hipLaunchKernelGGL(grad_scale_kernel<true>, grid, dim3(kBlock), 0, st, pl.desc, pl.grad, pl.vstart,
                           pl.chunk_first, pl.n_tensors, d_scale);
    else
        hipLaunchKernelGGL(grad_scale_kernel<false>, grid, dim3(kBlock), 0, st, pl.desc, pl.grad, pl.vstart,
                           pl.chunk_first, pl.n_tensors, d_scale);
    return launch_status(fn, "scale");
}

}  // extern "C"
