// adana_pow.h -- x ** y for Dana-Star's per-element effective-time factor,
// evaluated in binary64 and rounded once to binary32.
//
// Reference call site: ``(effective_time ** (1 - kappa))`` on the per-element
// tensor effective_time = clamp(tau * step, min=1) (src/optim/dana_star_mk4.py
// :159, :170/:174).  The exponent is the binary32 rounding of 1 - kappa.
//
// Method (table-driven argument reduction, all arithmetic in binary64):
//   x = 2^e * m, m in [1, 2);  j = top 7 bits of m's fraction
//   r = m * invc[j] - 1 (exact: invc has 12 significant bits), |r| < 0.0043
//   (invc[j] and -ln invc[j] sit side by side: one 16-byte table load)
//   ln x = e*ln2 + (-ln invc[j]) + log1p(r),  log1p by its degree-7 series
//   t = y * ln x;  k = rint(t * 128 / ln2);  r' = t - k * ln2/128 (|r'| < 0.0028)
//   x^y = 2^(k >> 7) * 2^((k & 127) / 128) * (1 + expm1(r')), degree-5 series
// Series truncation is below 2^-60; table entries are correctly rounded
// binary64 values (gen_pow_tables.py).  The binary64 result is within about
// (|t| + 4) binary64 ulps of x^y, so its binary32 rounding is the correctly
// rounded binary32 x^y unless the result lies next to a binary32 rounding
// boundary.
//
// Two entry points: pow_f32_unit_exp (0 < y < 1, the kernel's hot path; see
// there why it needs no slow path) and pow_f32_via_f64 (any y: results next
// to a rounding boundary -- about 1e-7 of inputs, and every input whose x^y
// is exactly a boundary -- and inputs outside 1 <= x < 3e38 are re-evaluated
// with the platform's binary64 pow).  Usable from host code: the CPU test
// suite checks both against the C library's pow.
#ifndef ADANA_POW_H
#define ADANA_POW_H

#include <cmath>
#include <cstdint>
#include <cstring>

#if defined(__HIPCC__) || defined(__HIP__)
#define ADANA_HD __host__ __device__
#define ADANA_TABLE_ATTR __device__ __constant__
#else
#define ADANA_HD
#define ADANA_TABLE_ATTR static
#endif

#include "adana_pow_tables.h"

namespace adana {

template <typename To, typename From>
ADANA_HD inline To bits_as(From v) {
    static_assert(sizeof(To) == sizeof(From), "size");
    To o;
    std::memcpy(&o, &v, sizeof o);
    return o;
}

// fma(a, b, c) with c a wave-uniform constant: on the GPU, v_fma_f64 reading
// c from an SGPR pair.  (Left to itself the compiler copies each 64-bit
// polynomial coefficient into a VGPR pair for the accumulator form -- two VALU
// moves per Horner step.)  The same IEEE fused multiply-add either way.
#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ double fma_uc(double a, double b, double c) {
    double d;
    asm("v_fma_f64 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "s"(c));
    return d;
}
#else
inline double fma_uc(double a, double b, double c) { return std::fma(a, b, c); }
#endif

// binary64 x ** y for 1 <= x < 3e38 (finite).  Writes t = y * ln x.  The
// tables are passed in so that a kernel can read them from a copy in LDS (the
// per-lane gathers then stay off the vector-memory path that the streaming
// loads use); pow_core_f64 reads the global tables.
ADANA_HD inline double pow_core_tab(float x, float y, double &t_out, const LogPair *log_tab,
                                    const double *exp_tab) {
    const uint32_t xb = bits_as<uint32_t>(x);
    const int e = static_cast<int>(xb >> 23) - 127;
    const int j = static_cast<int>((xb >> 16) & 127u);
    const double m = static_cast<double>(bits_as<float>((xb & 0x007fffffu) | 0x3f800000u));
    const LogPair c = log_tab[j];
    const double r = std::fma(m, c.inv_c, -1.0);
    // log1p(r) = r + r^2 * (-1/2 + r/3 - r^2/4 + r^3/5 - r^4/6 + r^5/7)
    double q = 1.0 / 7.0;
    q = fma_uc(q, r, -1.0 / 6.0);
    q = fma_uc(q, r, 1.0 / 5.0);
    q = fma_uc(q, r, -1.0 / 4.0);
    q = fma_uc(q, r, 1.0 / 3.0);
    q = fma_uc(q, r, -0.5);
    const double lp = std::fma(r * r, q, r);
    // ln 2 split so that e * LN2_HI and k * LN2_HI / 128 are exact
    const double LN2_HI = 6.93147180369123816490e-01;
    const double LN2_LO = 1.90821492927058770002e-10;
    const double ed = static_cast<double>(e);
    const double lnx = std::fma(ed, LN2_HI, c.neg_log) + std::fma(ed, LN2_LO, lp);
    const double t = static_cast<double>(y) * lnx;
    // e^t = 2^(k/128) e^r'
    const double kd = std::rint(t * 184.66496523378731);        // 128 / ln 2
    double rr = std::fma(-kd, LN2_HI / 128.0, t);
    rr = std::fma(-kd, LN2_LO / 128.0, rr);
    double p = 1.0 / 120.0;
    p = fma_uc(p, rr, 1.0 / 24.0);
    p = fma_uc(p, rr, 1.0 / 6.0);
    p = fma_uc(p, rr, 0.5);
    p = std::fma(rr * rr, p, rr);                                // expm1(r')
    const int k = static_cast<int>(kd);
    const double tj = exp_tab[k & 127];
    t_out = t;
    return std::ldexp(std::fma(tj, p, tj), k >> 7);
}

ADANA_HD inline double pow_core_f64(float x, float y, double &t_out) {
    return pow_core_tab(x, y, t_out, kLog, kExp2J);
}

// True when fp32(res) may differ from the correctly rounded binary32 x ** y:
// binary32 rounding drops the low 29 of the 52 fraction bits, and res is
// within 8 * (|t| + 4) binary64 ulps of the half-way pattern (or outside
// binary32's normal range).
ADANA_HD inline bool near_boundary(double res, double t) {
    const uint32_t dropped = static_cast<uint32_t>(bits_as<uint64_t>(res)) & 0x1fffffffu;
    const int32_t dist = static_cast<int32_t>(dropped) - 0x10000000;
    const int32_t w = 32 + 8 * static_cast<int32_t>(std::fabs(t));
    return (dist <= w && dist >= -w) || !(res >= 1.1754943508222875e-38);
}

// The platform's binary64 pow, rounded once: the slow path.
ADANA_HD inline float pow_f32_slow(float x, float y) {
    return static_cast<float>(std::pow(static_cast<double>(x), static_cast<double>(y)));
}

// x ** y for an exponent 0 < y < 1 and x >= 1 (NaN and +inf pass through,
// as pow gives them for such y).  Branch-free: the core runs on every x (its
// table indices are 7-bit fields of x's bits, in range for any x) and the
// result is selected afterwards, so a thread's pows can overlap their table
// loads.  No slow path: for 0 < y < 1, x ** y is
// never exactly a binary32 half-way point (x^p = M^q would need a 25-bit odd
// M with M^q, q > p, fitting x's 24 bits), so fp32(core) differs from the
// correctly rounded result only when x ** y lies within the core's error
// (~2^-51 relative) of a half-way point -- measured 1 in 2e8 inputs against
// the C library's pow (tests/pow_harness.cpp).
ADANA_HD inline float pow_f32_unit_exp_tab(float x, float y, const LogPair *log_tab, const double *exp_tab) {
    double t;
    const float r = static_cast<float>(pow_core_tab(x, y, t, log_tab, exp_tab));
    return (x < 3.0e38f) ? r : x;
}

ADANA_HD inline float pow_f32_unit_exp(float x, float y) { return pow_f32_unit_exp_tab(x, y, kLog, kExp2J); }

// Any exponent: the core, and the slow path next to rounding boundaries and
// outside the core's domain.
ADANA_HD inline float pow_f32_via_f64(float x, float y) {
    if (x >= 1.0f && x < 3.0e38f) {
        double t;
        const double res = pow_core_f64(x, y, t);
        if (!near_boundary(res, t)) return static_cast<float>(res);
    }
    return pow_f32_slow(x, y);
}

}  // namespace adana

#endif  // ADANA_POW_H
