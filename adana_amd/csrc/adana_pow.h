// adana_pow.h -- x ** y for Dana-Star's per-element effective-time factor,
// evaluated in binary64 and rounded once to binary32.
//
// Reference call site: ``(effective_time ** (1 - kappa))`` on the per-element
// tensor effective_time = clamp(tau * step, min=1) (src/optim/dana_star_mk4.py
// :159, :170/:174).  The exponent is the binary32 rounding of 1 - kappa.
//
// Method (standard argument reduction, all in binary64):
//   x = 2^k * m, m in [sqrt(1/2), sqrt(2))
//   ln m = 2u (1 + u^2/3 + u^4/5 + ... + u^22/23),  u = (m-1)/(m+1), |u| < 0.1716
//   ln x = k*ln2_hi + (k*ln2_lo + ln m)
//   t = y * ln x;  n = rint(t / ln2);  r = t - n*ln2 (two-step, |r| <= 0.347)
//   e^r = sum_{j<=13} r^j / j!;  x^y = 2^n * e^r
// Truncation errors are below 2^-56 relative for both series; the result
// before the final rounding is within a few binary64 ulps of x^y, so the
// binary32 result equals the correctly rounded one except when x^y lies
// within ~2^-50 (relative) of a binary32 rounding boundary.
//
// Domain of the fast path: 1 <= x < 3e38 (finite).  Anything else (NaN,
// +inf), and results next to a binary32 rounding boundary, go to the
// platform's binary64 pow.  Usable from host code (the CPU
// test suite checks it against the C library's pow).
#ifndef ADANA_POW_H
#define ADANA_POW_H

#include <cmath>

#if defined(__HIPCC__) || defined(__HIP__)
#define ADANA_HD __host__ __device__
#else
#define ADANA_HD
#endif

namespace adana {

ADANA_HD inline double pow_core_f64(double x, double y) {
    // x = m * 2^k with m in [0.5, 1)
    int k;
    double m = std::frexp(x, &k);
    if (m < 0.70710678118654752440) {   // move m to [sqrt(1/2), sqrt(2))
        m = m + m;
        k -= 1;
    }
    const double u = (m - 1.0) / (m + 1.0);
    const double w = u * u;
    // Q(w) = 1/3 + w/5 + ... + w^10/23
    double q = 1.0 / 23.0;
    q = std::fma(q, w, 1.0 / 21.0);
    q = std::fma(q, w, 1.0 / 19.0);
    q = std::fma(q, w, 1.0 / 17.0);
    q = std::fma(q, w, 1.0 / 15.0);
    q = std::fma(q, w, 1.0 / 13.0);
    q = std::fma(q, w, 1.0 / 11.0);
    q = std::fma(q, w, 1.0 / 9.0);
    q = std::fma(q, w, 1.0 / 7.0);
    q = std::fma(q, w, 1.0 / 5.0);
    q = std::fma(q, w, 1.0 / 3.0);
    const double s = u + u;
    const double lnm = std::fma(s * w, q, s);
    // ln 2 split so that k * LN2_HI is exact for |k| < 2^11
    const double LN2_HI = 6.93147180369123816490e-01;
    const double LN2_LO = 1.90821492927058770002e-10;
    const double kd = static_cast<double>(k);
    const double lnx = kd * LN2_HI + (kd * LN2_LO + lnm);
    const double t = y * lnx;
    // e^t = 2^n e^r
    const double n = std::rint(t * 1.44269504088896338700);
    double r = std::fma(-n, LN2_HI, t);
    r = std::fma(-n, LN2_LO, r);
    double e = 1.0 / 6227020800.0;               // 1/13!
    e = std::fma(e, r, 1.0 / 479001600.0);       // 1/12!
    e = std::fma(e, r, 1.0 / 39916800.0);
    e = std::fma(e, r, 1.0 / 3628800.0);
    e = std::fma(e, r, 1.0 / 362880.0);
    e = std::fma(e, r, 1.0 / 40320.0);
    e = std::fma(e, r, 1.0 / 5040.0);
    e = std::fma(e, r, 1.0 / 720.0);
    e = std::fma(e, r, 1.0 / 120.0);
    e = std::fma(e, r, 1.0 / 24.0);
    e = std::fma(e, r, 1.0 / 6.0);
    e = std::fma(e, r, 0.5);
    e = std::fma(e, r, 1.0);
    e = std::fma(e, r, 1.0);
    return std::ldexp(e, static_cast<int>(n));
}

// binary32 x ** y as fp32(x ** y evaluated in binary64).  When the core's
// result lies within 2^-46 (relative) of a binary32 rounding boundary -- about
// 2e-7 of inputs, and every case where x ** y is exactly a boundary -- the
// rounding is decided by the platform's binary64 pow instead.
ADANA_HD inline float pow_f32_via_f64(float x, float y) {
    if (x >= 1.0f && x < 3.0e38f) {
        const double d = pow_core_f64(static_cast<double>(x), static_cast<double>(y));
        const float f = static_cast<float>(d);
        const double fd = static_cast<double>(f);
        const double err = std::fabs(d - fd);
        // half the binary32 spacing above fd, and below it (a power of two has
        // a spacing below that is half the spacing above)
        const double half_up = std::ldexp(1.0, std::ilogb(fd) - 24);
        const double tol = d * 1.4210854715202004e-14;    // 2^-46
        if (std::fabs(err - half_up) > tol && std::fabs(err - 0.5 * half_up) > tol) return f;
    }
    return static_cast<float>(std::pow(static_cast<double>(x), static_cast<double>(y)));
}

}  // namespace adana

#endif  // ADANA_POW_H
