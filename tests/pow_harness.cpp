// Host harness for adana_amd/csrc/adana_pow.h: compares both entry points with
// the C library's binary64 pow rounded the same way, over x in [1, 2^24] for
// the exponents given on the command line.  Prints
//   <mismatches of pow_f32_via_f64> <mismatches of pow_f32_unit_exp> <total>
// (the second only counted for 0 < y < 1).
#include "../adana_amd/csrc/adana_pow.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

int main(int argc, char **argv) {
    const long per = argc > 1 ? atol(argv[1]) : 1000000;
    std::mt19937_64 rng(12345);
    long mism = 0, mism_unit = 0, total = 0;
    for (int a = 2; a < argc; ++a) {
        const float y = static_cast<float>(atof(argv[a]));
        const bool unit = y > 0.0f && y < 1.0f;
        for (long i = 0; i < per; ++i) {
            float x;
            if (i % 4 == 0) {
                x = 1.0f + static_cast<float>(i % 100003) * 0.173f;       // tau * step-like
            } else if (i % 4 == 1) {
                x = 1.0f + static_cast<float>(i % 16777216) * 0.015625f;  // multiples of 1/64
            } else {
                const double lx = std::uniform_real_distribution<double>(0.0, 16.6355)(rng);
                x = static_cast<float>(std::exp(lx));
                if (x < 1.0f) x = 1.0f;
            }
            const float ref = static_cast<float>(std::pow(static_cast<double>(x), static_cast<double>(y)));
            const float got = adana::pow_f32_via_f64(x, y);
            if (memcmp(&got, &ref, 4) != 0) {
                if (mism < 5) printf("mismatch x=%.9g y=%.9g got=%.9g ref=%.9g\n", x, y, got, ref);
                ++mism;
            }
            if (unit) {
                const float gu = adana::pow_f32_unit_exp(x, y);
                if (memcmp(&gu, &ref, 4) != 0) {
                    if (mism_unit < 5) printf("unit mismatch x=%.9g y=%.9g got=%.9g ref=%.9g\n", x, y, gu, ref);
                    ++mism_unit;
                }
            }
            ++total;
        }
    }
    const float nanv = adana::pow_f32_unit_exp(__builtin_nanf(""), 0.15f);
    const float infv = adana::pow_f32_unit_exp(__builtin_inff(), 0.15f);
    if (!(nanv != nanv) || infv != __builtin_inff()) { printf("special values wrong\n"); return 1; }
    printf("%ld %ld %ld\n", mism, mism_unit, total);
    return 0;
}
