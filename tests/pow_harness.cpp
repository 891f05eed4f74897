// Host harness for adana_amd/csrc/adana_pow.h: compares the binary64-core pow
// (rounded once to binary32) with the C library's binary64 pow rounded the
// same way, over x in [1, 2^24] and the exponents given on the command line.
#include "../adana_amd/csrc/adana_pow.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>

int main(int argc, char **argv) {
    const long per = argc > 1 ? atol(argv[1]) : 1000000;
    std::mt19937_64 rng(12345);
    long mism = 0, total = 0;
    for (int a = 2; a < argc; ++a) {
        const float y = static_cast<float>(atof(argv[a]));
        for (long i = 0; i < per; ++i) {
            float x;
            if (i % 4 == 0) {
                x = 1.0f + static_cast<float>(i % 100003) * 0.173f;       // tau * step-like
            } else {
                const double lx = std::uniform_real_distribution<double>(0.0, 16.6355)(rng);
                x = static_cast<float>(std::exp(lx));
                if (x < 1.0f) x = 1.0f;
            }
            const float got = adana::pow_f32_via_f64(x, y);
            const float ref = static_cast<float>(std::pow(static_cast<double>(x), static_cast<double>(y)));
            if (memcmp(&got, &ref, 4) != 0) {
                if (mism < 5) printf("mismatch x=%.9g y=%.9g got=%.9g ref=%.9g\n", x, y, got, ref);
                ++mism;
            }
            ++total;
        }
    }
    printf("%ld %ld\n", mism, total);
    return 0;
}
