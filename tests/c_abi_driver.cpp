// c_abi_driver.cpp -- the optimizer step's C ABI driven from plain C++, as a
// non-Python host (a Go, Java or C++ training loop binding
// include/adana_mta.h) would drive it: its own HIP allocations, the layout,
// the chunk index, the workspace, then adana_mta_step per step, checked
// against the CPU oracle (oracle/adana_oracle.c) after every step.
//
// Test infrastructure: built by tests/Makefile, run by
// tests/test_gpu_c_abi.py.  Exit status 0 and a last line "c_abi_driver: ok"
// when every step matches; 1 with the first mismatch otherwise; 2 on a HIP or
// library error.
//
// Bars (as the Python parity tests): m, v, tau bit-exact; p bit-exact except
// at most 2 elements per tensor per step whose pow lies on a rounding
// boundary, each within 2 ulps of max(|p_before|, |p_after|); diagnostics
// within 1e-5 relative of the oracle's binary64 sums.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "adana_mta.h"
#include "adana_oracle.h"

namespace {

#define HIP_OK(x)                                                                      \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            std::printf("HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
            std::exit(2);                                                              \
        }                                                                              \
    } while (0)

#define LIB_OK(x)                                                                      \
    do {                                                                               \
        int r_ = (x);                                                                  \
        if (r_ != ADANA_OK) {                                                          \
            char msg_[512];                                                            \
            adana_last_error(msg_, sizeof msg_);                                       \
            std::printf("library error %d: %s (%s:%d)\n", r_, msg_, __FILE__, __LINE__); \
            std::exit(2);                                                              \
        }                                                                              \
    } while (0)

// Seeded standard normals (xorshift64* and Box-Muller), scaled by sd.
struct Rng {
    uint64_t s;
    double u() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return ((s * 0x2545F4914F6CDD1DULL) >> 11) * (1.0 / 9007199254740992.0);
    }
    float normal(double sd) {
        const double a = u() + 1e-300, b = u();
        return static_cast<float>(sd * std::sqrt(-2.0 * std::log(a)) * std::cos(6.283185307179586 * b));
    }
};

uint32_t bits(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    return b;
}

// The oracle's element math takes the same binary32 scalars the library
// computed for the kernel (the scalars themselves are pinned separately,
// bit for bit, by tests/test_host_cpu.py).
adana_oracle_scalars to_oracle(const adana_step_scalars &s) {
    adana_oracle_scalars o{};
    o.a = s.a;
    o.oma = s.oma;
    o.s = s.s;
    o.eps = s.eps;
    o.pw = s.pw;
    o.min_p = s.min_p;
    o.clip = s.clip;
    o.has_clip = s.has_clip;
    o.c3 = s.c3;
    o.cg2 = s.cg2;
    o.opw = s.opw;
    o.star_exp = s.star_exp;
    o.pow_mode = s.pow_mode;
    o.pow_int = s.pow_int;
    o.compiled = 1;          // the library's default numerics (no ADANA_NUMERICS_EAGER)
    return o;
}

}  // namespace

int main() {
    const std::vector<int64_t> numel = {1000, 37 * 19, 5, 4096 + 3, 70000};
    const int n = static_cast<int>(numel.size());
    const int kSteps = 6;
    HIP_OK(hipSetDevice(0));
    std::printf("c_abi_driver: ABI %d, %d tensors, %d Dana-Star-MK4 steps\n", adana_abi_version(), n, kSteps);
    std::fflush(stdout);

    // host state (the oracle's) and device state (the library's)
    Rng rng{0x1234567ULL};
    std::vector<std::vector<float>> p(n), g(n), m(n), v(n), tau(n);
    std::vector<float *> dp(n), dg(n), dm(n), dv(n), dtau(n);
    for (int i = 0; i < n; ++i) {
        const size_t k = static_cast<size_t>(numel[i]);
        p[i].resize(k);
        for (auto &x : p[i]) x = rng.normal(0.02);
        g[i].assign(k, 0.0f);
        m[i].assign(k, 0.0f);
        v[i].assign(k, 0.0f);
        tau[i].assign(k, 0.0f);
        HIP_OK(hipMalloc(&dp[i], 4 * k));
        HIP_OK(hipMalloc(&dg[i], 4 * k));
        HIP_OK(hipMalloc(&dm[i], 4 * k));
        HIP_OK(hipMalloc(&dv[i], 4 * k));
        HIP_OK(hipMalloc(&dtau[i], 4 * k));
        HIP_OK(hipMemcpy(dp[i], p[i].data(), 4 * k, hipMemcpyHostToDevice));
        HIP_OK(hipMemset(dm[i], 0, 4 * k));
        HIP_OK(hipMemset(dv[i], 0, 4 * k));
        HIP_OK(hipMemset(dtau[i], 0, 4 * k));
    }

    // layout, descriptors, chunk index, workspace
    std::vector<int64_t> vstart(n + 1);
    std::vector<int32_t> fold_first(n + 1);
    int64_t n_folds = 0;
    const int64_t n_chunks = adana_plan_layout(numel.data(), n, vstart.data(), fold_first.data(), &n_folds);
    if (n_chunks < 0) LIB_OK(static_cast<int>(n_chunks));
    std::vector<adana_tensor_desc> desc(n);
    for (int i = 0; i < n; ++i)
        desc[i] = adana_tensor_desc{dp[i], nullptr, dm[i], dv[i], dtau[i], nullptr, numel[i], 0, ADANA_DESC_VEC_OK};
    std::vector<const void *> gptr(dg.begin(), dg.end());
    adana_tensor_desc *d_desc;
    const void **d_grad;
    int64_t *d_vstart;
    int32_t *d_fold_first, *d_chunk_first;
    HIP_OK(hipMalloc(&d_desc, sizeof(adana_tensor_desc) * n));
    HIP_OK(hipMalloc(&d_grad, sizeof(void *) * n));
    HIP_OK(hipMemcpy(d_grad, gptr.data(), sizeof(void *) * n, hipMemcpyHostToDevice));
    HIP_OK(hipMalloc(&d_vstart, 8 * (n + 1)));
    HIP_OK(hipMalloc(&d_fold_first, 4 * (n + 1)));
    HIP_OK(hipMalloc(&d_chunk_first, 4 * n_chunks));
    HIP_OK(hipMemcpy(d_desc, desc.data(), sizeof(adana_tensor_desc) * n, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_vstart, vstart.data(), 8 * (n + 1), hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(d_fold_first, fold_first.data(), 4 * (n + 1), hipMemcpyHostToDevice));
    hipStream_t stream;
    HIP_OK(hipStreamCreate(&stream));
    LIB_OK(adana_plan_index(d_vstart, n, n_chunks, d_chunk_first, stream));
    adana_plan plan{};
    plan.desc = d_desc;
    plan.grad = d_grad;
    plan.vstart = d_vstart;
    plan.chunk_first = d_chunk_first;
    plan.fold_first = d_fold_first;
    plan.n_tensors = n;
    plan.n_chunks = n_chunks;
    plan.n_folds = n_folds;
    const size_t ws_bytes = adana_workspace_bytes(&plan);
    void *d_ws;
    float *d_diag;
    HIP_OK(hipMalloc(&d_ws, ws_bytes));
    HIP_OK(hipMalloc(&d_diag, 4 * 5 * n));

    // the launcher's hyper-parameters (scripts/launch.sh: kappa 0.85, delta 8,
    // clipsnr 2, weight decay omega / wd_ts with wd_decaying)
    adana_hparams hp{};
    hp.peak_lr = 1e-3;
    hp.delta = 8.0;
    hp.kappa = 0.85;
    hp.epsilon = 1e-8;
    hp.weight_decay = 0.4;
    hp.clipsnr = 2.0;
    hp.wd_ts = 10.0;
    hp.gamma_3_factor = 1.0;
    hp.has_clip = 1;
    hp.wd_decaying = 1;

    std::vector<float> got(70000 + 8);
    std::vector<float> gdiag(5 * n);
    for (int t = 1; t <= kSteps; ++t) {
        for (int i = 0; i < n; ++i) {
            for (auto &x : g[i]) x = rng.normal(1e-3);
            HIP_OK(hipMemcpyAsync(dg[i], g[i].data(), 4 * numel[i], hipMemcpyHostToDevice, stream));
        }
        adana_step_scalars sc;
        LIB_OK(adana_step_scalars_init(&sc, &hp, hp.peak_lr, t));
        LIB_OK(adana_mta_step(&plan, &sc, 1, ADANA_VARIANT_STAR, d_ws, ws_bytes, d_diag, stream));
        HIP_OK(hipMemcpyAsync(gdiag.data(), d_diag, 4 * 5 * n, hipMemcpyDeviceToHost, stream));
        HIP_OK(hipStreamSynchronize(stream));
        const adana_oracle_scalars osc = to_oracle(sc);
        for (int i = 0; i < n; ++i) {
            const size_t k = static_cast<size_t>(numel[i]);
            const std::vector<float> before = p[i];
            double dsum[4];
            adana_oracle_star_step(numel[i], p[i].data(), g[i].data(), m[i].data(), v[i].data(), tau[i].data(),
                                   &osc, dsum);
            const std::vector<float> *want[3] = {&m[i], &v[i], &tau[i]};
            float *const have[3] = {dm[i], dv[i], dtau[i]};
            const char *name[3] = {"m", "v", "tau"};
            for (int s = 0; s < 3; ++s) {
                HIP_OK(hipMemcpy(got.data(), have[s], 4 * k, hipMemcpyDeviceToHost));
                for (size_t e = 0; e < k; ++e)
                    if (bits(got[e]) != bits((*want[s])[e])) {
                        std::printf("step %d tensor %d: %s[%zu] = %.9g, oracle %.9g\n", t, i, name[s], e, got[e],
                                    (*want[s])[e]);
                        return 1;
                    }
            }
            HIP_OK(hipMemcpy(got.data(), dp[i], 4 * k, hipMemcpyDeviceToHost));
            int hard = 0;
            for (size_t e = 0; e < k; ++e) {
                if (bits(got[e]) == bits(p[i][e])) continue;
                const double scale = std::fmax(std::fabs(before[e]), std::fabs(p[i][e]));
                const double ulp = std::nextafter(static_cast<float>(scale), INFINITY) - static_cast<float>(scale);
                if (++hard > 2 || std::fabs(static_cast<double>(got[e]) - p[i][e]) > 2 * ulp) {
                    std::printf("step %d tensor %d: p[%zu] = %.9g, oracle %.9g\n", t, i, e, got[e], p[i][e]);
                    return 1;
                }
            }
            p[i].assign(got.begin(), got.begin() + k);                // continue from the GPU's p
            const double nd = static_cast<double>(k);
            const double ref[5] = {dsum[0] / nd, std::sqrt(dsum[1]), dsum[2] / nd, (dsum[0] / nd) / (dsum[2] / nd),
                                   std::sqrt(dsum[3])};
            for (int c = 0; c < 5; ++c)
                if (std::fabs(gdiag[5 * i + c] - ref[c]) > 1e-5 * std::fabs(ref[c]) + 1e-30) {
                    std::printf("step %d tensor %d: diagnostic %d = %.9g, oracle %.9g\n", t, i, c, gdiag[5 * i + c],
                                ref[c]);
                    return 1;
                }
        }
        std::printf("step %d: every tensor matches\n", t);
        std::fflush(stdout);
    }
    for (int i = 0; i < n; ++i) {
        HIP_OK(hipFree(dp[i]));
        HIP_OK(hipFree(dg[i]));
        HIP_OK(hipFree(dm[i]));
        HIP_OK(hipFree(dv[i]));
        HIP_OK(hipFree(dtau[i]));
    }
    HIP_OK(hipFree(d_desc));
    HIP_OK(hipFree(d_grad));
    HIP_OK(hipFree(d_vstart));
    HIP_OK(hipFree(d_fold_first));
    HIP_OK(hipFree(d_chunk_first));
    HIP_OK(hipFree(d_ws));
    HIP_OK(hipFree(d_diag));
    HIP_OK(hipStreamDestroy(stream));
    std::printf("c_abi_driver: ok\n");
    return 0;
}
