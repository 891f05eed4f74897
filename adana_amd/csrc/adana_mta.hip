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
//     (chunk, tensor) segment with wave shuffles and an LDS combine, written to
//     partials[chunk + tensor], and combined per tensor in binary64 by a
//     one-workgroup-per-tensor finalize kernel (deterministic, no atomics).
//
// Element arithmetic follows the reference's op order with every op one
// correctly rounded binary32 operation (built with -ffp-contract=off); the
// only fused multiply-adds are the ones ATen's lerp_ and addcmul_ perform.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "adana_mta.h"
#include "adana_pow.h"

namespace {

thread_local char g_err[512] = "";

int set_err(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / 64;
constexpr int kChunk = ADANA_CHUNK_ELEMS;
static_assert(kChunk == 4 * kBlock, "one 4-element vector per thread per chunk");
static_assert(ADANA_ALIGN_ELEMS == 4, "tensors start on vector boundaries");
static_assert(sizeof(adana_tensor_desc) == 64, "descriptor layout");
static_assert(sizeof(adana_step_scalars) == 64, "scalar layout");

struct ScalarPack {
    adana_step_scalars c[ADANA_MAX_CLASSES];
};

// ---------------------------------------------------------------------------
// Element math
// ---------------------------------------------------------------------------

__device__ __forceinline__ float sign_f(float x) {  // torch.sign: 0 for +-0, NaN
    return x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
}
__device__ __forceinline__ float clamp_max(float x, float c) { return x > c ? c : x; }
__device__ __forceinline__ float clamp_min(float x, float c) { return x < c ? c : x; }
__device__ __forceinline__ float relu_f(float x) { return x < 0.0f ? 0.0f : x; }

__device__ __forceinline__ float bf16_to_f32(unsigned short h) {
    return __uint_as_float(static_cast<unsigned int>(h) << 16);
}
// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ unsigned short f32_to_bf16(float f) {
    unsigned int u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<unsigned short>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<unsigned short>(u >> 16);
}

// x ** e with ATen's exponent specialisations (pow(Tensor, Scalar)); the
// general case is evaluated in binary64 and rounded once (adana_pow.h).
__device__ __forceinline__ float pow_aten(float x, const adana_step_scalars &sc) {
    if (sc.pow_mode == ADANA_POW_GENERAL) return adana::pow_f32_via_f64(x, sc.star_exp);
    switch (sc.pow_mode) {
    case ADANA_POW_ONE: return 1.0f;
    case ADANA_POW_SQRT: return sqrtf(x);
    case ADANA_POW_RSQRT: return 1.0f / sqrtf(x);
    case ADANA_POW_RECIP: return 1.0f / x;
    case ADANA_POW_SQUARE: return x * x;
    case ADANA_POW_CUBE: return (x * x) * x;
    case ADANA_POW_INVSQ: return 1.0f / (x * x);
    default: return adana::pow_f32_via_f64(x, sc.star_exp);
    }
}

// One element.  ADana / Dana-MK4: src/optim/adana.py:101-143.
// Dana-Star / Dana-Star-MK4: src/optim/dana_star_mk4.py:137-195.
template <bool STAR>
__device__ __forceinline__ float update_elem(float p, float g, float &m, float &v, float &tau,
                                             const adana_step_scalars &sc, float (&acc)[4]) {
    // m.lerp_(grad, alpha): ATen computes fma(w, end - self, self) for |w| < 0.5
    // and fma(w - 1, end - self, end) otherwise.
    const float mn_ = __builtin_fmaf(sc.lerp_coef, g - m, sc.lerp_small ? m : g);
    // v.mul_(1 - alpha).addcmul_(grad, grad, value=alpha) = fma(alpha*g, g, v*(1-alpha))
    const float vn = __builtin_fmaf(sc.a * g, g, v * sc.oma);
    const float se = sqrtf(vn) + sc.eps;
    float nt, mfac, af, inner;
    if constexpr (!STAR) {
        nt = 1.0f / se;                                   // adana.py:110
        mfac = fabsf(mn_) * nt;                           // :111, :115
        af = sc.pw * mfac;                                // :119 / :123
        if (sc.has_clip) af = clamp_max(af, sc.clip);
        inner = sign_f(mn_) * af + mn_ * nt;              // :126
    } else {
        const float ag = fabsf(g);                        // dana_star_mk4.py:147
        const float tu = ag / (ag + se);                  // :148
        const float tn = __builtin_fmaf(sc.lerp_coef, tu - tau, sc.lerp_small ? tau : tu);
        const float ct = clamp_max(tn, 0.5f);             // :152
        const float pe = ct / (1.0f - ct);                // :153
        const float tr = sc.min_p + relu_f(pe - sc.min_p);  // :154-156
        const float et = clamp_min(tn * sc.s, 1.0f);      // :159
        nt = sqrtf(tr) / se;                              // :163-164
        const float mnt = fabsf(mn_) * nt;                // :165
        mfac = mnt / tr;                                  // :167
        af = pow_aten(et, sc) * mfac;                     // :170 / :174
        if (sc.has_clip) af = clamp_max(af, sc.clip);
        inner = sign_f(mn_) * (tr * af + mnt);            // :177
        tau = tn;
    }
    const float g3t = sc.c3 * inner;                      // (-g3) * gamma_3_factor * (...)
    const float g2t = (sc.cg2 * g) * nt;                  // (-g2) * grad * norm_term
    float pn = p + (g2t + g3t);                           // p.add_(update)
    pn = pn * sc.opw;                                     // p.mul_(1 + wd_factor)
    m = mn_;
    v = vn;
    acc[0] += af;
    acc[1] += g * g;
    acc[2] += mfac;
    acc[3] += mn_ * mn_;
    return pn;
}

// ---------------------------------------------------------------------------
// Memory access: global (not flat) 16-byte vectors, non-temporal for the
// streamed arrays (each byte is touched once per step).
// ---------------------------------------------------------------------------

#define GLOBAL_AS __attribute__((address_space(1)))
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ v4f ld4(const float *p) {
    return __builtin_nontemporal_load((const GLOBAL_AS v4f *)(p));
}
__device__ __forceinline__ void st4(float *p, v4f x) {
    __builtin_nontemporal_store(x, (GLOBAL_AS v4f *)(p));
}
__device__ __forceinline__ v2u ld2u(const void *p) {
    return __builtin_nontemporal_load((const GLOBAL_AS v2u *)(p));
}
__device__ __forceinline__ void st2u(void *p, v2u x) {
    __builtin_nontemporal_store(x, (GLOBAL_AS v2u *)(p));
}

template <bool GBF16>
__device__ __forceinline__ v4f load_grad4(const void *g, int64_t off) {
    if constexpr (GBF16) {
        const v2u r = ld2u(static_cast<const unsigned short *>(g) + off);
        v4f o;
        o.x = __uint_as_float(r.x << 16);
        o.y = __uint_as_float(r.x & 0xffff0000u);
        o.z = __uint_as_float(r.y << 16);
        o.w = __uint_as_float(r.y & 0xffff0000u);
        return o;
    } else {
        return ld4(static_cast<const float *>(g) + off);
    }
}
template <bool GBF16>
__device__ __forceinline__ float load_grad1(const void *g, int64_t off) {
    if constexpr (GBF16) return bf16_to_f32(static_cast<const unsigned short *>(g)[off]);
    else return static_cast<const float *>(g)[off];
}

// ---------------------------------------------------------------------------
// Main multi-tensor kernel: one 1024-element chunk per 256-thread workgroup,
// one 16-byte vector per thread per array, a single load -> update -> store
// pass (waves exit right after their stores; looping waves would wait on
// their own stores, which the gfx9 vmcnt counter orders with later loads).
// ---------------------------------------------------------------------------

template <bool STAR, bool GBF16, bool PBF16>
__global__ __launch_bounds__(kBlock) void mta_step_kernel(const adana_tensor_desc *__restrict__ desc,
                                                          const int64_t *__restrict__ vstart,
                                                          const int32_t *__restrict__ chunk_first,
                                                          int32_t n, ScalarPack pack,
                                                          float *__restrict__ partials) {
    __shared__ float red[kWaves][4];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t chunk = blockIdx.x;
    const int64_t lo = chunk * kChunk;
    const int64_t hi = lo + kChunk;
    const int64_t mine = lo + 4 * tid;   // virtual index of this thread's 4 elements

    for (int i = chunk_first[chunk]; i < n; ++i) {
        const int64_t vs = vstart[i];
        if (vs >= hi) break;
        const adana_tensor_desc d = desc[i];
        const int64_t ve = vs + d.numel;
        if (ve <= lo) continue;                                    // uniform across the block
        const adana_step_scalars &sc = pack.c[d.sclass];
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (mine >= vs && mine < ve) {
            const int64_t off = mine - vs;                         // multiple of 4
            float *pp = static_cast<float *>(d.param) + off;
            float *mp = d.m + off;
            float *vp = d.v + off;
            float *tp = STAR ? d.tau + off : nullptr;
            const int cnt = (ve - mine) < 4 ? static_cast<int>(ve - mine) : 4;
            if (cnt == 4 && (d.flags & ADANA_DESC_VEC_OK)) {
                const v4f P = ld4(pp);
                const v4f G = load_grad4<GBF16>(d.grad, off);
                v4f M = ld4(mp);
                v4f V = ld4(vp);
                v4f T = {0.0f, 0.0f, 0.0f, 0.0f};
                if constexpr (STAR) T = ld4(tp);
                v4f O;
                float t0 = T.x, t1 = T.y, t2 = T.z, t3 = T.w;
                float m0 = M.x, m1 = M.y, m2 = M.z, m3 = M.w;
                float v0 = V.x, v1 = V.y, v2 = V.z, v3 = V.w;
                O.x = update_elem<STAR>(P.x, G.x, m0, v0, t0, sc, acc);
                O.y = update_elem<STAR>(P.y, G.y, m1, v1, t1, sc, acc);
                O.z = update_elem<STAR>(P.z, G.z, m2, v2, t2, sc, acc);
                O.w = update_elem<STAR>(P.w, G.w, m3, v3, t3, sc, acc);
                M.x = m0; M.y = m1; M.z = m2; M.w = m3;
                V.x = v0; V.y = v1; V.z = v2; V.w = v3;
                st4(pp, O);
                st4(mp, M);
                st4(vp, V);
                if constexpr (STAR) {
                    T.x = t0; T.y = t1; T.z = t2; T.w = t3;
                    st4(tp, T);
                }
                if constexpr (PBF16) {
                    v2u b;
                    b.x = static_cast<unsigned int>(f32_to_bf16(O.x)) |
                          (static_cast<unsigned int>(f32_to_bf16(O.y)) << 16);
                    b.y = static_cast<unsigned int>(f32_to_bf16(O.z)) |
                          (static_cast<unsigned int>(f32_to_bf16(O.w)) << 16);
                    st2u(static_cast<unsigned short *>(d.param_lp) + off, b);
                }
            } else {
                // unaligned tensor, or the last (<4) elements of a tensor
                for (int e = 0; e < cnt; ++e) {
                    float mm = mp[e], vv = vp[e], tt = STAR ? tp[e] : 0.0f;
                    const float o = update_elem<STAR>(pp[e], load_grad1<GBF16>(d.grad, off + e), mm, vv,
                                                      tt, sc, acc);
                    pp[e] = o;
                    mp[e] = mm;
                    vp[e] = vv;
                    if constexpr (STAR) tp[e] = tt;
                    if constexpr (PBF16) static_cast<unsigned short *>(d.param_lp)[off + e] = f32_to_bf16(o);
                }
            }
        }
        // (chunk, tensor) segment sums: wave butterfly, fixed-order wave combine.
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float x = acc[k];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
            if (lane == 0) red[wave][k] = x;
        }
        __syncthreads();
        if (tid == 0) {
            float4 q;
            q.x = ((red[0][0] + red[1][0]) + red[2][0]) + red[3][0];
            q.y = ((red[0][1] + red[1][1]) + red[2][1]) + red[3][1];
            q.z = ((red[0][2] + red[1][2]) + red[2][2]) + red[3][2];
            q.w = ((red[0][3] + red[1][3]) + red[2][3]) + red[3][3];
            reinterpret_cast<float4 *>(partials)[chunk + i] = q;
        }
        __syncthreads();
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

// One workgroup per tensor: binary64 sum of the tensor's (chunk, tensor)
// partials in a fixed order, then the five diagnostics
// (src/optim/adana.py:146-151, :221-225).
__global__ __launch_bounds__(kBlock) void finalize_kernel(const adana_tensor_desc *__restrict__ desc,
                                                          const int64_t *__restrict__ vstart,
                                                          int32_t n, const float *__restrict__ partials,
                                                          float *__restrict__ diag) {
    __shared__ double red[kWaves][4];
    const int i = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t numel = desc[i].numel;
    const int64_t vs = vstart[i];
    double s0 = 0.0, s1 = 0.0, s2 = 0.0, s3 = 0.0;
    if (numel > 0) {
        const int64_t b0 = vs / kChunk, b1 = (vs + numel - 1) / kChunk;
        const float4 *p4 = reinterpret_cast<const float4 *>(partials);
        for (int64_t b = b0 + tid; b <= b1; b += kBlock) {
            const float4 q = p4[b + i];
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
    if (lane == 0) { red[wave][0] = s0; red[wave][1] = s1; red[wave][2] = s2; red[wave][3] = s3; }
    __syncthreads();
    if (tid == 0) {
        s0 = ((red[0][0] + red[1][0]) + red[2][0]) + red[3][0];
        s1 = ((red[0][1] + red[1][1]) + red[2][1]) + red[3][1];
        s2 = ((red[0][2] + red[1][2]) + red[2][2]) + red[3][2];
        s3 = ((red[0][3] + red[1][3]) + red[2][3]) + red[3][3];
        const double nd = static_cast<double>(numel);
        const float ca = static_cast<float>(s0 / nd);     // alpha_factor.mean()
        const float afm = static_cast<float>(s2 / nd);    // mfac.mean()
        float *o = diag + 5 * static_cast<int64_t>(i);
        o[0] = ca;
        o[1] = static_cast<float>(sqrt(s1));              // grad.norm()
        o[2] = afm;
        o[3] = ca / afm;                                  // current_alpha / auto_factor_mean
        o[4] = static_cast<float>(sqrt(s3));              // m.norm()
    }
}

template <bool STAR, bool GBF16, bool PBF16>
void launch_main(int64_t n_chunks, hipStream_t st, const adana_tensor_desc *d, const int64_t *vs,
                 const int32_t *cf, int32_t n, const ScalarPack &pack, float *partials) {
    hipLaunchKernelGGL((mta_step_kernel<STAR, GBF16, PBF16>), dim3(static_cast<unsigned>(n_chunks)),
                       dim3(kBlock), 0, st, d, vs, cf, n, pack, partials);
}

// ---------------------------------------------------------------------------
// Host scalar code
// ---------------------------------------------------------------------------

int pow_mode_of(double e) {
    if (e == 0.0) return ADANA_POW_ONE;
    if (e == 0.5) return ADANA_POW_SQRT;
    if (e == -0.5) return ADANA_POW_RSQRT;
    if (e == -1.0) return ADANA_POW_RECIP;
    if (e == 2.0) return ADANA_POW_SQUARE;
    if (e == 3.0) return ADANA_POW_CUBE;
    if (e == -2.0) return ADANA_POW_INVSQ;
    return ADANA_POW_GENERAL;
}

// ATen pow(Tensor, Scalar) on a 0-d float tensor: specialisations as above,
// otherwise std::pow(float, double) evaluated in binary64.
float pow0d(float x, double e) {
    switch (pow_mode_of(e)) {
    case ADANA_POW_ONE: return 1.0f;
    case ADANA_POW_SQRT: return std::sqrt(x);
    case ADANA_POW_RSQRT: return 1.0f / std::sqrt(x);
    case ADANA_POW_RECIP: return 1.0f / x;
    case ADANA_POW_SQUARE: return x * x;
    case ADANA_POW_CUBE: return (x * x) * x;
    case ADANA_POW_INVSQ: return 1.0f / (x * x);
    default: return static_cast<float>(std::pow(static_cast<double>(x), e));
    }
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
    if (!out || !hp) return set_err(ADANA_E_INVALID, "adana_step_scalars_init: null pointer");
    if (step < 1) return set_err(ADANA_E_INVALID, "adana_step_scalars_init: step %lld < 1",
                                 static_cast<long long>(step));
    if (!(hp->peak_lr != 0.0))
        return set_err(ADANA_E_INVALID, "adana_step_scalars_init: peak lr must be nonzero");
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
    out->pw = pow0d(one_p_s, 1.0 - hp->kappa);
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
    out->pow_mode = pow_mode_of(1.0 - hp->kappa);
    return ADANA_OK;
}

int64_t adana_plan_layout(const int64_t *numel, int32_t n, int64_t *vstart) {
    if (n < 0 || (n > 0 && (!numel || !vstart)))
        return set_err(ADANA_E_INVALID, "adana_plan_layout: bad arguments");
    int64_t off = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (numel[i] < 0) return set_err(ADANA_E_INVALID, "adana_plan_layout: numel[%d] < 0", i);
        vstart[i] = off;
        off += (numel[i] + ADANA_ALIGN_ELEMS - 1) / ADANA_ALIGN_ELEMS * ADANA_ALIGN_ELEMS;
    }
    if (vstart) vstart[n] = off;
    const int64_t chunks = (off + kChunk - 1) / kChunk;
    if (chunks > 0x7fffffffLL) return set_err(ADANA_E_UNSUPPORTED, "adana_plan_layout: list too large");
    return chunks;
}

int adana_plan_index(const int64_t *d_vstart, int32_t n_tensors, int64_t n_chunks,
                     int32_t *d_chunk_first, void *stream) {
    if (n_tensors < 0 || n_chunks < 0 || n_chunks > 0x7fffffffLL)
        return set_err(ADANA_E_INVALID, "adana_plan_index: bad sizes");
    if (n_chunks == 0) return ADANA_OK;
    if (n_tensors == 0 || !d_vstart || !d_chunk_first)
        return set_err(ADANA_E_INVALID, "adana_plan_index: null pointer or no tensors");
    const unsigned blocks = static_cast<unsigned>((n_chunks + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(chunk_index_kernel, dim3(blocks), dim3(kBlock), 0,
                       static_cast<hipStream_t>(stream), d_vstart, n_tensors, n_chunks, d_chunk_first);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return set_err(ADANA_E_HIP, "adana_plan_index: launch failed: %s", hipGetErrorString(err));
    return ADANA_OK;
}

int64_t adana_partials_floats(int32_t n_tensors, int64_t n_chunks) {
    return 4 * (static_cast<int64_t>(n_tensors) + n_chunks);
}

int adana_mta_step(const adana_tensor_desc *d_desc, const int64_t *d_vstart,
                   const int32_t *d_chunk_first, int32_t n_tensors, int64_t n_chunks,
                   const adana_step_scalars *h_scalars, int32_t n_classes, uint32_t variant_flags,
                   float *d_partials, float *d_diag, void *stream) {
    if (n_tensors < 0 || n_chunks < 0 || n_chunks > 0x7fffffffLL)
        return set_err(ADANA_E_INVALID, "adana_mta_step: bad sizes (n_tensors=%d, n_chunks=%lld)",
                       n_tensors, static_cast<long long>(n_chunks));
    if (variant_flags & ~(ADANA_VARIANT_STAR | ADANA_GRAD_BF16 | ADANA_PARAM_BF16))
        return set_err(ADANA_E_INVALID, "adana_mta_step: unknown variant flags 0x%x", variant_flags);
    if (n_tensors == 0) return ADANA_OK;
    if (!d_desc || !d_vstart || !d_partials || !d_diag || !h_scalars ||
        (n_chunks > 0 && !d_chunk_first))
        return set_err(ADANA_E_INVALID, "adana_mta_step: null pointer argument");
    if (n_classes < 1 || n_classes > ADANA_MAX_CLASSES)
        return set_err(ADANA_E_INVALID, "adana_mta_step: n_classes=%d outside [1, %d]", n_classes,
                       ADANA_MAX_CLASSES);
    ScalarPack pack;
    memset(&pack, 0, sizeof pack);
    memcpy(pack.c, h_scalars, sizeof(adana_step_scalars) * static_cast<size_t>(n_classes));
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool star = variant_flags & ADANA_VARIANT_STAR;
    const bool gb = variant_flags & ADANA_GRAD_BF16;
    const bool pb = variant_flags & ADANA_PARAM_BF16;
    if (n_chunks > 0) {
        if (star) {
            if (gb) { if (pb) launch_main<true, true, true>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials);
                      else launch_main<true, true, false>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials); }
            else    { if (pb) launch_main<true, false, true>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials);
                      else launch_main<true, false, false>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials); }
        } else {
            if (gb) { if (pb) launch_main<false, true, true>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials);
                      else launch_main<false, true, false>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials); }
            else    { if (pb) launch_main<false, false, true>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials);
                      else launch_main<false, false, false>(n_chunks, st, d_desc, d_vstart, d_chunk_first, n_tensors, pack, d_partials); }
        }
        hipError_t err = hipGetLastError();
        if (err != hipSuccess)
            return set_err(ADANA_E_HIP, "adana_mta_step: main launch failed: %s", hipGetErrorString(err));
    }
    hipLaunchKernelGGL(finalize_kernel, dim3(static_cast<unsigned>(n_tensors)), dim3(kBlock), 0, st, d_desc, d_vstart,
                       n_tensors, d_partials, d_diag);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess)
        return set_err(ADANA_E_HIP, "adana_mta_step: finalize launch failed: %s", hipGetErrorString(err));
    return ADANA_OK;
}

}  // extern "C"
