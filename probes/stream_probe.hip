// stream_probe.hip -- the achievable HBM rate of the optimizer step's access
// pattern with the arithmetic taken out, for bench.py's roofline report.
//
// The Dana-Star step streams 5 fp32 arrays in (p, g, m, v, tau) and 4 back
// out in place (p, m, v, tau), and ends each 1024-element chunk with a
// workgroup reduction and one 16-byte partial-sum store.  This kernel moves
// exactly those bytes in exactly the step kernel's way -- one 256-thread
// workgroup per chunk, one 16-byte non-temporal global load per array per
// thread, 16-byte sc1|nt buffer stores, the end-of-chunk barrier and partial
// store, a residency cap imposed with unused dynamic LDS -- and computes only
// a sum.  Its rate is the ceiling that memory-system effects (stream count,
// read/write mix) leave for the step itself.  (The end-of-chunk barrier and
// store are part of the pattern: without them the same stream measured about
// 5% slower on MI355X.)
//
// A second kernel does the same for the bf16-master ADana step (fp32 master,
// m, v and bf16 gradient in; fp32 master, m, v and bf16 parameter out).
//
// Not part of the optimizer's interface: built as a separate library
// (probes/libadana_probe.so) and loaded only by bench.py.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

namespace {

typedef float F4 __attribute__((ext_vector_type(4)));
typedef unsigned int U4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) F4 GF4;

constexpr int kChunk = 1024;
constexpr int kThreads = 256;

__device__ __forceinline__ void store_stream(float *chunk_base, int byte_off, F4 x) {
    U4 u;
    u.x = __float_as_uint(x.x);
    u.y = __float_as_uint(x.y);
    u.z = __float_as_uint(x.z);
    u.w = __float_as_uint(x.w);
    __builtin_amdgcn_raw_buffer_store_b128(
        u, __builtin_amdgcn_make_buffer_rsrc(chunk_base, 0, 0x7fffffff, 0x00020000), byte_off, 0, 16 | 2);
}

// The chunk's sum of s over the workgroup, stored by thread 0 as one float4.
__device__ __forceinline__ void chunk_partial(F4 s, float4 *partials) {
    __shared__ float red[kThreads / 64][4];
    float t[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
#pragma unroll
        for (int k = 0; k < 4; ++k) t[k] += __shfl_xor(t[k], o, 64);
    }
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) red[threadIdx.x >> 6][k] = t[k];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float4 q = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int w = 0; w < kThreads / 64; ++w) {
            q.x += red[w][0];
            q.y += red[w][1];
            q.z += red[w][2];
            q.w += red[w][3];
        }
        partials[blockIdx.x] = q;
    }
}

// arrays a[0..R-1] are read; a[0..W-1] are written back (in place).
// R = 5, W = 4: the Dana-Star step (p, g, m, v, tau in; p, m, v, tau out);
// R = 4, W = 3: the fp32 ADana step (p, g, m, v in; p, m, v out);
// R = 5, W = 0 and R = 0, W = 4: the same streams read only / written only.
template <int R, int W>
__global__ __launch_bounds__(kThreads) void stream_rw_kernel(float *a0, float *a1, float *a2, float *a3,
                                                            float *a4, float4 *partials) {
    float *const a[5] = {a0, a1, a2, a3, a4};
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * kChunk;
    const int64_t i = lo + 4 * threadIdx.x;
    F4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < R; ++k) s += __builtin_nontemporal_load((const GF4 *)(a[k] + i));
#pragma unroll
    for (int k = 0; k < W; ++k) {
        F4 o = s;
        o.x += static_cast<float>(k);
        store_stream(a[k] + lo, 16 * threadIdx.x, o);
    }
    chunk_partial(s, partials);
}

// The bf16-master ADana step's pattern (config C4): fp32 master, m, v and the
// bf16 gradient read; fp32 master, m, v written back in place and the bf16
// parameter written, with the step's policies (8-byte non-temporal loads and
// stores for the bf16 arrays, as the step's vector path) and end of chunk.
typedef unsigned int U2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(1))) U2 GU2;

__global__ __launch_bounds__(kThreads) void stream_master_kernel(float *master, const unsigned short *g, float *m,
                                                                float *v, unsigned short *p16, float4 *partials) {
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * kChunk;
    const int64_t i = lo + 4 * threadIdx.x;
    const F4 a = __builtin_nontemporal_load((const GF4 *)(master + i));
    const F4 b = __builtin_nontemporal_load((const GF4 *)(m + i));
    const F4 c = __builtin_nontemporal_load((const GF4 *)(v + i));
    const U2 h = __builtin_nontemporal_load((const GU2 *)(g + i));
    F4 s = a + b + c;
    s.x += __uint_as_float(h.x << 16);
    s.y += __uint_as_float(h.y << 16);
    store_stream(master + lo, 16 * threadIdx.x, s);
    F4 o = s;
    o.x += 1.0f;
    store_stream(m + lo, 16 * threadIdx.x, o);
    o.x += 1.0f;
    store_stream(v + lo, 16 * threadIdx.x, o);
    U2 q;
    q.x = __float_as_uint(s.z) >> 16;
    q.y = __float_as_uint(s.w) >> 16;
    __builtin_nontemporal_store(q, (GU2 *)(p16 + i));
    chunk_partial(s, partials);
}

// STREAM copy in the same style: dst[i] = src[i], with the same end of chunk
__global__ __launch_bounds__(kThreads) void stream_copy_kernel(float *dst, const float *src, float4 *partials) {
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * kChunk;
    const F4 x = __builtin_nontemporal_load((const GF4 *)(src + lo + 4 * threadIdx.x));
    store_stream(dst + lo, 16 * threadIdx.x, x);
    chunk_partial(x, partials);
}

// Dynamic LDS bytes for a cap of `wgs` resident workgroups per CU (0: none);
// -1 when the device cannot be queried or the cap is not expressible.
int64_t cap_lds(int wgs) {
    if (wgs == 0) return 0;
    int dev = 0, per_cu = 0, per_block = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
        hipDeviceGetAttribute(&per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        return -1;
    const int64_t l = static_cast<int64_t>(per_cu) / wgs - 1024;
    return (l > 0 && l <= per_block) ? l : -1;
}

template <int R, int W>
int launch_rw(float *const *arrays, int64_t n, float4 *partials, int wgs_per_cu, hipStream_t stream) {
    if (!arrays || !partials || n <= 0 || n % kChunk != 0 || n / kChunk > 0x7fffffff || wgs_per_cu < 0)
        return -1;
    for (int k = 0; k < (R > W ? R : W); ++k)
        if (!arrays[k] || reinterpret_cast<uintptr_t>(arrays[k]) % 16 != 0) return -1;
    const int64_t lds = cap_lds(wgs_per_cu);
    if (lds < 0) return -1;
    hipLaunchKernelGGL((stream_rw_kernel<R, W>), dim3(static_cast<unsigned>(n / kChunk)), dim3(kThreads),
                       static_cast<unsigned>(lds), stream, arrays[0], arrays[1], arrays[2], arrays[3],
                       R > 4 ? arrays[4] : nullptr, partials);
    return static_cast<int>(hipGetLastError());
}

}  // namespace

// One launch over n elements of each array (n a positive multiple of 1024;
// the arrays 16-byte aligned, n elements each, distinct; `partials` room for
// n / 1024 float4), capped at `wgs_per_cu` resident workgroups per CU (0: no
// cap).  Returns 0 or a HIP error code; -1 for bad arguments.
extern "C" int adana_probe_stream_5r4w(float *const *arrays, int64_t n, float4 *partials, int wgs_per_cu,
                                       hipStream_t stream) {
    return launch_rw<5, 4>(arrays, n, partials, wgs_per_cu, stream);
}

// The 5 arrays read only (no stores) and 4 written only (no loads), in the
// one-shot style of adana_probe_stream_5r4w (same conditions).
extern "C" int adana_probe_stream_5r0w(float *const *arrays, int64_t n, float4 *partials, int wgs_per_cu,
                                       hipStream_t stream) {
    return launch_rw<5, 0>(arrays, n, partials, wgs_per_cu, stream);
}
extern "C" int adana_probe_stream_0r4w(float *const *arrays, int64_t n, float4 *partials, int wgs_per_cu,
                                       hipStream_t stream) {
    return launch_rw<0, 4>(arrays, n, partials, wgs_per_cu, stream);
}

// The fp32 ADana pattern: arrays[0..3] read, arrays[0..2] written back (same
// conditions as above for those 4 arrays).
extern "C" int adana_probe_stream_4r3w(float *const *arrays, int64_t n, float4 *partials, int wgs_per_cu,
                                       hipStream_t stream) {
    return launch_rw<4, 3>(arrays, n, partials, wgs_per_cu, stream);
}

// The bf16-master pattern over n elements: master, m, v fp32 (16-byte aligned),
// g and p16 bfloat16 (8-byte aligned), all distinct, n a positive multiple of
// 1024; `partials` room for n / 1024 float4.
extern "C" int adana_probe_stream_master(float *master, const void *g, float *m, float *v, void *p16, int64_t n,
                                         float4 *partials, int wgs_per_cu, hipStream_t stream) {
    if (!master || !g || !m || !v || !p16 || !partials || n <= 0 || n % kChunk != 0 || n / kChunk > 0x7fffffff ||
        wgs_per_cu < 0)
        return -1;
    for (const void *q : {static_cast<const void *>(master), static_cast<const void *>(m), static_cast<const void *>(v)})
        if (reinterpret_cast<uintptr_t>(q) % 16 != 0) return -1;
    if (reinterpret_cast<uintptr_t>(g) % 8 != 0 || reinterpret_cast<uintptr_t>(p16) % 8 != 0) return -1;
    const int64_t lds = cap_lds(wgs_per_cu);
    if (lds < 0) return -1;
    hipLaunchKernelGGL(stream_master_kernel, dim3(static_cast<unsigned>(n / kChunk)), dim3(kThreads),
                       static_cast<unsigned>(lds), stream, master, static_cast<const unsigned short *>(g), m, v,
                       static_cast<unsigned short *>(p16), partials);
    return static_cast<int>(hipGetLastError());
}

// STREAM copy of n elements (same conditions as above; dst and src distinct).
extern "C" int adana_probe_copy(float *dst, const float *src, int64_t n, float4 *partials, int wgs_per_cu,
                                hipStream_t stream) {
    if (!dst || !src || !partials || dst == src || n <= 0 || n % kChunk != 0 || n / kChunk > 0x7fffffff ||
        wgs_per_cu < 0 ||
        reinterpret_cast<uintptr_t>(dst) % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0)
        return -1;
    const int64_t lds = cap_lds(wgs_per_cu);
    if (lds < 0) return -1;
    hipLaunchKernelGGL(stream_copy_kernel, dim3(static_cast<unsigned>(n / kChunk)), dim3(kThreads),
                       static_cast<unsigned>(lds), stream, dst, src, partials);
    return static_cast<int>(hipGetLastError());
}
