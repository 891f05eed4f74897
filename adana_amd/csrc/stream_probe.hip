// stream_probe.hip -- the achievable HBM rate of the optimizer step's access
// pattern with the arithmetic taken out, for bench.py's roofline report.
//
// The Dana-Star step streams 5 fp32 arrays in (p, g, m, v, tau) and 4 back
// out in place (p, m, v, tau).  This kernel moves exactly those bytes in
// exactly the step kernel's way -- one 256-thread workgroup per 1024-element
// chunk, one 16-byte non-temporal global load per array per thread, 16-byte
// sc1|nt buffer stores, a residency cap imposed with unused dynamic LDS --
// and computes only a sum.  Its rate is the ceiling that memory-system
// effects (stream count, read/write mix) leave for the step itself.
//
// Not part of the optimizer's interface: built as a separate library
// (libadana_probe.so) and loaded only by bench.py.
#include <hip/hip_runtime.h>

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

// arrays a[0..4] are read; a[0..3] are written back (in place)
__global__ __launch_bounds__(kThreads) void stream_5r4w_kernel(float *a0, float *a1, float *a2, float *a3,
                                                              float *a4) {
    float *const a[5] = {a0, a1, a2, a3, a4};
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * kChunk;
    const int64_t i = lo + 4 * threadIdx.x;
    F4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < 5; ++k) s += __builtin_nontemporal_load((const GF4 *)(a[k] + i));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        F4 o = s;
        o.x += static_cast<float>(k);
        store_stream(a[k] + lo, 16 * threadIdx.x, o);
    }
}

}  // namespace

// One launch over n elements of each array (n a positive multiple of 1024;
// the arrays 16-byte aligned, n elements each, distinct), capped at
// `wgs_per_cu` resident workgroups per CU (0: no cap).  Returns 0 or a HIP
// error code; -1 for bad arguments.
extern "C" int adana_probe_stream_5r4w(float *const *arrays, int64_t n, int wgs_per_cu, hipStream_t stream) {
    if (!arrays || n <= 0 || n % kChunk != 0 || n / kChunk > 0x7fffffff || wgs_per_cu < 0) return -1;
    for (int k = 0; k < 5; ++k)
        if (!arrays[k] || reinterpret_cast<uintptr_t>(arrays[k]) % 16 != 0) return -1;
    size_t lds = 0;
    if (wgs_per_cu > 0) {
        int dev = 0, per_cu = 0, per_block = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) != hipSuccess ||
            hipDeviceGetAttribute(&per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
            return -1;
        const size_t l = static_cast<size_t>(per_cu) / static_cast<size_t>(wgs_per_cu) - 1024;
        if (l > static_cast<size_t>(per_block)) return -1;
        lds = l;
    }
    hipLaunchKernelGGL(stream_5r4w_kernel, dim3(static_cast<unsigned>(n / kChunk)), dim3(kThreads),
                       static_cast<unsigned>(lds), stream, arrays[0], arrays[1], arrays[2], arrays[3], arrays[4]);
    return static_cast<int>(hipGetLastError());
}
