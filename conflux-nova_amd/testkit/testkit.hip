// testkit.hip -- seeded synthetic K/V for tests and benchmarks (gfx950).
//
// Not part of the reference interface: the reference fills its cache from a
// model; the benchmarks here need tens of GB of N(0,1) fp16 K/V resident in
// HBM without a host round trip.  Element e of a fill gets
//     u = splitmix64(seed + e * 0x9E3779B97F4A7C15)
//     x = sqrt(-2 ln u1) * cos(2 pi u2)    (Box-Muller, u1,u2 from the two halves)
// rounded to fp16 (RNE).  Tests never regenerate these values on the host:
// they download what the device holds, so the device math need not match libm.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "check.h"
#include "hal.h"
#include "nova_testkit.h"

namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_f16_kernel(uint16_t* __restrict__ p, uint64_t n, uint64_t seed, float scale) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t e = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; e < n; e += stride) {
        const uint64_t u = splitmix64(seed ^ (e * 0x9E3779B97F4A7C15ull));
        const float u1 = ((float)(uint32_t)(u >> 40) + 0.5f) * (1.0f / 16777216.0f);
        const float u2 = (float)(uint32_t)(u & 0xFFFFFFu) * (1.0f / 16777216.0f);
        const float x = sqrtf(-2.0f * logf(u1)) * cospif(2.0f * u2) * scale;
        const _Float16 h = (_Float16)x;
        p[e] = __builtin_bit_cast(uint16_t, h);
    }
}

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__global__ void copy16_kernel(u4* __restrict__ dst, const u4* __restrict__ src, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t e = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; e < n; e += stride) dst[e] = src[e];
}

// Contiguous streaming read of n 16-byte units by the whole grid, grid-stride
// (consecutive threads on consecutive 16 B), 4 loads per lane in flight per
// round, non-temporal (the decode kernel's load policy), one sink word per
// thread.  Measured on one MI355X over 127 MB per launch (28 launches in a
// graph): 512 workgroups of 256 threads reach 19.7 us, 80.6% of 8 TB/s, the
// best of 256-2048 workgroups x 256-1024 threads x 2, 4 or 8 loads in flight;
// one 512-thread workgroup per CU reading its own contiguous piece with 16
// loads in flight took 22.8 us.
constexpr int kStreamDepth = 4;
constexpr int kStreamThreads = 256;
__global__ void __launch_bounds__(kStreamThreads) stream_read_kernel(const u4* __restrict__ src, uint64_t n,
                                                                     uint32_t* __restrict__ sink) {
    const uint64_t stride = (uint64_t)gridDim.x * kStreamThreads;
    u4 acc = {0u, 0u, 0u, 0u};
    uint64_t e = (uint64_t)blockIdx.x * kStreamThreads + threadIdx.x;
    for (; e + (kStreamDepth - 1) * stride < n; e += kStreamDepth * stride) {
        u4 x[kStreamDepth];
#pragma unroll
        for (int k = 0; k < kStreamDepth; ++k) x[k] = __builtin_nontemporal_load(src + e + k * stride);
#pragma unroll
        for (int k = 0; k < kStreamDepth; ++k) acc += x[k];
    }
    for (; e < n; e += stride) acc += __builtin_nontemporal_load(src + e);
    sink[(uint64_t)blockIdx.x * kStreamThreads + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

}  // namespace

extern "C" {

void testkit_stream_read(const void* src, uint64_t bytes, int workgroups, uint32_t* sink, nova_stream_t s) {
    NOVA_REQUIRE(src && sink && bytes % 16 == 0 && workgroups >= 1);
    hipLaunchKernelGGL(stream_read_kernel, dim3(workgroups), dim3(kStreamThreads), 0, reinterpret_cast<hipStream_t>(s),
                       static_cast<const u4*>(src), bytes / 16, sink);
    NOVA_LAUNCHED();
}


// Plain 16-byte-per-lane copy of `bytes` (a multiple of 16): the reference
// kernel of known traffic that calibrates the HBM byte counters.
void testkit_copy(void* dst, const void* src, uint64_t bytes, nova_stream_t s) {
    NOVA_REQUIRE(bytes % 16 == 0);
    const uint64_t n = bytes / 16;
    if (n == 0) return;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL(copy16_kernel, dim3((unsigned)blocks), dim3(256), 0, reinterpret_cast<hipStream_t>(s),
                       static_cast<u4*>(dst), static_cast<const u4*>(src), n);
    NOVA_LAUNCHED();
}

// Fill n fp16 values at p with seeded N(0, scale^2) draws.
void testkit_fill_normal_f16(uint16_t* p, uint64_t n, uint64_t seed, float scale, nova_stream_t s) {
    if (n == 0) return;
    uint64_t blocks = (n + 255) / 256;
    if (blocks > 1u << 20) blocks = 1u << 20;
    hipLaunchKernelGGL(fill_normal_f16_kernel, dim3((unsigned)blocks), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), p, n, seed, scale);
    NOVA_LAUNCHED();
}

}  // extern "C"
