// q4k.hip -- Q4_K weight x int8 activation GEMV for one decode token, and the
// activation quantiser it consumes (gfx950).
//
// Reference: src/kernel/q4k_gemv.cu.  Weights are ggml block_q4_K super-blocks
// (include/nova/quant/q4_k.h:19-25): 144 B per 256 weights -- fp16 d, fp16
// dmin, 12 B of packed 6-bit (scale, min) for 8 sub-blocks of 32, and 128 B of
// nibbles (bytes 32g..32g+31 hold sub-block 2g in the low nibbles and 2g+1 in
// the high nibbles).  Activations are ActQ8 (include/nova/kernel/types.h:24-28):
// int8 codes, an fp32 scale per 32 and the int sum of each 16 codes, so that
//   w . x = sum over sub-blocks of dx * (d*sc*sum(q*c) - dmin*m*sum(c)).
//
// gfx950 design (HBM-bound on the weights, 4.5 bits each):
//  * A workgroup of 4 waves stages the whole activation (codes, scales, sums)
//    in LDS once and then walks rows (grid-stride), one row per wave at a
//    time, so the activation is read from L2 once per workgroup, not per row.
//  * A wave covers 8 super-blocks per step: lane (j, c) = (lane >> 3, lane & 7)
//    takes the 16 nibble bytes at offset 16c of super-block 8s + j -- 16 weights
//    of sub-block 2(c>>1) (low nibbles) and 16 of sub-block 2(c>>1)+1 (high).
//    Rows of up to 4 steps (cols <= 8192: the hidden widths 1536, 3584,
//    5120) use a kernel whose step loop is unrolled at compile time, all of a
//    row's loads issued before any is consumed; wider rows (the FFN widths)
//    take 4 steps in flight at a time.  One row per wave either way; ~70-80
//    registers keep 6-7 waves per SIMD resident.
//  * Products: v_dot4_i32_i8 on nibbles unpacked with a mask and a shift
//    (8 per lane per super-block); the per-sub-block float combination is the
//    reference's; the row sum is a wave reduction.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "check.h"
#include "nova_kernel.h"

namespace nova {
namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef int32_t i4 __attribute__((ext_vector_type(4)));

constexpr int kQK = 256;                       // weights per super-block
constexpr int kBlockBytes = 144;
constexpr int QT = 256;                        // threads per workgroup
constexpr int kBatch = 4;                      // steps (8 super-blocks each) in flight per wave
constexpr int kMaxCols = 32768;                // the activation (and its scales, sums) fits LDS

// ---------------------------------------------------------------- quant
// quant_kernel, q4k_gemv.cu:9-33: one thread per 32-element block.
__global__ void quant_kernel(int8_t* __restrict__ qs, float* __restrict__ d, int32_t* __restrict__ sums,
                             const float* __restrict__ x, int rows, int cols) {
    const int nb = cols / 32;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * nb) return;
    const int64_t row = idx / nb;
    const int b = (int)(idx - row * nb);
    const float* xp = x + row * cols + 32 * b;
    float v[32];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(xp + i);
        v[i] = t.x; v[i + 1] = t.y; v[i + 2] = t.z; v[i + 3] = t.w;
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    const float scale = amax * (1.f / 127.f);
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    int s0 = 0, s1 = 0;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int q = (int)rintf(v[i] * inv);
        if (i < 16) s0 += q; else s1 += q;
        if ((i & 3) == 0) packed[i >> 2] = 0;
        packed[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
    }
    u4* qp = reinterpret_cast<u4*>(qs + row * cols + 32 * b);
    qp[0] = u4{packed[0], packed[1], packed[2], packed[3]};
    qp[1] = u4{packed[4], packed[5], packed[6], packed[7]};
    d[row * nb + b] = scale;
    sums[row * (cols / 16) + 2 * b] = s0;
    sums[row * (cols / 16) + 2 * b + 1] = s1;
}

// ---------------------------------------------------------------- gemv
__device__ __forceinline__ float half_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// get_scale_min_k4, q4_k.h:44-52, for sub-block j of the 12 scale bytes
// held as three little-endian words
__device__ __forceinline__ void scale_min(int j, const uint32_t sw[3], uint32_t& sc, uint32_t& m) {
    auto byte = [&](int k) -> uint32_t { return (sw[k >> 2] >> (8 * (k & 3))) & 0xFFu; };
    if (j < 4) {
        sc = byte(j) & 63;
        m = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// one lane's share of super-block sb (header hd, nibbles nb16) against the
// activation staged in LDS: the two sub-block terms of the reference's sum
__device__ __forceinline__ float sb_terms(const u4 hd, const u4 nb16, int sb, int grp, int elo,
                                          const int8_t* s_q, const float* s_d, const int32_t* s_s) {
    const int k0 = sb * kQK + elo;             // low-nibble elements k0..k0+15, high k0+32..
    const i4 alo = *reinterpret_cast<const i4*>(s_q + k0);
    const i4 ahi = *reinterpret_cast<const i4*>(s_q + k0 + 32);
    int dlo = 0, dhi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        dlo = __builtin_amdgcn_sdot4((int)(nb16[e] & 0x0F0F0F0Fu), alo[e], dlo, false);
        dhi = __builtin_amdgcn_sdot4((int)((nb16[e] >> 4) & 0x0F0F0F0Fu), ahi[e], dhi, false);
    }
    const uint32_t sw[3] = {hd[1], hd[2], hd[3]};
    uint32_t scl, mcl, sch, mch;
    scale_min(2 * grp, sw, scl, mcl);
    scale_min(2 * grp + 1, sw, sch, mch);
    const float dd = half_to_float(hd[0] & 0xFFFFu);
    const float dm = half_to_float(hd[0] >> 16);
    const float dxl = s_d[k0 >> 5], dxh = s_d[(k0 + 32) >> 5];
    const int sml = s_s[k0 >> 4], smh = s_s[(k0 + 32) >> 4];
    return dxl * ((dd * (float)scl) * (float)dlo - (dm * (float)mcl) * (float)sml) +
           dxh * ((dd * (float)sch) * (float)dhi - (dm * (float)mch) * (float)smh);
}

__device__ __forceinline__ void stage_activation(int cols, const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                 const int32_t* __restrict__ xs, int8_t* s_q, float* s_d,
                                                 int32_t* s_s) {
    for (int i = threadIdx.x; i < cols / 16; i += QT)
        *reinterpret_cast<u4*>(s_q + 16 * i) = *reinterpret_cast<const u4*>(xq + 16 * i);
    for (int i = threadIdx.x; i < cols / 32; i += QT) s_d[i] = xd[i];
    for (int i = threadIdx.x; i < cols / 16; i += QT) s_s[i] = xs[i];
    __syncthreads();
}

// Rows of at most 4 steps (8 super-blocks per step, cols <= 8192): the step
// loop is unrolled at compile time, one row per wave, all of the row's loads
// issued before any is consumed.  (Measured on gfx950: taking 2 or 4 rows per
// wave at once keeps more bytes in flight per wave but costs occupancy and is
// slower; so is a compile-time kernel for the 10-step rows of the FFN width.)
template <int STEPS>
__global__ void __launch_bounds__(QT) gemv_fixed_kernel(const uint8_t* __restrict__ w, int64_t rows, int cols,
                                                         const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                         const int32_t* __restrict__ xs, float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) unsigned char s_x[];
    int8_t* s_q = reinterpret_cast<int8_t*>(s_x);
    float* s_d = reinterpret_cast<float*>(s_x + cols);
    int32_t* s_s = reinterpret_cast<int32_t*>(s_x + cols + 4 * (cols / 32));
    stage_activation(cols, xq, xd, xs, s_q, s_d, s_s);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane >> 3, c = lane & 7, grp = c >> 1;
    const int elo = grp * 64 + (c & 1) * 16;
    const int nsb = cols / kQK;
    const int64_t row_bytes = (int64_t)nsb * kBlockBytes;

    for (int64_t r = (int64_t)blockIdx.x * 4 + wave; r < rows; r += (int64_t)gridDim.x * 4) {
        u4 hdr[STEPS], nib[STEPS];
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const int sb = 8 * t + j;
            if (sb < nsb) {
                const uint8_t* blk = w + r * row_bytes + (int64_t)sb * kBlockBytes;
                hdr[t] = *reinterpret_cast<const u4*>(blk);
                nib[t] = *reinterpret_cast<const u4*>(blk + 16 + 16 * c);
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const int sb = 8 * t + j;
            if (sb < nsb) acc += sb_terms(hdr[t], nib[t], sb, grp, elo, s_q, s_d, s_s);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) out[r] = acc;
    }
}

// Any width: one row per wave, 4 steps of loads in flight at a time.
__global__ void __launch_bounds__(QT) gemv_kernel(const uint8_t* __restrict__ w, int64_t rows, int cols,
                                                   const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                   const int32_t* __restrict__ xs, float* __restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) unsigned char s_x[];
    int8_t* s_q = reinterpret_cast<int8_t*>(s_x);
    float* s_d = reinterpret_cast<float*>(s_x + cols);
    int32_t* s_s = reinterpret_cast<int32_t*>(s_x + cols + 4 * (cols / 32));
    stage_activation(cols, xq, xd, xs, s_q, s_d, s_s);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int j = lane >> 3;                   // super-block within the step
    const int c = lane & 7;                    // 16-byte slice of its nibbles
    const int grp = c >> 1;                    // sub-blocks 2grp (low) and 2grp+1 (high)
    const int elo = grp * 64 + (c & 1) * 16;   // first element (low nibbles) inside the super-block
    const int nsb = cols / kQK;
    const int steps = (nsb + 7) / 8;
    const int64_t row_bytes = (int64_t)nsb * kBlockBytes;

    for (int64_t r = (int64_t)blockIdx.x * 4 + wave; r < rows; r += (int64_t)gridDim.x * 4) {
        const uint8_t* wr = w + r * row_bytes;
        float acc = 0.f;
        for (int t0 = 0; t0 < steps; t0 += kBatch) {
            u4 hdr[kBatch], nib[kBatch];
#pragma unroll
            for (int t = 0; t < kBatch; ++t) {
                const int sb = 8 * (t0 + t) + j;
                if (sb < nsb) {
                    const uint8_t* blk = wr + (int64_t)sb * kBlockBytes;
                    hdr[t] = *reinterpret_cast<const u4*>(blk);
                    nib[t] = *reinterpret_cast<const u4*>(blk + 16 + 16 * c);
                }
            }
#pragma unroll
            for (int t = 0; t < kBatch; ++t) {
                const int sb = 8 * (t0 + t) + j;
                if (sb < nsb) acc += sb_terms(hdr[t], nib[t], sb, grp, elo, s_q, s_d, s_s);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) out[r] = acc;
    }
}

int gemv_grid(int64_t rows) {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        NOVA_HIP(hipGetDevice(&dev));
        NOVA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    }
    const int64_t want = (rows + 3) / 4;       // one row per wave
    const int64_t cap = (int64_t)cus * 8;      // grid-stride beyond 8 workgroups per CU
    return (int)(want < cap ? want : cap);
}

template <int STEPS>
void launch_fixed(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                  const int32_t* xs, float* out, size_t lds, hipStream_t s) {
    hipLaunchKernelGGL(gemv_fixed_kernel<STEPS>, dim3((unsigned)gemv_grid(rows)), dim3(QT), lds, s, blocks, rows,
                       cols, xq, xd, xs, out);
}

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {

void launch_quant_q8(int8_t* qs, float* d, int32_t* sums, const float* x, int rows, int cols, nova_stream_t s) {
    NOVA_REQUIRE(qs && d && sums && x && rows >= 0 && cols > 0 && cols % 32 == 0);
    const int64_t total = (int64_t)rows * (cols / 32);
    if (total == 0) return;
    hipLaunchKernelGGL(quant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), qs, d, sums, x, rows, cols);
    NOVA_LAUNCHED();
}

void launch_gemv_q4k(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                     const int32_t* xs, float* out, nova_stream_t s) {
    NOVA_REQUIRE(blocks && xq && xd && xs && out && rows >= 0);
    NOVA_REQUIRE(cols > 0 && cols % kQK == 0 && cols <= kMaxCols);
    if (rows == 0) return;
    const size_t lds = (size_t)cols + 4 * (size_t)(cols / 32) + 4 * (size_t)(cols / 16);
    const hipStream_t st = reinterpret_cast<hipStream_t>(s);
    switch ((cols / kQK + 7) / 8) {            // steps of 8 super-blocks
        case 1: launch_fixed<1>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 2: launch_fixed<2>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 3: launch_fixed<3>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 4: launch_fixed<4>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        default:
            hipLaunchKernelGGL(gemv_kernel, dim3((unsigned)gemv_grid(rows)), dim3(QT), lds, st, blocks, rows, cols,
                               xq, xd, xs, out);
    }
    NOVA_LAUNCHED();
}

}  // extern "C"
