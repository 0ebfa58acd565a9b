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
//  * One token: a wave covers 16 super-blocks per step: lane (j, c) =
//    (lane >> 2, lane & 3) takes the 32 nibble bytes at offset 32c of
//    super-block 16s + j -- all 32 weights of sub-block 2c (low nibbles) and
//    of 2c+1 (high).  (The four-token kernel uses half-width lanes, 8
//    super-blocks per step.)  Rows of up to 4 steps (cols <= 16384: the
//    hidden widths 1536, 3584, 5120) are one wave's, with the step loop unrolled at compile time and
//    all of a row's loads issued before any is consumed; wider rows (the FFN
//    widths) are shared by the 4 waves of a workgroup, at most 4 steps each,
//    reduced through LDS in a fixed order.  Grids are sized to what is
//    resident at once and grid-stride beyond.
//  * Products: v_dot4_i32_i8 on nibbles unpacked with a mask and a shift
//    (8 per lane per super-block); the per-sub-block float combination is the
//    reference's; the row sum is a wave reduction.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <mutex>

#include "check.h"
#include "nova_kernel.h"

namespace nova {
namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef int32_t i4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

constexpr int kQK = 256;                       // weights per super-block
constexpr int kBlockBytes = 144;
constexpr int QT = 256;                        // threads per workgroup
constexpr int kMaxCols = 32768;                // the activation (and its scales, sums) fits LDS
// Lane geometry, LPS = lanes per super-block.  LPS = 4 (one token): a lane
// owns the 32 nibble bytes of one sub-block pair (64 weights: sub-block 2c in
// the low nibbles, 2c+1 in the high), 16 super-blocks per wave step.  LPS = 8
// (four tokens): half of that, 8 super-blocks per step.  Measured: the wide
// lanes take a 7B layer's projections from 50.8 to 48.7 us (fewer, larger
// steps per row), but make the four-token kernel 11% slower.
template <int LPS>
struct Lanes {
    static_assert(LPS == 4 || LPS == 8, "4 or 8 lanes per super-block");
    static constexpr int kSbPerStep = 64 / LPS;
    static constexpr int kNibWords = 32 / LPS;   // nibble dwords per lane
    static constexpr int grp(int c) { return LPS == 4 ? c : c >> 1; }
    static constexpr int elo(int c) { return LPS == 4 ? 64 * c : (c >> 1) * 64 + (c & 1) * 16; }
};
constexpr int kLps1 = 4;                       // one-token kernels
constexpr int kLps4 = 8;                       // four-token kernel
template <int LPS>
struct Nib {
    uint32_t w[Lanes<LPS>::kNibWords];
};

// ---------------------------------------------------------------- quant
// One 32-element block of quant_kernel, q4k_gemv.cu:9-33: d = amax / 127,
// codes rint(x * 127 / amax), the int sums of the two 16-code halves.  Shared
// by the quant kernel and the GEMV's in-kernel staging, so both produce the
// same bits.
__device__ __forceinline__ void quant_block(const float* __restrict__ xp, u4& lo, u4& hi, float& scale, int& s0,
                                            int& s1) {
    float v[32];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(xp + i);
        v[i] = t.x; v[i + 1] = t.y; v[i + 2] = t.z; v[i + 3] = t.w;
    }
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
    scale = amax * (1.f / 127.f);
    const float inv = amax > 0.f ? 127.f / amax : 0.f;
    s0 = 0;
    s1 = 0;
    uint32_t packed[8];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int q = (int)rintf(v[i] * inv);
        if (i < 16) s0 += q; else s1 += q;
        if ((i & 3) == 0) packed[i >> 2] = 0;
        packed[i >> 2] |= ((uint32_t)q & 0xFFu) << (8 * (i & 3));
    }
    lo = u4{packed[0], packed[1], packed[2], packed[3]};
    hi = u4{packed[4], packed[5], packed[6], packed[7]};
}

// quant_kernel: one thread per 32-element block.
__global__ void quant_kernel(int8_t* __restrict__ qs, float* __restrict__ d, int32_t* __restrict__ sums,
                             const float* __restrict__ x, int rows, int cols) {
    const int nb = cols / 32;
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * nb) return;
    const int64_t row = idx / nb;
    const int b = (int)(idx - row * nb);
    u4 lo, hi;
    float scale;
    int s0, s1;
    quant_block(x + row * cols + 32 * b, lo, hi, scale, s0, s1);
    u4* qp = reinterpret_cast<u4*>(qs + row * cols + 32 * b);
    qp[0] = lo;
    qp[1] = hi;
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

// One lane's share of a super-block, split in two so that several
// activations can reuse one weight load: sb_prep unpacks the lane's 16 nibble
// bytes (16 weights of sub-block 2grp in the low nibbles, 16 of 2grp+1 in the
// high) and the two (d*scale, dmin*min) pairs; sb_dot takes the products with
// one activation staged in LDS (codes, scales per 32, sums per 16).  The
// float combination is the reference's: dx * (d*sc*sum(q*c) - dmin*m*sum(c)).
template <int LPS>
struct SbW {
    static constexpr int NW = Lanes<LPS>::kNibWords;
    int lo[NW], hi[NW];                // nibbles as int8 lanes for v_dot4_i32_i8
    float al, bl, ah, bh;              // d*sc and dmin*m of the two sub-blocks
};

template <int LPS>
__device__ __forceinline__ Nib<LPS> load_nib(const uint8_t* blk, int c) {
    constexpr int NW = Lanes<LPS>::kNibWords;
    Nib<LPS> n;
    const uint8_t* p = blk + 16 + 4 * NW * c;
#pragma unroll
    for (int h = 0; h < NW / 4; ++h) {
        const u4 v = *reinterpret_cast<const u4*>(p + 16 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) n.w[4 * h + e] = v[e];
    }
    return n;
}

template <int LPS>
__device__ __forceinline__ SbW<LPS> sb_prep(const u4 hd, const Nib<LPS>& nb, int grp) {
    SbW<LPS> w;
#pragma unroll
    for (int e = 0; e < SbW<LPS>::NW; ++e) {
        w.lo[e] = (int)(nb.w[e] & 0x0F0F0F0Fu);
        w.hi[e] = (int)((nb.w[e] >> 4) & 0x0F0F0F0Fu);
    }
    const uint32_t sw[3] = {hd[1], hd[2], hd[3]};
    uint32_t scl, mcl, sch, mch;
    scale_min(2 * grp, sw, scl, mcl);
    scale_min(2 * grp + 1, sw, sch, mch);
    const float dd = half_to_float(hd[0] & 0xFFFFu);
    const float dm = half_to_float(hd[0] >> 16);
    w.al = dd * (float)scl;
    w.bl = dm * (float)mcl;
    w.ah = dd * (float)sch;
    w.bh = dm * (float)mch;
    return w;
}

// k0: the lane's first element (low nibbles) in the row; high nibbles at k0 + 32
template <int LPS>
__device__ __forceinline__ float sb_dot(const SbW<LPS>& w, int k0, const int8_t* s_q, const float* s_d,
                                        const float* s_s) {
    constexpr int NW = SbW<LPS>::NW;
    int dlo = 0, dhi = 0;
#pragma unroll
    for (int h = 0; h < NW / 4; ++h) {
        const i4 alo = *reinterpret_cast<const i4*>(s_q + k0 + 16 * h);
        const i4 ahi = *reinterpret_cast<const i4*>(s_q + k0 + 32 + 16 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            dlo = __builtin_amdgcn_sdot4(w.lo[4 * h + e], alo[e], dlo, false);
            dhi = __builtin_amdgcn_sdot4(w.hi[4 * h + e], ahi[e], dhi, false);
        }
    }
    const float dxl = s_d[k0 >> 5], dxh = s_d[(k0 + 32) >> 5];
    float sml = s_s[k0 >> 4], smh = s_s[(k0 + 32) >> 4];
    if constexpr (NW == 8) {                   // 32 elements: both 16-sums
        sml += s_s[(k0 >> 4) + 1];
        smh += s_s[((k0 + 32) >> 4) + 1];
    }
    return dxl * (w.al * (float)dlo - w.bl * sml) + dxh * (w.ah * (float)dhi - w.bh * smh);
}

template <int LPS>
__device__ __forceinline__ float sb_terms(const u4 hd, const Nib<LPS>& nb, int sb, int grp, int elo,
                                          const int8_t* s_q, const float* s_d, const float* s_s) {
    return sb_dot<LPS>(sb_prep<LPS>(hd, nb, grp), sb * kQK + elo, s_q, s_d, s_s);
}

// Up to 4 matrices of the same width that read one activation (q/k/v,
// gate/up), walked as one row space: matrix m owns rows [end[m-1], end[m]).
constexpr int kMaxMats = 4;
struct GemvSet {
    const uint8_t* w[kMaxMats];
    float* out[kMaxMats];
    int64_t end[kMaxMats];
    int n;
    int cols;
    const int8_t* xq;          // pre-quantised activation (ActQ8) ...
    const float* xd;
    const int32_t* xs;
    const float* x;            // ... or fp32, quantised while it is staged
};

__device__ __forceinline__ int mat_of(const GemvSet& g, int64_t r) {
    int m = 0;
#pragma unroll
    for (int k = 0; k < kMaxMats - 1; ++k) m += (k + 1 < g.n && r >= g.end[k]) ? 1 : 0;
    return m;
}

// The activation (codes, scales per 32, sums per 16) into LDS, once per
// workgroup; from ActQ8 as given, or quantised here from fp32.  The sums are
// kept as floats (exact: |sum| <= 16 * 127), so no dot product converts them.
// Copies an ActQ8 activation of n columns (codes, per-32 scales, per-16
// sums, the sums converted to exact floats) into LDS; NT threads, n <= MAXC.
// The loads of a round all go out before its LDS stores: a strided copy loop
// waits out one load latency per element, which at the FFN width was 3 us of
// the down projection's 11.4.  Codes go in rounds of 8 x 16 B per thread, the
// sums and scales as 16 B loads with the first round.  No barrier.
template <int NT, int MAXC>
__device__ __forceinline__ void stage_q8(const int8_t* xq, const float* xd, const int32_t* xs, int n, int8_t* s_q,
                                         float* s_d, float* s_s) {
    constexpr int NQ = (MAXC / 16 + NT - 1) / NT < 8 ? (MAXC / 16 + NT - 1) / NT : 8;
    constexpr int NS = (MAXC / 64 + NT - 1) / NT;
    constexpr int ND = (MAXC / 128 + NT - 1) / NT;
    const int t = threadIdx.x;
    i4 vs[NS];
    f4 vd[ND];
#pragma unroll
    for (int k = 0; k < NS; ++k)
        if (t + k * NT < n / 64) vs[k] = *reinterpret_cast<const i4*>(xs + 4 * (t + k * NT));
#pragma unroll
    for (int k = 0; k < ND; ++k)
        if (t + k * NT < n / 128) vd[k] = *reinterpret_cast<const f4*>(xd + 4 * (t + k * NT));
#pragma unroll 1
    for (int b = t; b < n / 16; b += NQ * NT) {
        u4 vq[NQ];
#pragma unroll
        for (int k = 0; k < NQ; ++k)
            if (b + k * NT < n / 16) vq[k] = *reinterpret_cast<const u4*>(xq + 16 * (b + k * NT));
#pragma unroll
        for (int k = 0; k < NQ; ++k)
            if (b + k * NT < n / 16) *reinterpret_cast<u4*>(s_q + 16 * (b + k * NT)) = vq[k];
    }
#pragma unroll
    for (int k = 0; k < NS; ++k)
        if (t + k * NT < n / 64) {
            const i4 v = vs[k];
            *reinterpret_cast<f4*>(s_s + 4 * (t + k * NT)) = f4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
        }
#pragma unroll
    for (int k = 0; k < ND; ++k)
        if (t + k * NT < n / 128) *reinterpret_cast<f4*>(s_d + 4 * (t + k * NT)) = vd[k];
}

template <bool kF32, int MAXC = kMaxCols>
__device__ __forceinline__ void stage_activation(const GemvSet& g, int8_t* s_q, float* s_d, float* s_s) {
    const int cols = g.cols;
    if constexpr (kF32) {
        for (int b = threadIdx.x; b < cols / 32; b += QT) {
            u4 lo, hi;
            float scale;
            int s0, s1;
            quant_block(g.x + 32 * b, lo, hi, scale, s0, s1);
            *reinterpret_cast<u4*>(s_q + 32 * b) = lo;
            *reinterpret_cast<u4*>(s_q + 32 * b + 16) = hi;
            s_d[b] = scale;
            s_s[2 * b] = (float)s0;
            s_s[2 * b + 1] = (float)s1;
        }
    } else {
        stage_q8<QT, MAXC>(g.xq, g.xd, g.xs, cols, s_q, s_d, s_s);
    }
    __syncthreads();
}

// Rows of at most 4 steps (16 super-blocks per step, cols <= 16384): the step
// loop is unrolled at compile time, one row per wave, all of the row's loads
// issued before any is consumed.  (Measured on gfx950: taking 2 or 4 rows per
// wave at once, or loading the next row while the current one is reduced,
// keeps more bytes in flight per wave but costs occupancy and is slower.)
template <int STEPS, bool kF32>
__global__ void __launch_bounds__(QT) gemv_fixed_kernel(GemvSet g) {
    constexpr int LPS_ = kLps1;
    extern __shared__ __attribute__((aligned(16))) unsigned char s_x[];
    const int cols = g.cols;
    int8_t* s_q = reinterpret_cast<int8_t*>(s_x);
    float* s_d = reinterpret_cast<float*>(s_x + cols);
    float* s_s = reinterpret_cast<float*>(s_x + cols + 4 * (cols / 32));   // 16-sums as exact floats
    stage_activation<kF32, STEPS * Lanes<kLps1>::kSbPerStep * kQK>(g, s_q, s_d, s_s);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar row addressing
    using L = Lanes<LPS_>;
    const int j = lane / LPS_, c = lane % LPS_, grp = L::grp(c);
    const int elo = L::elo(c);
    const int nsb = cols / kQK;
    const int64_t row_bytes = (int64_t)nsb * kBlockBytes;
    const int64_t rows = kF32 ? g.end[g.n - 1] : g.end[0];   // one matrix on the ActQ8 path

    for (int64_t r = (int64_t)blockIdx.x * 4 + wave; r < rows; r += (int64_t)gridDim.x * 4) {
        const int m = kF32 ? mat_of(g, r) : 0;
        const int64_t lr = m ? r - g.end[m - 1] : r;
        const uint8_t* wr = g.w[m] + lr * row_bytes;
        u4 hdr[STEPS];
        Nib<LPS_> nib[STEPS];
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const int sb = L::kSbPerStep * t + j;
            if (sb < nsb) {
                const uint8_t* blk = wr + (int64_t)sb * kBlockBytes;
                hdr[t] = *reinterpret_cast<const u4*>(blk);
                nib[t] = load_nib<LPS_>(blk, c);
            }
        }
        float acc = 0.f;
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const int sb = L::kSbPerStep * t + j;
            if (sb < nsb) acc += sb_terms<LPS_>(hdr[t], nib[t], sb, grp, elo, s_q, s_d, s_s);
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) g.out[m][lr] = acc;
    }
}

// Rows wider than 4 steps (the FFN widths): KS waves share a row, each with
// at most STEPS steps whose loads all go out at once; the KS partial sums
// meet in LDS and are added in a fixed order.  4 / KS rows per workgroup
// iteration.
template <int STEPS, int KS, bool kF32>
__global__ void __launch_bounds__(QT) gemv_split_kernel(GemvSet g) {
    constexpr int LPS_ = kLps1;
    extern __shared__ __attribute__((aligned(16))) unsigned char s_x[];
    __shared__ float s_part[4];
    const int cols = g.cols;
    int8_t* s_q = reinterpret_cast<int8_t*>(s_x);
    float* s_d = reinterpret_cast<float*>(s_x + cols);
    float* s_s = reinterpret_cast<float*>(s_x + cols + 4 * (cols / 32));   // 16-sums as exact floats
    stage_activation<kF32, (STEPS * Lanes<kLps1>::kSbPerStep * kQK * KS < kMaxCols ? STEPS * Lanes<kLps1>::kSbPerStep * kQK * KS : kMaxCols)>(g, s_q, s_d, s_s);

    constexpr int RPI = 4 / KS;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar row addressing
    const int part = wave % KS;
    using L = Lanes<LPS_>;
    const int j = lane / LPS_, c = lane % LPS_, grp = L::grp(c);
    const int elo = L::elo(c);
    const int nsb = cols / kQK;
    const int sb0 = L::kSbPerStep * STEPS * part + j;
    const int64_t row_bytes = (int64_t)nsb * kBlockBytes;
    const int64_t rows = kF32 ? g.end[g.n - 1] : g.end[0];   // one matrix on the ActQ8 path
    const int64_t stride = (int64_t)gridDim.x * RPI;

    for (int64_t base = (int64_t)blockIdx.x * RPI; base < rows; base += stride) {   // uniform per workgroup
        const int64_t r = base + wave / KS;
        const int m = (kF32 && r < rows) ? mat_of(g, r) : 0;
        const int64_t lr = m ? r - g.end[m - 1] : r;
        float acc = 0.f;
        if (r < rows) {
            const uint8_t* wr = g.w[m] + lr * row_bytes;
            u4 hdr[STEPS];
            Nib<LPS_> nib[STEPS];
#pragma unroll
            for (int t = 0; t < STEPS; ++t) {
                const int sb = sb0 + L::kSbPerStep * t;
                if (sb < nsb) {
                    const uint8_t* blk = wr + (int64_t)sb * kBlockBytes;
                    hdr[t] = *reinterpret_cast<const u4*>(blk);
                    nib[t] = load_nib<LPS_>(blk, c);
                }
            }
#pragma unroll
            for (int t = 0; t < STEPS; ++t) {
                const int sb = sb0 + L::kSbPerStep * t;
                if (sb < nsb) acc += sb_terms<LPS_>(hdr[t], nib[t], sb, grp, elo, s_q, s_d, s_s);
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
        if (lane == 0) s_part[wave] = acc;
        __syncthreads();
        if (part == 0 && lane == 0 && r < rows) {
            float sum = s_part[wave];
#pragma unroll
            for (int p = 1; p < KS; ++p) sum += s_part[wave + p];
            g.out[m][lr] = sum;
        }
        __syncthreads();
    }
}

// Four tokens at once (the reference's gemv4_kernel, q4k_gemv.cu:98-180, as
// Engine::decode_batch uses it for every projection, model.cpp:270-311):
// each weight load and its scale unpacking serve four activations.  The four
// activations (4 x 1.375 B per column) sit in LDS, 104 KB at the FFN width,
// so a workgroup is 16 waves to keep the CU's waves up.  Lanes are half as
// wide as in the one-token kernels (8 per super-block), so each token's sum
// is taken in another order than launch_gemv_q4k's (same terms).
constexpr int kTok4 = 4;
constexpr int QT4 = 1024;                      // threads per workgroup
constexpr int kMaxCols4 = 28672;               // 4 activations within 160 KB of LDS

template <int STEPS, int KS>
__global__ void __launch_bounds__(QT4) gemv4_kernel(const uint8_t* __restrict__ w, int64_t rows, int cols,
                                                     const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                     const int32_t* __restrict__ xs, float* __restrict__ out) {
    constexpr int LPS_ = kLps4;
    extern __shared__ __attribute__((aligned(16))) unsigned char s_x[];
    __shared__ float s_part[QT4 / 64][kTok4];
    int8_t* s_q = reinterpret_cast<int8_t*>(s_x);                                   // [4][cols]
    float* s_d = reinterpret_cast<float*>(s_x + kTok4 * cols);                       // [4][cols/32]
    float* s_s = reinterpret_cast<float*>(s_x + kTok4 * cols + 4 * kTok4 * (cols / 32));   // [4][cols/16]
    stage_q8<QT4, kTok4 * kMaxCols4>(xq, xd, xs, kTok4 * cols, s_q, s_d, s_s);
    __syncthreads();

    constexpr int WAVES4 = QT4 / 64;
    constexpr int RPI = WAVES4 / KS;           // rows per workgroup iteration
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int part = wave % KS;
    using L = Lanes<LPS_>;
    const int j = lane / LPS_, c = lane % LPS_, grp = L::grp(c);
    const int elo = L::elo(c);
    const int nsb = cols / kQK;
    const int sb0 = L::kSbPerStep * STEPS * part + j;
    const int64_t row_bytes = (int64_t)nsb * kBlockBytes;
    const int64_t stride = (int64_t)gridDim.x * RPI;

    for (int64_t base = (int64_t)blockIdx.x * RPI; base < rows; base += stride) {   // uniform per workgroup
        const int64_t r = base + wave / KS;
        float acc[kTok4] = {0.f, 0.f, 0.f, 0.f};
        if (r < rows) {
            const uint8_t* wr = w + r * row_bytes;
            u4 hdr[STEPS];
            Nib<LPS_> nib[STEPS];
#pragma unroll
            for (int t = 0; t < STEPS; ++t) {
                const int sb = sb0 + L::kSbPerStep * t;
                if (sb < nsb) {
                    const uint8_t* blk = wr + (int64_t)sb * kBlockBytes;
                    hdr[t] = *reinterpret_cast<const u4*>(blk);
                    nib[t] = load_nib<LPS_>(blk, c);
                }
            }
#pragma unroll
            for (int t = 0; t < STEPS; ++t) {
                const int sb = sb0 + L::kSbPerStep * t;
                if (sb < nsb) {
                    const SbW<LPS_> wv = sb_prep<LPS_>(hdr[t], nib[t], grp);
#pragma unroll
                    for (int k = 0; k < kTok4; ++k)
                        acc[k] += sb_dot<LPS_>(wv, sb * kQK + elo, s_q + k * cols, s_d + k * (cols / 32),
                                         s_s + k * (cols / 16));
                }
            }
        }
#pragma unroll
        for (int k = 0; k < kTok4; ++k)
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) acc[k] += __shfl_xor(acc[k], o, 64);
        if constexpr (KS == 1) {
            if (lane == 0 && r < rows)
#pragma unroll
                for (int k = 0; k < kTok4; ++k) out[k * rows + r] = acc[k];
        } else {
            if (lane == 0)
#pragma unroll
                for (int k = 0; k < kTok4; ++k) s_part[wave][k] = acc[k];
            __syncthreads();
            if (part == 0 && lane < kTok4 && r < rows) {
                float sum = s_part[wave][lane];
#pragma unroll
                for (int p = 1; p < KS; ++p) sum += s_part[wave + p][lane];
                out[lane * rows + r] = sum;
            }
            __syncthreads();
        }
    }
}

// Workgroups: one per rows_per_wg rows, but no more than can be resident at
// once (this kernel's occupancy at this LDS size times the CUs); beyond that
// the kernels grid-stride, so no second partial round of workgroups forms a
// tail (measured: gate projection 9.8 -> 9.0 us against a fixed cap of 8
// workgroups per CU, of which 7 fit).
template <typename K>
int gemv_grid(K kernel, int64_t rows, int rows_per_wg, size_t lds, int block = QT) {
    int dev = 0, cus = 0, per_cu = 0;
    NOVA_HIP(hipGetDevice(&dev));
    NOVA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    NOVA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, block, lds));
    if (per_cu < 1) per_cu = 1;
    const int64_t want = (rows + rows_per_wg - 1) / rows_per_wg;
    const int64_t cap = (int64_t)per_cu * cus;
    return (int)(want < cap ? want : cap);
}


// Four tokens on the matrix cores.  v_mfma_i32_16x16x64_i8 multiplies the
// codes (A: lane (g,r) with r = 4j + t holds token t's 16 codes at positions
// 16(g&1).. of sub-block 2p + (g>>1) when j is that sub-block's index within
// its half super-block, zeros otherwise) by 16 weight rows (B: lane (g,c)
// holds row c's 16 nibble bytes of sub-block pair p at offset 16(g&1), low
// nibbles for g < 2 and high nibbles for g >= 2: the same positions).  Two
// MFMAs (pairs 2h, 2h+1) give one C tile of integer dot products whose rows
// are (sub-block 4h+j, token t) and columns the weight rows, so lane (g,c)
// holds the four tokens of sub-block 4h+g for row c: one header load and one
// scale decode serve four values, which the float combination of sb_dot turns
// into dx * (d*sc*sum(q*c) - dmin*m*sum(c)).  The VALU keeps the nibble
// unpacking and that epilogue; the dot products move to the matrix core.  ks
// waves split a 16-row block's super-blocks and add their sums through LDS in
// a fixed order; 16 / ks blocks per workgroup iteration.
template <int STEPS>
__global__ void __launch_bounds__(QT4) gemv4_mfma_kernel(const uint8_t* __restrict__ w, int64_t rows, int cols,
                                                          const int8_t* __restrict__ xq, const float* __restrict__ xd,
                                                          const int32_t* __restrict__ xs, float* __restrict__ out,
                                                          int ks) {
    extern __shared__ __attribute__((aligned(16))) unsigned char s_x[];
    __shared__ f4 s_part[QT4 / 64][16];
    int8_t* s_q = reinterpret_cast<int8_t*>(s_x);                                   // [4][cols]
    float* s_d = reinterpret_cast<float*>(s_x + kTok4 * cols);                       // [4][cols/32]
    float* s_s = reinterpret_cast<float*>(s_x + kTok4 * cols + 4 * kTok4 * (cols / 32));   // [4][cols/16]
    stage_q8<QT4, kTok4 * kMaxCols4>(xq, xd, xs, kTok4 * cols, s_q, s_d, s_s);
    __syncthreads();

    constexpr int WAVES4 = QT4 / 64;
    const int rbi = WAVES4 / ks;                   // 16-row blocks per workgroup iteration
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int part = wave % ks, rbl = wave / ks;   // rbl >= rbi: an idle wave
    const int g = lane >> 4, c = lane & 15;
    const int t = c & 3, j = c >> 2;               // A role: row (j, t)
    const int nsb = cols / kQK;
    const int sb_a = part * nsb / ks, sb_b = (part + 1) * nsb / ks;
    const int64_t row_bytes = (int64_t)nsb * kBlockBytes;
    const int64_t n_rb = (rows + 15) / 16;
    const int sh = 4 * (g >> 1);
    const int8_t* aq = s_q + t * cols + 16 * g;
    const int cols32 = cols / 32, cols16 = cols / 16;

    for (int64_t base = (int64_t)blockIdx.x * rbi; base < n_rb; base += (int64_t)gridDim.x * rbi) {   // uniform
        const int64_t rb = base + rbl;
        const bool live = rbl < rbi && rb < n_rb;
        const int64_t r0 = rb * 16;
        const int64_t rw = live && r0 + c < rows ? r0 + c : rows - 1;
        const uint8_t* wr = w + rw * row_bytes;
        f4 acc = {0.f, 0.f, 0.f, 0.f};             // tokens 0..3 of row c, sub-blocks 4h+g
        if (live) {
            for (int sb0 = sb_a; sb0 < sb_b; sb0 += STEPS) {
                u4 raw[STEPS][4], hdr[STEPS];
#pragma unroll
                for (int u = 0; u < STEPS; ++u) {
                    const int sb = sb0 + u < sb_b ? sb0 + u : sb0;
                    const uint8_t* blk = wr + (int64_t)sb * kBlockBytes;
                    hdr[u] = *reinterpret_cast<const u4*>(blk);
#pragma unroll
                    for (int p = 0; p < 4; ++p) raw[u][p] = *reinterpret_cast<const u4*>(blk + 16 + 32 * p + 16 * (g & 1));
                }
#pragma unroll
                for (int u = 0; u < STEPS; ++u) {
                    if (sb0 + u >= sb_b) break;
                    const int sb = sb0 + u;
                    const uint32_t sw[3] = {hdr[u][1], hdr[u][2], hdr[u][3]};
                    const float dd = half_to_float(hdr[u][0] & 0xFFFFu);
                    const float dm = half_to_float(hdr[u][0] >> 16);
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        i4 cacc = {0, 0, 0, 0};
#pragma unroll
                        for (int q = 0; q < 2; ++q) {
                            const int p = 2 * h + q;
                            i4 b;
#pragma unroll
                            for (int e = 0; e < 4; ++e) b[e] = (int)((raw[u][p][e] >> sh) & 0x0F0F0F0Fu);
                            i4 a = {0, 0, 0, 0};
                            if (j == 2 * q + (g >> 1)) a = *reinterpret_cast<const i4*>(aq + sb * kQK + 64 * p);
                            cacc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, cacc, 0, 0, 0);
                        }
                        const int sub = 4 * h + g;                 // this lane's sub-block
                        uint32_t sc, mn;
                        scale_min(sub, sw, sc, mn);
                        const float al = dd * (float)sc, bl = dm * (float)mn;
                        const int k0 = sb * kQK + 32 * sub;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const float dx = s_d[i * cols32 + (k0 >> 5)];
                            const float sm = s_s[i * cols16 + (k0 >> 4)] + s_s[i * cols16 + (k0 >> 4) + 1];
                            acc[i] += dx * (al * (float)cacc[i] - bl * sm);
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[i] += __shfl_xor(acc[i], 16, 64);
            acc[i] += __shfl_xor(acc[i], 32, 64);
        }
        if (g == 0) s_part[wave][c] = acc;
        __syncthreads();
        if (part == 0 && g == 0 && live && r0 + c < rows) {
            f4 sum = s_part[wave][c];
            for (int pp = 1; pp < ks; ++pp) sum += s_part[wave + pp][c];
#pragma unroll
            for (int i = 0; i < 4; ++i) out[(int64_t)i * rows + r0 + c] = sum[i];
        }
        __syncthreads();
    }
}

template <int STEPS, bool kF32>
void launch_fixed(const GemvSet& g, size_t lds, hipStream_t s) {
    auto k = gemv_fixed_kernel<STEPS, kF32>;
    hipLaunchKernelGGL(k, dim3((unsigned)gemv_grid(k, g.end[g.n - 1], 4, lds)), dim3(QT), lds, s, g);
}

template <int STEPS, bool kF32>
void launch_split(const GemvSet& g, size_t lds, hipStream_t s) {
    auto k = gemv_split_kernel<STEPS, 4, kF32>;
    hipLaunchKernelGGL(k, dim3((unsigned)gemv_grid(k, g.end[g.n - 1], 1, lds)), dim3(QT), lds, s, g);
}

template <int STEPS, int KS>
void launch_gemv4_shape(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                        const int32_t* xs, float* out, size_t lds, hipStream_t s) {
    auto k = gemv4_kernel<STEPS, KS>;
    static std::once_flag once;                // dynamic LDS beyond 64 KB must be allowed per kernel
    std::call_once(once, [&] {
        NOVA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)(kTok4 * (size_t)kMaxCols4 * 11 / 8)));
    });
    hipLaunchKernelGGL(k, dim3((unsigned)gemv_grid(k, rows, (QT4 / 64) / KS, lds, QT4)), dim3(QT4), lds, s, blocks,
                       rows, cols, xq, xd, xs, out);
}

// Matrices of at least this many weights take the MFMA kernel.  Measured
// (7B shapes, four tokens): gate 18944 x 3584 18.9 -> 11.7 us, down
// 3584 x 18944 23.2 -> 15.1 us; the 3584 x 3584 and 512 x 3584 projections
// stay a little faster on the dot4 kernel (5.9 vs 6.0 us, 5.4 vs 5.65 us):
// 224 or fewer 16-row blocks are too few to fill the chip's 16-wave
// workgroups.
constexpr int64_t kMfma4MinWeights = (int64_t)32 << 20;
void launch_gemv4_mfma(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                       const int32_t* xs, float* out, size_t lds, hipStream_t s) {
    auto k = gemv4_mfma_kernel<2>;             // 2 super-blocks per load batch (3: gate slower, 4: both)
    static std::once_flag once;                // dynamic LDS beyond 64 KB must be allowed per kernel
    std::call_once(once, [&] {
        NOVA_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)(kTok4 * (size_t)kMaxCols4 * 11 / 8)));
    });
    int dev = 0, cus = 0, per_cu = 0;
    NOVA_HIP(hipGetDevice(&dev));
    NOVA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    NOVA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, QT4, lds));
    if (per_cu < 1) per_cu = 1;
    const int64_t n_rb = (rows + 15) / 16;
    const int64_t cap = (int64_t)per_cu * cus;
    const int nsb = cols / kQK;
    // waves per 16-row block (1..16; 16 / ks blocks per workgroup iteration,
    // the rest of the 16 waves idle): the fewest rounds of resident
    // workgroups times super-blocks per wave
    int ks = 1;
    int64_t best = INT64_MAX;
    for (int kk = 1; kk <= QT4 / 64; ++kk) {
        const int64_t wgs = (n_rb + (QT4 / 64) / kk - 1) / ((QT4 / 64) / kk);
        const int64_t cost = (wgs + cap - 1) / cap * ((nsb + kk - 1) / kk);
        if (cost < best) {
            best = cost;
            ks = kk;
        }
    }
    const int rbi = (QT4 / 64) / ks;
    const int64_t want = (n_rb + rbi - 1) / rbi;
    hipLaunchKernelGGL(k, dim3((unsigned)(want < cap ? want : cap)), dim3(QT4), lds, s, blocks, rows, cols, xq, xd, xs,
                       out, ks);
}

template <bool kF32>
void launch_set(const GemvSet& g, hipStream_t st) {
    const int cols = g.cols;
    const size_t lds = (size_t)cols + 4 * (size_t)(cols / 32) + 4 * (size_t)(cols / 16);
    constexpr int SPS = Lanes<kLps1>::kSbPerStep;
    switch ((cols / kQK + SPS - 1) / SPS) {    // steps of SPS super-blocks
        case 1: launch_fixed<1, kF32>(g, lds, st); break;
        case 2: launch_fixed<2, kF32>(g, lds, st); break;
        case 3: launch_fixed<3, kF32>(g, lds, st); break;
        case 4: launch_fixed<4, kF32>(g, lds, st); break;
        // wider rows: 4 waves per row, at most 4 steps each (measured: down
        // projection 3584 x 18944, 12.7 -> 11.7 us against one wave per row)
        case 5: case 6: case 7: case 8: launch_split<2, kF32>(g, lds, st); break;
        case 9: case 10: case 11: case 12: launch_split<3, kF32>(g, lds, st); break;
        default: launch_split<4, kF32>(g, lds, st); break;
    }
    NOVA_LAUNCHED();
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
    NOVA_REQUIRE(aligned16(xq) && aligned16(xd) && aligned16(xs));   // staged with 16 B loads
    if (rows == 0) return;
    GemvSet g{};
    g.w[0] = blocks;
    g.out[0] = out;
    g.end[0] = rows;
    g.n = 1;
    g.cols = cols;
    g.xq = xq;
    g.xd = xd;
    g.xs = xs;
    launch_set<false>(g, reinterpret_cast<hipStream_t>(s));
}

void launch_gemv4_q4k(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                      const int32_t* xs, float* out, nova_stream_t s) {
    NOVA_REQUIRE(blocks && xq && xd && xs && out && rows >= 0);
    NOVA_REQUIRE(cols > 0 && cols % kQK == 0 && cols <= kMaxCols4);
    NOVA_REQUIRE(aligned16(xq) && aligned16(xd) && aligned16(xs));   // staged with 16 B loads
    if (rows == 0) return;
    const size_t lds = kTok4 * ((size_t)cols + 4 * (size_t)(cols / 32) + 4 * (size_t)(cols / 16));
    const hipStream_t st = reinterpret_cast<hipStream_t>(s);
    if (rows * (int64_t)cols >= kMfma4MinWeights) {
        launch_gemv4_mfma(blocks, rows, cols, xq, xd, xs, out, lds, st);
        NOVA_LAUNCHED();
        return;
    }
    constexpr int SPS = Lanes<kLps4>::kSbPerStep;
    switch ((cols / kQK + SPS - 1) / SPS) {    // steps of SPS super-blocks: the row shapes
        case 1: launch_gemv4_shape<1, 1>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 2: launch_gemv4_shape<2, 1>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 3: launch_gemv4_shape<3, 1>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 4: launch_gemv4_shape<4, 1>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 5: case 6: case 7: case 8: launch_gemv4_shape<2, 4>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
        case 9: case 10: case 11: case 12:
            launch_gemv4_shape<3, 4>(blocks, rows, cols, xq, xd, xs, out, lds, st);
            break;
        default: launch_gemv4_shape<4, 4>(blocks, rows, cols, xq, xd, xs, out, lds, st); break;
    }
    NOVA_LAUNCHED();
}

void launch_gemv_q4k_f32(const uint8_t* const* blocks, const int64_t* rows, float* const* outs, int n_mat,
                         int cols, const float* x, nova_stream_t s) {
    NOVA_REQUIRE(blocks && rows && outs && x && n_mat >= 1 && n_mat <= kMaxMats);
    NOVA_REQUIRE(cols > 0 && cols % kQK == 0 && cols <= kMaxCols);
    GemvSet g{};
    int64_t total = 0;
    for (int m = 0; m < n_mat; ++m) {
        NOVA_REQUIRE(blocks[m] && outs[m] && rows[m] >= 0);
        total += rows[m];
        g.w[m] = blocks[m];
        g.out[m] = outs[m];
        g.end[m] = total;
    }
    if (total == 0) return;
    g.n = n_mat;
    g.cols = cols;
    g.x = x;
    launch_set<true>(g, reinterpret_cast<hipStream_t>(s));
}

}  // extern "C"
