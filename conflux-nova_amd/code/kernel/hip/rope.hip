// rope.hip -- rotary position embedding, alone and fused with the paged append
// (gfx950).
//
// Reference: src/kernel/rope.cu.  The table kernel (rope.cu:9-18) fills
// cs/sn [rows][HD/2] with f_i = exp2f(-(float)i * (1/(HD/2)) * log2f(theta)),
// a = (float)pos * f_i, cs = cosf(a), sn = sinf(a).  Here every float step of
// that recipe is correctly rounded (the transcendentals run in double and are
// rounded once), so the table is fixed bit for bit and equals the CPU oracle's.
// The rotation (rope.cu:21-58) uses the NeoX pairs (i, i + HD/2) of the Qwen2
// family (include/nova/arch/traits.h:15-17) and evaluates x0*c - x1*s and
// x0*s + x1*c exactly as written (each product rounded, no fma).
//
// The fused entry points replace RopeKvOp (code/graph/dense.h:75-83), which
// runs rope_batch over q and k in place and then kv_store_paged reads k back:
// here one pass rotates q in place, rotates k in registers and writes it, with
// v, straight into the fp16 pages (round to nearest even).  The caller's k
// buffer is left unrotated: in the reference nothing reads it after the store.
//
// Layout: one workgroup per (token, session).  Work units are (head, quad):
// lane-unit u rotates elements 4j..4j+3 and their partners 64+4j.. of one
// head (float4 loads, 16 lanes per head); the fused kernel adds (kv head,
// octet) units that convert 8 values of v.  HBM-bound elementwise work.
#include <hip/hip_runtime.h>
#include <cmath>
#include <cstdint>

#include "check.h"
#include "model.h"
#include "nova_kernel.h"
#include "rope_math.h"

namespace nova {
namespace {

constexpr int NH = Model::NH, NKV = Model::NKV, HD = Model::HD, KVW = Model::KVW;
constexpr int HALF = HD / 2;
constexpr int QUADS = HALF / 4;                // float4 units per head
constexpr int OCTS = HD / 8;                   // 8-value v units per head
constexpr int RT = 256;                        // threads per workgroup
constexpr int kRopeCtx = 4096;                 // reference kCtx (include/nova/config.h:23)
static_assert(HALF % 4 == 0 && HD % 8 == 0, "vector units");

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

__global__ void rope_table_kernel(float* __restrict__ cs, float* __restrict__ sn, int rows, float l2) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)rows * HALF) return;
    const int pos = (int)(idx / HALF);
    const int i = (int)(idx - (int64_t)pos * HALF);
    const float e = -(float)i * (1.f / (float)HALF);
    const float t = e * l2;
    const float f = (float)exp2((double)t);
    const float a = (float)pos * f;
    cs[idx] = (float)cos((double)a);
    sn[idx] = (float)sin((double)a);
}

// four pairs at once, each through rope_rotate (every product rounded, no fma)
__device__ __forceinline__ void rotate(const f4 x0, const f4 x1, const f4 c, const f4 s, f4& y0, f4& y1) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float a, b;
        rope_rotate(x0[e], x1[e], c[e], s[e], a, b);
        y0[e] = a;
        y1[e] = b;
    }
}

__device__ __forceinline__ u2 to_f16x4(const f4 y) {
    u2 r;
    r[0] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[0]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[1]) << 16);
    r[1] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[2]) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)y[3]) << 16);
    return r;
}

struct RopeArgs {
    float* q;                  // [n_sess][n][NH][HD], rotated in place
    float* k;                  // [n_sess][n][NKV][HD]; rotated in place unless pool_k
    const float* v;            // [n_sess][n][NKV][HD] (fused only)
    const float* cs;
    const float* sn;
    uint16_t* pool_k;          // null: plain rope (reference launch_rope_batch)
    uint16_t* pool_v;
    const int32_t* tables;     // session i's table at tables + i * table_stride
    int64_t table_stride;
    const int32_t* pos0;       // device [n_sess] or null -> pos0_scalar
    int64_t pos0_scalar;
    int n;
    int layer;
    int nb;
};

template <bool kFused>
__global__ void __launch_bounds__(RT) rope_kernel(RopeArgs a) {
    const int t = blockIdx.x;
    const int sess = blockIdx.y;
    const int64_t pos = (a.pos0 ? (int64_t)a.pos0[sess] : a.pos0_scalar) + t;
    const int64_t tok = (int64_t)sess * a.n + t;
    const f4* cs4 = reinterpret_cast<const f4*>(a.cs + pos * HALF);
    const f4* sn4 = reinterpret_cast<const f4*>(a.sn + pos * HALF);
    int64_t row = 0;                                         // pool element offset of this token's row
    if constexpr (kFused) {
        const int32_t* table = a.tables + (int64_t)sess * a.table_stride;
        row = (((int64_t)a.layer * a.nb + table[pos >> kKvBlockShift]) * kKvBlock + (pos & kKvBlockMask)) * KVW;
    }
    constexpr int ROT = (NH + NKV) * QUADS;
    constexpr int UNITS = ROT + (kFused ? NKV * OCTS : 0);
    for (int u = threadIdx.x; u < UNITS; u += RT) {
        if (u < ROT) {
            const int h = u / QUADS, j = u - h * QUADS;
            const bool is_q = h < NH;
            float* base = is_q ? a.q + (tok * NH + h) * HD : a.k + (tok * NKV + (h - NH)) * HD;
            const f4 x0 = *reinterpret_cast<const f4*>(base + 4 * j);
            const f4 x1 = *reinterpret_cast<const f4*>(base + HALF + 4 * j);
            f4 y0, y1;
            rotate(x0, x1, cs4[j], sn4[j], y0, y1);
            if (kFused && !is_q) {
                uint16_t* dst = a.pool_k + row + (h - NH) * HD;
                *reinterpret_cast<u2*>(dst + 4 * j) = to_f16x4(y0);
                *reinterpret_cast<u2*>(dst + HALF + 4 * j) = to_f16x4(y1);
            } else {
                *reinterpret_cast<f4*>(base + 4 * j) = y0;
                *reinterpret_cast<f4*>(base + HALF + 4 * j) = y1;
            }
        } else if constexpr (kFused) {
            const int w = u - ROT;
            const int h = w / OCTS, j = w - h * OCTS;
            const float* src = a.v + (tok * NKV + h) * HD + 8 * j;
            const u2 lo = to_f16x4(*reinterpret_cast<const f4*>(src));
            const u2 hi = to_f16x4(*reinterpret_cast<const f4*>(src + 4));
            *reinterpret_cast<u4*>(a.pool_v + row + h * HD + 8 * j) = u4{lo[0], lo[1], hi[0], hi[1]};
        }
    }
}

void table(float* cs, float* sn, int rows, hipStream_t s) {
    NOVA_REQUIRE(cs && sn && rows >= 0);
    const int64_t total = (int64_t)rows * HALF;
    if (total == 0) return;
    const float l2 = (float)std::log2((double)(float)Model::kTheta);
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, cs, sn, rows, l2);
    NOVA_LAUNCHED();
}

void launch(const RopeArgs& a, int n_sess, hipStream_t s) {
    if (a.n == 0 || n_sess == 0) return;
    if (a.pool_k) hipLaunchKernelGGL(rope_kernel<true>, dim3(a.n, n_sess), dim3(RT), 0, s, a);
    else hipLaunchKernelGGL(rope_kernel<false>, dim3(a.n, n_sess), dim3(RT), 0, s, a);
    NOVA_LAUNCHED();
}

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {

void launch_rope_table(float* cs, float* sn, nova_stream_t s) {
    table(cs, sn, kRopeCtx, reinterpret_cast<hipStream_t>(s));
}

void launch_rope_table_rows(float* cs, float* sn, int rows, nova_stream_t s) {
    table(cs, sn, rows, reinterpret_cast<hipStream_t>(s));
}

void launch_rope_batch(float* q, float* k, int n, int64_t pos0, const float* cs, const float* sn,
                       nova_stream_t s) {
    NOVA_REQUIRE(q && k && cs && sn && n >= 0 && n <= 65535 && pos0 >= 0);
    RopeArgs a{};
    a.q = q;
    a.k = k;
    a.cs = cs;
    a.sn = sn;
    a.pos0_scalar = pos0;
    a.n = n;
    launch(a, 1, reinterpret_cast<hipStream_t>(s));
}

void launch_rope(float* q, float* k, int64_t pos, const float* cs, const float* sn, nova_stream_t s) {
    launch_rope_batch(q, k, 1, pos, cs, sn, s);
}

void launch_rope_kv_store_paged(float* q, const float* k, const float* v, const float* cs, const float* sn,
                                uint16_t* pool_k, uint16_t* pool_v, const int32_t* table, int layer, int nb,
                                int n, int64_t pos0, nova_stream_t s) {
    NOVA_REQUIRE(q && k && v && cs && sn && pool_k && pool_v && table);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n >= 0 && n <= 65535 && pos0 >= 0);
    RopeArgs a{};
    a.q = q;
    a.k = const_cast<float*>(k);
    a.v = v;
    a.cs = cs;
    a.sn = sn;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = table;
    a.pos0_scalar = pos0;
    a.n = n;
    a.layer = layer;
    a.nb = nb;
    launch(a, 1, reinterpret_cast<hipStream_t>(s));
}

void launch_rope_kv_store_paged_batch(float* q, const float* k, const float* v, const float* cs,
                                      const float* sn, uint16_t* pool_k, uint16_t* pool_v,
                                      const int32_t* tables, int table_stride, const int32_t* n_past,
                                      int n_sess, int n, int layer, int nb, nova_stream_t s) {
    NOVA_REQUIRE(q && k && v && cs && sn && pool_k && pool_v && tables && n_past);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n >= 0 && n <= 65535);
    NOVA_REQUIRE(n_sess >= 0 && n_sess <= 65535 && table_stride > 0);
    RopeArgs a{};
    a.q = q;
    a.k = const_cast<float*>(k);
    a.v = v;
    a.cs = cs;
    a.sn = sn;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = tables;
    a.table_stride = table_stride;
    a.pos0 = n_past;
    a.n = n;
    a.layer = layer;
    a.nb = nb;
    launch(a, n_sess, reinterpret_cast<hipStream_t>(s));
}

}  // extern "C"
