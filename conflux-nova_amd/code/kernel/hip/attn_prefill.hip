// attn_prefill.hip -- causal attention of a prefill chunk over a paged prefix,
// on gfx950 matrix cores.
//
// Computes what flash_paged_kernel<false> computes (reference
// src/kernel/attn.cu:293-357, launcher :514-525): query qi of the chunk sits at
// position n_past + qi and attends keys [0, n_past + qi] of its session, read
// through the block table.  The reference runs one warp per (query, head) and
// streams every key once per query; here the work is a dense contraction:
//
//  * Columns.  For one kv head the chunk has n_q*G (query, head) pairs, all
//    needing the same K/V rows.  A wave owns 4 blocks of 16 such columns
//    (col = qi*G + hh), a workgroup 4 waves.  Each K/V operand register a wave
//    loads feeds 4 column blocks.
//  * Tiles of 32 keys (2 pages).  S^T = K . Q^T (v_mfma_f32_16x16x32_f16, rows =
//    16 keys of a page, cols = 16 columns), then O^T += V^T . P^T with the same
//    instruction; S^T's C layout is P^T's B layout (see attn_decode.hip), so
//    the softmax runs per lane with two cross-lane steps per tile.
//  * Q is converted to fp16 once (scaled by 1/sqrt(HD)*log2 e); P is fp16; both
//    accumulate in fp32 (error analysis and the measured error are in the
//    tests).  kSplitQ switches Q to an exact hi+lo split at 1.5x the MFMA work.
//  * Lazy rescaling: a column's running max only moves when a tile's max
//    exceeds it by more than 8 (log2 units), bounding P by 2^8 in fp16, so the
//    O rescale (32 multiplies per column block) is skipped on most tiles.
//  * Causal mask per (key, column); tiles wholly beyond a wave's last query
//    are never visited.  Workgroups are launched heaviest-first.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "check.h"
#include "model.h"
#include "nova_kernel.h"

namespace nova {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int NH = Model::NH, NKV = Model::NKV, HD = Model::HD, G = Model::G, KVW = Model::KVW;
constexpr int WAVES = 4;
constexpr int THREADS = WAVES * 64;
constexpr int CB = 4;                          // 16-column blocks per wave
constexpr int COLS_WAVE = 16 * CB;
constexpr int COLS_WG = COLS_WAVE * WAVES;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;                  // rescale threshold, log2 units
constexpr int64_t kPageHalves = (int64_t)kKvBlock * KVW;
constexpr bool kSplitQ = false;

struct PrefillArgs {
    const float* q;            // [n_sess][n_q][NH][HD]
    const uint16_t* pool_k;
    const uint16_t* pool_v;
    const int32_t* tables;
    int64_t table_stride;
    const int32_t* n_past;     // device [n_sess] or null -> n_past_scalar
    int n_past_scalar;
    int n_q;
    int layer;
    int nb;
    float* o;                  // [n_sess][n_q][NH][HD]
};

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

__global__ void __launch_bounds__(THREADS)
prefill_kernel(PrefillArgs a) {
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int n_cols = a.n_q * G;
    const int n_cg = (n_cols + COLS_WG - 1) / COLS_WG;
    const int cg = n_cg - 1 - (int)blockIdx.x;           // heaviest (latest queries) first
    const int kvh = blockIdx.y;
    const int sess = blockIdx.z;
    const int n_past = a.n_past ? a.n_past[sess] : a.n_past_scalar;
    const int32_t* table = a.tables + (int64_t)sess * a.table_stride;
    const float* qs = a.q + (int64_t)sess * a.n_q * NH * HD;
    float* os = a.o + (int64_t)sess * a.n_q * NH * HD;

    const int col0 = cg * COLS_WG + wave * COLS_WAVE;
    if (col0 >= n_cols) return;
    const int col_last = min(col0 + COLS_WAVE, n_cols) - 1;
    const int key_end = n_past + col_last / G + 1;            // exclusive bound for this wave
    const int key_min_full = n_past + col0 / G + 1;           // keys < this are visible to all columns

    // ---- Q^T operands: lane (g,c) of block b holds column col0 + 16b + c ----
    h8 qhi[CB][4];
    h8 qlo[CB][4];
    int qpos[CB];
#pragma unroll
    for (int b = 0; b < CB; ++b) {
        const int col = col0 + 16 * b + c;
        const bool real = col < n_cols;
        const int qi = real ? col / G : 0;
        const int hh = real ? col - qi * G : 0;
        qpos[b] = real ? n_past + qi : -1;
        const float* qp = qs + ((int64_t)qi * NH + kvh * G + hh) * HD + 8 * g;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = real ? qp[32 * ks + j] * (kScale * kLog2e) : 0.f;
                const _Float16 h = (_Float16)x;
                qhi[b][ks][j] = h;
                qlo[b][ks][j] = (_Float16)(x - (float)h);
            }
    }

    float m[CB], lsum[CB];
    f4 acc[CB][8];
#pragma unroll
    for (int b = 0; b < CB; ++b) {
        m[b] = -INFINITY;
        lsum[b] = 0.f;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[b][cb] = f4{0.f, 0.f, 0.f, 0.f};
    }

    const int64_t layer_base = (int64_t)a.layer * a.nb;
    const int n_tiles = (key_end + 31) >> 5;
    for (int t = 0; t < n_tiles; ++t) {
        const int pg0 = 2 * t;
        const bool two = (pg0 + 1) * kKvBlock < key_end;
        const int pg1 = two ? pg0 + 1 : pg0;
        const int phys0 = __builtin_amdgcn_readfirstlane(table[pg0]);
        const int phys1 = __builtin_amdgcn_readfirstlane(table[pg1]);
        const uint16_t* kb0 = a.pool_k + (layer_base + phys0) * kPageHalves + kvh * HD;
        const uint16_t* kb1 = a.pool_k + (layer_base + phys1) * kPageHalves + kvh * HD;
        const uint16_t* vb0 = a.pool_v + (layer_base + phys0) * kPageHalves + kvh * HD;
        const uint16_t* vb1 = a.pool_v + (layer_base + phys1) * kPageHalves + kvh * HD;
        u4 k0[4], k1[4], vl[8];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            k0[ks] = *reinterpret_cast<const u4*>(kb0 + c * KVW + 32 * ks + 8 * g);
            k1[ks] = *reinterpret_cast<const u4*>(kb1 + c * KVW + 32 * ks + 8 * g);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int slot = 4 * g + (j & 3);
            vl[j] = *reinterpret_cast<const u4*>((j < 4 ? vb0 : vb1) + slot * KVW + 8 * c);
        }
        const int key_base = t * 32;
        const bool full = key_base + 32 <= key_min_full;       // no causal mask in this tile
        // keys that exist at all (the tail of the last page may be unwritten)
        bool kok[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int key = key_base + (j < 4 ? 0 : 16) + 4 * g + (j & 3);
            kok[j] = key < key_end && (j < 4 || two);
            if (!kok[j]) vl[j] = u4{0u, 0u, 0u, 0u};
        }

        h8 va[8];
#pragma unroll
        for (int cb = 0; cb < 8; ++cb)
#pragma unroll
            for (int j = 0; j < 8; ++j) va[cb][j] = __builtin_bit_cast(h8, vl[j])[cb];

#pragma unroll
        for (int b = 0; b < CB; ++b) {
            f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, k0[ks]), qhi[b][ks], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, k1[ks]), qhi[b][ks], s1, 0, 0, 0);
                if constexpr (kSplitQ) {
                    s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, k0[ks]), qlo[b][ks], s0, 0, 0, 0);
                    s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, k1[ks]), qlo[b][ks], s1, 0, 0, 0);
                }
            }
            float s[8];
            bool ok[8];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                s[ii] = s0[ii];
                s[4 + ii] = s1[ii];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = key_base + (j < 4 ? 0 : 16) + 4 * g + (j & 3);
                ok[j] = kok[j] && (full || key <= qpos[b]);
            }
            float bm = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) bm = ok[j] ? fmaxf(bm, s[j]) : bm;
            bm = fmaxf(bm, shfl_xor_f(bm, 16));
            bm = fmaxf(bm, shfl_xor_f(bm, 32));
            const bool need = bm > m[b] + kLazy;
            if (__builtin_amdgcn_ballot_w64(need)) {
                const float mn = need ? bm : m[b];
                const float corr = exp2f(m[b] - mn);
                lsum[b] *= corr;
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) acc[b][cb] *= corr;
                m[b] = mn;
            }
            float ps = 0.f;
            h8 ph;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = ok[j] ? exp2f(s[j] - m[b]) : 0.f;
                const _Float16 hp = (_Float16)p;
                ph[j] = hp;
                ps += (float)hp;       // normalise with the weights actually applied
            }
            lsum[b] += ps;
#pragma unroll
            for (int cb = 0; cb < 8; ++cb)
                acc[b][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[cb], ph, acc[b][cb], 0, 0, 0);
        }
    }

    // ---- normalise and store: lane (g,c) of block b holds d = 8*(4g+i) + cb ----
#pragma unroll
    for (int b = 0; b < CB; ++b) {
        float L = lsum[b];
        L += shfl_xor_f(L, 16);
        L += shfl_xor_f(L, 32);
        const int col = col0 + 16 * b + c;
        if (col >= n_cols) continue;
        const int qi = col / G, hh = col - qi * G;
        float* op = os + ((int64_t)qi * NH + kvh * G + hh) * HD;
        const float inv = 1.f / L;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            f4 lo4, hi4;
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                lo4[cb] = acc[b][cb][ii] * inv;
                hi4[cb] = acc[b][cb + 4][ii] * inv;
            }
            *reinterpret_cast<f4*>(op + 8 * (4 * g + ii)) = lo4;
            *reinterpret_cast<f4*>(op + 8 * (4 * g + ii) + 4) = hi4;
        }
    }
}

void launch(const PrefillArgs& a, int n_sess, hipStream_t s) {
    const int n_cg = (a.n_q * G + COLS_WG - 1) / COLS_WG;
    hipLaunchKernelGGL(prefill_kernel, dim3(n_cg, NKV, n_sess), dim3(THREADS), 0, s, a);
    NOVA_LAUNCHED();
}

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {

void launch_attn_prefill_paged(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                               const int32_t* table, int layer, int nb, int n_q, int n_past, float* o,
                               nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && table && o);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n_q >= 0 && n_past >= 0);
    if (n_q == 0) return;
    PrefillArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = table;
    a.table_stride = 0;
    a.n_past = nullptr;
    a.n_past_scalar = n_past;
    a.n_q = n_q;
    a.layer = layer;
    a.nb = nb;
    a.o = o;
    launch(a, 1, reinterpret_cast<hipStream_t>(s));
}

void launch_attn_prefill_paged_batch(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                                     const int32_t* tables, int table_stride, const int32_t* n_past,
                                     int n_sess, int n_q, int layer, int nb, float* o, nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && tables && n_past && o);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n_q >= 0 && n_sess >= 1 && n_sess <= 65535);
    NOVA_REQUIRE(table_stride > 0);
    if (n_q == 0) return;
    PrefillArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = tables;
    a.table_stride = table_stride;
    a.n_past = n_past;
    a.n_q = n_q;
    a.layer = layer;
    a.nb = nb;
    a.o = o;
    launch(a, n_sess, reinterpret_cast<hipStream_t>(s));
}

}  // extern "C"
