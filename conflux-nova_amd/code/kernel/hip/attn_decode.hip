// attn_decode.hip -- paged split-K flash-decode for gfx950 (MI355X).
//
// Computes what fa_split_paged_kernel + fa_combine_kernel compute
// (reference src/kernel/attn.cu:163-289, launcher :498-512): for every query head
// h of a session, softmax(q_h . K^T * 1/sqrt(HD)) . V over keys [0, n_keys),
// gathering K/V through the session's block table.  The arithmetic is laid out
// for CDNA4 instead of the reference's one-warp-per-head scan:
//
//  * Work split (stream-K).  The pages of all sessions of a layer form one list
//    of T pages; workgroup w owns pages [w*T/Gw, (w+1)*T/Gw).  Every workgroup
//    does the same number of pages whatever the context lengths, so a ragged
//    batch fills all CUs evenly.  A range that crosses a session boundary
//    yields one partial (m, l, acc[HD]) per session touched.
//  * One workgroup = 8 wave64s.  Wave w serves kv head w % NKV and takes every
//    R-th pair of pages (R = 8/NKV), so the workgroup reads whole 16-token pages
//    (all kv heads) and each wave streams 256 B rows of its head.
//  * GQA on the matrix cores.  For a pair of pages (32 keys) a wave forms
//    S = K . Q^T with v_mfma_f32_16x16x32_f16 (rows = 16 keys of a page, cols =
//    the G query heads of its kv head padded to 16) and O^T += V^T . P^T with the
//    same instruction (rows = 16 head-dim columns, k = the 32 keys).  The C
//    layout of S (lane (g,c) holds keys 4g..4g+3 of head c) is exactly the B
//    layout P^T needs, so no cross-lane shuffles sit between the two products,
//    and the V operand is read as 16 B per lane straight from 256 B rows.
//  * fp32-grade accuracy from fp16 operands.  K and V are fp16 in the pool (exact
//    MFMA inputs).  Q (fp32) is split q = hi + lo into two fp16 terms after a
//    per-head power-of-two scaling, P (fp32 softmax weights) likewise; each
//    product is two MFMAs accumulating in fp32, leaving ~2^-22 relative error
//    per operand instead of fp16's 2^-11.
//  * Online softmax in the log2 domain (exp2f), scale*log2(e) folded into the
//    per-head factor.  Split partials merge with the reference's combine rule
//    (max, then l- and acc-weighted sums; rows with l == 0 are skipped).
//  * Merge: the batched entry point merges in the last workgroup to finish a
//    session (device-scope counter, self-resetting); the single-session entry
//    point keeps the reference's scratch contract and uses a combine kernel.
//  * Fused append: the batched entry point can take the layer's new token; the
//    workgroup that owns the session's last page writes it to the pool and
//    every lane that needs that row reads it from the input buffer instead, so
//    no lane ever reads the slot being written.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <mutex>

#include "check.h"
#include "model.h"
#include "nova_kernel.h"

namespace nova {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int NH = Model::NH, NKV = Model::NKV, HD = Model::HD, G = Model::G, KVW = Model::KVW;
constexpr int WAVES = 8;
constexpr int THREADS = WAVES * 64;
constexpr int R = WAVES / NKV;           // waves per kv head
static_assert(WAVES % NKV == 0, "kv heads must divide the 8 waves of a workgroup");
constexpr int PW = HD + 2;               // partial row: m, l, acc[HD]
constexpr int kMaxBatch = 1024;          // sessions per batched launch
constexpr float kLog2e = 1.4426950408889634f;
constexpr int64_t kPageHalves = (int64_t)kKvBlock * KVW;

struct DecodeArgs {
    const float* q;          // [n_sess][NH][HD]
    const uint16_t* pool_k;
    const uint16_t* pool_v;
    uint16_t* wpool_k;       // append targets (== pool_k/pool_v) or null
    uint16_t* wpool_v;
    const int32_t* tables;
    int64_t table_stride;
    const int32_t* n_keys;   // device [n_sess] or null -> n_keys_scalar
    int n_keys_scalar;
    int n_sess;
    int layer;
    int nb;
    const uint16_t* k_new;   // [n_sess][NKV][HD] or null
    const uint16_t* v_new;
    float* o;                // [n_sess][NH][HD]
    float* part;             // [(Gw + n_sess)][NH][PW]
    int* counters;           // [n_sess], zero between launches
    int gw;                  // workgroups in the grid
};

__device__ __forceinline__ int owner_of(int64_t page, int64_t T, int gw) {
    // largest w with floor(w*T/gw) <= page
    return (int)(((page + 1) * gw - 1) / T);
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

template <bool kInlineMerge>
__global__ void __launch_bounds__(THREADS)
decode_kernel(DecodeArgs a) {
    __shared__ int s_cu[kMaxBatch + 1];
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ float s_acc[WAVES][G][HD];
    __shared__ int s_flag;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;      // 0..3
    const int c = lane & 15;      // 0..15
    const int kvh = wave % NKV;
    const int r = wave / NKV;
    const int w = blockIdx.x;

    // ---- page prefix over sessions (cu[i] = first page of session i) ----
    const int ns = a.n_sess;
    if (wave == 0) {
        int carry = 0;
        for (int base = 0; base < ns; base += 64) {
            const int i = base + lane;
            int nk = 0;
            if (i < ns) nk = a.n_keys ? a.n_keys[i] : a.n_keys_scalar;
            int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
            int incl = pg;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            if (i < ns) s_cu[i + 1] = carry + incl;
            carry += __shfl(incl, 63, 64);
        }
        if (lane == 0) s_cu[0] = 0;
    }
    __syncthreads();
    const int64_t T = s_cu[ns];

    if (kInlineMerge && w == 0) {
        // sessions without keys produce a zero row (fa_combine: l == 0 -> 0)
        for (int i = 0; i < ns; ++i)
            if (s_cu[i + 1] == s_cu[i])
                for (int idx = tid; idx < NH * HD; idx += THREADS) a.o[(int64_t)i * NH * HD + idx] = 0.f;
    }
    if (T == 0) return;
    // with fewer pages than workgroups, only the first T workgroups take work,
    // so every participating range is non-empty and owner_of counts arrivals
    const int gw = a.gw < T ? a.gw : (int)T;
    if (w >= gw) return;
    int64_t lo = (int64_t)w * T / gw;
    const int64_t hi = (int64_t)(w + 1) * T / gw;

    // first session whose pages reach past lo
    int i = 0;
    while (s_cu[i + 1] <= lo) ++i;

    while (lo < hi) {
        const int64_t seg_hi = hi < (int64_t)s_cu[i + 1] ? hi : (int64_t)s_cu[i + 1];
        const int pa = (int)(lo - s_cu[i]);              // session-local pages [pa, pb)
        const int pb = (int)(seg_hi - s_cu[i]);
        const int n_keys = a.n_keys ? a.n_keys[i] : a.n_keys_scalar;
        const int last_page = (n_keys - 1) >> kKvBlockShift;
        const int new_slot = (n_keys - 1) & kKvBlockMask;
        const bool has_new = a.k_new != nullptr;
        const int32_t* table = a.tables + (int64_t)i * a.table_stride;

        // fused append: the owner of the session's last page stores the new token
        if (has_new && pb == last_page + 1 && a.wpool_k) {
            const int phys = table[last_page];
            const int64_t dst = ((int64_t)a.layer * a.nb + phys) * kPageHalves + (int64_t)new_slot * KVW;
            const int64_t src = (int64_t)i * KVW;
            for (int e = tid; e < KVW / 8; e += THREADS) {
                *reinterpret_cast<u4*>(a.wpool_k + dst + 8 * e) =
                    *reinterpret_cast<const u4*>(a.k_new + src + 8 * e);
                *reinterpret_cast<u4*>(a.wpool_v + dst + 8 * e) =
                    *reinterpret_cast<const u4*>(a.v_new + src + 8 * e);
            }
        }

        // ---- this wave's query group as split fp16 B operands ----
        // lane (g,c): head kvh*G + c, dims d = 32*ks + 8*g + j
        h8 qhi[4], qlo[4];
        float qf;
        {
            float qv[4][8];
            float amax = 0.f;
            const bool real = c < G;
            const float* qp = a.q + ((int64_t)i * NH + kvh * G + (real ? c : 0)) * HD + 8 * g;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = real ? qp[32 * ks + j] : 0.f;
                    qv[ks][j] = x;
                    amax = fmaxf(amax, fabsf(x));
                }
            amax = fmaxf(amax, shfl_xor_f(amax, 16));
            amax = fmaxf(amax, shfl_xor_f(amax, 32));
            int ex = 0;
            if (amax > 0.f) (void)frexpf(amax, &ex);
            const int k2 = amax > 0.f ? 15 - ex : 0;    // amax * 2^k2 in [2^14, 2^15)
            const float up = ldexpf(1.f, k2);
            qf = kScale * kLog2e * ldexpf(1.f, -k2);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = qv[ks][j] * up;
                    const _Float16 h = (_Float16)x;
                    qhi[ks][j] = h;
                    qlo[ks][j] = (_Float16)(x - (float)h);
                }
        }

        float m = -INFINITY, lsum = 0.f;
        f4 acc[8];
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[cb] = f4{0.f, 0.f, 0.f, 0.f};

        const int npairs = (pb - pa + 1) >> 1;
        const int64_t layer_base = (int64_t)a.layer * a.nb;
        const uint16_t* knew_row = has_new ? a.k_new + (int64_t)i * KVW + kvh * HD : nullptr;
        const uint16_t* vnew_row = has_new ? a.v_new + (int64_t)i * KVW + kvh * HD : nullptr;

        for (int qp = r; qp < npairs; qp += R) {
            const int pg0 = pa + 2 * qp;
            const bool two = pg0 + 1 < pb;
            const int pg1 = two ? pg0 + 1 : pg0;
            const int phys0 = __builtin_amdgcn_readfirstlane(table[pg0]);
            const int phys1 = __builtin_amdgcn_readfirstlane(table[pg1]);
            const uint16_t* kb0 = a.pool_k + (layer_base + phys0) * kPageHalves + kvh * HD;
            const uint16_t* kb1 = a.pool_k + (layer_base + phys1) * kPageHalves + kvh * HD;
            const uint16_t* vb0 = a.pool_v + (layer_base + phys0) * kPageHalves + kvh * HD;
            const uint16_t* vb1 = a.pool_v + (layer_base + phys1) * kPageHalves + kvh * HD;

            // K operand: row c of each page, halves [32ks + 8g, +8)
            const uint16_t* kr0 = (has_new && pg0 == last_page && c == new_slot) ? knew_row : kb0 + c * KVW;
            const uint16_t* kr1 = (has_new && pg1 == last_page && c == new_slot) ? knew_row : kb1 + c * KVW;
            u4 k0[4], k1[4];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                k0[ks] = *reinterpret_cast<const u4*>(kr0 + 32 * ks + 8 * g);
                k1[ks] = *reinterpret_cast<const u4*>(kr1 + 32 * ks + 8 * g);
            }
            // V operand: rows kappa(g,j) = page j/4, slot 4g + j%4; halves [8c, 8c+8)
            u4 vl[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int slot = 4 * g + (j & 3);
                const int pg = j < 4 ? pg0 : pg1;
                const uint16_t* vb = j < 4 ? vb0 : vb1;
                const uint16_t* vr = (has_new && pg == last_page && slot == new_slot) ? vnew_row : vb + slot * KVW;
                vl[j] = *reinterpret_cast<const u4*>(vr + 8 * c);
            }

            // S = K . Q^T  (C layout: lane (g,c) holds keys 4g+i of head c)
            f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const h8 ka = __builtin_bit_cast(h8, k0[ks]);
                const h8 kc = __builtin_bit_cast(h8, k1[ks]);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi[ks], s0, 0, 0, 0);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo[ks], s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, qhi[ks], s1, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, qlo[ks], s1, 0, 0, 0);
            }

            // mask keys >= n_keys and the missing second page
            float s[8];
            bool ok[8];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                const int key0 = (pg0 << kKvBlockShift) + 4 * g + ii;
                const int key1 = (pg1 << kKvBlockShift) + 4 * g + ii;
                ok[ii] = key0 < n_keys;
                ok[4 + ii] = two && key1 < n_keys;
                s[ii] = s0[ii] * qf;
                s[4 + ii] = s1[ii] * qf;
            }
            float bm = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) bm = ok[j] ? fmaxf(bm, s[j]) : bm;
            bm = fmaxf(bm, shfl_xor_f(bm, 16));
            bm = fmaxf(bm, shfl_xor_f(bm, 32));
            const float mn = fmaxf(m, bm);
            const float corr = exp2f(m - mn);
            float p[8];
            float ps = 0.f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                p[j] = ok[j] ? exp2f(s[j] - mn) : 0.f;
                ps += p[j];
            }
            lsum = fmaf(lsum, corr, ps);
            m = mn;
            h8 phi, plo;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const _Float16 h = (_Float16)p[j];
                phi[j] = h;
                plo[j] = (_Float16)(p[j] - (float)h);
            }
            // masked V rows are zeroed so garbage (NaN/Inf) in unused slots cannot leak
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (!ok[j]) vl[j] = u4{0u, 0u, 0u, 0u};

            // O^T += V^T . P^T   (A: lane (g,c) holds V[kappa(g,j)][8c + cb], j = 0..7)
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                h8 va;
#pragma unroll
                for (int j = 0; j < 8; ++j) va[j] = __builtin_bit_cast(h8, vl[j])[cb];
                acc[cb] *= corr;
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, phi, acc[cb], 0, 0, 0);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, plo, acc[cb], 0, 0, 0);
            }
        }

        // ---- merge the R waves of each kv head in LDS ----
        lsum += shfl_xor_f(lsum, 16);
        lsum += shfl_xor_f(lsum, 32);
        if (g == 0) {
            s_m[wave][c] = m;
            s_l[wave][c] = lsum;
        }
        if (c < G) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii)
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) s_acc[wave][c][8 * (4 * g + ii) + cb] = acc[cb][ii];
        }
        __syncthreads();

        // partial slot of (workgroup w, session i): unique because the segment
        // path is monotone in both w and i
        float* pout = a.part + (int64_t)(w + i) * NH * PW;
        for (int idx = tid; idx < NH * HD; idx += THREADS) {
            const int h = idx / HD, d = idx - h * HD;
            const int hk = h / G, hc = h - hk * G;
            float M = -INFINITY;
#pragma unroll
            for (int rr = 0; rr < R; ++rr) M = fmaxf(M, s_m[hk + NKV * rr][hc]);
            float L = 0.f, A = 0.f;
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int ww = hk + NKV * rr;
                const float lw = s_l[ww][hc];
                const float f = lw > 0.f ? exp2f(s_m[ww][hc] - M) : 0.f;
                L = fmaf(lw, f, L);
                A = fmaf(s_acc[ww][hc][d], f, A);
            }
            pout[(int64_t)h * PW + 2 + d] = A;
            if (d == 0) {
                pout[(int64_t)h * PW] = M;
                pout[(int64_t)h * PW + 1] = L;
            }
        }

        if constexpr (kInlineMerge) {
            const int w_first = owner_of(s_cu[i], T, gw);
            const int w_last = owner_of((int64_t)s_cu[i + 1] - 1, T, gw);
            const int nseg = w_last - w_first + 1;
            __threadfence();
            __syncthreads();
            if (tid == 0) {
                const int old = atomicAdd(a.counters + i, 1);
                s_flag = (old == nseg - 1);
            }
            __syncthreads();
            if (s_flag) {
                __threadfence();
                float* orow = a.o + (int64_t)i * NH * HD;
                for (int idx = tid; idx < NH * HD; idx += THREADS) {
                    const int h = idx / HD, d = idx - h * HD;
                    float M = -INFINITY;
                    for (int ww = w_first; ww <= w_last; ++ww)
                        M = fmaxf(M, __builtin_nontemporal_load(a.part + ((int64_t)(ww + i) * NH + h) * PW));
                    float L = 0.f, A = 0.f;
                    for (int ww = w_first; ww <= w_last; ++ww) {
                        const float* pr = a.part + ((int64_t)(ww + i) * NH + h) * PW;
                        const float ls = __builtin_nontemporal_load(pr + 1);
                        const float f = ls > 0.f ? exp2f(__builtin_nontemporal_load(pr) - M) : 0.f;
                        L = fmaf(ls, f, L);
                        A = fmaf(__builtin_nontemporal_load(pr + 2 + d), f, A);
                    }
                    orow[idx] = L > 0.f ? A / L : 0.f;
                }
                if (tid == 0) a.counters[i] = 0;
            }
        }
        __syncthreads();   // LDS reuse by the next segment
        lo = seg_hi;
        ++i;
        while (i < ns && s_cu[i + 1] == s_cu[i]) ++i;   // skip empty sessions
    }
}

// Combine for the single-session entry point: nsplit partial rows per head ->
// O[h][d] (fa_combine_kernel, attn.cu:163-191), partials in the log2 domain.
__global__ void __launch_bounds__(HD) combine_kernel(const float* __restrict__ part, float* __restrict__ o,
                                                     int nsplit) {
    const int h = blockIdx.x, d = threadIdx.x;
    float M = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, part[((int64_t)sp * NH + h) * PW]);
    float L = 0.f, A = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
        const float* pr = part + ((int64_t)sp * NH + h) * PW;
        const float f = pr[1] > 0.f ? exp2f(pr[0] - M) : 0.f;
        L = fmaf(pr[1], f, L);
        A = fmaf(pr[2 + d], f, A);
    }
    o[h * HD + d] = L > 0.f ? A / L : 0.f;
}

int batch_workgroups() {
    static int gw = 0;
    static std::once_flag once;
    std::call_once(once, [] {
        int per_cu = 2;
        if (const char* e = std::getenv("NOVA_DECODE_WG_PER_CU")) per_cu = std::atoi(e);
        if (per_cu < 1) per_cu = 1;
        int dev = 0, cus = 0;
        NOVA_HIP(hipGetDevice(&dev));
        NOVA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        gw = cus * per_cu;
    });
    return gw;
}

size_t counters_bytes(int n_sess) { return ((size_t)n_sess * 4 + 255) / 256 * 256; }

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {

size_t attn_decode_batch_workspace_bytes(int n_sess) {
    NOVA_REQUIRE(n_sess >= 1 && n_sess <= kMaxBatch);
    return counters_bytes(n_sess) + (size_t)(batch_workgroups() + n_sess) * NH * PW * sizeof(float);
}

void launch_attn_decode_paged_batch(const float* q, uint16_t* pool_k, uint16_t* pool_v,
                                    const int32_t* tables, int table_stride, const int32_t* n_keys,
                                    int n_sess, int layer, int nb, const uint16_t* k_new,
                                    const uint16_t* v_new, float* o, void* workspace, nova_stream_t s) {
    NOVA_REQUIRE(n_sess >= 1 && n_sess <= kMaxBatch);
    NOVA_REQUIRE(q && pool_k && pool_v && tables && n_keys && o && workspace);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && table_stride > 0);
    NOVA_REQUIRE((k_new == nullptr) == (v_new == nullptr));
    DecodeArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.wpool_k = pool_k;
    a.wpool_v = pool_v;
    a.tables = tables;
    a.table_stride = table_stride;
    a.n_keys = n_keys;
    a.n_sess = n_sess;
    a.layer = layer;
    a.nb = nb;
    a.k_new = k_new;
    a.v_new = v_new;
    a.o = o;
    a.counters = static_cast<int*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + counters_bytes(n_sess));
    a.gw = batch_workgroups();
    hipLaunchKernelGGL(decode_kernel<true>, dim3(a.gw), dim3(THREADS), 0,
                       reinterpret_cast<hipStream_t>(s), a);
    NOVA_LAUNCHED();
}

void launch_attn_decode_paged(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                              const int32_t* table, int layer, int nb, int n_keys, float* o,
                              float* scratch, nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && table && o && scratch);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n_keys >= 1);
    const int pages = (n_keys + kKvBlock - 1) >> kKvBlockShift;
    // scratch holds NH*32*(HD+2) floats (reference contract): at most 32 splits
    int gw = pages / 2;
    if (gw > kMaxSplit) gw = kMaxSplit;
    if (gw < 1) gw = 1;
    DecodeArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = table;
    a.table_stride = 1;
    a.n_keys = nullptr;
    a.n_keys_scalar = n_keys;
    a.n_sess = 1;
    a.layer = layer;
    a.nb = nb;
    a.o = o;
    a.part = scratch;
    a.gw = gw;
    hipStream_t st = reinterpret_cast<hipStream_t>(s);
    hipLaunchKernelGGL(decode_kernel<false>, dim3(gw), dim3(THREADS), 0, st, a);
    NOVA_LAUNCHED();
    hipLaunchKernelGGL(combine_kernel, dim3(NH), dim3(HD), 0, st, scratch, o, gw);
    NOVA_LAUNCHED();
}

}  // extern "C"
