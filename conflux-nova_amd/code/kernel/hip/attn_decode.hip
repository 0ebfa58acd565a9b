// attn_decode.hip -- paged split-K flash-decode for gfx950 (MI355X).
//
// Computes what fa_split_paged_kernel + fa_combine_kernel compute
// (reference src/kernel/attn.cu:163-289, launcher :498-512): for every query head
// h of a session, softmax(q_h . K^T * 1/sqrt(HD)) . V over keys [0, n_keys),
// gathering K/V through the session's block table.  The arithmetic is laid out
// for CDNA4 instead of the reference's one-warp-per-head scan:
//
//  * Work split (session-aligned, balanced).  With T pages in the batch and Gw
//    target workgroups, session i (P_i pages) gets k_i = ceil(P_i / ceil(T/Gw))
//    workgroups (the share is at least 4 pages, and raised until the
//    workgroups fit in Gw), each owning a contiguous page range of that
//    session.  Every workgroup does at most that share whatever
//    the context lengths, so
//    a ragged batch fills all CUs evenly, and a workgroup never straddles two
//    sessions.  In the batched path a workgroup writes one partial
//    (m, l, acc[HD]) per head: with two waves per kv head (7B) the two merge
//    through LDS first, each keeping half of the head dims and signalling the
//    other with an LDS flag rather than a workgroup barrier; with four (1.5B)
//    each wave row writes its own slot (the four-way exchange costs more than
//    the bytes it saves).  The reference-signature path writes one partial per
//    head and page range (its scratch holds 32 rows per head; there each page
//    range runs as NKV workgroups, one per kv head, so one single-session call
//    spreads over 31 * NKV CUs).
//    Every wave derives the partition itself from one load of n_keys.
//  * One workgroup = 8 wave64s, one workgroup per CU.  Wave w serves kv head
//    w % NKV and takes every R-th pair of pages (R = 8/NKV), so the workgroup
//    reads whole 16-token pages (all kv heads) and each wave streams 256 B rows
//    of its head; the CU keeps 8 pairs (128 KiB) of K/V outstanding.  The
//    query operands live once per kv head in LDS.
//  * Latency hiding inside a wave: the segment's block-table slice is fetched
//    once (one coalesced load, then v_readlane per page), so no pair waits on
//    a table lookup.  Every wave issues its loads in one fixed order -- the
//    appended token's page and row, the query rows (and the RoPE rows), then
//    its first pair -- so that the vector-memory counter, which drains in
//    issue order, lets the query conversion and the append wait only for what
//    they use, not for the pair.
//    Page bases are wave-uniform (SGPR) and lane
//    offsets are fixed 32-bit values, so the loop does no per-lane 64-bit
//    address arithmetic.
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
//    per operand instead of fp16's 2^-11.  The matrix cores have the slack:
//    the kernel is bound by HBM, not by MFMA issue.
//  * Online softmax in the log2 domain (raw v_exp_f32), scale*log2(e) folded
//    into the per-head factor, with a lazy running max: it moves only when a
//    score exceeds it by more than 8, so most pairs skip the cross-lane max
//    and the accumulator rescale.  Split partials merge with the reference's combine rule
//    (max, then l- and acc-weighted sums; rows with l == 0 are skipped) in a
//    second, small kernel: the kernel boundary publishes the partials, so no
//    workgroup pays for a device-scope fence (an L2 writeback on this part).
//  * Fused append: the batched entry point can take the layer's new token; the
//    workgroup that owns the session's last page stores it into the pool and
//    publishes it to its own waves with a workgroup barrier before any wave
//    reads that page; no other workgroup reads that page.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "check.h"
#include "model.h"
#include "nova_kernel.h"
#ifdef NOVA_TESTKIT
#include "nova_testkit.h"
#endif
#include "rope_math.h"

namespace nova {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int NH = Model::NH, NKV = Model::NKV, HD = Model::HD, G = Model::G, KVW = Model::KVW;
#ifndef NOVA_DECODE_WAVES
#define NOVA_DECODE_WAVES 8
#endif
constexpr int WAVES = NOVA_DECODE_WAVES;
constexpr int THREADS = WAVES * 64;
constexpr int R = WAVES / NKV;           // waves per kv head
static_assert(WAVES % NKV == 0, "kv heads must divide the waves of a workgroup");
constexpr int PW = HD + 2;               // partial row of the reference-signature scratch: m, l, acc[HD]
#ifndef NOVA_DECODE_PWB
#define NOVA_DECODE_PWB (HD + 4)
#endif
constexpr int PWB = NOVA_DECODE_PWB;     // batched workspace row: m, l, pad, pad, acc[HD] (16-byte aligned acc)
constexpr int kMaxBatch = 1024;          // sessions per batched launch
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;            // running-max slack, log2 units (weights <= 2^8)
constexpr int64_t kPageBytes = (int64_t)kKvBlock * KVW * 2;
constexpr int kRowBytes = KVW * 2;

struct DecodeArgs {
    const float* q;          // [n_sess][NH][HD]
    const uint16_t* pool_k;
    const uint16_t* pool_v;
    const int32_t* tables;
    int64_t table_stride;
    const int32_t* n_keys;   // device [n_sess] or null -> n_keys_scalar
    int n_keys_scalar;
    int n_sess;
    int layer;
    int nb;
    const uint16_t* k_new;   // [n_sess][NKV][HD] or null
    const uint16_t* v_new;
    const float* k_new32;    // fused RoPE: new token fp32 [n_sess][NKV][HD], rotated here
    const float* v_new32;
    const float* cs;         // RoPE table rows [pos][HD/2] (null: no rotation)
    const float* sn;
    float* part;             // [(Gw + n_sess) * (wave_parts ? R : 1)][NH][PW]
    const int32_t* plan;     // per-step plan (null: derive the partition in-kernel)
    int gw;                  // workgroups in the grid
    int wave_parts;          // 1: a partial slot per (workgroup, wave row), no in-workgroup merge
    int kv_split;            // 1: grid.x = kv head, all waves of a workgroup on that head
    float* o;                // solo launches: the output [n_sess][NH][HD], written by the split kernel
    int tab_read;            // solo launches: block-table entries of a row that may be read before n_keys is known
    int spin;                // polls of the in-workgroup exchange before it gives up (kSpinLimit)
    int pw;                  // floats per partial row: {m, l, [pad,] acc[HD]}
    int po;                  // offset of acc[0] in a row (2, or 4: 16-byte aligned acc)
    int32_t* status;         // batched path: the plan's status word (null: none)
};

// Bound of the LDS-flag wait in the one-slot partial exchange.  The partner
// wave of a kv head always arrives (every wave of the workgroup reaches the
// exchange), so the bound only guards against a hang; if it ever runs out,
// the keeper sets kStatusExchange in the plan's status word and writes NaN
// into its partial row, so the affected heads come out NaN, never silently
// wrong.
constexpr int kSpinLimit = 1 << 22;
constexpr int32_t kStatusExchange = 1;

// Per-step plan, written once per decode step by decode_plan_kernel (n_keys
// and block tables are the same for every layer of a step):
//   session table: n_sess x {kc, k, n_keys, pages}
//   one record per workgroup slot: {phys[64], sess, pa, pb, n_keys}
// so a layer's split kernel starts with one load instead of a dependent
// n_keys -> partition -> block-table chain.
constexpr int kRecPages = 64;
constexpr int kRec = kRecPages + 8;            // phys[64], {sess, pa, pb, n_keys, partial slot, 0, 0, 0}
// Workgroup slots and XCDs.  Workgroup w runs on XCD w % 8.  The first
// 8 * ceil(gw / 8) slots take the workgroups' logical indices XCD by XCD:
// with S = sum k_i workgroups in the step and per = ceil(S / 8), slot w holds
// logical L = (w % 8) * per + w / 8 (none if w / 8 >= per), so a session's
// workgroups, which are consecutive logical indices, share one or two XCDs
// and their partial rows stay in those XCDs' L2 for the combine, while a
// small step still spreads over all 8 XCDs.  Slots past 8 ceil(gw / 8) map to
// themselves (only used when the sessions outnumber what one round of gw
// workgroups can split).
__host__ __device__ constexpr int xcd_per(int gw) { return (gw + 7) / 8; }
__host__ __device__ constexpr int split_slots(int n_sess, int gw) { return 8 * xcd_per(gw) + n_sess; }
__host__ __device__ __forceinline__ int xcd_stride(int sumk, int gw) {
    const int per = (sumk + 7) / 8;
    return per < 1 ? 1 : per < xcd_per(gw) ? per : xcd_per(gw);
}
__host__ __device__ __forceinline__ int logical_of(int w, int stride, int gw) {
    if (w >= 8 * xcd_per(gw)) return w;
    return (w >> 3) < stride ? (w & 7) * stride + (w >> 3) : -1;
}
// plan: [session table n_sess x 4 | combine map n_sess*NH x {kc, k, sess | head << 16, pages} | records]
__host__ __device__ constexpr int64_t plan_map_off(int n_sess) { return (int64_t)n_sess * 4; }
__host__ __device__ constexpr int64_t plan_rec_off(int n_sess) { return (int64_t)n_sess * 4 + (int64_t)n_sess * NH * 4; }
// one status word after the records: cleared by every plan launch, OR-ed
// with kStatus* by the kernels of the step's layers
__host__ __device__ constexpr int64_t plan_status_off(int n_sess, int gw) {
    return plan_rec_off(n_sess) + (int64_t)split_slots(n_sess, gw) * kRec;
}
__host__ __device__ constexpr int64_t plan_ints(int n_sess, int gw) { return plan_status_off(n_sess, gw) + 1; }

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }

// K/V page loads go out non-temporal: each byte is read once per launch, and
// every load instruction covers whole 128 B lines (V: 256 B row slices; K:
// 8 rows x 128 B, see k_operand).  Measured: page-sized non-temporal
// streaming reaches 6.9 TB/s against 6.1 TB/s with the default policy; V
// non-temporal took the config-2 step 0.905 -> 0.875 ms, K with whole-line
// loads 0.834-0.841 -> 0.826 ms (config 4: 6.21 -> 6.37-6.55 TB/s).  K
// loaded the MFMA's way (64 B of 16 rows per instruction, the other half of
// each line by the next one) is slower non-temporal: 0.97 ms.
// Each page is a buffer resource: the loads take the page base in SGPRs and a
// 32-bit lane offset with an immediate, instead of a 64-bit VGPR address per
// load (the double-buffered solo loop: 254 -> 217 VGPRs, and its prefetch no
// longer waits on address registers still being loaded).  num_records bounds
// every load to its page; num_records = 0 makes a load return zero without a
// memory access (a prefetch slot with no pair left).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t page_rsrc(const char* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ u4 ldb16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));   // aux 2: nt
}

// Pages per workgroup: the even share ceil(T / gw), but at least kMinShare so
// that small batches do not spread one or two pages per workgroup (each extra
// workgroup costs a partial row and a combine term).  4 pages = one pair per
// wave row: measured on config 1 (one session, 65 pages) 0.287 -> 0.275 ms per
// step against 8; batches of 2048 pages and more are not affected.
constexpr int kMinShare = 4;
__host__ __device__ __forceinline__ int share_of(int T, int gw) {
    const int even = (T + gw - 1) / gw;
    return even > kMinShare ? even : kMinShare;
}

// Page range of workgroup j of a session with `pages` pages split over k
// workgroups: [j*pages/k, (j+1)*pages/k).  The plan kernel, the in-kernel
// partition and the combine's row count all take it from here, so a range
// never exceeds range_max_pages(pages, k).
__host__ __device__ __forceinline__ int range_begin(int j, int pages, int k) {
    return (int)((int64_t)j * pages / k);
}
__host__ __device__ __forceinline__ int range_max_pages(int pages, int k) { return (pages + k - 1) / k; }

// The batch partition, derived by one wave from n_keys (every wave that needs
// it computes it; no LDS, no barrier).  P_i = pages of session i, T = sum P_i,
// target = max(ceil(T / gw), 4), k_i = ceil(P_i / target) workgroups for session i,
// kc_i = k_0 + ... + k_{i-1} its first workgroup (= its first partial slot).
// Sum k_i <= gw + n_sess, so the grid launches gw + n_sess workgroups.
struct Part {
    int sess;      // session of this workgroup, -1 if the workgroup is idle
    int n_keys;    // keys of that session
    int pages;     // P_i
    int k;         // k_i
    int kc;        // kc_i
};

__device__ __forceinline__ int nkeys_of(const DecodeArgs& a, int i) {
    return a.n_keys ? a.n_keys[i] : a.n_keys_scalar;
}

// Pages per workgroup for the batch: the even share, raised until the
// sessions' workgroups (sum of ceil(P_i / share)) fit in gw, i.e. in one
// round of one workgroup per CU (a second round would start after the first
// has streamed its pages).  Bounded: with more sessions than gw no share fits
// and the loop gives up.  Wave-uniform; one wave's lanes take 64 sessions at
// a time.
__device__ int plan_share(const DecodeArgs& a, int T) {
    const int lane = threadIdx.x & 63;
    int target = share_of(T, a.gw);
    for (int it = 0; it < 64; ++it) {
        int sumk = 0;
        for (int base = 0; base < a.n_sess; base += 64) {
            const int i = base + lane;
            const int nk = i < a.n_sess ? nkeys_of(a, i) : 0;
            const int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
            int k = (pg + target - 1) / target;
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) k += __shfl_xor(k, o, 64);
            sumk += k;
        }
        if (sumk <= a.gw) break;
        ++target;
    }
    return target;
}

// Find the session that owns workgroup slot w (find_slot) or the partition
// entry of session `want` (want >= 0).
__device__ Part partition(const DecodeArgs& a, int w, int want) {
    const int lane = threadIdx.x & 63;
    int T = 0;
    for (int base = 0; base < a.n_sess; base += 64) {
        const int i = base + lane;
        const int nk = i < a.n_sess ? nkeys_of(a, i) : 0;
        int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) pg += __shfl_xor(pg, o, 64);
        T += pg;
    }
    Part r{-1, 0, 0, 0, 0};
    if (T == 0) return r;
    const int target = plan_share(a, T);
    int carry = 0;
    for (int base = 0; base < a.n_sess; base += 64) {
        const int i = base + lane;
        const int nk = i < a.n_sess ? nkeys_of(a, i) : 0;
        const int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
        const int k = (pg + target - 1) / target;
        int incl = k;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_up(incl, o, 64);
            if (lane >= o) incl += t;
        }
        const int kc = carry + incl - k;
        const bool hit = want >= 0 ? (i == want) : (i < a.n_sess && k > 0 && kc <= w && w < kc + k);
        const uint64_t b = __builtin_amdgcn_ballot_w64(hit);
        if (b) {
            const int src = __builtin_ctzll(b);
            r.sess = base + src;
            r.n_keys = __shfl(nk, src, 64);
            r.pages = __shfl(pg, src, 64);
            r.k = __shfl(k, src, 64);
            r.kc = __shfl(kc, src, 64);
            return r;
        }
        carry += __shfl(incl, 63, 64);
    }
    return r;
}

// Workgroups of the batch, sum of k_i (one wave).
__device__ int sum_k(const DecodeArgs& a) {
    const int lane = threadIdx.x & 63;
    int T = 0;
    for (int base = 0; base < a.n_sess; base += 64) {
        const int i = base + lane;
        const int nk = i < a.n_sess ? nkeys_of(a, i) : 0;
        int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) pg += __shfl_xor(pg, o, 64);
        T += pg;
    }
    if (T == 0) return 0;
    const int target = plan_share(a, T);
    int sumk = 0;
    for (int base = 0; base < a.n_sess; base += 64) {
        const int i = base + lane;
        const int nk = i < a.n_sess ? nkeys_of(a, i) : 0;
        const int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
        int k = (pg + target - 1) / target;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) k += __shfl_xor(k, o, 64);
        sumk += k;
    }
    return sumk;
}

// K and V operands of one pair of pages, as loaded
struct PairRegs {
    u4 k0[4], k1[4];   // K of page 0 / page 1 as whole-line loads (k_operand)
    u4 v[8];           // V rows kappa(g,j) = (page j/4, slot 4g + j%4), halves [8c, +8)
};

// K operand ks of one page from the whole-line loads.  Load 2h+0 (X) holds,
// in lane (g,c), row c&7 at bytes 128h + 16(g + 4(c>>3)); load 2h+1 (Y) the
// same for rows 8 + (c&7).  The MFMA wants row c at bytes 64ks + 16g: for
// even ks that is X in lanes c < 8 and Y of lane c-8 in lanes c >= 8; for odd
// ks, X of lane c+8 in lanes c < 8 and Y in lanes c >= 8.  A row_ror:8 DPP
// move writing only the banks (4-lane groups) of the lanes that need it
// builds each operand dword in one instruction.
__device__ __forceinline__ u4 k_operand(const u4* kl, int ks) {
    const u4 x = kl[ks & 2], y = kl[(ks & 2) + 1];
    u4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (ks & 1)
            r[e] = (uint32_t)__builtin_amdgcn_update_dpp((int)y[e], (int)x[e], 0x128, 0xF, 0x3, false);
        else
            r[e] = (uint32_t)__builtin_amdgcn_update_dpp((int)x[e], (int)y[e], 0x128, 0xF, 0xC, false);
    }
    return r;
}

// kSolo (with kKvSplit): one workgroup per (kv head, session) streams all of
// the session's pages for that head, merges its waves in LDS and writes the
// output rows itself -- no partial rows, no combine launch.  For steps whose
// sessions are short enough that one CU streams a session's head in about
// the time a second launch would cost.
// kSingle (planned launches of one session): the session is known before the
// plan record arrives, so the query rows and the new token's row are loaded
// beside the record instead of one round trip after it.
template <bool kRope, bool kKvSplit, bool kSolo = false, bool kSingle = false>
__global__ void __launch_bounds__(THREADS)
decode_split_kernel(DecodeArgs a) {
    static_assert(!kSolo || kKvSplit, "solo workgroups serve one kv head");
    static_assert(!kSingle || !kKvSplit, "single-session launches use the planned grid");
    // two page pairs in flight per wave (the next pair's loads go out before
    // this pair's arithmetic): solo workgroups only.  The split grid is
    // slower with it even at 242 VGPRs with no spills and the prefetch in
    // flight (config 2 split kernel 26.5-27.0 vs 23.6-24.6 us, config 1
    // 8.0 vs 6.15 us, config 4 unchanged): its 8 waves per CU already keep
    // enough of the chip's bytes in flight.
    constexpr bool kDB = kSolo;
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ float s_acc[(R > 1 || kKvSplit) ? WAVES : 1][G][HD];
    __shared__ u4 s_q[NKV][4][2][64];            // Q^T hi/lo operands per kv head
    __shared__ float s_qf[NKV][16];              // per-head score factor
    __shared__ int s_ready[WAVES];               // a wave's exchange rows are in LDS (one-slot partials)

    const int tid = threadIdx.x;
    // solo: the wave index (and the pair loop) kept in scalar registers
    const int wave = kDB ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int lane = tid & 63;
    const int g = lane >> 4;      // 0..3
    const int c = lane & 15;      // 0..15
    // kv-split: workgroup (w, kv head) streams that head's rows of its page
    // range with all waves; otherwise wave w serves kv head w % NKV
    // kv-split grid is (NKV, ranges): block id kvh + NKV * range runs on XCD
    // (kvh + NKV * range) % 8, so one kv head's workgroups share the XCDs
    // congruent to kvh mod NKV, where its combine blocks run too
    const int kvh = kKvSplit ? (int)blockIdx.x : wave % NKV;
    const int r = kKvSplit ? wave : wave / NKV;
    constexpr int RS = kKvSplit ? WAVES : R;        // waves per kv head = pair stride
    const int w = kKvSplit ? (int)blockIdx.y : (int)blockIdx.x;

    int i, n_keys, pa, pb, tv, slot = w;        // slot: this workgroup's partial row index
    int tv2 = 0;                                 // solo: table entries 64..127

    // The appended token's row piece of this thread and the query rows of
    // session `sess`.  Every wave issues the same loads in the same order,
    // whatever its role, so that the compiler's waits count exactly: a wave
    // without a use for one reads a valid line and drops it.
    // (a kv-split workgroup appends its own kv head's part of the row)
    constexpr int kAppW = kKvSplit ? HD : KVW;      // halfs of the row this workgroup appends
    const int app_off = kKvSplit ? kvh * HD : 0;
    const bool app_lane = !kRope && tid < kAppW / 8;
    const bool qreal = c < G;
    u4 knew, vnew;
    f4 qraw[8];
    auto issue_new = [&](int sess) {
        const uint16_t* ks = a.k_new ? a.k_new : reinterpret_cast<const uint16_t*>(a.q);
        const uint16_t* vs = a.v_new ? a.v_new : reinterpret_cast<const uint16_t*>(a.q);
        const int64_t src = app_lane ? (int64_t)sess * KVW + app_off + 8 * tid : 0;
        knew = *reinterpret_cast<const u4*>(ks + src);
        vnew = *reinterpret_cast<const u4*>(vs + src);
    };
    auto issue_q = [&](int sess) {
        // the converting wave of each kv head (r == 0) reads its rows; the others one line
        const int64_t qoff = r == 0 ? ((int64_t)sess * NH + kvh * G + (qreal ? c : 0)) * HD + 8 * g : (int64_t)sess * NH * HD;
        const int step = r == 0 ? 1 : 0;
        const float* qp = a.q + qoff;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            qraw[2 * ks] = *reinterpret_cast<const f4*>(qp + step * (32 * ks));
            qraw[2 * ks + 1] = *reinterpret_cast<const f4*>(qp + step * (32 * ks + 4));
        }
    };
    if constexpr (kSolo) {
        // session w, all its pages; the first table entries load beside n_keys
        // (tab_read entries of every row are readable), not after it
        i = w;
        const int32_t* trow = a.tables + (int64_t)i * a.table_stride;
        tv = lane < a.tab_read ? trow[lane] : 0;
        tv2 = 64 + lane < a.tab_read ? trow[64 + lane] : 0;
        n_keys = nkeys_of(a, i);
        pa = 0;
        pb = n_keys > 0 ? (n_keys + kKvBlock - 1) >> kKvBlockShift : 0;
        if (n_keys <= 0) {                       // no keys: zero rows (uniform)
            float* orow = a.o + ((int64_t)i * NH + kvh * G) * HD;
            for (int e = tid; e < G * HD / 4; e += THREADS) reinterpret_cast<f4*>(orow)[e] = f4{0.f, 0.f, 0.f, 0.f};
            return;
        }
    } else if (a.plan) {
        // one load: lane t holds phys[t]; lanes 0..3 the header
        const int32_t* rec = a.plan + plan_rec_off(a.n_sess) + (int64_t)w * kRec;
        tv = rec[lane];
        int hv = rec[kRecPages + (lane & 7)];
        if constexpr (kSingle) {
            // in flight while the record travels (issued after it, so the
            // wait for the record below does not wait for them); the move
            // keeps the compiler from sinking them below that wait
            issue_new(0);
            issue_q(0);
            asm volatile("v_mov_b32 %0, %1" : "=v"(hv) : "v"(hv) : "memory");
        }
        i = __builtin_amdgcn_readlane(hv, 0);
        if (i < 0) return;                       // idle workgroup (uniform)
        pa = __builtin_amdgcn_readlane(hv, 1);
        pb = __builtin_amdgcn_readlane(hv, 2);
        n_keys = __builtin_amdgcn_readlane(hv, 3);
        slot = __builtin_amdgcn_readlane(hv, 4);
    } else {
        const Part pt = partition(a, w, -1);
        if (pt.sess < 0) return;                 // idle workgroup (uniform)
        i = pt.sess;
        n_keys = pt.n_keys;
        const int j = w - pt.kc;                 // this workgroup's share of session i
        pa = range_begin(j, pt.pages, pt.k);
        pb = range_begin(j + 1, pt.pages, pt.k);
        tv = (pa + lane < pb) ? a.tables[(int64_t)i * a.table_stride + pa + lane] : 0;
    }
    // settle the slice register here (one wait, nothing else in flight yet):
    // otherwise the compiler's wait before its first read, after the query and
    // first-pair loads below are issued, would be a wait for all of them
    asm volatile("v_mov_b32 %0, %1" : "=v"(tv) : "v"(tv));
    if constexpr (kSolo) asm volatile("v_mov_b32 %0, %1" : "=v"(tv2) : "v"(tv2));
    const int last_page = (n_keys - 1) >> kKvBlockShift;
    const int32_t* table = a.tables + (int64_t)i * a.table_stride;

    // lane-constant byte offsets inside a page
    const uint32_t koff = (uint32_t)((c & 7) * kRowBytes + kvh * HD * 2 + 16 * (g + 4 * (c >> 3)));
    uint32_t voff[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) voff[jj] = (uint32_t)((4 * g + jj) * kRowBytes + kvh * HD * 2 + 16 * c);

    const char* pk = reinterpret_cast<const char*>(a.pool_k);
    const char* pv = reinterpret_cast<const char*>(a.pool_v);
    const int64_t layer_page0 = (int64_t)a.layer * a.nb;

    {
        // block-table slice of this workgroup: lane t holds table[pa + 64*chunk + t]
        int tchunk = 0;
        auto phys_of = [&](int pg) -> int {
            const int rel = pg - pa;
            if constexpr (kDB) {
                // the first 64 (solo: 128) entries sit in tv (, tv2); later
                // pages come one at a time through the scalar cache.  No vector
                // load in the pair loop but the pairs', so the compiler's waits
                // count exactly and the prefetched pair stays in flight during
                // the arithmetic.
                if (rel < 64) return __builtin_amdgcn_readlane(tv, rel);
                if (kSolo && rel < 128) return __builtin_amdgcn_readlane(tv2, rel - 64);
                return *(const __attribute__((address_space(4))) int32_t*)(uintptr_t)(table + pg);
            }
            if ((rel >> 6) != tchunk) {          // rare: ranges longer than 64 pages
                tchunk = rel >> 6;
                const int e = pa + 64 * tchunk + lane;
                tv = e < pb ? table[e] : 0;
            }
            return __builtin_amdgcn_readlane(tv, rel & 63);
        };

        const int npairs = (pb - pa + 1) >> 1;
        // kFirst: a wave's first pair (pages < 16 into the range) takes its pages
        // straight from the slice register, with no reload branch: a reload's
        // load would make the first pair's issue wait for every load before it
        // live == false: the same 16 loads with an empty resource (they
        // return zero, no memory access), for a prefetch slot with no pair
        // left -- a load under a branch would make the compiler drain every
        // load in flight before the next use of any of them
        auto load_pair = [&](auto first_tag, int qp, PairRegs& pr, bool live = true) {
            constexpr bool kFirst = decltype(first_tag)::value;
            const int pg0 = pa + 2 * qp;
            const int pg1 = pg0 + 1 < pb ? pg0 + 1 : pg0;   // a lone last page loads itself twice
            const int ph0 = kFirst ? __builtin_amdgcn_readlane(tv, pg0 - pa) : phys_of(pg0);
            const int ph1 = kFirst ? __builtin_amdgcn_readlane(tv, pg1 - pa) : phys_of(pg1);
            const int64_t b0 = (layer_page0 + ph0) * kPageBytes;
            const int64_t b1 = (layer_page0 + ph1) * kPageBytes;
            const int nr = live ? (int)kPageBytes : 0;
            const auto rk0 = page_rsrc(pk + b0, nr), rk1 = page_rsrc(pk + b1, nr);
            const auto rv0 = page_rsrc(pv + b0, nr), rv1 = page_rsrc(pv + b1, nr);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const uint32_t o = koff + (ks & 1) * 8 * kRowBytes + (ks >> 1) * 128;
                pr.k0[ks] = ldb16_nt(rk0, o);
                pr.k1[ks] = ldb16_nt(rk1, o);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pr.v[j] = ldb16_nt(rv0, voff[j]);
                pr.v[4 + j] = ldb16_nt(rv1, voff[j]);
            }
        };

        // Issue order: the appended token's row and the query rows first, then
        // the first pair (unless the fused append is about to write into it:
        // then after the barrier).  The vector-memory counter drains in issue
        // order, so waiting for the query or the token row waits only for what
        // was issued before it -- issued after the pair, the query conversion
        // (and the barrier behind it) would wait for the whole pair to arrive.
        const bool appends = (kRope || a.k_new) && pb == last_page + 1;
        const bool early = !(appends && pa + 2 * r + 1 >= last_page);
        const int phys_last = table[last_page];     // the appended token's page (may lie past the slice register)
        static_assert(KVW / 8 <= THREADS, "one 16-byte piece of the appended row per thread");
        const bool app_thread = app_lane && appends;
        if constexpr (!kSingle) {
            issue_new(i);
            issue_q(i);
        }
        // fused RoPE: the cos/sin row of position n_keys - 1 for this lane's q
        // dims, and this thread's piece of the new k (one NeoX pair) and v
        f4 rcs[4], rsn[4];
        float rk0 = 0.f, rk1 = 0.f, rc = 0.f, rs = 0.f;
        float2 rv = {0.f, 0.f};
        static_assert(!kRope || (NKV * (HD / 2) <= THREADS && KVW <= 2 * THREADS), "one k pair and two v values per thread");
        const bool rope_k = kRope && appends && tid < (kAppW / HD) * (HD / 2);
        const bool rope_v = kRope && appends && 2 * tid < kAppW;
        if constexpr (kRope) {
            const int64_t row = (int64_t)(n_keys - 1) * (HD / 2);
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                rcs[2 * ks] = *reinterpret_cast<const f4*>(a.cs + row + 32 * ks + 8 * g);
                rcs[2 * ks + 1] = *reinterpret_cast<const f4*>(a.cs + row + 32 * ks + 8 * g + 4);
                rsn[2 * ks] = *reinterpret_cast<const f4*>(a.sn + row + 32 * ks + 8 * g);
                rsn[2 * ks + 1] = *reinterpret_cast<const f4*>(a.sn + row + 32 * ks + 8 * g + 4);
            }
            const int h = kKvSplit ? kvh : tid / (HD / 2), d = kKvSplit ? tid : tid - h * (HD / 2);
            const int64_t kr = rope_k ? (int64_t)i * KVW + h * HD + d : 0;
            rk0 = a.k_new32[kr];
            rk1 = a.k_new32[kr + HD / 2];
            rc = a.cs[row + (rope_k ? d : 0)];
            rs = a.sn[row + (rope_k ? d : 0)];
            rv = *reinterpret_cast<const float2*>(a.v_new32 + (rope_v ? (int64_t)i * KVW + app_off + 2 * tid : 0));
        }
        asm volatile("" ::: "memory");   // keep the loads above ahead of the pair's in issue order
        PairRegs cur;
        static_assert(2 * (8 - 1) + 1 < 64, "a first pair lies in the slice register");
        // the first pair (a wave without one, or whose pair the append is about
        // to write, loads page pa's pair and reloads after the barrier)
        load_pair(std::true_type{}, (r < npairs && early) ? r : 0, cur);

        // fused append: the owner of the session's last page stores the new
        // token; the barrier below publishes it to the waves of this workgroup
        if (appends) {
            const int phys = phys_last;
            const int64_t dst = ((layer_page0 + phys) * kPageBytes + (int64_t)((n_keys - 1) & kKvBlockMask) * kRowBytes) / 2;
            const int64_t src = (int64_t)i * KVW;
            if constexpr (kRope) {
                // RopeKvOp (code/graph/dense.h:75-83): k rotated at position
                // n_keys - 1, k and v rounded to fp16 (nearest even)
                uint16_t* pk16 = const_cast<uint16_t*>(a.pool_k) + dst;
                uint16_t* pv16 = const_cast<uint16_t*>(a.pool_v) + dst;
                (void)src;
                if (rope_k) {
                    const int h = kKvSplit ? kvh : tid / (HD / 2), d = kKvSplit ? tid : tid - h * (HD / 2);
                    float y0, y1;
                    rope_rotate(rk0, rk1, rc, rs, y0, y1);
                    pk16[h * HD + d] = __builtin_bit_cast(uint16_t, (_Float16)y0);
                    pk16[h * HD + d + HD / 2] = __builtin_bit_cast(uint16_t, (_Float16)y1);
                }
                if (rope_v) {
                    pv16[app_off + 2 * tid] = __builtin_bit_cast(uint16_t, (_Float16)rv.x);
                    pv16[app_off + 2 * tid + 1] = __builtin_bit_cast(uint16_t, (_Float16)rv.y);
                }
            } else if (app_thread) {
                (void)src;
                *reinterpret_cast<u4*>(const_cast<uint16_t*>(a.pool_k) + dst + app_off + 8 * tid) = knew;
                *reinterpret_cast<u4*>(const_cast<uint16_t*>(a.pool_v) + dst + app_off + 8 * tid) = vnew;
            }
        }

        // ---- the query group of each kv head as split fp16 B operands, in LDS ----
        // lane (g,c): head kvh*G + c, dims d = 32*ks + 8*g + j.  The first wave of
        // each kv head converts; the R waves of that head read them per pair.
        if (r == 0) {
            float qv[4][8];
            float amax = 0.f;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    qv[ks][jj] = qreal ? qraw[2 * ks][jj] : 0.f;
                    qv[ks][4 + jj] = qreal ? qraw[2 * ks + 1][jj] : 0.f;
                }
            }
            if constexpr (kRope) {
                // RoPE of q at position n_keys - 1: lane (g,c) holds dims
                // 32ks + 8g + jj, so the pair (d, d + 64) is (ks, ks + 2) in
                // the same lane; the caller's q is left as it is
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        float y0, y1;
                        rope_rotate(qv[ks][jj], qv[ks + 2][jj], rcs[2 * ks + (jj >> 2)][jj & 3],
                                    rsn[2 * ks + (jj >> 2)][jj & 3], y0, y1);
                        qv[ks][jj] = y0;
                        qv[ks + 2][jj] = y1;
                    }
                }
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) amax = fmaxf(amax, fabsf(qv[ks][jj]));
            }
            amax = fmaxf(amax, shfl_xor_f(amax, 16));
            amax = fmaxf(amax, shfl_xor_f(amax, 32));
            int ex = 0;
            if (amax > 0.f) (void)frexpf(amax, &ex);
            const int k2 = amax > 0.f ? 15 - ex : 0;    // amax * 2^k2 in [2^14, 2^15)
            const float up = ldexpf(1.f, k2);
            if (g == 0) s_qf[kvh][c] = kScale * kLog2e * ldexpf(1.f, -k2);
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                h8 hi, lo;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    const float x = qv[ks][jj] * up;
                    const _Float16 h = (_Float16)x;
                    hi[jj] = h;
                    lo[jj] = (_Float16)(x - (float)h);
                }
                s_q[kvh][ks][0][lane] = __builtin_bit_cast(u4, hi);
                s_q[kvh][ks][1][lane] = __builtin_bit_cast(u4, lo);
            }
        }
        if (lane == 0) s_ready[wave] = 0;
        __syncthreads();
        const float qf = s_qf[kvh][c];

        float m = -INFINITY, lsum = 0.f;
        f4 acc[8];
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[cb] = f4{0.f, 0.f, 0.f, 0.f};

        auto compute_pair = [&](int qp, PairRegs& cur) {
            const int pg0 = pa + 2 * qp;
            const bool two = pg0 + 1 < pb;
            // keys that exist: all of them except in the session's last pair
            const bool tail = !two || (((pg0 + 2) << kKvBlockShift) > n_keys);

            // S = K . Q^T  (C layout: lane (g,c) holds keys 4g+i of head c)
            // hi and lo products in separate accumulators: four chains of four
            // dependent MFMAs instead of two of eight
            f4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
            f4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const h8 ka = __builtin_bit_cast(h8, k_operand(cur.k0, ks));
                const h8 kc = __builtin_bit_cast(h8, k_operand(cur.k1, ks));
                const h8 qhi = __builtin_bit_cast(h8, s_q[kvh][ks][0][lane]);
                const h8 qlo = __builtin_bit_cast(h8, s_q[kvh][ks][1][lane]);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qhi, s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, qhi, s1, 0, 0, 0);
                t0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qlo, t0, 0, 0, 0);
                t1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, qlo, t1, 0, 0, 0);
            }
            s0 += t0;
            s1 += t1;
            float s[8];
            bool ok[8];
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                s[ii] = s0[ii] * qf;
                s[4 + ii] = s1[ii] * qf;
                ok[ii] = true;
                ok[4 + ii] = true;
            }
            if (tail) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    ok[ii] = (pg0 << kKvBlockShift) + 4 * g + ii < n_keys;
                    ok[4 + ii] = two && ((pg0 + 1) << kKvBlockShift) + 4 * g + ii < n_keys;
                }
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (!ok[j]) cur.v[j] = u4{0u, 0u, 0u, 0u};   // unwritten slots may hold NaN bits
            }
            // Lazy max: the running max m of a head only moves when a score
            // exceeds it by more than kLazy (log2 units), so weights stay
            // <= 2^kLazy (exact in the hi/lo fp16 split) and the common pair
            // needs one lane-local test and a ballot -- no cross-lane max, no
            // rescale of the accumulators.  The first pair (m = -inf) always
            // moves it.
            float lm = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) lm = ok[j] ? fmaxf(lm, s[j]) : lm;
            if (__builtin_amdgcn_ballot_w64(lm > m + kLazy)) {
                float bm = fmaxf(lm, shfl_xor_f(lm, 16));
                bm = fmaxf(bm, shfl_xor_f(bm, 32));
                const float mn = fmaxf(m, bm);
                const float corr = __builtin_amdgcn_exp2f(m - mn);   // m = -inf: 0
                lsum *= corr;
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) acc[cb] *= corr;
                m = mn;
            }
            float ps = 0.f;
            h8 phi, plo;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = ok[j] ? __builtin_amdgcn_exp2f(s[j] - m) : 0.f;
                ps += p;
                const _Float16 h = (_Float16)p;
                phi[j] = h;
                plo[j] = (_Float16)(p - (float)h);
            }
            lsum += ps;

            // O^T += V^T . P^T   (A: lane (g,c) holds V[kappa(g,j)][8c + cb], j = 0..7)
#pragma unroll
            for (int cb = 0; cb < 8; ++cb) {
                // column cb of the 8 loaded rows: half cb of each 16 B row, paired
                // into dwords with v_perm (low or high half of dword cb/2)
                const uint32_t sel = (cb & 1) ? 0x07060302u : 0x05040100u;
                u4 vw;
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    vw[u] = __builtin_amdgcn_perm(cur.v[2 * u + 1][cb >> 1], cur.v[2 * u][cb >> 1], sel);
                const h8 va = __builtin_bit_cast(h8, vw);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, phi, acc[cb], 0, 0, 0);
                acc[cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, plo, acc[cb], 0, 0, 0);
            }
        };

        // each wave keeps one pair (16 KiB) in flight; the 8 waves of the CU
        // overlap each other's latency (measured: a second pair prefetched
        // before the query conversion only delays the query rows further
        // behind the chip's first burst, 0.778 -> 0.791 ms per config-2 step)
        if constexpr (kDB) {
            // the next pair's loads go out before this pair's arithmetic (two
            // pairs in flight per wave), so the wave's stream does not stop at
            // every pair
            // Two register sets take turns (no copy between them: a copy would
            // wait for the prefetch to land).
            if (!early && r < npairs) load_pair(std::false_type{}, r, cur);
            PairRegs alt;
            for (int qp = r; qp < npairs; qp += 2 * RS) {
                const bool m1 = qp + RS < npairs;
                load_pair(std::false_type{}, m1 ? qp + RS : qp, alt, m1);
                // issued before the waits for this pair (the counter drains in
                // issue order): without the pin the scheduler sinks them below
                __builtin_amdgcn_sched_barrier(0);
                compute_pair(qp, cur);
                if (!m1) break;
                const bool m2 = qp + 2 * RS < npairs;
                load_pair(std::false_type{}, m2 ? qp + 2 * RS : qp, cur, m2);
                __builtin_amdgcn_sched_barrier(0);
                compute_pair(qp + RS, alt);
            }
        } else {
            for (int qp = r; qp < npairs; qp += RS) {
                if (qp != r || !early) load_pair(std::false_type{}, qp, cur);
                compute_pair(qp, cur);
            }
        }

        lsum += shfl_xor_f(lsum, 16);
        lsum += shfl_xor_f(lsum, 32);
        // this wave's G rows of a partial slot, straight from the accumulators
        auto write_rows = [&](float* pout) {
            if (c < G) {
                float* row = pout + (int64_t)(kvh * G + c) * a.pw;
                if (g == 0) {
                    row[0] = m;
                    row[1] = lsum;
                }
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    f4 lo4, hi4;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        lo4[cb] = acc[cb][ii];
                        hi4[cb] = acc[cb + 4][ii];
                    }
                    float* dst = row + a.po + 8 * (4 * g + ii);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dst[e] = lo4[e];
                        dst[4 + e] = hi4[e];
                    }
                }
            }
        };
        if constexpr (R == 1 && !kKvSplit) {
            write_rows(a.part + (int64_t)slot * NH * a.pw);
        } else if (a.wave_parts == 2 && !kKvSplit) {
            // one partial slot per workgroup: the R waves of a kv head merge
            // through LDS with no serial pass.  Lane group g (head dims
            // [32g, 32g + 32)) of wave r keeps its dims when g*R/4 == r and
            // hands them to that wave otherwise; each keeper merges the R rows
            // of its 32 dims by the combine rule and stores them.
            const int keeper = (g * R) >> 2;
            if (g == 0) {
                s_m[wave][c] = m;
                s_l[wave][c] = lsum;
            }
            if (keeper != r && c < G) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    f4 lo4, hi4;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        lo4[cb] = acc[cb][ii];
                        hi4[cb] = acc[cb + 4][ii];
                    }
                    *reinterpret_cast<f4*>(&s_acc[wave][c][8 * (4 * g + ii)]) = lo4;
                    *reinterpret_cast<f4*>(&s_acc[wave][c][8 * (4 * g + ii) + 4]) = hi4;
                }
            }
            // publish to the other waves of this kv head only (no workgroup
            // barrier: a wave waits for its R - 1 partners, not for the
            // slowest wave of the workgroup); bounded wait, every wave of the
            // workgroup reaches this point
            if (lane == 0) __hip_atomic_store(&s_ready[wave], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            bool gave_up = false;
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                const int ww = kvh + NKV * rr;
                if (ww == wave) continue;
                bool seen = false;
                for (int it = 0; it < a.spin; ++it) {
                    const int f = __hip_atomic_load(&s_ready[ww], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
                    if (__builtin_amdgcn_readfirstlane(f)) {
                        seen = true;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
                gave_up |= !seen;
            }
            if (gave_up && keeper == r && lane == 0 && a.status)
                __hip_atomic_fetch_or(a.status, kStatusExchange, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (keeper == r && c < G) {
                float M = -INFINITY;
#pragma unroll
                for (int rr = 0; rr < R; ++rr) {
                    const int ww = kvh + NKV * rr;
                    if (s_l[ww][c] > 0.f) M = fmaxf(M, s_m[ww][c]);
                }
                float L = 0.f;
                f4 A[8];
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) A[cb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int rr = 0; rr < R; ++rr) {
                    const int ww = kvh + NKV * rr;
                    const float lw = s_l[ww][c];
                    const float f = lw > 0.f ? exp2f(s_m[ww][c] - M) : 0.f;
                    L = fmaf(lw, f, L);
                    if (rr == r) {
#pragma unroll
                        for (int cb = 0; cb < 8; ++cb) A[cb] += acc[cb] * f;
                    } else {
#pragma unroll
                        for (int ii = 0; ii < 4; ++ii) {
                            const f4 lo4 = *reinterpret_cast<const f4*>(&s_acc[ww][c][8 * (4 * g + ii)]);
                            const f4 hi4 = *reinterpret_cast<const f4*>(&s_acc[ww][c][8 * (4 * g + ii) + 4]);
#pragma unroll
                            for (int cb = 0; cb < 4; ++cb) {
                                A[cb][ii] = fmaf(lo4[cb], f, A[cb][ii]);
                                A[cb + 4][ii] = fmaf(hi4[cb], f, A[cb + 4][ii]);
                            }
                        }
                    }
                }
                float* row = a.part + ((int64_t)slot * NH + kvh * G + c) * a.pw;
                if (gave_up) {
                    // the partner's rows may not be in LDS: poison this slot so
                    // that the combine's output for these heads is NaN
                    M = 0.f;
                    L = 1.f;
#pragma unroll
                    for (int cb = 0; cb < 8; ++cb) A[cb] = f4{NAN, NAN, NAN, NAN};
                }
                if (g == 0) {
                    row[0] = M;
                    row[1] = L;
                }
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    f4 lo4, hi4;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        lo4[cb] = A[cb][ii];
                        hi4[cb] = A[cb + 4][ii];
                    }
                    *reinterpret_cast<f4*>(row + a.po + 8 * (4 * g + ii)) = lo4;
                    *reinterpret_cast<f4*>(row + a.po + 8 * (4 * g + ii) + 4) = hi4;
                }
            }
        } else if (a.wave_parts) {
            // slot w*R + r: the combine merges the R rows with the workgroups'
            write_rows(a.part + ((int64_t)slot * R + r) * NH * a.pw);
        } else {
            // merge the waves of each kv head in LDS (kv-split: the G heads of
            // this workgroup's kv head over all its waves)
            float* pout = kSolo ? nullptr : a.part + (int64_t)w * NH * a.pw;
            if (g == 0) {
                s_m[wave][c] = m;
                s_l[wave][c] = lsum;
            }
            if (c < G) {
#pragma unroll
                for (int ii = 0; ii < 4; ++ii) {
                    f4 lo4, hi4;
#pragma unroll
                    for (int cb = 0; cb < 4; ++cb) {
                        lo4[cb] = acc[cb][ii];
                        hi4[cb] = acc[cb + 4][ii];
                    }
                    *reinterpret_cast<f4*>(&s_acc[wave][c][8 * (4 * g + ii)]) = lo4;
                    *reinterpret_cast<f4*>(&s_acc[wave][c][8 * (4 * g + ii) + 4]) = hi4;
                }
            }
            __syncthreads();
            const int h0 = kKvSplit ? kvh * G : 0;
            constexpr int n_out = kKvSplit ? G * HD : NH * HD;
            for (int idx = tid; idx < n_out; idx += THREADS) {
                const int h = h0 + idx / HD, d = idx - (idx / HD) * HD;
                const int hk = h / G, hc = h - hk * G;
                float M = -INFINITY;
#pragma unroll
                for (int rr = 0; rr < WAVES; ++rr)
                    if (rr < RS) M = fmaxf(M, s_m[kKvSplit ? rr : hk + NKV * rr][hc]);
                float L = 0.f, A = 0.f;
#pragma unroll
                for (int rr = 0; rr < WAVES; ++rr) {
                    if (rr >= RS) break;
                    const int ww = kKvSplit ? rr : hk + NKV * rr;
                    const float lw = s_l[ww][hc];
                    const float f = lw > 0.f ? exp2f(s_m[ww][hc] - M) : 0.f;
                    L = fmaf(lw, f, L);
                    A = fmaf(s_acc[ww][hc][d], f, A);
                }
                if constexpr (kSolo) {
                    a.o[((int64_t)i * NH + h) * HD + d] = L > 0.f ? A / L : 0.f;
                } else {
                    pout[(int64_t)h * a.pw + a.po + d] = A;
                    if (d == 0) {
                        pout[(int64_t)h * a.pw] = M;
                        pout[(int64_t)h * a.pw + 1] = L;
                    }
                }
            }
        }
    }
}

#ifdef NOVA_TESTKIT
// Stream floor (test kit): the planned split grid reading exactly the split
// kernel's bytes -- the same plan records, page pairs per wave row, lane
// offsets and non-temporal 16-byte loads -- with no arithmetic but a running
// sum, one 4-byte word per thread stored into the partial area.  Its time is
// the HBM floor of this partition on the part, to set the split kernel's
// time against.
__global__ void __launch_bounds__(THREADS)
decode_stream_floor_kernel(DecodeArgs a) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, c = lane & 15;
    const int kvh = wave % NKV, r = wave / NKV;
    const int w = (int)blockIdx.x;
    const int32_t* rec = a.plan + plan_rec_off(a.n_sess) + (int64_t)w * kRec;
    int tv = rec[lane];
    const int hv = rec[kRecPages + (lane & 7)];
    const int i = __builtin_amdgcn_readlane(hv, 0);
    if (i < 0) return;
    const int pa = __builtin_amdgcn_readlane(hv, 1);
    const int pb = __builtin_amdgcn_readlane(hv, 2);
    const int32_t* table = a.tables + (int64_t)i * a.table_stride;
    const uint32_t koff = (uint32_t)((c & 7) * kRowBytes + kvh * HD * 2 + 16 * (g + 4 * (c >> 3)));
    uint32_t voff[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) voff[jj] = (uint32_t)((4 * g + jj) * kRowBytes + kvh * HD * 2 + 16 * c);
    const char* pk = reinterpret_cast<const char*>(a.pool_k);
    const char* pv = reinterpret_cast<const char*>(a.pool_v);
    const int64_t layer_page0 = (int64_t)a.layer * a.nb;
    int tchunk = 0;
    auto phys_of = [&](int pg) -> int {
        const int rel = pg - pa;
        if ((rel >> 6) != tchunk) {
            tchunk = rel >> 6;
            const int e = pa + 64 * tchunk + lane;
            tv = e < pb ? table[e] : 0;
        }
        return __builtin_amdgcn_readlane(tv, rel & 63);
    };
    u4 sum = {0u, 0u, 0u, 0u};
    const int npairs = (pb - pa + 1) >> 1;
    for (int qp = r; qp < npairs; qp += R) {
        const int pg0 = pa + 2 * qp;
        const int pg1 = pg0 + 1 < pb ? pg0 + 1 : pg0;
        const int64_t b0 = (layer_page0 + phys_of(pg0)) * kPageBytes;
        const int64_t b1 = (layer_page0 + phys_of(pg1)) * kPageBytes;
        const auto rk0 = page_rsrc(pk + b0, (int)kPageBytes), rk1 = page_rsrc(pk + b1, (int)kPageBytes);
        const auto rv0 = page_rsrc(pv + b0, (int)kPageBytes), rv1 = page_rsrc(pv + b1, (int)kPageBytes);
        u4 x[16];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const uint32_t o = koff + (ks & 1) * 8 * kRowBytes + (ks >> 1) * 128;
            x[ks] = ldb16_nt(rk0, o);
            x[4 + ks] = ldb16_nt(rk1, o);
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            x[8 + jj] = ldb16_nt(rv0, voff[jj]);
            x[12 + jj] = ldb16_nt(rv1, voff[jj]);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) sum += x[e];
    }
    reinterpret_cast<uint32_t*>(a.part)[(int64_t)w * THREADS + tid] = sum[0] + sum[1] + sum[2] + sum[3];
}

#endif  // NOVA_TESTKIT

// Combine: one workgroup per (session, head) merges the session's k_i
// partials (slots kc_i .. kc_i+k_i-1) with the rule of fa_combine_kernel
// (attn.cu:163-191): M = max m_s, L = sum over l_s > 0 of l_s*2^(m_s-M),
// O = sum acc_s*2^(m_s-M) / L; a session without keys gets O = 0.  Its 8
// groups of 32 threads (a thread owns 4 consecutive head-dim columns) take
// every 8th slot, 8 slots per group with all loads in flight, and the 8 group
// results are merged through LDS by the same rule.  Measured against one
// workgroup per (session, kv head) walking all slots: 448 instead of 64
// workgroups for config 2, 0.876 -> 0.859 ms per step.
static_assert(8 % NKV == 0, "kv heads must divide the 8 XCDs");
constexpr int CT = 256;                       // combine threads
constexpr int kCombGroups = CT / (HD / 4);

__global__ void __launch_bounds__(CT)
decode_combine_kernel(DecodeArgs a, float* __restrict__ o) {
    const int t = blockIdx.x;
    int i, h;
    const int tid = threadIdx.x, g = tid / (HD / 4), q4 = tid - g * (HD / 4);
    __shared__ float s_m[kCombGroups], s_l[kCombGroups];
    __shared__ f4 s_a[kCombGroups][HD / 4];
    Part pt;
    if (a.plan) {
        // block t (XCD t % 8) serves the (session, head) the plan placed on it
        const int4 e = *reinterpret_cast<const int4*>(a.plan + plan_map_off(a.n_sess) + (int64_t)t * 4);
        pt.kc = e.x;
        pt.k = e.y;
        i = e.z & 0xffff;
        h = e.z >> 16;
        pt.pages = e.w;
        pt.sess = i;
    } else {
        if (a.kv_split) {
            // single session: head kvh * G + m runs on a block whose XCD
            // (t % 8) is congruent to kvh mod NKV, next to its split workgroups
            constexpr int per8 = 8 / NKV;
            const int x = t & 7, kv = x % NKV;
            const int m = (t >> 3) * per8 + x / NKV;
            if (m >= G) return;                  // padding block
            i = 0;
            h = kv * G + m;
        } else {
            i = t % a.n_sess;
            h = t / a.n_sess;
        }
        pt = partition(a, 0, i);
    }
    f4* orow = reinterpret_cast<f4*>(o + ((int64_t)i * NH + h) * HD) + q4;
    if (pt.sess < 0 || pt.k == 0) {
        if (g == 0) *orow = f4{0.f, 0.f, 0.f, 0.f};
        return;
    }
    const int64_t SEG = (int64_t)NH * a.pw;
    constexpr int kChunk = 8;
    // partial slots per split workgroup; with one per wave row, only the rows
    // that can hold a page pair are read (a workgroup has at most
    // ceil(pages / k) pages; rows past its pairs hold l = 0): config 1 reads
    // 34 rows in one round instead of 68 in two
    const int stride = a.wave_parts == 1 ? R : 1;
    const int used = a.wave_parts == 1 ? min(R, (range_max_pages(pt.pages, pt.k) + 1) >> 1) : 1;
    const int n_rows = pt.k * used;
    const float* base = a.part + (int64_t)pt.kc * stride * SEG + (int64_t)h * a.pw;
    float M = -INFINITY, L = 0.f;
    f4 A = {0.f, 0.f, 0.f, 0.f};
    for (int s0 = g; s0 < n_rows; s0 += kCombGroups * kChunk) {
        float ms[kChunk], ls[kChunk];
        f4 as[kChunk];
#pragma unroll
        for (int jj = 0; jj < kChunk; ++jj) {
            const int sl0 = s0 + jj * kCombGroups;
            const bool in = sl0 < n_rows;
            const int sl = in ? sl0 : s0;
            const int wg = sl / used;
            const float* row = base + (int64_t)(wg * stride + (sl - wg * used)) * SEG;
            ms[jj] = row[0];
            ls[jj] = in ? row[1] : 0.f;
            as[jj] = *reinterpret_cast<const f4*>(row + a.po + 4 * q4);
        }
        float mc = M;
#pragma unroll
        for (int jj = 0; jj < kChunk; ++jj)
            if (ls[jj] > 0.f) mc = fmaxf(mc, ms[jj]);
        const float rescale = L > 0.f ? exp2f(M - mc) : 0.f;
        L *= rescale;
        A *= rescale;
#pragma unroll
        for (int jj = 0; jj < kChunk; ++jj) {
            const float f = ls[jj] > 0.f ? exp2f(ms[jj] - mc) : 0.f;
            L = fmaf(ls[jj], f, L);
            A += as[jj] * f;
        }
        M = mc;
    }
    if (q4 == 0) {
        s_m[g] = M;
        s_l[g] = L;
    }
    s_a[g][q4] = A;
    __syncthreads();
    if (g != 0) return;
    float Mx = -INFINITY;
#pragma unroll
    for (int gg = 0; gg < kCombGroups; ++gg)
        if (s_l[gg] > 0.f) Mx = fmaxf(Mx, s_m[gg]);
    float Lx = 0.f;
    f4 Ax = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gg = 0; gg < kCombGroups; ++gg) {
        const float f = s_l[gg] > 0.f ? exp2f(s_m[gg] - Mx) : 0.f;
        Lx = fmaf(s_l[gg], f, Lx);
        Ax += s_a[gg][q4] * f;
    }
    const float inv = Lx > 0.f ? 1.f / Lx : 0.f;
    *orow = Ax * inv;
}

// Per-step plan: block w (< split_slots) writes the record of workgroup slot w;
// the last block also writes the session table and the combine map.  64
// threads per block.
__global__ void __launch_bounds__(64)
decode_plan_kernel(DecodeArgs a, int32_t* __restrict__ plan) {
    const int w = blockIdx.x, lane = threadIdx.x;
    const int n_slots = split_slots(a.n_sess, a.gw);
    if (w == n_slots) {
        if (lane == 0) plan[plan_status_off(a.n_sess, a.gw)] = 0;
        __shared__ int s_kc[kMaxBatch], s_k[kMaxBatch], s_mid[kMaxBatch], s_home[kMaxBatch], s_rank[kMaxBatch],
            s_pg[kMaxBatch];
        // session table: the same prefix as partition(), one lane per session
        int T = 0;
        for (int base = 0; base < a.n_sess; base += 64) {
            const int ii = base + lane;
            const int nk = ii < a.n_sess ? nkeys_of(a, ii) : 0;
            int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) pg += __shfl_xor(pg, o, 64);
            T += pg;
        }
        const int target = plan_share(a, T);
        int carry = 0;
        for (int base = 0; base < a.n_sess; base += 64) {
            const int ii = base + lane;
            const int nk = ii < a.n_sess ? nkeys_of(a, ii) : 0;
            const int pg = nk > 0 ? (nk + kKvBlock - 1) >> kKvBlockShift : 0;
            const int k = (pg + target - 1) / target;
            int incl = k;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int t = __shfl_up(incl, o, 64);
                if (lane >= o) incl += t;
            }
            if (ii < a.n_sess) {
                int32_t* e = plan + (int64_t)ii * 4;
                const int kc = carry + incl - k;
                e[0] = kc;
                e[1] = k;
                e[2] = nk;
                e[3] = pg;
                s_kc[ii] = kc;
                s_k[ii] = k;
                s_mid[ii] = kc + (k > 0 ? (k - 1) / 2 : 0);
                s_pg[ii] = pg;
            }
            carry += __shfl(incl, 63, 64);
        }
        // combine map: block t runs on XCD t % 8; each XCD first takes the
        // (session, head) pairs of its own sessions, the overflow fills the
        // blocks other XCDs leave free
        __shared__ int s_cap[8], s_dem[8], s_ovpre[8], s_freepre[8];
        __syncthreads();
        // home XCD: the one that runs the session's middle workgroup
        {
            const int stride = xcd_stride(carry, a.gw);
            for (int ii = lane; ii < a.n_sess; ii += 64)
                s_home[ii] = s_mid[ii] < 8 * stride ? s_mid[ii] / stride : 0;
        }
        __syncthreads();
        const int NT = a.n_sess * NH;
        if (lane == 0) {
            int cnt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int ii = 0; ii < a.n_sess; ++ii) s_rank[ii] = cnt[s_home[ii]]++;
            int ov = 0, fr = 0;
            for (int x = 0; x < 8; ++x) {
                const int cap = NT > x ? (NT - x + 7) / 8 : 0;
                const int dem = NH * cnt[x];
                s_cap[x] = cap;
                s_dem[x] = dem;
                s_ovpre[x] = ov;
                s_freepre[x] = fr;
                ov += dem > cap ? dem - cap : 0;
                fr += cap > dem ? cap - dem : 0;
            }
        }
        __syncthreads();
        int4* map = reinterpret_cast<int4*>(plan + plan_map_off(a.n_sess));
        for (int pr = lane; pr < NT; pr += 64) {
            const int ii = pr / NH, hh = pr - ii * NH;
            const int x = s_home[ii];
            const int rk = NH * s_rank[ii] + hh;
            int t;
            if (rk < s_cap[x]) {
                t = x + 8 * rk;
            } else {
                const int o = s_ovpre[x] + (rk - s_cap[x]);
                int x2 = 0;
                for (int y = 0; y < 8; ++y) {
                    const int fy = s_cap[y] > s_dem[y] ? s_cap[y] - s_dem[y] : 0;
                    if (o >= s_freepre[y] && o < s_freepre[y] + fy) x2 = y;
                }
                t = x2 + 8 * (s_dem[x2] + (o - s_freepre[x2]));
            }
            map[t] = int4{s_kc[ii], s_k[ii], ii | (hh << 16), s_pg[ii]};
        }
        return;
    }
    const int L = logical_of(w, xcd_stride(sum_k(a), a.gw), a.gw);
    const Part pt = L >= 0 ? partition(a, L, -1) : Part{-1, 0, 0, 0, 0};
    int32_t* rec = plan + plan_rec_off(a.n_sess) + (int64_t)w * kRec;
    if (pt.sess < 0) {
        if (lane == 0) rec[kRecPages] = -1;
        return;
    }
    const int j = L - pt.kc;
    const int pa = range_begin(j, pt.pages, pt.k);
    const int pb = range_begin(j + 1, pt.pages, pt.k);
    rec[lane] = pa + lane < pb ? a.tables[(int64_t)pt.sess * a.table_stride + pa + lane] : 0;
    if (lane < 5) {
        const int v = lane == 0 ? pt.sess : lane == 1 ? pa : lane == 2 ? pb : lane == 3 ? pt.n_keys : L;
        rec[kRecPages + lane] = v;
    }
}

// Split workgroups of the batched path: one per CU (an 8-wave workgroup fills
// the CU's share of waves at this kernel's register count; measured: 2 or 3
// per CU are slower, 0.97 -> 1.20 -> 1.43 ms per config-2 step).
int batch_workgroups() {
    static int gw = 0;
    static std::once_flag once;
    std::call_once(once, [] {
        int dev = 0, cus = 0;
        NOVA_HIP(hipGetDevice(&dev));
        NOVA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        gw = cus;
    });
    return gw;
}

void launch_split(const DecodeArgs& a, int n_sess, hipStream_t st) {
    const dim3 grid = a.kv_split ? dim3(NKV, a.gw + n_sess)
                                 : dim3(a.plan ? split_slots(n_sess, a.gw) : a.gw + n_sess);
    const bool single = a.plan && n_sess == 1;
    if (a.kv_split) hipLaunchKernelGGL((decode_split_kernel<false, true>), grid, dim3(THREADS), 0, st, a);
    else if (a.cs && single) hipLaunchKernelGGL((decode_split_kernel<true, false, false, true>), grid, dim3(THREADS), 0, st, a);
    else if (a.cs) hipLaunchKernelGGL((decode_split_kernel<true, false>), grid, dim3(THREADS), 0, st, a);
    else if (single) hipLaunchKernelGGL((decode_split_kernel<false, false, false, true>), grid, dim3(THREADS), 0, st, a);
    else hipLaunchKernelGGL((decode_split_kernel<false, false>), grid, dim3(THREADS), 0, st, a);
    NOVA_LAUNCHED();
}

// Solo launch: grid (kv head, session), the output written by the split
// kernel.  Up to this many pages the reference-signature decode runs as one
// solo launch instead of the split + combine pair.  Measured per layer (the
// reference's launch_kv_store_paged + launch_attn_decode_paged, graph of 28
// layers): 64 tokens 7.9 vs 14.4 us, 512 tokens 12.3 vs 14.2 us, 768 tokens
// 14.8 vs 14.3 us (1.5B; 7B alike).  One CU's arithmetic, ~2.3 us per round
// of one page pair per wave, is what limits a solo workgroup.
#ifndef NOVA_DECODE_SOLO_PAGES
#define NOVA_DECODE_SOLO_PAGES 40
#endif
constexpr int kSoloMaxPages = NOVA_DECODE_SOLO_PAGES;
void launch_solo(const DecodeArgs& a, int n_sess, hipStream_t st) {
    NOVA_REQUIRE(a.o && a.tab_read >= 1 && a.tab_read <= 128 && n_sess >= 1 && n_sess <= 65535);
    const dim3 grid(NKV, n_sess);
    if (a.cs) hipLaunchKernelGGL((decode_split_kernel<true, true, true>), grid, dim3(THREADS), 0, st, a);
    else hipLaunchKernelGGL((decode_split_kernel<false, true, true>), grid, dim3(THREADS), 0, st, a);
    NOVA_LAUNCHED();
}

void launch_pair(const DecodeArgs& a, int n_sess, float* o, hipStream_t st) {
    launch_split(a, n_sess, st);
    const int comb = a.plan ? n_sess * NH : a.kv_split ? 8 * ((NH + 7) / 8) : n_sess * NH;
    hipLaunchKernelGGL(decode_combine_kernel, dim3(comb), dim3(CT), 0, st, a, o);
    NOVA_LAUNCHED();
}

// workspace of the batched path: [plan | partials], each 256-byte aligned
size_t plan_bytes(int n_sess) { return ((size_t)plan_ints(n_sess, batch_workgroups()) * 4 + 255) / 256 * 256; }

DecodeArgs batch_args(const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess, void* workspace) {
    NOVA_REQUIRE(n_sess >= 1 && n_sess <= kMaxBatch);
    NOVA_REQUIRE(tables && workspace && table_stride > 0);
    DecodeArgs a{};
    a.tables = tables;
    a.table_stride = table_stride;
    a.n_keys = n_keys;
    a.n_sess = n_sess;
    a.gw = batch_workgroups();
    a.plan = static_cast<const int32_t*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + plan_bytes(n_sess));
    a.spin = kSpinLimit;
    a.status = static_cast<int32_t*>(workspace) + plan_status_off(n_sess, a.gw);
    a.pw = PWB;
    a.po = PWB - HD;
    // Partial slots: with two waves per kv head (7B) they merge through LDS
    // into one slot per workgroup (half the partial bytes, same step time);
    // with four (1.5B) the exchange costs more than it saves: one slot per
    // wave row (measured on config 1: 8.5 vs 6.4 us per split launch).
#ifndef NOVA_DECODE_PART_MODE
#define NOVA_DECODE_PART_MODE (R == 2 ? 2 : 1)
#endif
    a.wave_parts = R > 1 ? NOVA_DECODE_PART_MODE : 1;
    return a;
}

#ifndef NOVA_TESTKIT
// ---- workspace without allocation: a file-scope device array ----
// For callers that cannot allocate (code under graph capture, serving loops,
// harnesses that forbid hipMalloc): the batched decode with its plan and
// partials in this array instead of a caller workspace.  Sized for
// kStaticMaxSess sessions on a device of at most kStaticMaxCUs CUs.  Each
// device holds its own copy for the life of the process; every call on a
// device shares it, so calls that overlap on one device race.  Nothing in it
// needs initial contents: the plan kernel writes every record and combine-map
// entry it later reads, and the split kernel writes every partial row.
constexpr int kStaticMaxSess = 64;
constexpr int kStaticMaxCUs = 256;
constexpr size_t kStaticPlanBytes = ((size_t)plan_ints(kStaticMaxSess, kStaticMaxCUs) * 4 + 255) / 256 * 256;
constexpr size_t kStaticBytes =
    kStaticPlanBytes + (size_t)split_slots(kStaticMaxSess, kStaticMaxCUs) * R * NH * PWB * sizeof(float);
__device__ __align__(256) unsigned char scratch[kStaticBytes];

// Device address of `scratch` on the current device, looked up once per device
// with that device current (the host-side name is only a stand-in).
void* scratch_address() {
    constexpr int kMaxDevices = 64;
    static void* ptr[kMaxDevices] = {};
    static std::once_flag once[kMaxDevices];
    int dev = 0;
    NOVA_HIP(hipGetDevice(&dev));
    NOVA_REQUIRE(dev >= 0 && dev < kMaxDevices);
    std::call_once(once[dev], [dev] {
        void* p = nullptr;
        NOVA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        NOVA_REQUIRE(p != nullptr);
        ptr[dev] = p;
    });
    return ptr[dev];
}

#endif  // !NOVA_TESTKIT

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {


#ifndef NOVA_TESTKIT

size_t attn_decode_batch_workspace_bytes(int n_sess) {
    NOVA_REQUIRE(n_sess >= 1 && n_sess <= kMaxBatch);
    return plan_bytes(n_sess) + (size_t)split_slots(n_sess, batch_workgroups()) * R * NH * PWB * sizeof(float);
}

void launch_attn_decode_plan(const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess,
                             void* workspace, nova_stream_t s) {
    NOVA_REQUIRE(n_keys);
    DecodeArgs a = batch_args(tables, table_stride, n_keys, n_sess, workspace);
    a.plan = nullptr;   // the plan kernel derives the partition itself
    hipLaunchKernelGGL(decode_plan_kernel, dim3(split_slots(n_sess, a.gw) + 1), dim3(64), 0, reinterpret_cast<hipStream_t>(s),
                       a, static_cast<int32_t*>(workspace));
    NOVA_LAUNCHED();
}

void launch_attn_decode_paged_planned(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                      int table_stride, int n_sess, int layer, int nb, const uint16_t* k_new,
                                      const uint16_t* v_new, float* o, void* workspace, nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && o);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0);
    NOVA_REQUIRE((k_new == nullptr) == (v_new == nullptr));
    DecodeArgs a = batch_args(tables, table_stride, nullptr, n_sess, workspace);
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.layer = layer;
    a.nb = nb;
    a.k_new = k_new;
    a.v_new = v_new;
    launch_pair(a, n_sess, o, reinterpret_cast<hipStream_t>(s));
}

void launch_attn_decode_paged_rope_planned(const float* q, const float* k_new, const float* v_new, const float* cs,
                                           const float* sn, uint16_t* pool_k, uint16_t* pool_v,
                                           const int32_t* tables, int table_stride, int n_sess, int layer, int nb,
                                           float* o, void* workspace, nova_stream_t s) {
    NOVA_REQUIRE(q && k_new && v_new && cs && sn && pool_k && pool_v && o);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0);
    DecodeArgs a = batch_args(tables, table_stride, nullptr, n_sess, workspace);
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.layer = layer;
    a.nb = nb;
    a.k_new32 = k_new;
    a.v_new32 = v_new;
    a.cs = cs;
    a.sn = sn;
    launch_pair(a, n_sess, o, reinterpret_cast<hipStream_t>(s));
}

void launch_attn_decode_paged_rope_batch(const float* q, const float* k_new, const float* v_new, const float* cs,
                                         const float* sn, uint16_t* pool_k, uint16_t* pool_v,
                                         const int32_t* tables, int table_stride, const int32_t* n_keys,
                                         int n_sess, int layer, int nb, float* o, void* workspace,
                                         nova_stream_t s) {
    launch_attn_decode_plan(tables, table_stride, n_keys, n_sess, workspace, s);
    launch_attn_decode_paged_rope_planned(q, k_new, v_new, cs, sn, pool_k, pool_v, tables, table_stride, n_sess,
                                          layer, nb, o, workspace, s);
}

void launch_attn_decode_paged_batch(const float* q, uint16_t* pool_k, uint16_t* pool_v,
                                    const int32_t* tables, int table_stride, const int32_t* n_keys,
                                    int n_sess, int layer, int nb, const uint16_t* k_new,
                                    const uint16_t* v_new, float* o, void* workspace, nova_stream_t s) {
    launch_attn_decode_plan(tables, table_stride, n_keys, n_sess, workspace, s);
    launch_attn_decode_paged_planned(q, pool_k, pool_v, tables, table_stride, n_sess, layer, nb, k_new, v_new, o,
                                     workspace, s);
}

void launch_attn_decode_paged_batch_noalloc(const float* q, uint16_t* pool_k, uint16_t* pool_v,
                                            const int32_t* tables, int table_stride, const int32_t* n_keys,
                                            int n_sess, int layer, int nb, const uint16_t* k_new,
                                            const uint16_t* v_new, float* o, nova_stream_t s) {
    // checked on the host before anything is launched (sessions first: no HIP call)
    const int cus = (n_sess >= 1 && n_sess <= kStaticMaxSess) ? batch_workgroups() : 0;
    if (cus < 1 || cus > kStaticMaxCUs) {
        std::fflush(stdout);
        std::fprintf(stderr,
                     "[nova] FATAL launch_attn_decode_paged_batch_noalloc: the static workspace (%zu bytes) "
                     "covers 1..%d sessions on at most %d CUs; called with n_sess %d%s. Use "
                     "launch_attn_decode_paged_batch with a workspace instead.\n",
                     kStaticBytes, kStaticMaxSess, kStaticMaxCUs, n_sess, cus > kStaticMaxCUs ? " on a larger device" : "");
        std::fflush(stderr);
        std::abort();
    }
    NOVA_REQUIRE(attn_decode_batch_workspace_bytes(n_sess) <= kStaticBytes);
    void* ws = scratch_address();
    launch_attn_decode_plan(tables, table_stride, n_keys, n_sess, ws, s);
    launch_attn_decode_paged_planned(q, pool_k, pool_v, tables, table_stride, n_sess, layer, nb, k_new, v_new, o,
                                     ws, s);
}

void launch_attn_decode_paged(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                              const int32_t* table, int layer, int nb, int n_keys, float* o,
                              float* scratch, nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && table && o && scratch);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n_keys >= 1);
    const int pages = (n_keys + kKvBlock - 1) >> kKvBlockShift;
    if (pages <= kSoloMaxPages) {
        // short context: NKV workgroups stream the whole table and write o
        // directly (one launch; scratch is not touched)
        DecodeArgs a{};
        a.q = q;
        a.pool_k = pool_k;
        a.pool_v = pool_v;
        a.tables = table;
        a.table_stride = pages;
        a.n_keys_scalar = n_keys;
        a.n_sess = 1;
        a.layer = layer;
        a.nb = nb;
        a.kv_split = 1;
        a.o = o;
        a.tab_read = pages < 128 ? pages : 128;
        a.spin = kSpinLimit;
        launch_solo(a, 1, reinterpret_cast<hipStream_t>(s));
        return;
    }
    // scratch holds NH*32*(HD+2) floats (reference contract): at most 32
    // partial slots, and the partition uses at most gw + 1 of them
    int gw = (pages + 1) / 2;
    if (gw > kMaxSplit - 1) gw = kMaxSplit - 1;
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
    a.part = scratch;
    a.gw = gw;
    a.kv_split = 1;   // NKV workgroups per partial slot: 31 * NKV CUs per call
    a.spin = kSpinLimit;
    a.pw = PW;        // the reference's scratch holds NH*32*(HD+2) floats
    a.po = 2;
    launch_pair(a, 1, o, reinterpret_cast<hipStream_t>(s));
}

void launch_attn_decode_paged_solo(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                   int table_stride, const int32_t* n_keys, int n_sess, int layer, int nb,
                                   const uint16_t* k_new, const uint16_t* v_new, float* o, nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && tables && n_keys && o);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && table_stride > 0);
    NOVA_REQUIRE(n_sess >= 1 && n_sess <= 65535);
    NOVA_REQUIRE((k_new == nullptr) == (v_new == nullptr));
    DecodeArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = tables;
    a.table_stride = table_stride;
    a.n_keys = n_keys;
    a.n_sess = n_sess;
    a.layer = layer;
    a.nb = nb;
    a.k_new = k_new;
    a.v_new = v_new;
    a.kv_split = 1;
    a.o = o;
    a.tab_read = table_stride < 128 ? table_stride : 128;
    a.spin = kSpinLimit;
    launch_solo(a, n_sess, reinterpret_cast<hipStream_t>(s));
}

void launch_attn_decode_paged_rope_solo(const float* q, const float* k_new, const float* v_new, const float* cs,
                                        const float* sn, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                        int table_stride, const int32_t* n_keys, int n_sess, int layer, int nb,
                                        float* o, nova_stream_t s) {
    NOVA_REQUIRE(q && k_new && v_new && cs && sn && pool_k && pool_v && tables && n_keys && o);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && table_stride > 0);
    NOVA_REQUIRE(n_sess >= 1 && n_sess <= 65535);
    DecodeArgs a{};
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.tables = tables;
    a.table_stride = table_stride;
    a.n_keys = n_keys;
    a.n_sess = n_sess;
    a.layer = layer;
    a.nb = nb;
    a.k_new32 = k_new;
    a.v_new32 = v_new;
    a.cs = cs;
    a.sn = sn;
    a.kv_split = 1;
    a.o = o;
    a.tab_read = table_stride < 128 ? table_stride : 128;
    a.spin = kSpinLimit;
    launch_solo(a, n_sess, reinterpret_cast<hipStream_t>(s));
}

int attn_decode_batch_status(const void* workspace, int n_sess) {
    NOVA_REQUIRE(workspace && n_sess >= 1 && n_sess <= kMaxBatch);
    int32_t v = 0;
    NOVA_HIP(hipDeviceSynchronize());
    NOVA_HIP(hipMemcpy(&v, static_cast<const int32_t*>(workspace) + plan_status_off(n_sess, batch_workgroups()),
                       sizeof(v), hipMemcpyDeviceToHost));
    return v;
}

#endif  // !NOVA_TESTKIT

#ifdef NOVA_TESTKIT

void testkit_attn_decode_split_only(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                    int table_stride, int n_sess, int layer, int nb, const uint16_t* k_new,
                                    const uint16_t* v_new, void* workspace, nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0);
    NOVA_REQUIRE((k_new == nullptr) == (v_new == nullptr));
    DecodeArgs a = batch_args(tables, table_stride, nullptr, n_sess, workspace);
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.layer = layer;
    a.nb = nb;
    a.k_new = k_new;
    a.v_new = v_new;
    launch_split(a, n_sess, reinterpret_cast<hipStream_t>(s));
}

void testkit_decode_stream_floor(const uint16_t* pool_k, const uint16_t* pool_v, const int32_t* tables,
                                 int table_stride, int n_sess, int layer, int nb, void* workspace, nova_stream_t s) {
    NOVA_REQUIRE(pool_k && pool_v);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0);
    DecodeArgs a = batch_args(tables, table_stride, nullptr, n_sess, workspace);
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.layer = layer;
    a.nb = nb;
    static_assert(THREADS <= R * NH * PWB, "one sink word per thread fits in a workgroup's partial slots");
    hipLaunchKernelGGL(decode_stream_floor_kernel, dim3(split_slots(n_sess, a.gw)), dim3(THREADS), 0,
                       reinterpret_cast<hipStream_t>(s), a);
    NOVA_LAUNCHED();
}


void testkit_attn_decode_planned_spin(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                      int table_stride, int n_sess, int layer, int nb, const uint16_t* k_new,
                                      const uint16_t* v_new, float* o, void* workspace, int spin_limit,
                                      nova_stream_t s) {
    NOVA_REQUIRE(q && pool_k && pool_v && o && spin_limit >= 0);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0);
    NOVA_REQUIRE((k_new == nullptr) == (v_new == nullptr));
    DecodeArgs a = batch_args(tables, table_stride, nullptr, n_sess, workspace);
    a.q = q;
    a.pool_k = pool_k;
    a.pool_v = pool_v;
    a.layer = layer;
    a.nb = nb;
    a.k_new = k_new;
    a.v_new = v_new;
    a.spin = spin_limit;
    launch_pair(a, n_sess, o, reinterpret_cast<hipStream_t>(s));
}

#endif  // NOVA_TESTKIT

}  // extern "C"
