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
//    needing the same K/V rows.  A wave owns NB blocks of 16 such columns
//    (col = qi*G + hh); a workgroup of 4 waves owns 64*NB consecutive columns
//    of one (session, kv head); two workgroups share a CU (2 waves per SIMD, so
//    one wave's softmax overlaps the other's MFMAs).  NB = 2 when the launch
//    has enough (session, column group) items to fill the chip, NB = 1 (twice
//    the workgroups) for small launches such as one session's chunk.  Those
//    small launches also split the keys: their workgroups hold two groups of 4
//    waves over the same columns, group g taking key tiles g, g+2, ..., each
//    with its own LDS ring, and the two partial (O, l, m) are merged through
//    LDS at the end (measured: one session's chunk 16% faster; with NB = 2
//    the second group spills registers and is 26% slower, so wide launches
//    keep one group).
//  * K/V tiles of 32 keys (2 pages) are staged ONCE per workgroup in LDS by
//    direct global->LDS loads (global_load_lds_dwordx4: no staging
//    registers), four buffers: while tile t's softmax runs, the scores of
//    tile t+1 are on the matrix core and tiles t+2, t+3 are loading; one
//    barrier per tile.  The loop is unrolled by four so that every LDS
//    operand address is a lane offset plus a compile-time constant.
//    Rows keep their 256 B but the 16 B chunks are XOR-swizzled by row
//    (K: chunk k of row r at position k ^ (r & 15); V: k ^ 2 (r & 7)), so the
//    operand reads below are free of LDS bank conflicts.
//  * S^T = K . Q^T with v_mfma_f32_16x16x32_f16 (rows = 16 keys, cols = 16
//    columns); every K operand read from LDS feeds both column blocks.  S^T's
//    C layout is the B layout P^T needs, so O^T += V^T . P^T follows without
//    moving P between lanes; each V operand read feeds both blocks too.  The
//    V^T operand (8 keys of one d per lane) comes straight out of LDS with the
//    gfx950 transposing read ds_read_b64_tr_b16: within each 16-lane group,
//    lane i's element j is element (i & 3) of what lane 4j + (i >> 2) points
//    at, so lane s of group g points at key row 4g + (s >> 2), halfs
//    d0 + 4 (s & 3) .. +3, and receives V[4g + j][d0 + s], j = 0..3.
//  * Rows past the workgroup's last key (unwritten slots may hold NaN bits)
//    are loaded from the last key's row instead, so masked weights never
//    meet NaN operands.
//  * Q (scaled by 1/sqrt(HD)*log2 e and a per-column power of two) is split
//    once into hi + lo fp16 terms, each with its own score MFMA, so scores
//    carry ~2^-22 relative error per operand instead of fp16's 2^-11 (real
//    post-RoPE queries are far from unit scale); P is fp16; accumulation is
//    fp32.  The row sums l are sums of exactly the fp16 weights applied to V
//    (four v_dot2 per lane and block against (1, 1), reduced over the column's
//    four lanes at the end).
//  * Lazy rescaling: a column's running max m only moves when a tile's max
//    exceeds it by more than 8 (log2 units), bounding P by 2^8 in fp16, so the
//    O rescale (32 multiplies per block) is skipped on most tiles.  Each score
//    becomes s - m in one fma (undoing the column's power-of-two scale); the
//    common case is one lane-local comparison against 8 and a wave ballot,
//    and only a rescale takes the row max across the four 16-lane rows
//    (v_permlane16/32_swap, no LDS round trip).  The weights are computed before
//    that (rare) branch, assuming no max moves, so the exponentials overlap the
//    next tile's score MFMAs; the PV MFMA burst runs at raised wave priority.
//    Exponentials use the raw v_exp_f32; tiles wholly below the causal
//    diagonal run a mask-free path.
//  * The workgroup's slice of the block table sits in LDS (windows of 2048
//    pages), read a tile ahead, so a page lookup never waits on the vector-memory counter that
//    the tile loads in flight occupy; causal masking is per (key, column);
//    tiles past the workgroup's last query are never visited.
//  * Scheduling.  A work item is (session, column group); its cost is its
//    number of key tiles.  Workgroups take items in decreasing cost order
//    (longest-processing-time first: the dispatcher hands out workgroups in
//    index order, so the long items start first and the short ones fill the
//    tail); each workgroup ranks the items itself with an LDS histogram of
//    the costs.  Kv heads are pinned to XCDs (workgroup w runs on XCD w % 8),
//    so the column groups that re-read one kv head's K/V share an L2.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <type_traits>

#include "check.h"
#include "model.h"
#include "nova_kernel.h"

namespace nova {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef __fp16 tr4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) tr4 lds_tr4;

constexpr int NH = Model::NH, NKV = Model::NKV, HD = Model::HD, G = Model::G, KVW = Model::KVW;
constexpr int NBUF = 4;                        // K/V tile buffers in LDS
constexpr int WAVES = 4;
constexpr int THREADS = WAVES * 64;
constexpr int TILE = 32;                       // keys per stage (2 pages)
constexpr int ROWB = HD * 2;                   // 256 B per K or V row of one kv head
constexpr int STAGE_BYTES = 2 * TILE * ROWB;   // K then V
constexpr int CHUNKS = STAGE_BYTES / 16;       // 16 B chunks per stage
constexpr int LOADS = CHUNKS / THREADS;        // staging loads per thread per tile
static_assert(CHUNKS % THREADS == 0, "stage must split evenly over the workgroup");
static_assert(THREADS == 256 && LOADS == 4, "staging layout: one page row per 16 lanes, K then V");
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazy = 8.0f;                  // rescale threshold, log2 units
constexpr int64_t kPageBytes = (int64_t)kKvBlock * KVW * 2;

static_assert(8 % NKV == 0, "kv heads are pinned to groups of 8 / NKV XCDs");
constexpr int kXcd = 8;                        // XCDs; workgroup w is dispatched to XCD w % 8
constexpr int kXcdPerHead = kXcd / NKV;
constexpr int kBuckets = 4096;                 // cost histogram (tiles; longer items share the top bucket)
constexpr int kRankMax = 4096;                  // beyond this many items: natural order
constexpr int kTabWin = 2048;                   // block-table entries held in LDS

struct PrefillArgs {
    const float* q;            // [n_sess][n_q][NH][HD]
    const uint16_t* pool_k;
    const uint16_t* pool_v;
    const int32_t* tables;
    int64_t table_stride;
    const int32_t* n_past;     // device [n_sess] or null -> n_past_scalar
    int n_past_scalar;
    int n_sess;
    int n_q;
    int layer;
    int nb;
    float* o;                  // [n_sess][n_q][NH][HD]
};

__device__ __forceinline__ int n_past_of(const PrefillArgs& a, int sess) {
    return a.n_past ? a.n_past[sess] : a.n_past_scalar;
}

// cost (key tiles) of item j = sess * n_cg + cg, clamped to the histogram
__device__ __forceinline__ int item_bucket(const PrefillArgs& a, int j, int n_cg, int n_cols, int cols_wg) {
    const int sess = j / n_cg, cg = j - sess * n_cg;
    const int last_col = min(cg * cols_wg + cols_wg, n_cols) - 1;
    const int key_end = n_past_of(a, sess) + last_col / G + 1;
    return min((key_end + TILE - 1) / TILE, kBuckets - 1);
}

// The item of rank r in decreasing cost order (ties in index order).  Every
// thread of the workgroup calls it (it has barriers) and gets the same answer.
// s_i: LDS scratch of kBuckets + NT + 16 ints; NT threads in the workgroup.
template <int NT>
__device__ int lpt_item(const PrefillArgs& a, int r, int n_cg, int n_cols, int cols_wg, int* s_i) {
    const int N = a.n_sess * n_cg;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int* hist = s_i;
    int* part = s_i + kBuckets;
    int* res = part + NT;          // [0] group, [1] ranks above it, [2] item, [4..] wave counts
    for (int b = tid; b < kBuckets; b += NT) hist[b] = 0;
    __syncthreads();
    for (int j = tid; j < N; j += NT) atomicAdd(&hist[item_bucket(a, j, n_cg, n_cols, cols_wg)], 1);
    __syncthreads();
    constexpr int PER = kBuckets / NT;
    int sum = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) sum += hist[PER * tid + u];
    part[tid] = sum;
    __syncthreads();
    constexpr int GPL = NT / 64;   // groups per lane
    if (wave == 0) {
        // lane l covers groups GPL*l .. GPL*l+GPL-1; ranks run from the highest group down
        int ls = 0;
#pragma unroll
        for (int u = 0; u < GPL; ++u) ls += part[GPL * lane + u];
        int incl = ls;                                // sum over lanes >= l
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int t = __shfl_down(incl, o, 64);
            if (lane + o < 64) incl += t;
        }
        int above = incl - ls;
#pragma unroll
        for (int u = GPL - 1; u >= 0; --u) {
            const int gsum = part[GPL * lane + u];
            if (r >= above && r < above + gsum) {
                res[0] = GPL * lane + u;
                res[1] = above;
            }
            above += gsum;
        }
    }
    __syncthreads();
    const int grp = res[0];
    int base = res[1], bucket = PER * grp + PER - 1, o = 0;
    for (int u = PER - 1; u >= 0; --u) {
        const int h = hist[PER * grp + u];
        if (r >= base && r < base + h) {
            bucket = PER * grp + u;
            o = r - base;
        }
        base += h;
    }
    // the o-th item (index order) whose cost falls in that bucket
    for (int j0 = 0; j0 < N; j0 += NT) {
        const int j = j0 + tid;
        const bool f = j < N && item_bucket(a, j, n_cg, n_cols, cols_wg) == bucket;
        const uint64_t bal = __builtin_amdgcn_ballot_w64(f);
        if (lane == 0) res[4 + wave] = __builtin_popcountll(bal);
        __syncthreads();
        int before = 0, total = 0;
#pragma unroll
        for (int ww = 0; ww < NT / 64; ++ww) {
            const int n = res[4 + ww];
            before += ww < wave ? n : 0;
            total += n;
        }
        before += __builtin_popcountll(bal & ((1ull << lane) - 1));
        if (f && before == o) res[2] = j;
        __syncthreads();
        if (o < total) break;
        o -= total;
    }
    const int item = res[2];
    __syncthreads();                    // the scratch is reused for K/V tiles
    return item;
}

// The four direct global -> LDS loads of a tile stage, 16 B per lane: load u
// makes the wave write 1 KiB at LDS byte address lds + 16*THREADS*u
// (wave-uniform), taken from m0 when the load issues.
// Issued as inline asm so that the compiler's own vmcnt bookkeeping does not
// see them: the builtin makes the compiler drain every pending load (including
// the tiles still meant to be in flight) before each LDS read it cannot prove
// disjoint.  The pipeline waits for these loads explicitly (tile_barrier);
// the compiler's waits for its own loads stay correct, as the counter drains
// in issue order.  m0 is a register the compiler reserves (it cannot be
// declared clobbered), so the statement saves and restores it.
__device__ __forceinline__ void dma16x4(const void* s0, const void* s1, const void* s2, const void* s3,
                                        uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %5\n\tglobal_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %6\n\tglobal_load_lds_dwordx4 %2, off\n\t"
        "s_mov_b32 m0, %7\n\tglobal_load_lds_dwordx4 %3, off\n\t"
        "s_mov_b32 m0, %8\n\tglobal_load_lds_dwordx4 %4, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(s0), "v"(s1), "v"(s2), "v"(s3), "s"(lds), "s"(lds + 16u * THREADS), "s"(lds + 32u * THREADS),
          "s"(lds + 48u * THREADS)
        : "memory");
}

// The same four loads for a tile with no row past the last key: wave-uniform
// page bases in SGPR pairs (K page 0, K page 1, V page 0, V page 1) and the
// lane's 32-bit offsets inside a page (one for K, one for V), so the loop
// keeps two offset registers instead of four 64-bit addresses per tile.
__device__ __forceinline__ void dma16x4_s(const void* k0, const void* k1, const void* v0, const void* v1,
                                          uint32_t off_k, uint32_t off_v, uint32_t lds) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %7\n\tglobal_load_lds_dwordx4 %5, %1\n\t"
        "s_mov_b32 m0, %8\n\tglobal_load_lds_dwordx4 %5, %2\n\t"
        "s_mov_b32 m0, %9\n\tglobal_load_lds_dwordx4 %6, %3\n\t"
        "s_mov_b32 m0, %10\n\tglobal_load_lds_dwordx4 %6, %4\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(k0), "s"(k1), "s"(v0), "s"(v1), "v"(off_k), "v"(off_v), "s"(lds), "s"(lds + 16u * THREADS),
          "s"(lds + 32u * THREADS), "s"(lds + 48u * THREADS)
        : "memory");
}

// LDS byte address of a __shared__ location
__device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
    return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const unsigned char*)p;
}

// workgroup barrier for the tile pipeline: the wave's own direct loads of the
// next tile are complete (vmcnt <= pending, the later tiles may stay in
// flight), then s_barrier; the empty asm statements keep the compiler from
// moving LDS accesses across it
template <int kPending>
__device__ __forceinline__ void tile_barrier() {
    if constexpr (kPending == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kPending) : "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// max / sum over the 4 rows of 16 lanes (lanes c, c+16, c+32, c+48) with the
// gfx950 row swaps instead of LDS permutes: op(a, b) over the two swap results
// is the xor-16 (then xor-32) combination for a symmetric op.
__device__ __forceinline__ float rows_max(float v) {
    auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(x[0]), __uint_as_float(x[1]));
    auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(y[0]), __uint_as_float(y[1]));
}

// 4 halfs of a 16-bit matrix, transposed across each group of 16 lanes
__device__ __forceinline__ u2 lds_read_tr(const unsigned char* p) {
    const auto lp = (lds_tr4*)(__attribute__((address_space(3))) unsigned char*)p;
    return __builtin_bit_cast(u2, __builtin_amdgcn_ds_read_tr16_b64_v4f16(lp));
}

// Swizzles: the 16 B chunk k of tile row r sits at position k ^ f(r) of the
// row.  K half: f(r) = r & 15 -- the score operand reads have the 16 lanes of
// a group on 16 different rows at one chunk.  V half: f(r) = 2 (r & 7) -- the
// transposing reads have each group on 4 consecutive rows at a chunk pair
// (2cb, 2cb+1), and 8 consecutive rows must land on 16 distinct positions.
// Both patterns are then free of bank conflicts.
__device__ __forceinline__ uint32_t swz_k(int row, int chunk) {
    return (uint32_t)(row * ROWB + ((chunk ^ (row & 15)) << 4));
}
__device__ __forceinline__ uint32_t swz_v(int row, int chunk) {
    return (uint32_t)(row * ROWB + ((chunk ^ (2 * (row & 7))) << 4));
}


// NB: 16-column blocks per wave.  KS: key groups -- KS groups of 4 waves
// share the workgroup's columns; group k takes the key tiles KS*i + k with
// its own ring of tile buffers, and the groups' softmax states are merged at
// the end.  2 waves per SIMD either way (<= 256 VGPRs): two 4-wave
// workgroups per CU (KS = 1) or one 8-wave workgroup (KS = 2); while one wave
// runs its softmax on the VALU the other keeps the matrix core busy.
template <int NB, int KS>
__global__ void __launch_bounds__(THREADS * KS, 2)
prefill_kernel(PrefillArgs a) {
    constexpr int NT = THREADS * KS;
    constexpr int COLS_WAVE = 16 * NB;
    constexpr int COLS_WG = COLS_WAVE * WAVES;
    __shared__ __attribute__((aligned(16))) unsigned char s_kv[KS][NBUF][STAGE_BYTES];
    __shared__ int32_t s_tab[kTabWin];
    static_assert((kBuckets + NT + 16) * 4 <= (int)sizeof(s_kv), "ranking scratch fits the tile buffers");
    static_assert(4 + NT / 64 <= 16 && kBuckets % NT == 0, "ranking scratch layout");
    static_assert(KS == 1 || KS * 64 * NB * 34 * 4 * WAVES / KS <= (int)sizeof(s_kv), "merge scratch");

    const int tid = threadIdx.x;
    const int kg = tid / THREADS;                // key group
    const int wave = (tid >> 6) & (WAVES - 1);   // wave within the group: its columns
    const int gtid = tid & (THREADS - 1);
    const int lane = tid & 63;
    const int g = lane >> 4;
    const int c = lane & 15;
    const int n_cols = a.n_q * G;
    const int n_cg = (n_cols + COLS_WG - 1) / COLS_WG;
    const int N = a.n_sess * n_cg;
    // workgroup -> (kv head, rank): kv head h runs on XCDs [h*kXcdPerHead, +kXcdPerHead)
    const int xcd = (int)blockIdx.x % kXcd;
    const int kvh = xcd / kXcdPerHead;
    const int rank = ((int)blockIdx.x / kXcd) * kXcdPerHead + xcd % kXcdPerHead;
    if (rank >= N) return;                                  // grid padding (uniform)
    int item;
    if (a.n_sess == 1 || N > kRankMax) item = (rank / n_cg) * n_cg + (n_cg - 1 - rank % n_cg);
    else item = lpt_item<NT>(a, rank, n_cg, n_cols, COLS_WG, reinterpret_cast<int*>(&s_kv[0][0][0]));
    const int sess = item / n_cg;
    const int cg = item - sess * n_cg;
    const int n_past = n_past_of(a, sess);
    const int32_t* table = a.tables + (int64_t)sess * a.table_stride;
    const float* qs = a.q + (int64_t)sess * a.n_q * NH * HD;
    float* os = a.o + (int64_t)sess * a.n_q * NH * HD;

    const int wg_col0 = cg * COLS_WG;
    const int wg_col_last = min(wg_col0 + COLS_WG, n_cols) - 1;
    const int key_end = n_past + wg_col_last / G + 1;         // keys the workgroup needs
    const int n_tiles = (key_end + TILE - 1) / TILE;
    const int n_steps = (n_tiles + KS - 1) / KS;               // tiles per key group (rounded up)
    const int col0 = wg_col0 + wave * COLS_WAVE;
    const int wave_last = min(col0 + COLS_WAVE, n_cols) - 1;
    const int wave_key_end = col0 < n_cols ? n_past + wave_last / G + 1 : 0;
    const int key_min_full = n_past + col0 / G + 1;           // keys below: visible to all columns

    // ---- staging ----
    // Stage chunk q = tid + THREADS*u (u = 0..3): K for u < 2, V for u >= 2;
    // page u & 1 of the tile; row (tid >> 4) of that page; LDS position
    // tid & 15 of the row holds global chunk (tid & 15) ^ f(tid >> 4), with the
    // K or V swizzle f.  So a lane's offset inside a page is one of two values
    // for all four loads, and each load instruction of a wave covers 4 rows of
    // one page (wave-uniform base).
    const char* pk = reinterpret_cast<const char*>(a.pool_k);
    const char* pv = reinterpret_cast<const char*>(a.pool_v);
    const int64_t layer_page0 = (int64_t)a.layer * a.nb;
    const int n_pages = (key_end + kKvBlock - 1) >> kKvBlockShift;
    const int srow = gtid >> 4;                              // row inside the page
    const int schunk_k = (gtid & 15) ^ srow;                 // global chunk this lane moves (K, V)
    const int schunk_v = (gtid & 15) ^ (2 * (srow & 7));
    const uint32_t loff_k = (uint32_t)(srow * (KVW * 2) + 16 * schunk_k);
    const uint32_t loff_v = (uint32_t)(srow * (KVW * 2) + 16 * schunk_v);
    const uint32_t wave_s = __builtin_amdgcn_readfirstlane(wave);
    int win0 = 0;                                            // first page of the LDS table window
    auto load_window = [&](int first) {                      // every thread, uniform
        for (int e = tid; e < kTabWin && first + e < n_pages; e += NT) s_tab[e] = table[first + e];
        __syncthreads();
        win0 = first;
    };
    load_window(0);
    // physical pages of this group's tile of step i (tile KS*i + kg), read
    // from the LDS table a step before the loads that use them.  Every wave
    // calls this at the same points with the same i, so the window (which
    // only moves forward, between barriers) is moved by all of them together.
    struct Pages { int p0, p1; };
    auto read_pages = [&](int i) -> Pages {
        const int pg_first = 2 * KS * i;                     // first page of step i's tiles
        if (pg_first < n_pages && pg_first + 2 * KS - 1 - win0 >= kTabWin) {
            __syncthreads();                                 // every wave is done with the old window
            load_window(pg_first);
        }
        const int T = KS * i + kg;
        if (T >= n_tiles) return Pages{0, 0};                // no such tile for this group
        const int pg0 = 2 * T;
        const int pg1 = pg0 + 1 < n_pages ? pg0 + 1 : pg0;   // a lone last page loads itself twice
        return Pages{s_tab[pg0 - win0], s_tab[pg1 - win0]};
    };
    auto load_tile = [&](auto buf_tag, int T, Pages pp) {
        constexpr int BI = decltype(buf_tag)::value;
        const int64_t b0 = (layer_page0 + __builtin_amdgcn_readfirstlane(pp.p0)) * kPageBytes + kvh * ROWB;
        const int64_t b1 = (layer_page0 + __builtin_amdgcn_readfirstlane(pp.p1)) * kPageBytes + kvh * ROWB;
        const uint32_t m0base = __builtin_amdgcn_readfirstlane(lds_addr(&s_kv[kg][BI][0])) + 1024u * wave_s;
        if (TILE * (T + 1) <= key_end) {
            dma16x4_s(pk + b0, pk + b1, pv + b0, pv + b1, loff_k, loff_v, m0base);
        } else {
            // the tile holding the last key: rows past it (never written, may
            // hold NaN bits) load the last key's row instead; their weights are
            // masked to zero
            const int rl = key_end - 1 - TILE * T;           // in [0, TILE)
            const int64_t bl = ((rl >> 4) ? b1 : b0) + (int64_t)(rl & 15) * (KVW * 2);
            const void* src[LOADS];
#pragma unroll
            for (int u = 0; u < LOADS; ++u) {
                const int row = srow + 16 * (u & 1);
                const char* pool = u < 2 ? pk + 16 * schunk_k : pv + 16 * schunk_v;
                const int64_t rowoff = (int64_t)srow * (KVW * 2);
                src[u] = TILE * T + row < key_end ? pool + ((u & 1) ? b1 : b0) + rowoff : pool + bl;
            }
            dma16x4(src[0], src[1], src[2], src[3], m0base);
        }
    };

    // the group's tiles of steps 0, 1, 2 start loading; step 3's pages are read
    Pages pp = read_pages(0);
    if (kg < n_tiles) load_tile(std::integral_constant<int, 0>{}, kg, pp);
    pp = read_pages(1);
    if (KS + kg < n_tiles) load_tile(std::integral_constant<int, 1>{}, KS + kg, pp);
    pp = read_pages(2);
    if (2 * KS + kg < n_tiles) load_tile(std::integral_constant<int, 2>{}, 2 * KS + kg, pp);
    pp = read_pages(3);

    // ---- Q^T operands: lane (g,c) of block b holds column col0 + 16b + c ----
    // x = q * (1/sqrt(HD) * log2 e) is split x = hi + lo into two fp16 terms
    // after scaling the column by a power of two up = 2^k (the column's largest
    // |x| lands in [2^14, 2^15)), so lo keeps the bits hi drops (~2^-22 of the
    // column's scale instead of fp16's 2^-11) and stays a normal number; the
    // score MFMAs run once per term, and the scores come out multiplied by up,
    // which qf = 1/up undoes per lane.
    h8 qh[NB][4], ql[NB][4];
    float qf[NB];
    int qpos[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int col = col0 + 16 * b + c;
        const bool real = col < n_cols;
        const int qi = real ? col / G : 0;
        const int hh = real ? col - qi * G : 0;
        qpos[b] = real ? n_past + qi : -1;
        const float* qp = qs + ((int64_t)qi * NH + kvh * G + hh) * HD + 8 * g;
        float xv[4][8];
        float amax = 0.f;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const f4 x0 = *reinterpret_cast<const f4*>(qp + 32 * ks);
            const f4 x1 = *reinterpret_cast<const f4*>(qp + 32 * ks + 4);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                xv[ks][j] = real ? x0[j] * (kScale * kLog2e) : 0.f;
                xv[ks][4 + j] = real ? x1[j] * (kScale * kLog2e) : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(xv[ks][j]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 16, 64));   // the column's 128 dims sit in lanes c, c+16, c+32, c+48
        amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
        int ex = 0;
        if (amax > 0.f) (void)frexpf(amax, &ex);
        const int k2 = amax > 0.f ? 15 - ex : 0;
        const float up = ldexpf(1.f, k2);
        qf[b] = ldexpf(1.f, -k2);
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float x = xv[ks][j] * up;
                const _Float16 h = (_Float16)x;
                qh[b][ks][j] = h;
                ql[b][ks][j] = (_Float16)(x - (float)h);
            }
        }
    }

    // Running max m of the lane's column (log2 units); x = s - m is formed as
    // one fma of the raw (scaled) MFMA score with qf and -m.  m starts at 0;
    // the wave's first tile always rescales.
    float m[NB];
    float lsum[NB];       // this lane's share (its 8 keys of each tile) of column c's row sum
    f4 acc[NB][8];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        m[b] = 0.f;
        lsum[b] = 0.f;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[b][cb] = f4{0.f, 0.f, 0.f, 0.f};
    }

    // operand addresses inside a stage (the buffer adds a compile-time offset):
    // K rows c (page 0) and 16 + c (page 1), chunk 4ks + g; V^T: lane s of
    // group g reads key row 4g + (s >> 2) (and +16, the second page), halfs
    // 16cb + 4 (s & 3) .. +3 of it
    // (the group's ring is folded into the lane offsets)
    uint32_t koff[4], voff[8];
    const uint32_t ring = (uint32_t)kg * NBUF * STAGE_BYTES;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) koff[ks] = ring + swz_k(c, 4 * ks + g);
    {
        const int vr = 4 * g + (c >> 2);
        const int vh = (c >> 1) & 1;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) voff[cb] = ring + TILE * ROWB + swz_v(vr, 2 * cb + vh) + 8 * (c & 1);
    }
    const unsigned char* s_ring0 = &s_kv[0][0][0];

    // the group's tiles of steps 0 and 1 resident (step 2's may still be loading)
    if (2 * KS + kg < n_tiles) tile_barrier<LOADS>();
    else tile_barrier<0>();

    // S^T = K . Q^T for both pages of the tile in buffer BI and all blocks
    auto compute_s = [&](auto buf_tag, f4 (&s0)[NB], f4 (&s1)[NB]) {
        constexpr int BI = decltype(buf_tag)::value;
        const unsigned char* sk = s_ring0 + BI * STAGE_BYTES;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const h8 k0 = __builtin_bit_cast(h8, *reinterpret_cast<const u4*>(sk + koff[ks]));
            const h8 k1 = __builtin_bit_cast(h8, *reinterpret_cast<const u4*>(sk + koff[ks] + 16 * ROWB));
            // the hi terms of every accumulator, then the lo terms: 2*NB
            // independent MFMAs between two that share an accumulator
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                s0[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qh[b][ks], ks ? s0[b] : f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                s1[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qh[b][ks], ks ? s1[b] : f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            }
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                s0[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, ql[b][ks], s0[b], 0, 0, 0);
                s1[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, ql[b][ks], s1[b], 0, 0, 0);
            }
        }
    };
    // One tile: online softmax of the scores c (buffer BI) and O^T += V^T . P^T,
    // with the next tile's score MFMAs (buffer NI, into n) issued in the same
    // basic block as this tile's row maxima so that the matrix core and the
    // VALU work side by side.  kMask selects the causal masking (only tiles
    // that cross the diagonal or the end of the keys need it).
    auto tile = [&](auto mask_tag, auto buf_tag, auto next_tag, int key_base, bool first, const f4 (&c0)[NB],
                    const f4 (&c1)[NB], f4 (&n0)[NB], f4 (&n1)[NB]) {
        constexpr bool kMask = decltype(mask_tag)::value;
        constexpr int BI = decltype(buf_tag)::value;
        const unsigned char* sv = s_ring0 + BI * STAGE_BYTES;
        // V^T operands: va[cb] row c = d 16cb + c, k = keys kappa(g, j) =
        // (page j / 4, slot 4g + j % 4), the k order of P^T below
        h8 va[8];                // read after the next tile's score MFMAs (below)
        compute_s(next_tag, n0, n1);
        // x = s - m; the common case only asks whether any score of the wave
        // exceeds its column's max by more than kLazy (a lane-local test)
        float x[NB][8];
        bool ok[NB][8];
        float lmax[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) {
                x[b][ii] = fmaf(c0[b][ii], qf[b], -m[b]);
                x[b][4 + ii] = fmaf(c1[b][ii], qf[b], -m[b]);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int key = key_base + (j < 4 ? 0 : 16) + 4 * g + (j & 3);
                ok[b][j] = !kMask || key <= qpos[b];
            }
            float v = -INFINITY;
#pragma unroll
            for (int j = 0; j < 8; ++j) v = ok[b][j] ? fmaxf(v, x[b][j]) : v;
            lmax[b] = v;
        }
        // the weights, assuming no column's max moves (recomputed below if one
        // does): computed here so that they overlap the next tile's MFMAs
        h8 ph[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int j = 0; j < 8; ++j) ph[b][j] = (_Float16)(ok[b][j] ? __builtin_amdgcn_exp2f(x[b][j]) : 0.f);
        // score MFMAs of the next tile interleaved with the work above
#ifndef NOVA_PREFILL_SCHED_VALU
#define NOVA_PREFILL_SCHED_VALU 6
#endif
#pragma unroll
        for (int i = 0; i < 16 * NB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA (hi or lo term)
            __builtin_amdgcn_sched_group_barrier(0x002, NOVA_PREFILL_SCHED_VALU, 0);
        }
        // the V^T operands, read here rather than at the start of the tile:
        // 32 registers fewer across the score MFMAs and the softmax (7 spilled
        // registers instead of 16 at 256 VGPRs), 184.5 -> 182.3 us per config-5 layer
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) {
            const u2 lo = lds_read_tr(sv + voff[cb]);
            const u2 hi = lds_read_tr(sv + voff[cb] + 16 * ROWB);
            va[cb] = __builtin_bit_cast(h8, u4{lo[0], lo[1], hi[0], hi[1]});
        }
        bool over = false;
#pragma unroll
        for (int b = 0; b < NB; ++b) over |= lmax[b] > kLazy;
        if (__builtin_amdgcn_ballot_w64(over) || first) {
            // rare (and the group's first tile): move the max of every column whose
            // tile max exceeds it by more than kLazy.  bm = -inf: no key of the
            // column in this tile, nothing moves.
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const float bm = rows_max(lmax[b]);
                const bool need = bm > -INFINITY && (first || bm > kLazy);
                const float shift = need ? bm : 0.f;
                const float corr = first ? 0.f : __builtin_amdgcn_exp2f(-shift);
                lsum[b] *= corr;
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) acc[b][cb] *= corr;
                m[b] += shift;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    ph[b][j] = (_Float16)(ok[b][j] ? __builtin_amdgcn_exp2f(x[b][j] - shift) : 0.f);
            }
        }
        __builtin_amdgcn_s_setprio(1);   // the PV MFMAs go first on the SIMD
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            // l += the lane's 8 fp16 weights, exactly those applied below,
            // summed in fp32 by four v_dot2 against (1, 1)
#pragma unroll
            for (int j = 0; j < 8; j += 2)
                lsum[b] = __builtin_amdgcn_fdot2(h2{ph[b][j], ph[b][j + 1]}, h2{(_Float16)1.0f, (_Float16)1.0f},
                                                 lsum[b], false);
#pragma unroll
            for (int cb = 0; cb < 8; ++cb)
                acc[b][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va[cb], ph[b], acc[b][cb], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
    };

    // Tile pipeline over NBUF = 4 buffers per group.  Step i (buffer i % 4):
    // issue the loads of the group's tile of step i+3 into the buffer of step
    // i-1 and read step i+4's pages; run the group's tile of step i (softmax
    // and PV, with step i+1's score MFMAs alongside); then the barrier makes
    // step i+2's tile resident (step i+3's may stay in flight).  A wave's last
    // tile computes scores of a buffer it will not use: they are discarded.
    const int wave_tiles = (wave_key_end + TILE - 1) / TILE;   // tiles the wave's columns need
    f4 sa0[NB], sa1[NB], sb0[NB], sb1[NB];
    if (kg < wave_tiles) compute_s(std::integral_constant<int, 0>{}, sa0, sa1);
    auto step = [&](auto buf_tag, int i, f4 (&c0)[NB], f4 (&c1)[NB], f4 (&n0)[NB], f4 (&n1)[NB]) {
        constexpr int BI = decltype(buf_tag)::value;
        const int t = KS * i + kg;                           // the group's tile
        const bool ahead = t + 3 * KS < n_tiles;
        if (ahead) load_tile(std::integral_constant<int, (BI + 3) % NBUF>{}, t + 3 * KS, pp);
        if (i + 4 < n_steps) pp = read_pages(i + 4);         // every wave, same i
        if (t < wave_tiles) {
            const int key_base = t * TILE;
            constexpr auto next = std::integral_constant<int, (BI + 1) % NBUF>{};
            // a tile needs no mask when every key in it exists and is visible
            // to every column of the wave
            if (key_base + TILE <= key_min_full)
                tile(std::integral_constant<bool, false>{}, buf_tag, next, key_base, i == 0, c0, c1, n0, n1);
            else
                tile(std::integral_constant<bool, true>{}, buf_tag, next, key_base, i == 0, c0, c1, n0, n1);
        }
        if (ahead) tile_barrier<LOADS>();
        else tile_barrier<0>();
    };
    for (int i = 0; i < n_steps; i += NBUF) {               // unrolled: buffers and score registers rotate
        step(std::integral_constant<int, 0>{}, i, sa0, sa1, sb0, sb1);
        if (i + 1 < n_steps) step(std::integral_constant<int, 1>{}, i + 1, sb0, sb1, sa0, sa1);
        if (i + 2 < n_steps) step(std::integral_constant<int, 2>{}, i + 2, sa0, sa1, sb0, sb1);
        if (i + 3 < n_steps) step(std::integral_constant<int, 3>{}, i + 3, sb0, sb1, sa0, sa1);
    }

    // the column's row sum over its four 16-lane rows
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        lsum[b] += __shfl_xor(lsum[b], 16, 64);
        lsum[b] += __shfl_xor(lsum[b], 32, 64);
    }

    if constexpr (KS == 2) {
        // merge group 1's (m, l, acc) into group 0's through LDS (the tile
        // buffers are free: the last step ended with a barrier)
        float* xs = reinterpret_cast<float*>(&s_kv[0][0][0]) + (wave * 64 + lane) * (NB * 34);
        if (kg == 1) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) *reinterpret_cast<f4*>(xs + b * 34 + 4 * cb) = acc[b][cb];
                xs[b * 34 + 32] = lsum[b];
                xs[b * 34 + 33] = m[b];
            }
        }
        __syncthreads();
        if (kg == 1) return;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const float l1 = xs[b * 34 + 32], m1 = xs[b * 34 + 33], l0 = lsum[b];
            // a group without keys for this column has l = 0 and must not set the max
            const float mm = l1 > 0.f ? (l0 > 0.f ? fmaxf(m[b], m1) : m1) : m[b];
            const float f0 = l0 > 0.f ? __builtin_amdgcn_exp2f(m[b] - mm) : 0.f;
            const float f1 = l1 > 0.f ? __builtin_amdgcn_exp2f(m1 - mm) : 0.f;
#pragma unroll
            for (int cb = 0; cb < 8; ++cb)
                acc[b][cb] = acc[b][cb] * f0 + *reinterpret_cast<const f4*>(xs + b * 34 + 4 * cb) * f1;
            lsum[b] = l0 * f0 + l1 * f1;
        }
    }

    // ---- normalise and store: lane (g,c) of block b holds d = 16cb + 4g + i ----
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const float L = lsum[b];
        const int col = col0 + 16 * b + c;
        if (col >= n_cols) continue;
        const int qi = col / G, hh = col - qi * G;
        float* op = os + ((int64_t)qi * NH + kvh * G + hh) * HD;
        const float inv = 1.f / L;
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) *reinterpret_cast<f4*>(op + 16 * cb + 4 * g) = acc[b][cb] * inv;
    }
}

int compute_units() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        NOVA_HIP(hipGetDevice(&dev));
        NOVA_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    }
    return cus;
}

#ifndef NOVA_PREFILL_KS_WIDE
#define NOVA_PREFILL_KS_WIDE 1
#endif
#ifndef NOVA_PREFILL_KS_NARROW
#define NOVA_PREFILL_KS_NARROW 2
#endif
#ifndef NOVA_PREFILL_NB_WIDE
#define NOVA_PREFILL_NB_WIDE 2
#endif
constexpr int kNbWide = NOVA_PREFILL_NB_WIDE;      // 16-column blocks per wave in wide launches
constexpr int kKsWide = NOVA_PREFILL_KS_WIDE;      // key groups with 128-column workgroups
constexpr int kKsNarrow = NOVA_PREFILL_KS_NARROW;  // and with 64-column workgroups

// Column groups of 128 (2 blocks per wave) when the launch has enough work
// items to fill every workgroup slot of the chip (two 4-wave or one 8-wave
// workgroup per CU); otherwise of 64 (1 block per wave):
// twice the workgroups for a single session's chunk, each with half the
// columns (same key tiles, half the work per tile).
void launch(const PrefillArgs& a, int n_sess, hipStream_t s) {
    const int64_t slots = (int64_t)compute_units() * (2 / kKsWide);
    const int64_t items128 = (a.n_q * G + 127) / 128 * (int64_t)n_sess * NKV;
    const bool wide = items128 >= slots;
    const int cols_wg = wide ? 64 * kNbWide : 64;
    const int64_t n_cg = (a.n_q * G + cols_wg - 1) / cols_wg;
    const int64_t n_wg = (n_cg * n_sess * NKV + kXcd - 1) / kXcd * kXcd;
    NOVA_REQUIRE(n_wg < (int64_t)1 << 31);
    if (wide)
        hipLaunchKernelGGL((prefill_kernel<kNbWide, kKsWide>), dim3((unsigned)n_wg), dim3(THREADS * kKsWide), 0, s, a);
    else
        hipLaunchKernelGGL((prefill_kernel<1, kKsNarrow>), dim3((unsigned)n_wg), dim3(THREADS * kKsNarrow), 0, s, a);
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
    a.n_sess = 1;
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
    a.n_sess = n_sess;
    a.n_q = n_q;
    a.layer = layer;
    a.nb = nb;
    a.o = o;
    launch(a, n_sess, reinterpret_cast<hipStream_t>(s));
}

}  // extern "C"
