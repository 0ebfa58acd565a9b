// kv_pages.hip -- page-granular KV movement for gfx950: paged append, batched
// copy-on-write page copies, page clears and device block-table patches.
//
// All of it is HBM-bound byte movement, so every lane moves 16 B (one
// global_load/store_dwordx4) and consecutive lanes touch consecutive bytes.
//
//  * kv_store: replaces kv_store_paged_kernel (reference src/kernel/elem.cu:59-76,
//    launcher :93-98).  The reference maps one fp32 element per thread with a
//    (token, kv head) grid; here one lane moves 8 fp16 of a token row and a
//    workgroup covers whole rows, so the table is read once per row.
//  * cow_copy: replaces the 2L cudaMemcpyAsync of Engine::cow_guard
//    (src/model.cpp:171-191) with one launch for any number of COW pairs:
//    grid.y = pair, grid.x walks the 2*L pages (K and V per layer) of that pair.
//  * zero_pages: the per-page cudaMemsetAsync loop of SessionManager::create
//    (code/session.h:107-118) as one launch.
//  * table_patch: the 4-byte H2D table writes of cow_guard (model.cpp:188-190)
//    for a batch of COWs, done as a kernel so it orders with the copies on
//    the same stream without host round trips.
#include <hip/hip_runtime.h>
#include <cstdint>

#include "check.h"
#include "model.h"
#include "nova_kernel.h"

namespace nova {
namespace {

typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int KVW = Model::KVW;
constexpr int64_t kPageHalves = (int64_t)kKvBlock * KVW;
constexpr int kRowVecs = KVW / 8;            // 16 B vectors per token row
constexpr int kPageVecs = (int)(kPageHalves / 8);

__global__ void __launch_bounds__(256)
kv_store_kernel(uint16_t* __restrict__ pool_k, uint16_t* __restrict__ pool_v,
                const int32_t* __restrict__ table, int layer, int nb, int n, int64_t pos0,
                const uint16_t* __restrict__ k, const uint16_t* __restrict__ v) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // vector index
    if (e >= (int64_t)n * kRowVecs) return;
    const int t = (int)(e / kRowVecs);
    const int col = (int)(e - (int64_t)t * kRowVecs);
    const int64_t pos = pos0 + t;
    const int phys = table[pos >> kKvBlockShift];
    const int64_t dst = (((int64_t)layer * nb + phys) * kKvBlock + (pos & kKvBlockMask)) * KVW + 8 * col;
    const int64_t src = (int64_t)t * KVW + 8 * col;
    *reinterpret_cast<u4*>(pool_k + dst) = *reinterpret_cast<const u4*>(k + src);
    *reinterpret_cast<u4*>(pool_v + dst) = *reinterpret_cast<const u4*>(v + src);
}

// batched append: session i writes n tokens at positions pos0[i] .. pos0[i]+n-1
// through tables + i*stride; k/v are [n_sess][n][NKV][HD]
__global__ void __launch_bounds__(256)
kv_store_batch_kernel(uint16_t* __restrict__ pool_k, uint16_t* __restrict__ pool_v,
                      const int32_t* __restrict__ tables, int64_t stride, const int32_t* __restrict__ pos0,
                      int layer, int nb, int n, const uint16_t* __restrict__ k, const uint16_t* __restrict__ v) {
    const int sess = blockIdx.y;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= (int64_t)n * kRowVecs) return;
    const int t = (int)(e / kRowVecs);
    const int col = (int)(e - (int64_t)t * kRowVecs);
    const int64_t pos = (int64_t)pos0[sess] + t;
    const int phys = tables[sess * stride + (pos >> kKvBlockShift)];
    const int64_t dst = (((int64_t)layer * nb + phys) * kKvBlock + (pos & kKvBlockMask)) * KVW + 8 * col;
    const int64_t src = ((int64_t)sess * n + t) * KVW + 8 * col;
    *reinterpret_cast<u4*>(pool_k + dst) = *reinterpret_cast<const u4*>(k + src);
    *reinterpret_cast<u4*>(pool_v + dst) = *reinterpret_cast<const u4*>(v + src);
}

// grid: x = chunks over the 2*L pages of a pair, y = pair index
__global__ void __launch_bounds__(256)
cow_copy_kernel(uint16_t* __restrict__ pool_k, uint16_t* __restrict__ pool_v, int nb,
                const int32_t* __restrict__ src, const int32_t* __restrict__ dst) {
    const int pair = blockIdx.y;
    const int s = src[pair], d = dst[pair];
    const int64_t per_pair = 2LL * Model::L * kPageVecs;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per_pair;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = e / kPageVecs;          // 0..2L-1: (layer, K/V)
        const int64_t off = e - page * kPageVecs;
        const int layer = (int)(page >> 1);
        uint16_t* pool = (page & 1) ? pool_v : pool_k;
        const int64_t lb = (int64_t)layer * nb;
        const u4 x = *reinterpret_cast<const u4*>(pool + (lb + s) * kPageHalves + 8 * off);
        *reinterpret_cast<u4*>(pool + (lb + d) * kPageHalves + 8 * off) = x;
    }
}

__global__ void __launch_bounds__(256)
zero_pages_kernel(uint16_t* __restrict__ pool_k, uint16_t* __restrict__ pool_v, int nb,
                  const int32_t* __restrict__ pages) {
    const int pg = pages[blockIdx.y];
    const int64_t per = 2LL * Model::L * kPageVecs;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = e / kPageVecs;
        const int64_t off = e - page * kPageVecs;
        uint16_t* pool = (page & 1) ? pool_v : pool_k;
        *reinterpret_cast<u4*>(pool + ((int64_t)(page >> 1) * nb + pg) * kPageHalves + 8 * off) =
            u4{0u, 0u, 0u, 0u};
    }
}

__global__ void table_patch_kernel(int32_t* __restrict__ table, const int32_t* __restrict__ idx,
                                   const int32_t* __restrict__ val, int n) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n) table[idx[e]] = val[e];
}

constexpr int kOpsPerLaunch = 64;
struct CowOps {
    nova_cow_op op[kOpsPerLaunch];
};

// grid: x = chunks over the 2*L pages of an op, y = op index.  Block (0, y)
// also patches the table entry; the copy reads only pool pages, so the order
// between the two does not matter within the launch.
__global__ void __launch_bounds__(256)
cow_apply_kernel(uint16_t* __restrict__ pool_k, uint16_t* __restrict__ pool_v, int nb,
                 int32_t* __restrict__ tables, CowOps ops) {
    const nova_cow_op o = ops.op[blockIdx.y];
    if (blockIdx.x == 0 && threadIdx.x == 0 && tables) tables[o.table_index] = o.dst;
    const int64_t per_pair = 2LL * Model::L * kPageVecs;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < per_pair;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t page = e / kPageVecs;
        const int64_t off = e - page * kPageVecs;
        const int layer = (int)(page >> 1);
        uint16_t* pool = (page & 1) ? pool_v : pool_k;
        const int64_t lb = (int64_t)layer * nb;
        const u4 x = *reinterpret_cast<const u4*>(pool + (lb + o.src) * kPageHalves + 8 * off);
        *reinterpret_cast<u4*>(pool + (lb + o.dst) * kPageHalves + 8 * off) = x;
    }
}

int copy_chunks() {
    // 2L pages of 16 KiB..32 KiB per pair: spread each pair over several
    // workgroups so a handful of COWs still fill the chip.
    const int64_t per_pair = 2LL * Model::L * kPageVecs;
    int64_t chunks = (per_pair + 256 * 8 - 1) / (256 * 8);
    return (int)(chunks < 1 ? 1 : chunks);
}

}  // namespace
}  // namespace nova

using namespace nova;

extern "C" {

void launch_kv_store_paged(uint16_t* pool_k, uint16_t* pool_v, const int32_t* table, int layer, int nb,
                           int n, int64_t pos0, const uint16_t* k, const uint16_t* v, nova_stream_t s) {
    NOVA_REQUIRE(pool_k && pool_v && table && k && v);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n >= 0 && pos0 >= 0);
    if (n == 0) return;
    const int64_t vecs = (int64_t)n * kRowVecs;
    hipLaunchKernelGGL(kv_store_kernel, dim3((unsigned)((vecs + 255) / 256)), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), pool_k, pool_v, table, layer, nb, n, pos0, k, v);
    NOVA_LAUNCHED();
}

void launch_kv_store_paged_batch(uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables, int table_stride,
                                 const int32_t* pos0, int n_sess, int layer, int nb, int n, const uint16_t* k,
                                 const uint16_t* v, nova_stream_t s) {
    NOVA_REQUIRE(pool_k && pool_v && tables && pos0 && k && v);
    NOVA_REQUIRE(layer >= 0 && layer < Model::L && nb > 0 && n >= 0 && n_sess >= 1 && n_sess <= 65535);
    NOVA_REQUIRE(table_stride > 0);
    if (n == 0) return;
    const int64_t vecs = (int64_t)n * kRowVecs;
    hipLaunchKernelGGL(kv_store_batch_kernel, dim3((unsigned)((vecs + 255) / 256), n_sess), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), pool_k, pool_v, tables, (int64_t)table_stride, pos0, layer,
                       nb, n, k, v);
    NOVA_LAUNCHED();
}

void launch_kv_cow_copy(uint16_t* pool_k, uint16_t* pool_v, int nb, const int32_t* src, const int32_t* dst,
                        int n_pairs, nova_stream_t s) {
    NOVA_REQUIRE(pool_k && pool_v && nb > 0 && n_pairs >= 0 && n_pairs <= 65535);
    if (n_pairs == 0) return;
    NOVA_REQUIRE(src && dst);
    hipLaunchKernelGGL(cow_copy_kernel, dim3(copy_chunks(), n_pairs), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), pool_k, pool_v, nb, src, dst);
    NOVA_LAUNCHED();
}

void launch_kv_cow_apply(uint16_t* pool_k, uint16_t* pool_v, int nb, int32_t* tables_dev,
                         const nova_cow_op* ops, int n_ops, nova_stream_t s) {
    NOVA_REQUIRE(pool_k && pool_v && nb > 0 && n_ops >= 0);
    for (int base = 0; base < n_ops; base += kOpsPerLaunch) {
        const int n = n_ops - base < kOpsPerLaunch ? n_ops - base : kOpsPerLaunch;
        CowOps o{};
        for (int e = 0; e < n; ++e) {
            NOVA_REQUIRE(ops[base + e].src >= 0 && ops[base + e].src < nb);
            NOVA_REQUIRE(ops[base + e].dst >= 0 && ops[base + e].dst < nb);
            o.op[e] = ops[base + e];
        }
        hipLaunchKernelGGL(cow_apply_kernel, dim3(copy_chunks(), n), dim3(256), 0,
                           reinterpret_cast<hipStream_t>(s), pool_k, pool_v, nb, tables_dev, o);
        NOVA_LAUNCHED();
    }
}

void launch_kv_zero_pages(uint16_t* pool_k, uint16_t* pool_v, int nb, const int32_t* pages, int n_pages,
                          nova_stream_t s) {
    NOVA_REQUIRE(pool_k && pool_v && nb > 0 && n_pages >= 0 && n_pages <= 65535);
    if (n_pages == 0) return;
    NOVA_REQUIRE(pages);
    hipLaunchKernelGGL(zero_pages_kernel, dim3(copy_chunks(), n_pages), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), pool_k, pool_v, nb, pages);
    NOVA_LAUNCHED();
}

void launch_table_patch(int32_t* table_dev, const int32_t* idx, const int32_t* val, int n, nova_stream_t s) {
    NOVA_REQUIRE(n >= 0);
    if (n == 0) return;
    NOVA_REQUIRE(table_dev && idx && val);
    hipLaunchKernelGGL(table_patch_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(s), table_dev, idx, val, n);
    NOVA_LAUNCHED();
}

nova_geometry nova_model_geometry(void) {
    nova_geometry g;
    g.nh = Model::NH;
    g.nkv = Model::NKV;
    g.hd = Model::HD;
    g.n_layers = Model::L;
    g.kv_block = kKvBlock;
    g.max_split = kMaxSplit;
    g.name = kModelName;
    return g;
}

}  // extern "C"
