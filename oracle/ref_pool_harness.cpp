// ref_pool_harness.cpp -- C-ABI harness over the reference's own paging headers
// (TEST INFRASTRUCTURE).  Compiled by oracle/Makefile against the untouched
// sources under the reference tree into oracle/_ref/libnova_ref_pool.so; tests
// use it to pin the C oracle (oracle/nova_oracle.c) bit-exactly.
//
// Wrapped reference symbols: nova::KvPool (code/graph/kv_pool.h:68-197),
// nova::kv_hash_ids / kv_hash_text / kv_hash_hex (code/graph/kv_block.h:21-79),
// nova::BlockRegistry (code/graph/kv_registry.h:26-66).
#include <cstdint>
#include <cstring>
#include <vector>
#include "graph/kv_pool.h"
#include "graph/kv_block.h"
#include "graph/kv_registry.h"

namespace {
// KvPool keeps live slices in a reserved std::vector in acquisition order and
// release() erases by value, so element k of that vector sits at base + k.  The
// harness mirrors that order to re-derive each id's current KvSlice address.
struct Handle {
    nova::KvPool pool;
    nova::KvSlice* base = nullptr;
    std::vector<int> order;
    nova::KvSlice* slice(int id) {
        for (size_t k = 0; k < order.size(); ++k)
            if (order[k] == id) return base + k;
        return nullptr;
    }
};
}  // namespace

extern "C" {
void* ref_pool_new(int n_slices, int64_t ctx) {
    Handle* h = new Handle;
    h->pool.init(n_slices, ctx);
    return h;
}
void ref_pool_delete(void* p) { delete static_cast<Handle*>(p); }
int ref_pool_acquire(void* p) {
    Handle* h = static_cast<Handle*>(p);
    nova::KvSlice* s = h->pool.acquire();
    if (!s) return -1;
    if (h->order.empty()) h->base = s;
    h->order.push_back(s->id);
    return s->id;
}
int ref_pool_alloc_block(void* p) { return static_cast<Handle*>(p)->pool.alloc_block(); }
void ref_pool_free_block(void* p, int b) { static_cast<Handle*>(p)->pool.free_block(b); }
void ref_pool_ref_block(void* p, int b) { static_cast<Handle*>(p)->pool.ref_block(b); }
int ref_pool_refcnt(void* p, int b) { return static_cast<Handle*>(p)->pool.refcnt(b); }
void ref_pool_attach(void* p, int dst, int src, int k) {
    Handle* h = static_cast<Handle*>(p);
    h->pool.attach(*h->slice(dst), *h->slice(src), k);
}
void ref_pool_attach_prefix(void* p, int dst, int src, int64_t n) {
    Handle* h = static_cast<Handle*>(p);
    h->pool.attach_prefix(*h->slice(dst), *h->slice(src), n);
}
int ref_pool_cow_slice(void* p, int s, int64_t pos) {
    Handle* h = static_cast<Handle*>(p);
    return h->pool.cow_slice(*h->slice(s), pos);
}
void ref_pool_release(void* p, int s) {
    Handle* h = static_cast<Handle*>(p);
    nova::KvSlice* sl = h->slice(s);
    if (!sl) return;
    h->pool.release(sl);
    for (size_t k = 0; k < h->order.size(); ++k)
        if (h->order[k] == s) { h->order.erase(h->order.begin() + (long)k); break; }
}
int ref_pool_nblocks(void* p) { return static_cast<Handle*>(p)->pool.nblocks(); }
int ref_pool_nb_total(void* p) { return static_cast<Handle*>(p)->pool.nb_total(); }
int ref_pool_cow_count(void* p) { return static_cast<Handle*>(p)->pool.cow_count(); }
int ref_pool_free_blocks(void* p) { return static_cast<Handle*>(p)->pool.free_blocks(); }
int ref_pool_used(void* p) { return static_cast<Handle*>(p)->pool.used(); }
int ref_pool_free_slices(void* p) { return static_cast<Handle*>(p)->pool.free_slices(); }
// The free-block stack itself is private: recover it by draining alloc_block()
// on a copy of the pool (pop order = top..bottom).
int ref_pool_free_list(void* p, int* out, int cap) {
    nova::KvPool copy = static_cast<Handle*>(p)->pool;
    std::vector<int> popped;
    for (int b; (b = copy.alloc_block()) >= 0;) popped.push_back(b);
    const int n = (int)popped.size();
    for (int i = 0; i < n && i < cap; ++i) out[i] = popped[(size_t)(n - 1 - i)];
    return n;
}
int ref_pool_table(void* p, int s, int32_t* out, int cap) {
    nova::KvSlice* sl = static_cast<Handle*>(p)->slice(s);
    const int n = (int)sl->table.size();
    for (int i = 0; i < n && i < cap; ++i) out[i] = sl->table[(size_t)i];
    return n;
}
int64_t ref_pool_n_past(void* p, int s) { return static_cast<Handle*>(p)->slice(s)->n_past; }
int ref_pool_need_copy(void* p, int s, int* from, int* blk) {
    nova::KvSlice* sl = static_cast<Handle*>(p)->slice(s);
    *from = sl->need_copy_from;
    *blk = sl->need_copy_blk;
    return *from >= 0;
}

uint64_t ref_kv_hash_ids(const int* ids, size_t n) {
    return nova::kv_hash_ids(std::vector<int>(ids, ids + n));
}
uint64_t ref_kv_hash_text(const char* t, size_t n) { return nova::kv_hash_text(std::string(t, n)); }
void ref_kv_block_id(uint64_t a, uint64_t b, char* out) {
    const std::string s = nova::kv_block_id(a, b);
    std::memcpy(out, s.c_str(), s.size() + 1);
}

void* ref_registry_new(void) { return new nova::BlockRegistry; }
void ref_registry_delete(void* r) { delete static_cast<nova::BlockRegistry*>(r); }
void ref_registry_set_capacity(void* r, size_t n) { static_cast<nova::BlockRegistry*>(r)->set_capacity(n); }
void ref_registry_put(void* r, uint64_t prefix, uint64_t suffix, int session, int turn,
                      int64_t pos0, int64_t pos1) {
    nova::KvBlock b;
    b.prefix = prefix; b.suffix = suffix; b.session = session; b.turn = turn; b.pos0 = pos0; b.pos1 = pos1;
    static_cast<nova::BlockRegistry*>(r)->put(b);
}
int ref_registry_find(void* r, uint64_t prefix, uint64_t suffix, int* session, int* turn,
                      int64_t* pos0, int64_t* pos1) {
    const nova::KvBlock* b = static_cast<nova::BlockRegistry*>(r)->find(prefix, suffix);
    if (!b) return 0;
    *session = b->session; *turn = b->turn; *pos0 = b->pos0; *pos1 = b->pos1;
    return 1;
}
int ref_registry_live(void* r) { return static_cast<nova::BlockRegistry*>(r)->live(); }
int ref_registry_total(void* r) { return static_cast<nova::BlockRegistry*>(r)->total(); }
}
