// graph_capi.cpp -- C ABI over the host paging layer (include/nova_graph.h).
#include <cstring>
#include <string>
#include <vector>

#include "graph/kv_block.h"
#include "graph/kv_pool.h"
#include "graph/kv_registry.h"
#include "nova_graph.h"
#include "session_paged.h"

using nova::BlockRegistry;
using nova::KvPool;
using nova::KvSlice;
using nova::PagedKv;

namespace {
KvPool* P(nova_kvpool_t p) { return static_cast<KvPool*>(p); }
PagedKv* H(nova_paged_t h) { return static_cast<PagedKv*>(h); }
BlockRegistry* RG(nova_registry_t r) { return static_cast<BlockRegistry*>(r); }

KvSlice& S(KvPool* p, int id) {
    KvSlice* s = p->slice(id);
    if (!s) {
        std::fprintf(stderr, "[nova] FATAL: slice %d is not live\n", id);
        std::abort();
    }
    return *s;
}
int copy_out(const std::vector<int>& v, int* out, int cap) {
    const int n = (int)v.size();
    if (out) std::memcpy(out, v.data(), sizeof(int) * (size_t)(n < cap ? n : cap));
    return n;
}
}  // namespace

extern "C" {

nova_kvpool_t nova_kvpool_new(int n_slices, int64_t ctx) {
    KvPool* p = new KvPool;
    p->init(n_slices, ctx);
    return p;
}
void nova_kvpool_delete(nova_kvpool_t p) { delete P(p); }
int nova_kvpool_acquire(nova_kvpool_t p) {
    KvSlice* s = P(p)->acquire();
    return s ? s->id : -1;
}
int nova_kvpool_alloc_block(nova_kvpool_t p) { return P(p)->alloc_block(); }
void nova_kvpool_free_block(nova_kvpool_t p, int b) { P(p)->free_block(b); }
void nova_kvpool_ref_block(nova_kvpool_t p, int b) { P(p)->ref_block(b); }
int nova_kvpool_refcnt(nova_kvpool_t p, int b) { return P(p)->refcnt(b); }
void nova_kvpool_attach(nova_kvpool_t p, int dst, int src, int k) { P(p)->attach(S(P(p), dst), S(P(p), src), k); }
void nova_kvpool_attach_prefix(nova_kvpool_t p, int dst, int src, int64_t n) {
    P(p)->attach_prefix(S(P(p), dst), S(P(p), src), n);
}
int nova_kvpool_cow_slice(nova_kvpool_t p, int s, int64_t pos) { return P(p)->cow_slice(S(P(p), s), pos); }
void nova_kvpool_release(nova_kvpool_t p, int s) { P(p)->release(P(p)->slice(s)); }
int nova_kvpool_nblocks(nova_kvpool_t p) { return P(p)->nblocks(); }
int nova_kvpool_nb_total(nova_kvpool_t p) { return P(p)->nb_total(); }
int nova_kvpool_cow_count(nova_kvpool_t p) { return P(p)->cow_count(); }
int nova_kvpool_free_blocks(nova_kvpool_t p) { return P(p)->free_blocks(); }
int nova_kvpool_used(nova_kvpool_t p) { return P(p)->used(); }
int nova_kvpool_free_slices(nova_kvpool_t p) { return P(p)->free_slices(); }
int nova_kvpool_free_list(nova_kvpool_t p, int* out, int cap) { return copy_out(P(p)->free_list(), out, cap); }
int nova_kvpool_refcnts(nova_kvpool_t p, int* out, int cap) { return copy_out(P(p)->refcnts(), out, cap); }
int nova_kvpool_table(nova_kvpool_t p, int s, int32_t* out, int cap) {
    const auto& t = S(P(p), s).table;
    const int n = (int)t.size();
    if (out) std::memcpy(out, t.data(), sizeof(int32_t) * (size_t)(n < cap ? n : cap));
    return n;
}
int64_t nova_kvpool_n_past(nova_kvpool_t p, int s) { return S(P(p), s).n_past; }
void nova_kvpool_set_n_past(nova_kvpool_t p, int s, int64_t n) { S(P(p), s).n_past = n; }
int nova_kvpool_need_copy(nova_kvpool_t p, int s, int* from, int* blk) {
    const KvSlice& sl = S(P(p), s);
    *from = sl.need_copy_from;
    *blk = sl.need_copy_blk;
    return *from >= 0;
}

uint64_t nova_kv_hash_ids(const int* ids, size_t n) { return nova::kv_hash_ids(ids, n); }
uint64_t nova_kv_hash_text(const char* text, size_t n) { return nova::kv_hash_text(std::string(text, n)); }
void nova_kv_hash_hex(uint64_t v, char out[17]) {
    const std::string s = nova::kv_hash_hex(v);
    std::memcpy(out, s.c_str(), 17);
}
void nova_kv_block_id(uint64_t prefix, uint64_t suffix, char out[40]) {
    const std::string s = nova::kv_block_id(prefix, suffix);
    std::memcpy(out, s.c_str(), s.size() + 1);
}

nova_registry_t nova_registry_new(void) { return new BlockRegistry; }
void nova_registry_delete(nova_registry_t r) { delete RG(r); }
void nova_registry_set_capacity(nova_registry_t r, size_t n) { RG(r)->set_capacity(n); }
void nova_registry_put(nova_registry_t r, uint64_t prefix, uint64_t suffix, int session, int turn, int64_t pos0,
                       int64_t pos1) {
    nova::KvBlock b;
    b.prefix = prefix;
    b.suffix = suffix;
    b.session = session;
    b.turn = turn;
    b.pos0 = pos0;
    b.pos1 = pos1;
    RG(r)->put(b);
}
int nova_registry_find(nova_registry_t r, uint64_t prefix, uint64_t suffix, int* session, int* turn,
                       int64_t* pos0, int64_t* pos1) {
    const nova::KvBlock* b = RG(r)->find(prefix, suffix);
    if (!b) return 0;
    *session = b->session;
    *turn = b->turn;
    *pos0 = b->pos0;
    *pos1 = b->pos1;
    return 1;
}
int nova_registry_live(nova_registry_t r) { return RG(r)->live(); }
int nova_registry_total(nova_registry_t r) { return RG(r)->total(); }

nova_paged_t nova_paged_new(int n_slices, int64_t ctx) {
    PagedKv* h = new PagedKv;
    h->init(n_slices, ctx);
    return h;
}
void nova_paged_delete(nova_paged_t h) {
    H(h)->destroy();
    delete H(h);
}
nova_kvpool_t nova_paged_pool(nova_paged_t h) { return &H(h)->pool(); }
uint16_t* nova_paged_pool_k(nova_paged_t h) { return H(h)->k_base(); }
uint16_t* nova_paged_pool_v(nova_paged_t h) { return H(h)->v_base(); }
int32_t* nova_paged_tables(nova_paged_t h) { return H(h)->tables(); }
int nova_paged_nb(nova_paged_t h) { return H(h)->nb(); }
nova_stream_t nova_paged_stream(nova_paged_t h) { return H(h)->stream(); }
int nova_paged_create_session(nova_paged_t h, int clear_pages) { return H(h)->create_session(clear_pages != 0)->id; }
void nova_paged_destroy_session(nova_paged_t h, int s) { H(h)->destroy_session(H(h)->pool().slice(s)); }
void nova_paged_attach(nova_paged_t h, int dst, int src, int k) {
    H(h)->attach(S(&H(h)->pool(), dst), S(&H(h)->pool(), src), k);
}
void nova_paged_attach_prefix(nova_paged_t h, int dst, int src, int64_t n) {
    H(h)->attach_prefix(S(&H(h)->pool(), dst), S(&H(h)->pool(), src), n);
}
int nova_paged_cow_guard(nova_paged_t h, int s, int64_t pos, nova_stream_t st) {
    return H(h)->cow_guard(S(&H(h)->pool(), s), pos, st);
}
void nova_paged_session_cow(nova_paged_t h, int s, int64_t pos0, int n, nova_stream_t st) {
    H(h)->session_cow(S(&H(h)->pool(), s), pos0, n, st);
}
int nova_paged_cow_batch(nova_paged_t h, const int* sessions, const int64_t* pos0, const int* n, int count,
                         nova_stream_t st) {
    std::vector<KvSlice*> ss((size_t)count);
    for (int i = 0; i < count; ++i) ss[(size_t)i] = &S(&H(h)->pool(), sessions[i]);
    return H(h)->cow_batch(ss.data(), pos0, n, count, st);
}
int32_t* nova_paged_table_dev(nova_paged_t h, int s) { return S(&H(h)->pool(), s).table_dev; }
int nova_paged_create_sessions(nova_paged_t h, int count, int clear_pages, int* ids) {
    if (count < 0 || (count > 0 && !ids)) {
        std::fprintf(stderr, "[nova] FATAL: nova_paged_create_sessions: bad arguments\n");
        std::abort();
    }
    return H(h)->create_sessions(count, clear_pages != 0, ids);
}
void nova_paged_push_tables(nova_paged_t h, const int* ids, int count) {
    for (int i = 0; i < count; ++i) (void)S(&H(h)->pool(), ids[i]);   // validates every id
    H(h)->push_tables(ids, count);
}

}  // extern "C"
