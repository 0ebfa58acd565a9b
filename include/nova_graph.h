/*
 * nova_graph.h -- host paging layer of the paged KV-cache path (C ABI).
 *
 * Handles over the C++ classes in conflux-nova_amd/code/graph and
 * code/session_paged.h, so an FFI (ctypes here) can drive block tables,
 * refcounts, COW decisions and kv_block IDs exactly as the reference's C++
 * callers do.  All functions are host-side; the nova_paged_* ones also touch
 * the device through include/hal.h and include/nova_kernel.h.
 */
#ifndef NOVA_GRAPH_H
#define NOVA_GRAPH_H
#include <stddef.h>
#include <stdint.h>
#include "hal.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef void* nova_kvpool_t;
typedef void* nova_registry_t;
typedef void* nova_paged_t;

/* ---- nova::KvPool, code/graph/kv_pool.h:68-197 (slice handles are slice ids) ---- */
nova_kvpool_t nova_kvpool_new(int n_slices, int64_t ctx);        /* KvPool::init :70-84 */
void    nova_kvpool_delete(nova_kvpool_t p);
int     nova_kvpool_acquire(nova_kvpool_t p);                     /* :90-113, -1 when none */
int     nova_kvpool_alloc_block(nova_kvpool_t p);                 /* :116-122 */
void    nova_kvpool_free_block(nova_kvpool_t p, int b);           /* :123-126 */
void    nova_kvpool_ref_block(nova_kvpool_t p, int b);            /* :127 */
int     nova_kvpool_refcnt(nova_kvpool_t p, int b);               /* :128 */
void    nova_kvpool_attach(nova_kvpool_t p, int dst, int src, int k);            /* :132-138 */
void    nova_kvpool_attach_prefix(nova_kvpool_t p, int dst, int src, int64_t n); /* :141-148 */
int     nova_kvpool_cow_slice(nova_kvpool_t p, int s, int64_t pos);              /* :153-166 */
void    nova_kvpool_release(nova_kvpool_t p, int s);              /* :168-174 */
int     nova_kvpool_nblocks(nova_kvpool_t p);
int     nova_kvpool_nb_total(nova_kvpool_t p);
int     nova_kvpool_cow_count(nova_kvpool_t p);
int     nova_kvpool_free_blocks(nova_kvpool_t p);
int     nova_kvpool_used(nova_kvpool_t p);
int     nova_kvpool_free_slices(nova_kvpool_t p);
int     nova_kvpool_free_list(nova_kvpool_t p, int* out, int cap);   /* bottom..top; returns size */
int     nova_kvpool_refcnts(nova_kvpool_t p, int* out, int cap);
int     nova_kvpool_table(nova_kvpool_t p, int s, int32_t* out, int cap);
int64_t nova_kvpool_n_past(nova_kvpool_t p, int s);
void    nova_kvpool_set_n_past(nova_kvpool_t p, int s, int64_t n);
int     nova_kvpool_need_copy(nova_kvpool_t p, int s, int* from, int* blk);

/* ---- kv_block IDs, code/graph/kv_block.h:21-83 ---- */
uint64_t nova_kv_hash_ids(const int* ids, size_t n);
uint64_t nova_kv_hash_text(const char* text, size_t n);
void     nova_kv_hash_hex(uint64_t v, char out[17]);
void     nova_kv_block_id(uint64_t prefix, uint64_t suffix, char out[40]);

/* ---- nova::BlockRegistry, code/graph/kv_registry.h:26-66 ---- */
nova_registry_t nova_registry_new(void);
void    nova_registry_delete(nova_registry_t r);
void    nova_registry_set_capacity(nova_registry_t r, size_t n);
void    nova_registry_put(nova_registry_t r, uint64_t prefix, uint64_t suffix, int session, int turn,
                          int64_t pos0, int64_t pos1);
int     nova_registry_find(nova_registry_t r, uint64_t prefix, uint64_t suffix, int* session, int* turn,
                           int64_t* pos0, int64_t* pos1);
int     nova_registry_live(nova_registry_t r);
int     nova_registry_total(nova_registry_t r);

/* ---- device-backed pool + sessions (Engine pool views model.h:140-145,
 *      SessionManager::create/destroy session.h:84-142, session_attach*,
 *      session_cow session.h:156-180, Engine::cow_guard model.cpp:171-191) ---- */
nova_paged_t  nova_paged_new(int n_slices, int64_t ctx);
void          nova_paged_delete(nova_paged_t h);
nova_kvpool_t nova_paged_pool(nova_paged_t h);          /* its KvPool, for the getters above */
uint16_t*     nova_paged_pool_k(nova_paged_t h);
uint16_t*     nova_paged_pool_v(nova_paged_t h);
int32_t*      nova_paged_tables(nova_paged_t h);        /* all tables; slice s at + s*nblocks */
int           nova_paged_nb(nova_paged_t h);
nova_stream_t nova_paged_stream(nova_paged_t h);
int           nova_paged_create_session(nova_paged_t h, int clear_pages);
void          nova_paged_destroy_session(nova_paged_t h, int s);
void          nova_paged_attach(nova_paged_t h, int dst, int src, int k);
void          nova_paged_attach_prefix(nova_paged_t h, int dst, int src, int64_t n_tokens);
int           nova_paged_cow_guard(nova_paged_t h, int s, int64_t pos, nova_stream_t st);
void          nova_paged_session_cow(nova_paged_t h, int s, int64_t pos0, int n, nova_stream_t st);
int           nova_paged_cow_batch(nova_paged_t h, const int* sessions, const int64_t* pos0, const int* n,
                                   int count, nova_stream_t st);
int32_t*      nova_paged_table_dev(nova_paged_t h, int s);
/* Batched session manager (no single counterpart in the reference: it
 * replaces N calls of SessionManager::create's paging steps, session.h:84-142,
 * and N table uploads).  create_sessions acquires `count` slices in the order
 * serial creates would (ids out, -1 past pool exhaustion; returns the number
 * created), uploads their tables with one copy per run of consecutive ids and
 * clears all their pages in one launch.  push_tables re-uploads the host
 * tables of `count` sessions the same way. */
int           nova_paged_create_sessions(nova_paged_t h, int count, int clear_pages, int* ids);
void          nova_paged_push_tables(nova_paged_t h, const int* ids, int count);

#ifdef __cplusplus
}
#endif
#endif
