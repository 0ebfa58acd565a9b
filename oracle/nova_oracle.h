/*
 * nova_oracle.h -- CPU oracle for the paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is a plain-C restatement of the
 * reference algorithms (Conflux Nova, CUDA line) and exists to check the HIP
 * product.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it, and only as the checker / the timed CPU baseline; the
 * product library never links or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root).  Shapes are runtime arguments here (the
 * reference welds them at compile time); K/V are fp16 bit patterns widened to
 * fp32, Q/O are fp32, accumulation is fp32 unless the name says f64.
 */
#ifndef NOVA_ORACLE_H
#define NOVA_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- geometry ---------------- */
typedef struct {
    int nh;   /* query heads              */
    int nkv;  /* kv heads                 */
    int hd;   /* head dim (64 or 128)     */
    int kb;   /* tokens per page (8..64)  */
} or_geom;

/* ---------------- fp16 helpers ---------------- */
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);                 /* round-to-nearest-even */
void     or_f32_to_f16_n(const float* src, uint16_t* dst, size_t n);
void     or_f16_to_f32_n(const uint16_t* src, float* dst, size_t n);

/* ---------------- KvPool (code/graph/kv_pool.h:68-197) ---------------- */
typedef struct or_pool or_pool;
or_pool* or_pool_new(int n_slices, int64_t ctx);             /* KvPool::init   :70-84  */
void     or_pool_delete(or_pool* p);
int      or_pool_acquire(or_pool* p);                        /* :90-113, returns slice id or -1 */
int      or_pool_alloc_block(or_pool* p);                    /* :116-122 */
void     or_pool_free_block(or_pool* p, int b);              /* :123-126 */
void     or_pool_ref_block(or_pool* p, int b);               /* :127 */
int      or_pool_refcnt(const or_pool* p, int b);            /* :128 */
void     or_pool_attach(or_pool* p, int dst, int src, int k);              /* :132-138 */
void     or_pool_attach_prefix(or_pool* p, int dst, int src, int64_t n);  /* :141-148 */
int      or_pool_cow_slice(or_pool* p, int s, int64_t pos);  /* :153-166 */
void     or_pool_release(or_pool* p, int s);                 /* :168-174 */
int      or_pool_nblocks(const or_pool* p);
int      or_pool_nb_total(const or_pool* p);
int      or_pool_cow_count(const or_pool* p);
int      or_pool_free_blocks(const or_pool* p);
int      or_pool_used(const or_pool* p);
int      or_pool_free_slices(const or_pool* p);
/* state export for bit-exact comparisons */
int      or_pool_free_list(const or_pool* p, int* out, int cap);  /* free-block stack, bottom..top */
int      or_pool_refcnts(const or_pool* p, int* out, int cap);
int      or_pool_table(const or_pool* p, int s, int32_t* out, int cap);
int64_t  or_pool_n_past(const or_pool* p, int s);
void     or_pool_set_n_past(or_pool* p, int s, int64_t n);
int      or_pool_need_copy(const or_pool* p, int s, int* from, int* blk);

/* ---------------- kv_block IDs (code/graph/kv_block.h:21-83) ---------------- */
uint64_t or_kv_hash_ids(const int* ids, size_t n);           /* :21-64 */
uint64_t or_kv_hash_text(const char* text, size_t n);        /* :67-72 */
void     or_kv_hash_hex(uint64_t v, char out[17]);           /* :74-79 */
void     or_kv_block_id(uint64_t prefix, uint64_t suffix, char out[40]);  /* :81-83 */

/* ---------------- BlockRegistry (code/graph/kv_registry.h:26-66) ---------------- */
typedef struct or_registry or_registry;
or_registry* or_registry_new(void);
void     or_registry_delete(or_registry* r);
void     or_registry_set_capacity(or_registry* r, size_t n);
void     or_registry_put(or_registry* r, uint64_t prefix, uint64_t suffix, int session, int turn,
                         int64_t pos0, int64_t pos1);
int      or_registry_find(const or_registry* r, uint64_t prefix, uint64_t suffix,
                          int* session, int* turn, int64_t* pos0, int64_t* pos1);
int      or_registry_live(const or_registry* r);
int      or_registry_total(const or_registry* r);

/* ---------------- paged append (src/kernel/elem.cu:59-76,93-98) ---------------- */
void or_kv_store_paged(or_geom g, uint16_t* pool_k, uint16_t* pool_v, const int32_t* table,
                       int layer, int nb, int n, int64_t pos0,
                       const uint16_t* k, const uint16_t* v);
/* gather logical positions [0,n) of one layer into contiguous [n][nkv][hd] */
void or_kv_gather_paged(or_geom g, const uint16_t* pool, const int32_t* table, int layer, int nb,
                        int64_t n, uint16_t* out);

/* ---------------- RoPE (src/kernel/rope.cu) ----------------
 * Table: rope_table_kernel rope.cu:9-18, cs/sn [rows][half] with
 *   f_i = exp2f(-(float)i * (1/half) * log2f(theta)), a = (float)pos * f_i,
 *   cs = cosf(a), sn = sinf(a)
 * evaluated with every float operation correctly rounded (transcendentals in
 * double, rounded once), which fixes the table bit for bit.
 * Rotation: rope_batch_kernel rope.cu:39-58, NeoX pairs (i, i + half) for the
 * Qwen2 family (include/nova/arch/traits.h:15-17), x0*c - x1*s and x0*s + x1*c
 * without contraction.  q [n][nh][hd] and k [n][nkv][hd] fp32, rotated in place
 * at positions pos0 .. pos0+n-1. */
void or_rope_table(float* cs, float* sn, int rows, int half, double theta);
void or_rope_apply(or_geom g, float* q, float* k, int n, int64_t pos0, const float* cs, const float* sn);
/* RopeKvOp (code/graph/dense.h:75-83): rope_batch then kv_store_paged, with
 * the pool in fp16: q rotated in place, k rotated (its buffer untouched) and
 * appended with v as fp16 (round to nearest even) at pos0 .. pos0+n-1. */
void or_rope_kv_store_paged(or_geom g, float* q, const float* k, const float* v, const float* cs,
                            const float* sn, uint16_t* pool_k, uint16_t* pool_v, const int32_t* table,
                            int layer, int nb, int n, int64_t pos0);

/* ---------------- Q4_K GEMV (src/kernel/q4k_gemv.cu, include/nova/quant/q4_k.h) ----------------
 * Weights: rows x (cols/256) ggml block_q4_K (144 B: fp16 d, fp16 dmin,
 * 12 B of packed 6-bit (scale, min) for 8 sub-blocks of 32, 128 B of nibbles;
 * q4_k.h:19-25).  Activations ActQ8 (include/nova/kernel/types.h:24-28): per
 * row int8 qs[cols], float d[cols/32], int s[cols/16] (sum of each 16 int8). */
float or_q4k_half(uint16_t h);                                            /* q4_k.h:28-41 */
void  or_q4k_dequant_block(const uint8_t* block, float* y);              /* q4_k.h:55-73 */
/* quant_kernel q4k_gemv.cu:9-33: amax over 32, d = amax/127, q = rint(x*127/amax) */
void  or_quant_q8(const float* x, int rows, int cols, int8_t* qs, float* d, int32_t* s);
/* out[r] = sum_b dot(dequant(w[r]), x_q * x_d) in double: the value the GEMV
 * (gemv_kernel q4k_gemv.cu:35-91) computes in fp32 with its own order */
void  or_gemv_q4k(const uint8_t* w, int64_t rows, int64_t cols, const int8_t* qs, const float* d,
                  const int32_t* s, double* out);

/* ---------------- COW page copy (src/model.cpp:171-191) ---------------- */
void or_cow_copy(or_geom g, uint16_t* pool_k, uint16_t* pool_v, int n_layers, int nb,
                 int src, int dst);

/* ---------------- attention ----------------
 * decode: fa_split_paged_kernel + fa_combine_kernel (src/kernel/attn.cu:163-289),
 * split rule of launch_attn_decode_paged (attn.cu:498-512); emulates the 4-warp
 * ranges, the per-lane fma order and the shuffle-down reduction order.
 * q [nh][hd] f32, o [nh][hd] f32. */
void or_attn_decode_paged(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                          const int32_t* table, int layer, int nb, int n_keys, float* o);
/* textbook two-pass softmax attention in double (tests/sycl_bench.cpp:889-943 form) */
void or_attn_decode_paged_f64(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                              const int32_t* table, int layer, int nb, int n_keys, double* o);
/* prefill: flash_paged_kernel<false> (attn.cu:293-357): one (query, head) at a time,
 * causal keys [0, n_past+qi].  q/o [n_q][nh][hd]. */
void or_attn_prefill_paged(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                           const int32_t* table, int layer, int nb, int n_q, int n_past, float* o);
void or_attn_prefill_paged_f64(or_geom g, const float* q, const uint16_t* pool_k,
                               const uint16_t* pool_v, const int32_t* table, int layer, int nb,
                               int n_q, int n_past, double* o);

/* Batched decode over sessions for the CPU baseline: session i uses
 * tables + i*table_stride and n_keys[i]; q/o [n_sess][nh][hd].  Work units
 * (session, head) are spread over n_threads pthreads.  Same arithmetic as
 * or_attn_decode_paged. */
void or_attn_decode_batch(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                          const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess,
                          int layer, int nb, float* o, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
