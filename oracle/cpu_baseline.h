/* cpu_baseline.h -- TEST INFRASTRUCTURE: the CPU baseline that bench.py times
 * beside the GPU path (its `cpu_baseline` leg) and nothing else loads.
 *
 * A throughput-minded host restatement of the same arithmetic as the
 * reference's paged decode and prefill (src/kernel/attn.cu:163-357): fp16
 * pages converted with F16C, fp32 dot products and accumulation with AVX2
 * FMA, an online softmax per page of keys, and a thread pool over work units.
 * It is not the parity oracle (nova_oracle.c emulates the reference's
 * per-lane order); its outputs agree with it to the attention tolerance, which
 * tests/test_cpu_baseline.py checks. */
#ifndef NOVA_CPU_BASELINE_H
#define NOVA_CPU_BASELINE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry: nh query heads, nkv kv heads, hd head dim (a multiple of 8), kb
 * tokens per page.  Pools [layers][nb][kb][nkv][hd] fp16 bits. */
typedef struct {
    int nh, nkv, hd, kb;
} cb_geom;

/* Batched decode: session i attends q[i] (nh x hd) over keys [0, n_keys[i])
 * of its table (tables + i*table_stride) in `layer`; o[i] (nh x hd).  Work
 * units (session, kv head, split of at most 64 pages) go to n_threads
 * threads; the splits merge with fa_combine_kernel's rule (attn.cu:163-191).
 * A session with n_keys 0 gets zeros. */
void cb_attn_decode_batch(cb_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                          const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess,
                          int layer, int nb, float* o, int n_threads);

/* Batched causal prefill: session i has n_q queries (q + i*n_q*nh*hd) at
 * positions n_past[i] .. n_past[i]+n_q-1, each attending keys [0, pos];
 * o like q.  Work units (session, kv head, block of 16 queries) go to
 * n_threads threads. */
void cb_attn_prefill_batch(cb_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                           const int32_t* tables, int table_stride, const int32_t* n_past, int n_sess,
                           int n_q, int layer, int nb, float* o, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
