/* nova_testkit.h -- entry points of the test kit library, libnova_testkit_<model>.so.
 *
 * None of these is a reference surface and none ships in the product
 * libraries (libnova_hip_<model>.so): they exist for tests and benchmarks.
 * The test kit is built from the same kernel sources as the product library
 * of the same model, with the same flags, so a kernel timed through it is the
 * kernel a caller runs.  Device pointers and streams are shared with the
 * product library (one HIP runtime per process).
 */
#ifndef NOVA_TESTKIT_H
#define NOVA_TESTKIT_H

#include <stdint.h>

#include "hal.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Fill n fp16 values at p with seeded N(0, scale^2) draws (splitmix64 +
 * Box-Muller), so benchmarks hold tens of GB of K/V without a host round trip. */
void testkit_fill_normal_f16(uint16_t* p, uint64_t n, uint64_t seed, float scale, nova_stream_t s);

/* Plain 16-byte-per-lane copy of `bytes` (a multiple of 16): the kernel of
 * known traffic that calibrates the HBM byte counters. */
void testkit_copy(void* dst, const void* src, uint64_t bytes, nova_stream_t s);

/* Contiguous streaming read of `bytes` (a multiple of 16) by `workgroups`
 * workgroups of 256 threads, grid-stride non-temporal 16-byte loads with 4
 * per lane in flight, one sink word per thread into `sink` (workgroups * 256
 * uint32): the HBM floor of reading a layer's K/V bytes with no paging at
 * all (two workgroups per CU is the fastest shape measured). */
void testkit_stream_read(const void* src, uint64_t bytes, int workgroups, uint32_t* sink, nova_stream_t s);

/* Only the split kernel of launch_attn_decode_paged_planned (partials
 * written, o not), so that a benchmark can time the dominant kernel alone.
 * Needs the step's launch_attn_decode_plan. */
void testkit_attn_decode_split_only(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                    int table_stride, int n_sess, int layer, int nb, const uint16_t* k_new,
                                    const uint16_t* v_new, void* workspace, nova_stream_t s);

/* The HBM floor of the planned split: its grid reading the same pages with the
 * same loads and no arithmetic (one sink word per thread into the workspace's
 * partial area).  Needs the step's launch_attn_decode_plan. */
void testkit_decode_stream_floor(const uint16_t* pool_k, const uint16_t* pool_v, const int32_t* tables,
                                 int table_stride, int n_sess, int layer, int nb, void* workspace, nova_stream_t s);

/* launch_attn_decode_paged_planned with the bound of the in-workgroup
 * partial exchange set to `spin_limit` polls (the product uses 1 << 22).
 * With 0 the exchange gives up at once wherever it has more than one wave
 * per kv head, so a test can check from the host that a give-up is reported
 * (attn_decode_batch_status) and poisons the affected outputs with NaN. */
void testkit_attn_decode_planned_spin(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                      int table_stride, int n_sess, int layer, int nb, const uint16_t* k_new,
                                      const uint16_t* v_new, float* o, void* workspace, int spin_limit,
                                      nova_stream_t s);

#ifdef __cplusplus
}
#endif
#endif
