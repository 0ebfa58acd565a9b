/*
 * nova_kernel.h -- kernel-layer entry points of the paged KV-cache path (C ABI).
 *
 * One shared library per model geometry (libnova_hip_<model>.so), exactly as
 * the reference welds NH / NKV / HD / L and the page size at compile time
 * (include/nova/model/select.h:6-32, code/graph/kv_pool_cfg.h:12-33): there is
 * no runtime shape argument.  nova_model_geometry() reports what a library was
 * built for.
 *
 * Pool layout (unchanged from the reference, include/nova/model.h:140-145,
 * code/graph/kv_pool.h:8-15): separate K and V pools, each
 *     pool[layer][NB][KB][NKV][HD],  KB = 16 tokens per page,
 * address of token pos of a session = ((layer*NB + table[pos>>4])*KB + (pos&15))*NKV*HD.
 * K/V elements are IEEE fp16 bit patterns (uint16_t); the reference stores fp32
 * (dense.h:25-26), the build stores fp16.  Q and O stay fp32.
 *
 * All launches are asynchronous on the given stream and return nothing; bad
 * arguments abort before anything is launched (include/nova/config.h:42-63).
 */
#ifndef NOVA_KERNEL_H
#define NOVA_KERNEL_H
#include <stddef.h>
#include <stdint.h>
#include "hal.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Geometry the library was compiled for.  Not a reference surface: the
 * reference reads it from ActiveModel (select.h); an FFI needs it as a call. */
typedef struct {
    int nh, nkv, hd, n_layers, kv_block, max_split;
    const char* name;
} nova_geometry;
nova_geometry nova_model_geometry(void);

/* Append n tokens of K and V at logical positions pos0..pos0+n-1.
 * k, v: [n][NKV][HD] fp16.  table: the session's device block table.
 * Replaces nova::launch_kv_store_paged, include/nova/kernel.h:44-45
 * (kernel src/kernel/elem.cu:59-76, launcher :93-98). */
void launch_kv_store_paged(uint16_t* pool_k, uint16_t* pool_v, const int32_t* table, int layer, int nb,
                           int n, int64_t pos0, const uint16_t* k, const uint16_t* v, nova_stream_t s);

/* Single-session split-K decode over keys [0, n_keys) of one layer.
 * q, o: [NH][HD] fp32.  scratch: caller-owned, >= NH*32*(HD+2) floats
 * (src/model.cpp:114,148).  Replaces nova::launch_attn_decode_paged,
 * include/nova/kernel.h:62-64 (attn.cu:197-289 + combine :163-191, launcher :498-512). */
void launch_attn_decode_paged(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                              const int32_t* table, int layer, int nb, int n_keys,
                              float* o, float* scratch, nova_stream_t s);

/* Causal attention of n_q new queries at positions n_past..n_past+n_q-1 over
 * keys [0, n_past+qi] (the chunk must already be appended).  q, o:
 * [n_q][NH][HD] fp32.  Replaces nova::launch_attn_prefill_paged,
 * include/nova/kernel.h:65-67 (attn.cu:293-357, launcher :514-525). */
void launch_attn_prefill_paged(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                               const int32_t* table, int layer, int nb,
                               int n_q, int n_past, float* o, nova_stream_t s);

/* ---------------- extensions (no single reference counterpart) ---------------- */

/* Batched ragged decode: one launch for all sessions of a layer, optionally
 * fused with that layer's 1-token append.  Replaces the 2N per-session
 * launches of Engine::decode_batch (src/model.cpp:282-289).
 *   q, o     [n_sess][NH][HD] fp32
 *   tables   session i's block table is tables + i*table_stride (the
 *            reference keeps all tables in one array, model.cpp:95)
 *   n_keys   device int32[n_sess]; keys [0, n_keys[i]) are attended
 *   k_new, v_new  NULL, or [n_sess][NKV][HD] fp16: the token at position
 *            n_keys[i]-1 is written into the pool AND attended from these
 *            buffers in the same launch (append-then-attend, dense.h:75-95)
 *   workspace    from attn_decode_batch_workspace_bytes(): plan + split
 *            partials; no initial contents required.
 * Three launches on s: plan, split kernel, combine kernel.
 * n_keys[i] == 0 yields a zero output row. */
size_t attn_decode_batch_workspace_bytes(int n_sess);
/* Status word of the batched decode in `workspace` (n_sess as in the calls):
 * 0, or an OR of failure bits set by the layers since the step's plan launch
 * (1: a split workgroup's in-LDS partial exchange gave up waiting, and the
 * heads it served were written as NaN).  The plan launch clears it.  Waits for
 * the device to finish, then reads the word: a host-side check for tests and
 * serving loops, not for the hot path. */
int attn_decode_batch_status(const void* workspace, int n_sess);
/* The batched call above = launch_attn_decode_plan + launch_attn_decode_paged_planned.
 * A decode step has the same n_keys and block tables in every layer, so a
 * caller can plan once per step and run only the planned call per layer:
 * the plan records each workgroup's session, page range, physical pages and
 * partial slot (a session's workgroups are grouped on one or two XCDs) and
 * the (session, head) each combine block merges (on its session's XCD where
 * there is room), and the planned call starts from one load instead of a dependent
 * n_keys -> partition -> block-table chain.  The plan lives at the start of
 * `workspace`; it is valid until n_keys or the tables change. */
void launch_attn_decode_plan(const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess,
                             void* workspace, nova_stream_t s);
void launch_attn_decode_paged_planned(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                      int table_stride, int n_sess, int layer, int nb, const uint16_t* k_new,
                                      const uint16_t* v_new, float* o, void* workspace, nova_stream_t s);
void launch_attn_decode_paged_batch(const float* q, uint16_t* pool_k, uint16_t* pool_v,
                                    const int32_t* tables, int table_stride, const int32_t* n_keys,
                                    int n_sess, int layer, int nb,
                                    const uint16_t* k_new, const uint16_t* v_new,
                                    float* o, void* workspace, nova_stream_t s);
/* The batched decode above (plan + split + combine) with no workspace
 * argument and no allocation: the plan and partials live in a static device
 * array inside the library (about 10 MB per device, held until the process
 * ends).  No counterpart in the reference: it is for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Limits: n_sess <= 64 on a device of at most 256
 * CUs; anything else aborts with a message before launching.  Every call on
 * a device shares the array, so calls that overlap on one device (two
 * streams) race; calls in one stream order are safe.  Nothing in the array
 * needs clearing between calls. */
void launch_attn_decode_paged_batch_noalloc(const float* q, uint16_t* pool_k, uint16_t* pool_v,
                                            const int32_t* tables, int table_stride, const int32_t* n_keys,
                                            int n_sess, int layer, int nb, const uint16_t* k_new,
                                            const uint16_t* v_new, float* o, nova_stream_t s);
/* The batched decode with the step before it fused in: RopeKvOp
 * (code/graph/dense.h:75-83: rope_batch of q and k at position n_keys[i]-1,
 * src/kernel/rope.cu:21-58, then kv_store_paged of k and v) and the
 * attention of the planned call above, in one launch pair.  k_new, v_new:
 * the layer's new token, fp32 [n_sess][NKV][HD], unrotated; k is rotated with
 * the cs/sn table rows of launch_rope_table (every row used must exist) and
 * written with v as fp16 (nearest even) into the session's last page; q is
 * rotated in registers as it is loaded and the caller's q is not modified.
 * The appended rows are bit-identical to launch_rope_kv_store_paged_batch's;
 * n_keys[i] counts the new token and must be >= 1 for every session. */
void launch_attn_decode_paged_rope_planned(const float* q, const float* k_new, const float* v_new, const float* cs,
                                           const float* sn, uint16_t* pool_k, uint16_t* pool_v,
                                           const int32_t* tables, int table_stride, int n_sess, int layer, int nb,
                                           float* o, void* workspace, nova_stream_t s);
void launch_attn_decode_paged_rope_batch(const float* q, const float* k_new, const float* v_new, const float* cs,
                                         const float* sn, uint16_t* pool_k, uint16_t* pool_v,
                                         const int32_t* tables, int table_stride, const int32_t* n_keys,
                                         int n_sess, int layer, int nb, float* o, void* workspace,
                                         nova_stream_t s);

/* Batched decode in ONE launch for short contexts ("solo"): one workgroup
 * per (kv head, session) streams all of the session's pages for that head,
 * merges its waves on chip and writes the session's output rows itself: no
 * plan, no partials, no combine launch, no workspace.  Arguments as for
 * launch_attn_decode_paged_batch (k_new, v_new: NULL or the fused 1-token
 * append), except that `tables` must hold n_sess full rows of table_stride
 * readable entries (the first min(128, table_stride) entries of a row are read
 * before its n_keys is known).  One CU serves a session's kv head, so this
 * suits steps whose sessions hold up to about 40 pages (640 tokens); longer
 * sessions belong on the split path (on config 1's single 1025-key session
 * the split path is faster).  The reference's launch_attn_decode_paged takes
 * this route itself for contexts up to 40 pages.  The _rope_ form fuses RoPE
 * as launch_attn_decode_paged_rope_planned does. */
void launch_attn_decode_paged_solo(const float* q, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                   int table_stride, const int32_t* n_keys, int n_sess, int layer, int nb,
                                   const uint16_t* k_new, const uint16_t* v_new, float* o, nova_stream_t s);
void launch_attn_decode_paged_rope_solo(const float* q, const float* k_new, const float* v_new, const float* cs,
                                        const float* sn, uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables,
                                        int table_stride, const int32_t* n_keys, int n_sess, int layer, int nb,
                                        float* o, nova_stream_t s);

/* Batched append: session i writes n tokens at positions pos0[i]..pos0[i]+n-1
 * (pos0: device int32[n_sess]) through tables + i*table_stride; k, v:
 * [n_sess][n][NKV][HD] fp16.  One launch for a decode step's appends (or a
 * prefill chunk per session) instead of n_sess launch_kv_store_paged calls. */
void launch_kv_store_paged_batch(uint16_t* pool_k, uint16_t* pool_v, const int32_t* tables, int table_stride,
                                 const int32_t* pos0, int n_sess, int layer, int nb, int n, const uint16_t* k,
                                 const uint16_t* v, nova_stream_t s);

/* Batched chunked-prefill attention: n_sess sessions each with a chunk of n_q
 * queries at positions n_past[i]..n_past[i]+n_q-1 (device int32[n_sess]).
 * q, o: [n_sess][n_q][NH][HD] fp32; tables as for the batched decode.  One
 * launch instead of n_sess launch_attn_prefill_paged calls. */
void launch_attn_prefill_paged_batch(const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                                     const int32_t* tables, int table_stride, const int32_t* n_past,
                                     int n_sess, int n_q, int layer, int nb, float* o, nova_stream_t s);

/* Batched copy-on-write page copy: for every pair c, copy page src[c] to page
 * dst[c] in every layer of both pools (n_layers*2 pages per pair, one launch).
 * src/dst are device int32[n_pairs].  Replaces the 2L cudaMemcpyAsync calls of
 * Engine::cow_guard, src/model.cpp:178-187. */
void launch_kv_cow_copy(uint16_t* pool_k, uint16_t* pool_v, int nb, const int32_t* src,
                        const int32_t* dst, int n_pairs, nova_stream_t s);

/* Apply a batch of COW decisions in one launch: for each op, copy page src to
 * page dst in every layer of both pools, then set tables_dev[table_index] = dst.
 * ops is a HOST array (copied into the launch, 64 ops per kernel), so no
 * staging buffer or host sync is needed: the fused form of cow_guard's
 * 2L+1 copies (src/model.cpp:171-191) for any number of sessions. */
typedef struct { int32_t src, dst; int64_t table_index; } nova_cow_op;
void launch_kv_cow_apply(uint16_t* pool_k, uint16_t* pool_v, int nb, int32_t* tables_dev,
                         const nova_cow_op* ops, int n_ops, nova_stream_t s);

/* Clear pages (all layers, K and V) -- the per-page memsets of
 * SessionManager::create, code/session.h:107-118, as one launch.
 * pages: device int32[n_pages]. */
void launch_kv_zero_pages(uint16_t* pool_k, uint16_t* pool_v, int nb, const int32_t* pages,
                          int n_pages, nova_stream_t s);

/* Update single entries of device block tables: table_dev[idx[c]] = val[c]
 * for c < n (idx/val are device int32).  The H2D table patch of cow_guard
 * (model.cpp:188-190) for a whole batch of COWs. */
void launch_table_patch(int32_t* table_dev, const int32_t* idx, const int32_t* val, int n,
                        nova_stream_t s);

/* ---- RoPE (src/kernel/rope.cu), NeoX pairs (i, i+HD/2) of the Qwen2 family ---- */

/* cos/sin table [4096][HD/2] fp32 (the reference's kCtx rows, config.h:23).
 * Replaces nova::launch_rope_table, include/nova/kernel.h:47 (rope.cu:9-18,69-72).
 * Each float step of the reference recipe is correctly rounded. */
void launch_rope_table(float* cs, float* sn, nova_stream_t s);
/* The same table with `rows` positions, for contexts past the reference's
 * 4096-row table.  Not a reference surface. */
void launch_rope_table_rows(float* cs, float* sn, int rows, nova_stream_t s);
/* Rotate n tokens in place: q [n][NH][HD], k [n][NKV][HD] fp32 at positions
 * pos0..pos0+n-1.  Replaces nova::launch_rope_batch, kernel.h:48 (rope.cu:39-58,74-80). */
void launch_rope_batch(float* q, float* k, int n, int64_t pos0, const float* cs, const float* sn,
                       nova_stream_t s);
/* One token.  Replaces nova::launch_rope, kernel.h:49 (rope.cu:21-37,82-87). */
void launch_rope(float* q, float* k, int64_t pos, const float* cs, const float* sn, nova_stream_t s);
/* RopeKvOp fused (code/graph/dense.h:75-83: rope_batch, then kv_store_paged):
 * rotate q in place; rotate k and append it with v as fp16 at pos0..pos0+n-1
 * through the block table (k, v: [n][NKV][HD] fp32; k's buffer is left as
 * passed).  One launch and no round trip of K through memory. */
void launch_rope_kv_store_paged(float* q, const float* k, const float* v, const float* cs, const float* sn,
                                uint16_t* pool_k, uint16_t* pool_v, const int32_t* table, int layer, int nb,
                                int n, int64_t pos0, nova_stream_t s);
/* Batched form: session i rotates and appends n tokens at n_past[i]..
 * (device int32[n_sess]) through tables + i*table_stride; q [n_sess][n][NH][HD],
 * k, v [n_sess][n][NKV][HD] fp32.  A decode step's RoPE + append for all
 * sessions (n = 1) or a prefill chunk per session, in one launch. */
void launch_rope_kv_store_paged_batch(float* q, const float* k, const float* v, const float* cs,
                                      const float* sn, uint16_t* pool_k, uint16_t* pool_v,
                                      const int32_t* tables, int table_stride, const int32_t* n_past,
                                      int n_sess, int n, int layer, int nb, nova_stream_t s);

/* ---- Q4_K GEMV (src/kernel/q4k_gemv.cu), weights in ggml block_q4_K
 * (include/nova/quant/q4_k.h:19-25: 144 B per 256 weights, row-major,
 * rows x cols/256 blocks), activations as ActQ8 (include/nova/kernel/types.h:24-28)
 * passed as three plain arrays: int8 codes [rows][cols], fp32 scales
 * [rows][cols/32], int32 sums of each 16 codes [rows][cols/16].  The GEMVs
 * read the three activation arrays with 16-byte loads and abort on pointers
 * that are not 16-byte aligned (the reference's ActQ8 buffers come from its
 * arena, which aligns them). ---- */

/* Quantise rows x cols fp32 activations (cols % 32 == 0).  Replaces
 * nova::launch_quant / launch_quant_ffn, q4k_gemv.cu:196-207 (kernel :9-33),
 * which fix cols to D or FFN at compile time. */
void launch_quant_q8(int8_t* qs, float* d, int32_t* sums, const float* x, int rows, int cols, nova_stream_t s);
/* out[r] = row r of the Q4_K matrix . the quantised activation (one token),
 * cols % 256 == 0, cols <= 32768.  Replaces nova::launch_gemv<K, R>,
 * q4k_gemv.cu:209-213 (kernel :35-91; Q4KWeight = {blocks, rows, cols},
 * types.h:17-21, passed here as plain arguments). */
void launch_gemv_q4k(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                     const int32_t* xs, float* out, nova_stream_t s);
/* Four tokens: out[t][r] = row r . activation t for t = 0..3 -- the reference's
 * launch_gemv4<K, R> (q4k_gemv.cu:182-187, kernel :98-180), which
 * Engine::decode_batch uses for every projection (model.cpp:270-311).  The
 * four ActQ8 activations are stacked: xq [4][cols], xd [4][cols/32],
 * xs [4][cols/16]; out [4][rows].  Each weight is read once for the four
 * tokens; out[t] equals launch_gemv_q4k on token t up to fp32 summation
 * order (the same terms, summed in another order).
 * cols % 256 == 0, cols <= 28672. */
void launch_gemv4_q4k(const uint8_t* blocks, int64_t rows, int cols, const int8_t* xq, const float* xd,
                      const int32_t* xs, float* out, nova_stream_t s);
/* The quantisation and the GEMVs that share one activation in one launch:
 * n_mat (1..4) Q4_K matrices of the same width cols (blocks[m], rows[m],
 * outs[m]; host arrays) against fp32 x, quantised inside the launch with the
 * arithmetic of launch_quant_q8 (same codes, scales and sums, so outs[m] is
 * bit-identical to launch_quant_q8 followed by launch_gemv_q4k per matrix).
 * Replaces the reference's Kernel::quant (include/nova/kernel.h:80-86,
 * kernel q4k_gemv.cu:9-33) followed by gemm_q4k/launch_gemv for each of the
 * q/k/v or gate/up projections (kernel.h:29-34, q4k_gemv.cu:209-213). */
void launch_gemv_q4k_f32(const uint8_t* const* blocks, const int64_t* rows, float* const* outs, int n_mat,
                         int cols, const float* x, nova_stream_t s);

#ifdef __cplusplus
}
#endif
#endif
