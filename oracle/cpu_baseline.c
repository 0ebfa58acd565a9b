/* cpu_baseline.c -- TEST INFRASTRUCTURE: the CPU baseline of bench.py (see
 * cpu_baseline.h).  Built with -O3 -march=x86-64-v3 (AVX2, FMA, F16C).
 *
 * Core: a block of query vectors (pre-scaled by 1/sqrt(hd) * log2 e) against
 * the keys of a page range, one page at a time: the page's K rows are
 * converted to fp32 once for all queries of the block, the block's scores
 * come from AVX2 dot products, each query keeps a running max m, sum l and
 * accumulator acc (log2 domain, the recurrence of attn.cu:252-263 applied per
 * page instead of per key), and the page's V rows, converted once, are added
 * with the weights.  Splits of one (session, head) merge with the rule of
 * fa_combine_kernel (attn.cu:163-191). */
#include "cpu_baseline.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAX_KB 64
#define MAX_HD 256
#define SPLIT_PAGES 64          /* decode work unit: at most 64 pages of one (session, kv head) */
#define PQ 16                   /* prefill work unit: 16 queries (x G heads) of one kv head */

static const float kLog2e = 1.4426950408889634f;

/* 2^x for x <= 0 (and -inf -> 0): 2^floor(x) times a degree-8 Taylor
 * polynomial of e^(f ln 2) on [0, 1); relative error below 2e-7. */
static inline float exp2_neg(float x) {
    if (!(x > -126.f)) return 0.f;
    const float xi = floorf(x);
    const float f = x - xi;
    const float c1 = 0.6931471805599453f, c2 = 0.2402265069591007f, c3 = 0.05550410866482158f,
                c4 = 0.009618129107628477f, c5 = 0.0013333558146428443f, c6 = 1.5403530393381606e-4f,
                c7 = 1.525273380405984e-5f, c8 = 1.3215486790144307e-6f;
    const float p = 1.f + f * (c1 + f * (c2 + f * (c3 + f * (c4 + f * (c5 + f * (c6 + f * (c7 + f * c8)))))));
    return ldexpf(p, (int)xi);
}

/* n fp16 values (n a multiple of 8) to fp32 */
static inline void f16_row(const uint16_t* src, float* dst, int n) {
    for (int d = 0; d < n; d += 8)
        _mm256_storeu_ps(dst + d, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(src + d))));
}

static inline float hsum(__m256 v) {
    const __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    __m128 s = _mm_add_ps(lo, hi);
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

static inline float dot(const float* a, const float* b, int n) {
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    for (int d = 0; d < n; d += 16) {
        s0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + d), _mm256_loadu_ps(b + d), s0);
        s1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + d + 8), _mm256_loadu_ps(b + d + 8), s1);
    }
    return hsum(_mm256_add_ps(s0, s1));
}

/* acc[0..n) = acc * c + sum_j w[j] * rows[j][0..n) */
static inline void scale_add_rows(float* acc, float c, const float* w, const float* rows, int nrows, int n) {
    for (int d = 0; d < n; d += 8) {
        __m256 a = _mm256_mul_ps(_mm256_loadu_ps(acc + d), _mm256_set1_ps(c));
        for (int j = 0; j < nrows; ++j)
            a = _mm256_fmadd_ps(_mm256_set1_ps(w[j]), _mm256_loadu_ps(rows + (size_t)j * n + d), a);
        _mm256_storeu_ps(acc + d, a);
    }
}

/* nq query vectors qv (nq x hd, log2-domain scale applied) with causal limits
 * lim[r] (last visible key) against keys [k0, k1) of one kv head; updates
 * m, l, acc (nq x hd). */
static void attend(cb_geom g, const float* qv, const int64_t* lim, int nq, const uint16_t* pool_k,
                   const uint16_t* pool_v, const int32_t* table, int layer, int nb, int kvh, int64_t k0,
                   int64_t k1, float* m, float* l, float* acc, float* kf, float* vf, float* s) {
    const int hd = g.hd, kb = g.kb;
    const int64_t row = (int64_t)g.nkv * hd;
    for (int64_t p0 = k0 - k0 % kb; p0 < k1; p0 += kb) {
        const int64_t js = p0 > k0 ? p0 : k0, je = p0 + kb < k1 ? p0 + kb : k1;
        const int n = (int)(je - js);
        const int64_t page = ((int64_t)layer * nb + table[p0 / kb]) * kb;
        const uint16_t* kp = pool_k + (page + (js - p0)) * row + (int64_t)kvh * hd;
        const uint16_t* vp = pool_v + (page + (js - p0)) * row + (int64_t)kvh * hd;
        for (int j = 0; j < n; ++j) f16_row(kp + j * row, kf + (size_t)j * hd, hd);
        int any = 0;
        for (int r = 0; r < nq; ++r) {
            float* sr = s + (size_t)r * MAX_KB;
            float mt = -INFINITY;
            for (int j = 0; j < n; ++j) {
                const float v = js + j <= lim[r] ? dot(qv + (size_t)r * hd, kf + (size_t)j * hd, hd) : -INFINITY;
                sr[j] = v;
                mt = v > mt ? v : mt;
            }
            if (mt == -INFINITY) {            /* no visible key in this page */
                sr[0] = NAN;                  /* marks the row as skipped */
                continue;
            }
            any = 1;
            float corr = 1.f;
            if (mt > m[r]) {
                corr = exp2_neg(m[r] - mt);   /* m = -inf at start: corr 0 */
                m[r] = mt;
            }
            float ls = 0.f;
            for (int j = 0; j < n; ++j) {
                sr[j] = exp2_neg(sr[j] - m[r]);
                ls += sr[j];
            }
            l[r] = l[r] * corr + ls;
            sr[MAX_KB - 1] = corr;            /* n <= kb <= MAX_KB - 2: slot free */
        }
        if (!any) continue;
        for (int j = 0; j < n; ++j) f16_row(vp + j * row, vf + (size_t)j * hd, hd);
        for (int r = 0; r < nq; ++r) {
            float* sr = s + (size_t)r * MAX_KB;
            if (isnan(sr[0])) continue;
            scale_add_rows(acc + (size_t)r * hd, sr[MAX_KB - 1], sr, vf, n, hd);
        }
    }
}

/* allocation or thread-start failures abort with a message (the reference's
   abort-only convention): a lost unit would leave outputs uninitialised */
static void* must(void* p, const char* what) {
    if (!p) {
        fprintf(stderr, "cpu_baseline: %s failed\n", what);
        abort();
    }
    return p;
}

/* ---------------- thread pool over work units ---------------- */
typedef struct {
    void (*fn)(void* ctx, int unit, float* scratch);
    void* ctx;
    int n_units;
    atomic_int next;
    size_t scratch_floats;
} pool_job;

static void* pool_worker(void* p) {
    pool_job* j = (pool_job*)p;
    float* scratch = (float*)must(aligned_alloc(64, (j->scratch_floats * sizeof(float) + 63) / 64 * 64 + 64),
                                  "aligned_alloc");
    for (;;) {
        const int u = atomic_fetch_add(&j->next, 1);
        if (u >= j->n_units) break;
        j->fn(j->ctx, u, scratch);
    }
    free(scratch);
    return NULL;
}

static void run_pool(void (*fn)(void*, int, float*), void* ctx, int n_units, size_t scratch_floats, int n_threads) {
    pool_job j;
    j.fn = fn;
    j.ctx = ctx;
    j.n_units = n_units;
    atomic_init(&j.next, 0);
    j.scratch_floats = scratch_floats;
    if (n_threads < 1) n_threads = 1;
    if (n_threads > n_units) n_threads = n_units > 0 ? n_units : 1;
    pthread_t* th = (pthread_t*)must(malloc(sizeof(pthread_t) * (size_t)n_threads), "malloc");
    for (int t = 0; t < n_threads; ++t)
        if (pthread_create(&th[t], NULL, pool_worker, &j) != 0) must(NULL, "pthread_create");
    for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
    free(th);
}

/* ---------------- decode ---------------- */
typedef struct {
    cb_geom g;
    const float* q;
    const uint16_t *pool_k, *pool_v;
    const int32_t* tables;
    int table_stride;
    const int32_t* n_keys;
    int layer, nb;
    int* unit_sess;      /* per unit: session, kv head, first page, split index */
    int* unit_kvh;
    int* unit_page;
    int* unit_split;
    int* sess_split0;    /* first split slot of a session; splits per session */
    int* sess_nsplit;
    float* part;         /* [split slot][nh][2 + hd]: m, l, acc */
} dec_ctx;

static void dec_unit(void* p, int u, float* scratch) {
    const dec_ctx* c = (const dec_ctx*)p;
    const cb_geom g = c->g;
    const int hd = g.hd, G = g.nh / g.nkv;
    const int i = c->unit_sess[u], kvh = c->unit_kvh[u];
    const int64_t nk = c->n_keys[i];
    const int64_t k0 = (int64_t)c->unit_page[u] * g.kb;
    int64_t k1 = k0 + (int64_t)SPLIT_PAGES * g.kb;
    if (k1 > nk) k1 = nk;
    float* kf = scratch;
    float* vf = kf + MAX_KB * MAX_HD;
    float* s = vf + MAX_KB * MAX_HD;
    float* qv = s + (size_t)G * MAX_KB;
    float* acc = qv + (size_t)G * hd;
    float m[64], l[64];
    int64_t lim[64] = {0};
    const float sc = kLog2e / sqrtf((float)hd);
    for (int r = 0; r < G; ++r) {
        const float* qs = c->q + ((int64_t)i * g.nh + kvh * G + r) * hd;
        for (int d = 0; d < hd; ++d) qv[(size_t)r * hd + d] = qs[d] * sc;
        m[r] = -INFINITY;
        l[r] = 0.f;
        lim[r] = nk - 1;
    }
    memset(acc, 0, sizeof(float) * (size_t)G * hd);
    attend(g, qv, lim, G, c->pool_k, c->pool_v, c->tables + (int64_t)i * c->table_stride, c->layer, c->nb, kvh, k0,
           k1, m, l, acc, kf, vf, s);
    for (int r = 0; r < G; ++r) {
        float* pr = c->part + ((int64_t)(c->sess_split0[i] + c->unit_split[u]) * g.nh + kvh * G + r) * (hd + 2);
        pr[0] = m[r];
        pr[1] = l[r];
        memcpy(pr + 2, acc + (size_t)r * hd, sizeof(float) * hd);
    }
}

void cb_attn_decode_batch(cb_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                          const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess,
                          int layer, int nb, float* o, int n_threads) {
    const int hd = g.hd;
    if (g.kb > MAX_KB - 2 || hd > MAX_HD || hd % 16 || g.nh / g.nkv > 64) abort();
    int n_units = 0, n_slots = 0;
    int* sess_split0 = (int*)must(malloc(sizeof(int) * (size_t)(n_sess + 1)), "malloc");
    int* sess_nsplit = (int*)must(malloc(sizeof(int) * (size_t)(n_sess + 1)), "malloc");
    for (int i = 0; i < n_sess; ++i) {
        const int pages = (int)((n_keys[i] + g.kb - 1) / g.kb);
        const int ns = (pages + SPLIT_PAGES - 1) / SPLIT_PAGES;
        sess_split0[i] = n_slots;
        sess_nsplit[i] = ns;
        n_slots += ns;
        n_units += ns * g.nkv;
    }
    dec_ctx c;
    c.g = g;
    c.q = q;
    c.pool_k = pool_k;
    c.pool_v = pool_v;
    c.tables = tables;
    c.table_stride = table_stride;
    c.n_keys = n_keys;
    c.layer = layer;
    c.nb = nb;
    c.sess_split0 = sess_split0;
    c.sess_nsplit = sess_nsplit;
    c.unit_sess = (int*)must(malloc(sizeof(int) * (size_t)(n_units + 1) * 4), "malloc");
    c.unit_kvh = c.unit_sess + (n_units + 1);
    c.unit_page = c.unit_kvh + (n_units + 1);
    c.unit_split = c.unit_page + (n_units + 1);
    c.part = (float*)must(malloc(sizeof(float) * ((size_t)n_slots * g.nh * (hd + 2) + 1)), "malloc");
    int u = 0;
    for (int i = 0; i < n_sess; ++i)
        for (int sp = 0; sp < sess_nsplit[i]; ++sp)
            for (int h = 0; h < g.nkv; ++h, ++u) {
                c.unit_sess[u] = i;
                c.unit_kvh[u] = h;
                c.unit_page[u] = sp * SPLIT_PAGES;
                c.unit_split[u] = sp;
            }
    const int G = g.nh / g.nkv;
    const size_t scratch = (size_t)2 * MAX_KB * MAX_HD + (size_t)G * MAX_KB + (size_t)2 * G * hd;
    run_pool(dec_unit, &c, n_units, scratch, n_threads);
    /* merge the splits (attn.cu:163-191) */
    for (int i = 0; i < n_sess; ++i)
        for (int h = 0; h < g.nh; ++h) {
            float* out = o + ((int64_t)i * g.nh + h) * hd;
            float M = -INFINITY;
            for (int sp = 0; sp < sess_nsplit[i]; ++sp) {
                const float* pr = c.part + ((int64_t)(sess_split0[i] + sp) * g.nh + h) * (hd + 2);
                if (pr[1] > 0.f && pr[0] > M) M = pr[0];
            }
            float L = 0.f;
            for (int d = 0; d < hd; ++d) out[d] = 0.f;
            for (int sp = 0; sp < sess_nsplit[i]; ++sp) {
                const float* pr = c.part + ((int64_t)(sess_split0[i] + sp) * g.nh + h) * (hd + 2);
                if (!(pr[1] > 0.f)) continue;
                const float f = exp2_neg(pr[0] - M);
                L += pr[1] * f;
                for (int d = 0; d < hd; ++d) out[d] += pr[2 + d] * f;
            }
            const float inv = L > 0.f ? 1.f / L : 0.f;
            for (int d = 0; d < hd; ++d) out[d] *= inv;
        }
    free(c.part);
    free(c.unit_sess);
    free(sess_split0);
    free(sess_nsplit);
}

/* ---------------- prefill ---------------- */
typedef struct {
    cb_geom g;
    const float* q;
    const uint16_t *pool_k, *pool_v;
    const int32_t* tables;
    int table_stride;
    const int32_t* n_past;
    int n_q, layer, nb, qblocks;
    float* o;
} pre_ctx;

static void pre_unit(void* p, int u, float* scratch) {
    const pre_ctx* c = (const pre_ctx*)p;
    const cb_geom g = c->g;
    const int hd = g.hd, G = g.nh / g.nkv;
    const int per_sess = c->qblocks * g.nkv;
    const int i = u / per_sess, rem = u - i * per_sess;
    const int kvh = rem / c->qblocks, qb = rem - kvh * c->qblocks;
    const int q0 = qb * PQ, q1 = q0 + PQ < c->n_q ? q0 + PQ : c->n_q;
    const int nq = (q1 - q0) * G;
    const int64_t np = c->n_past[i];
    float* kf = scratch;
    float* vf = kf + MAX_KB * MAX_HD;
    float* s = vf + MAX_KB * MAX_HD;
    float* qv = s + (size_t)PQ * G * MAX_KB;
    float* acc = qv + (size_t)PQ * G * hd;
    float* m = acc + (size_t)PQ * G * hd;
    float* l = m + PQ * G;
    int64_t lim[PQ * 64];
    const float sc = kLog2e / sqrtf((float)hd);
    for (int qi = q0; qi < q1; ++qi)
        for (int r = 0; r < G; ++r) {
            const int v = (qi - q0) * G + r;
            const float* qs = c->q + (((int64_t)i * c->n_q + qi) * g.nh + kvh * G + r) * hd;
            for (int d = 0; d < hd; ++d) qv[(size_t)v * hd + d] = qs[d] * sc;
            m[v] = -INFINITY;
            l[v] = 0.f;
            lim[v] = np + qi;
        }
    memset(acc, 0, sizeof(float) * (size_t)nq * hd);
    attend(g, qv, lim, nq, c->pool_k, c->pool_v, c->tables + (int64_t)i * c->table_stride, c->layer, c->nb, kvh, 0,
           np + q1, m, l, acc, kf, vf, s);
    for (int qi = q0; qi < q1; ++qi)
        for (int r = 0; r < G; ++r) {
            const int v = (qi - q0) * G + r;
            float* out = c->o + (((int64_t)i * c->n_q + qi) * g.nh + kvh * G + r) * hd;
            const float inv = l[v] > 0.f ? 1.f / l[v] : 0.f;
            for (int d = 0; d < hd; ++d) out[d] = acc[(size_t)v * hd + d] * inv;
        }
}

void cb_attn_prefill_batch(cb_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                           const int32_t* tables, int table_stride, const int32_t* n_past, int n_sess,
                           int n_q, int layer, int nb, float* o, int n_threads) {
    const int hd = g.hd, G = g.nh / g.nkv;
    if (g.kb > MAX_KB - 2 || hd > MAX_HD || hd % 16 || G > 64) abort();
    if (n_q <= 0 || n_sess <= 0) return;
    pre_ctx c;
    c.g = g;
    c.q = q;
    c.pool_k = pool_k;
    c.pool_v = pool_v;
    c.tables = tables;
    c.table_stride = table_stride;
    c.n_past = n_past;
    c.n_q = n_q;
    c.layer = layer;
    c.nb = nb;
    c.qblocks = (n_q + PQ - 1) / PQ;
    c.o = o;
    const size_t scratch = (size_t)2 * MAX_KB * MAX_HD + (size_t)PQ * G * MAX_KB + (size_t)2 * PQ * G * hd +
                           (size_t)2 * PQ * G;
    run_pool(pre_unit, &c, n_sess * g.nkv * c.qblocks, scratch, n_threads);
}
