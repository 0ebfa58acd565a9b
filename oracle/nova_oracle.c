/*
 * nova_oracle.c -- CPU oracle for the paged KV-cache path (TEST INFRASTRUCTURE).
 *
 * A plain-C restatement of the reference's host bookkeeping and kernels, used
 * only as the checker in tests/ and smoke(), and as the CPU baseline in
 * bench.py.  The product never links it.  Citations are reference file:line.
 *
 * Pinning (what checks each function against something other than itself):
 *   - pool, hash, registry: bit-exact against the reference's own headers
 *     compiled into oracle/_ref (tests/test_oracle_pins.py), the golden
 *     vectors of tests/kv_block_test.cpp and a pool probe (init(3, 64), two
 *     slices, attach_prefix at 20 tokens, one COW to page 8), and the
 *     invariants of tests/cow_demo.cpp / cow_e2e_demo.cpp.
 *   - kv_store / gather / cow_copy: closed form (bit-exact copies) and a
 *     brute-force contiguous model.
 *   - decode / prefill: the reference's SYCL restatement of the same
 *     algorithm run through its own host shim (oracle/_ref), the f64
 *     textbook softmax, the n_keys==1 => O==V closed form
 *     (tests/gpu_misc.cu:41-65) and the prefill-row == decode identity.
 */
#define _GNU_SOURCE
#include "nova_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ======================= fp16 ======================= */
float or_f16_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) & 1u;
    const uint32_t e = (uint32_t)(h >> 10) & 31u;
    const uint32_t m = (uint32_t)h & 1023u;
    float v;
    if (e == 0)       v = ldexpf((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else              v = ldexpf((float)(m | 1024u), (int)e - 25);
    return s ? -v : v;
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);           /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);          /* overflow -> inf (RNE) */
    if (ax < 0x38800000u) {                                            /* subnormal / zero */
        /* value = ax as float; scale to units of 2^-24 and round-to-nearest-even */
        float a;
        memcpy(&a, &ax, 4);
        const float t = a * 16777216.0f;                               /* exact: power of two */
        float r = nearbyintf(t);                                       /* default mode = RNE */
        return (uint16_t)(sign | (uint32_t)r);
    }
    const uint32_t e = (ax >> 23) - 112u;                              /* rebias 127 -> 15 */
    const uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;           /* carries into exponent ok */
    return (uint16_t)(sign | h);
}

void or_f32_to_f16_n(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_f32_to_f16(src[i]);
}
void or_f16_to_f32_n(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = or_f16_to_f32(src[i]);
}

/* ======================= KvPool ======================= */
typedef struct {
    int live;
    int need_copy_from, need_copy_blk;
    int64_t n_past;
    int32_t* table;
} or_slice;

struct or_pool {
    int64_t ctx;
    int nblocks, n_slices, nb_total, cow_count;
    or_slice* s;            /* indexed by slice id */
    int* order;             /* live slice ids in acquisition order (slices_ vector) */
    int n_order;
    int* free_slices;       /* stack, back = next */
    int n_free_slices;
    int* free_blocks;       /* stack, back = next; grows: freeing an already free
                               page pushes it again (refcount clamps at 0) */
    int n_free_blocks, cap_free_blocks;
    int* refcnt;
};

or_pool* or_pool_new(int n_slices, int64_t ctx) {
    /* KvPool::init kv_pool.h:70-84 */
    or_pool* p = (or_pool*)calloc(1, sizeof(or_pool));
    p->ctx = ctx;
    p->nblocks = (int)((ctx + 16 - 1) / 16);   /* kKvBlock = 16 (kv_pool_cfg.h:14) */
    p->n_slices = n_slices;
    p->s = (or_slice*)calloc((size_t)(n_slices > 0 ? n_slices : 1), sizeof(or_slice));
    p->order = (int*)malloc(sizeof(int) * (size_t)(n_slices > 0 ? n_slices : 1));
    p->free_slices = (int*)malloc(sizeof(int) * (size_t)(n_slices > 0 ? n_slices : 1));
    for (int i = n_slices - 1; i >= 0; --i) p->free_slices[p->n_free_slices++] = i;
    p->nb_total = n_slices * p->nblocks;
    p->refcnt = (int*)calloc((size_t)(p->nb_total > 0 ? p->nb_total : 1), sizeof(int));
    /* free blocks pushed descending => back is the lowest id */
    p->cap_free_blocks = p->nb_total + 16;
    p->free_blocks = (int*)malloc(sizeof(int) * (size_t)p->cap_free_blocks);
    for (int b = p->nb_total - 1; b >= 0; --b) p->free_blocks[p->n_free_blocks++] = b;
    for (int i = 0; i < n_slices; ++i) {
        p->s[i].need_copy_from = -1;
        p->s[i].need_copy_blk = -1;
    }
    return p;
}

void or_pool_delete(or_pool* p) {
    if (!p) return;
    for (int i = 0; i < p->n_slices; ++i) free(p->s[i].table);
    free(p->s); free(p->order); free(p->free_slices); free(p->free_blocks); free(p->refcnt);
    free(p);
}

static void erase_free_block(or_pool* p, int phys) {
    /* std::find + erase: first occurrence, order of the rest preserved */
    for (int i = 0; i < p->n_free_blocks; ++i) {
        if (p->free_blocks[i] == phys) {
            memmove(p->free_blocks + i, p->free_blocks + i + 1,
                    sizeof(int) * (size_t)(p->n_free_blocks - i - 1));
            --p->n_free_blocks;
            return;
        }
    }
}

int or_pool_acquire(or_pool* p) {
    /* KvPool::acquire kv_pool.h:90-113 */
    if (p->n_free_slices == 0) return -1;
    const int id = p->free_slices[--p->n_free_slices];
    or_slice* s = &p->s[id];
    s->live = 1;
    s->need_copy_from = -1;   /* fresh KvSlice{} */
    s->need_copy_blk = -1;
    s->n_past = 0;
    free(s->table);
    s->table = (int32_t*)malloc(sizeof(int32_t) * (size_t)(p->nblocks > 0 ? p->nblocks : 1));
    for (int b = 0; b < p->nblocks; ++b) s->table[b] = (int32_t)(id * p->nblocks + b);
    p->order[p->n_order++] = id;
    for (int b = 0; b < p->nblocks && id * p->nblocks + b < p->nb_total; ++b) {
        const int phys = s->table[b];
        p->refcnt[phys] = 1;
        erase_free_block(p, phys);
    }
    return id;
}

int or_pool_alloc_block(or_pool* p) {
    /* kv_pool.h:116-122: LIFO pop */
    if (p->n_free_blocks == 0) return -1;
    const int b = p->free_blocks[--p->n_free_blocks];
    p->refcnt[b] = 1;
    return b;
}

void or_pool_free_block(or_pool* p, int b) {
    /* kv_pool.h:123-126 */
    if (b < 0 || b >= p->nb_total) return;
    if (--p->refcnt[b] <= 0) {
        p->refcnt[b] = 0;
        if (p->n_free_blocks == p->cap_free_blocks) {
            p->cap_free_blocks *= 2;
            p->free_blocks = (int*)realloc(p->free_blocks, sizeof(int) * (size_t)p->cap_free_blocks);
        }
        p->free_blocks[p->n_free_blocks++] = b;
    }
}

void or_pool_ref_block(or_pool* p, int b) {
    if (b >= 0 && b < p->nb_total) ++p->refcnt[b];
}

int or_pool_refcnt(const or_pool* p, int b) {
    return (b >= 0 && b < p->nb_total) ? p->refcnt[b] : 0;
}

void or_pool_attach(or_pool* p, int dst, int src, int k) {
    /* kv_pool.h:132-138 -- n_past is only touched inside the loop (k==0 leaves it) */
    for (int i = 0; i < k; ++i) {
        p->s[dst].table[i] = p->s[src].table[i];
        or_pool_ref_block(p, p->s[src].table[i]);
        p->s[dst].n_past = (int64_t)k * 16;
    }
}

void or_pool_attach_prefix(or_pool* p, int dst, int src, int64_t n) {
    /* kv_pool.h:141-148 */
    const int nb = (int)((n + 16 - 1) / 16);
    for (int i = 0; i < nb && i < p->nblocks; ++i) {
        p->s[dst].table[i] = p->s[src].table[i];
        or_pool_ref_block(p, p->s[src].table[i]);
    }
    p->s[dst].n_past = n;
}

int or_pool_cow_slice(or_pool* p, int sid, int64_t pos) {
    /* kv_pool.h:153-166 */
    or_slice* s = &p->s[sid];
    const int lb = (int)(pos >> 4);
    if (lb < 0 || lb >= p->nblocks) return -1;
    const int phys = s->table[lb];
    if (or_pool_refcnt(p, phys) <= 1) return -1;
    const int nb = or_pool_alloc_block(p);
    if (nb < 0) return -2;
    ++p->cow_count;
    s->need_copy_from = phys;
    s->need_copy_blk = nb;
    s->table[lb] = nb;
    or_pool_free_block(p, phys);
    return nb;
}

void or_pool_release(or_pool* p, int sid) {
    /* kv_pool.h:168-174 */
    if (sid < 0 || sid >= p->n_slices || !p->s[sid].live) return;
    for (int b = 0; b < p->nblocks; ++b) or_pool_free_block(p, p->s[sid].table[b]);
    p->free_slices[p->n_free_slices++] = sid;
    for (int i = 0; i < p->n_order; ++i) {
        if (p->order[i] == sid) {
            memmove(p->order + i, p->order + i + 1, sizeof(int) * (size_t)(p->n_order - i - 1));
            --p->n_order;
            break;
        }
    }
    p->s[sid].live = 0;
}

int or_pool_nblocks(const or_pool* p) { return p->nblocks; }
int or_pool_nb_total(const or_pool* p) { return p->nb_total; }
int or_pool_cow_count(const or_pool* p) { return p->cow_count; }
int or_pool_free_blocks(const or_pool* p) { return p->n_free_blocks; }
int or_pool_used(const or_pool* p) { return p->n_order; }
int or_pool_free_slices(const or_pool* p) { return p->n_free_slices; }

int or_pool_free_list(const or_pool* p, int* out, int cap) {
    const int n = p->n_free_blocks < cap ? p->n_free_blocks : cap;
    memcpy(out, p->free_blocks, sizeof(int) * (size_t)n);
    return p->n_free_blocks;
}
int or_pool_refcnts(const or_pool* p, int* out, int cap) {
    const int n = p->nb_total < cap ? p->nb_total : cap;
    memcpy(out, p->refcnt, sizeof(int) * (size_t)n);
    return p->nb_total;
}
int or_pool_table(const or_pool* p, int sid, int32_t* out, int cap) {
    const int n = p->nblocks < cap ? p->nblocks : cap;
    memcpy(out, p->s[sid].table, sizeof(int32_t) * (size_t)n);
    return p->nblocks;
}
int64_t or_pool_n_past(const or_pool* p, int sid) { return p->s[sid].n_past; }
void or_pool_set_n_past(or_pool* p, int sid, int64_t n) { p->s[sid].n_past = n; }
int or_pool_need_copy(const or_pool* p, int sid, int* from, int* blk) {
    *from = p->s[sid].need_copy_from;
    *blk = p->s[sid].need_copy_blk;
    return *from >= 0;
}

/* ======================= kv_block IDs ======================= */
uint64_t or_kv_hash_ids(const int* ids, size_t n) {
    /* kv_block.h:21-64: decimal text -> uppercase hex of its bytes -> 16-hex
     * chunks (last one right-padded with '0') -> pairwise end-fold */
    static const char HEX[] = "0123456789ABCDEF";
    if (n == 0) return 0;
    size_t cap = n * 24 + 16, len = 0;
    char* hex = (char*)malloc(cap);
    for (size_t i = 0; i < n; ++i) {
        char dec[16];
        const int dl = snprintf(dec, sizeof dec, "%d", ids[i]);
        for (int j = 0; j < dl; ++j) {
            const unsigned char c = (unsigned char)dec[j];
            hex[len++] = HEX[c >> 4];
            hex[len++] = HEX[c & 15];
        }
    }
    const size_t nblk = (len + 15) / 16;
    uint64_t* blk = (uint64_t*)malloc(sizeof(uint64_t) * (nblk ? nblk : 1));
    for (size_t b = 0; b < nblk; ++b) {
        uint64_t v = 0;
        for (size_t k = 0; k < 16; ++k) {
            const size_t j = b * 16 + k;
            const char c = j < len ? hex[j] : '0';
            const uint64_t d = (c >= '0' && c <= '9') ? (uint64_t)(c - '0') : (uint64_t)(c - 'A' + 10);
            v = (v << 4) | d;
        }
        blk[b] = v;
    }
    size_t m = nblk;
    while (m > 1) {
        const size_t half = m / 2;
        uint64_t mid = blk[half];
        for (size_t i = 0; i < half; ++i) blk[i] = blk[i] + blk[m - 1 - i];
        size_t nm = half;
        if (m & 1) blk[nm++] = mid;
        m = nm;
    }
    const uint64_t r = nblk ? blk[0] : 0;
    free(hex);
    free(blk);
    return r;
}

uint64_t or_kv_hash_text(const char* text, size_t n) {
    /* kv_block.h:67-72: each UTF-8 byte is an id */
    int* ids = (int*)malloc(sizeof(int) * (n ? n : 1));
    for (size_t i = 0; i < n; ++i) ids[i] = (int)(unsigned char)text[i];
    const uint64_t r = or_kv_hash_ids(ids, n);
    free(ids);
    return r;
}

void or_kv_hash_hex(uint64_t v, char out[17]) {
    static const char HEX[] = "0123456789ABCDEF";
    for (int i = 15; i >= 0; --i) { out[i] = HEX[v & 15]; v >>= 4; }
    out[16] = 0;
}

void or_kv_block_id(uint64_t prefix, uint64_t suffix, char out[40]) {
    char a[17], b[17];
    or_kv_hash_hex(prefix, a);
    or_kv_hash_hex(suffix, b);
    snprintf(out, 40, "{ %s . %s }", a, b);
}

/* ======================= BlockRegistry ======================= */
typedef struct {
    uint64_t prefix, suffix;
    int session, turn, alive;
    int64_t pos0, pos1;
} or_reg_entry;

struct or_registry {
    or_reg_entry* v;
    size_t n, cap_alloc, cap;
};

or_registry* or_registry_new(void) {
    or_registry* r = (or_registry*)calloc(1, sizeof(or_registry));
    r->cap = 64;                                  /* kv_registry.h:69 */
    return r;
}
void or_registry_delete(or_registry* r) { if (r) { free(r->v); free(r); } }

int or_registry_live(const or_registry* r) {
    int n = 0;
    for (size_t i = 0; i < r->n; ++i) n += r->v[i].alive;
    return n;
}
int or_registry_total(const or_registry* r) { return (int)r->n; }

static void reg_evict(or_registry* r) {
    /* kv_registry.h:57-62: oldest live entries die first */
    while ((size_t)or_registry_live(r) > r->cap) {
        for (size_t i = 0; i < r->n; ++i) if (r->v[i].alive) { r->v[i].alive = 0; break; }
    }
}

void or_registry_set_capacity(or_registry* r, size_t n) { r->cap = n ? n : 1; reg_evict(r); }

void or_registry_put(or_registry* r, uint64_t prefix, uint64_t suffix, int session, int turn,
                     int64_t pos0, int64_t pos1) {
    /* kv_registry.h:36-40 */
    for (size_t i = 0; i < r->n; ++i)
        if (r->v[i].alive && r->v[i].prefix == prefix && r->v[i].suffix == suffix) r->v[i].alive = 0;
    if (r->n == r->cap_alloc) {
        r->cap_alloc = r->cap_alloc ? 2 * r->cap_alloc : 16;
        r->v = (or_reg_entry*)realloc(r->v, sizeof(or_reg_entry) * r->cap_alloc);
    }
    or_reg_entry e = {prefix, suffix, session, turn, 1, pos0, pos1};
    r->v[r->n++] = e;
    reg_evict(r);
}

int or_registry_find(const or_registry* r, uint64_t prefix, uint64_t suffix,
                     int* session, int* turn, int64_t* pos0, int64_t* pos1) {
    for (size_t i = 0; i < r->n; ++i) {
        const or_reg_entry* x = &r->v[i];
        if (x->alive && x->prefix == prefix && x->suffix == suffix) {
            *session = x->session; *turn = x->turn; *pos0 = x->pos0; *pos1 = x->pos1;
            return 1;
        }
    }
    return 0;
}

/* ======================= paged append / gather / COW ======================= */
static inline int64_t page_base(or_geom g, int layer, int nb, int phys) {
    /* ((layer*NB + phys) * KB) * KVW  (include/nova/model.h:140-145, kv_pool.h:8-15) */
    return (((int64_t)layer * nb + phys) * g.kb) * (int64_t)g.nkv * g.hd;
}

void or_kv_store_paged(or_geom g, uint16_t* pool_k, uint16_t* pool_v, const int32_t* table,
                       int layer, int nb, int n, int64_t pos0, const uint16_t* k, const uint16_t* v) {
    /* kv_store_paged_kernel elem.cu:59-76 */
    const int64_t kvw = (int64_t)g.nkv * g.hd;
    for (int t = 0; t < n; ++t) {
        const int64_t pos = pos0 + t;
        const int phys = table[pos / g.kb];
        const int slot = (int)(pos % g.kb);
        const int64_t off = page_base(g, layer, nb, phys) + (int64_t)slot * kvw;
        memcpy(pool_k + off, k + (int64_t)t * kvw, sizeof(uint16_t) * (size_t)kvw);
        memcpy(pool_v + off, v + (int64_t)t * kvw, sizeof(uint16_t) * (size_t)kvw);
    }
}

/* ---- RoPE ---- */
void or_rope_table(float* cs, float* sn, int rows, int half, double theta) {
    /* rope_table_kernel rope.cu:9-18, each float step correctly rounded */
    const float l2 = (float)log2((double)(float)theta);
    for (int pos = 0; pos < rows; ++pos) {
        for (int i = 0; i < half; ++i) {
            const float e = -(float)i * (1.f / (float)half);
            const float t = e * l2;
            const float f = (float)exp2((double)t);
            const float a = (float)pos * f;
            cs[(int64_t)pos * half + i] = (float)cos((double)a);
            sn[(int64_t)pos * half + i] = (float)sin((double)a);
        }
    }
}

static void rope_row(float* base, int half, const float* c, const float* s) {
    /* rope_batch_kernel rope.cu:51-57 (NeoX: a = i, b = i + half) */
    for (int i = 0; i < half; ++i) {
        const float x0 = base[i], x1 = base[i + half];
        base[i] = x0 * c[i] - x1 * s[i];
        base[i + half] = x0 * s[i] + x1 * c[i];
    }
}

void or_rope_apply(or_geom g, float* q, float* k, int n, int64_t pos0, const float* cs, const float* sn) {
    /* launch_rope_batch rope.cu:74-80: grid (token, head), heads 0..nh-1 are q, then k */
    const int half = g.hd / 2;
    for (int t = 0; t < n; ++t) {
        const int64_t pos = pos0 + t;
        const float* c = cs + pos * half;
        const float* s = sn + pos * half;
        for (int h = 0; h < g.nh; ++h) rope_row(q + ((int64_t)t * g.nh + h) * g.hd, half, c, s);
        for (int h = 0; h < g.nkv; ++h) rope_row(k + ((int64_t)t * g.nkv + h) * g.hd, half, c, s);
    }
}

void or_rope_kv_store_paged(or_geom g, float* q, const float* k, const float* v, const float* cs,
                            const float* sn, uint16_t* pool_k, uint16_t* pool_v, const int32_t* table,
                            int layer, int nb, int n, int64_t pos0) {
    /* RopeKvOp dense.h:75-83 = launch_rope_batch + launch_kv_store_paged (elem.cu:59-76) */
    const int half = g.hd / 2;
    const int64_t kvw = (int64_t)g.nkv * g.hd;
    float* kr = (float*)malloc(sizeof(float) * (size_t)kvw);
    for (int t = 0; t < n; ++t) {
        const int64_t pos = pos0 + t;
        const float* c = cs + pos * half;
        const float* s = sn + pos * half;
        for (int h = 0; h < g.nh; ++h) rope_row(q + ((int64_t)t * g.nh + h) * g.hd, half, c, s);
        memcpy(kr, k + (int64_t)t * kvw, sizeof(float) * (size_t)kvw);
        for (int h = 0; h < g.nkv; ++h) rope_row(kr + (int64_t)h * g.hd, half, c, s);
        const int64_t off = page_base(g, layer, nb, table[pos / g.kb]) + (pos % g.kb) * kvw;
        for (int64_t e = 0; e < kvw; ++e) {
            pool_k[off + e] = or_f32_to_f16(kr[e]);
            pool_v[off + e] = or_f32_to_f16(v[(int64_t)t * kvw + e]);
        }
    }
    free(kr);
}

/* ---- Q4_K ---- */
float or_q4k_half(uint16_t h) {
    /* half_to_float q4_k.h:28-41 (host branch) */
    const int sgn = (h >> 15) & 1, e = (h >> 10) & 0x1F;
    const uint32_t m = h & 0x3FFu;
    double v;
    if (e == 0) v = ldexp((double)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = ldexp((double)(m | 0x400u), e - 25);
    return (float)(sgn ? -v : v);
}

static void q4k_scale_min(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    /* get_scale_min_k4 q4_k.h:44-52 */
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

void or_q4k_dequant_block(const uint8_t* block, float* y) {
    /* dequant_block q4_k.h:55-73: sub-block 2g from the low nibbles of
       qs[32g..32g+31], 2g+1 from the high nibbles */
    uint16_t hd, hm;
    memcpy(&hd, block, 2);
    memcpy(&hm, block + 2, 2);
    const float d = or_q4k_half(hd), dmin = or_q4k_half(hm);
    const uint8_t* scales = block + 4;
    const uint8_t* q = block + 16;
    for (int g = 0; g < 4; ++g) {
        uint8_t sc0, m0, sc1, m1;
        q4k_scale_min(2 * g, scales, &sc0, &m0);
        q4k_scale_min(2 * g + 1, scales, &sc1, &m1);
        const float d0 = d * (float)sc0, e0 = dmin * (float)m0;
        const float d1 = d * (float)sc1, e1 = dmin * (float)m1;
        for (int l = 0; l < 32; ++l) y[g * 64 + l] = d0 * (float)(q[32 * g + l] & 0xF) - e0;
        for (int l = 0; l < 32; ++l) y[g * 64 + 32 + l] = d1 * (float)(q[32 * g + l] >> 4) - e1;
    }
}

void or_quant_q8(const float* x, int rows, int cols, int8_t* qs, float* d, int32_t* s) {
    /* quant_kernel q4k_gemv.cu:9-33 */
    for (int r = 0; r < rows; ++r) {
        for (int b = 0; b < cols / 32; ++b) {
            const float* xp = x + (int64_t)r * cols + 32 * b;
            float amax = 0.f;
            for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xp[i]));
            const float scale = amax * (1.f / 127.f);
            const float inv = amax > 0.f ? 127.f / amax : 0.f;
            int s0 = 0, s1 = 0;
            for (int i = 0; i < 32; ++i) {
                const int v = (int)rintf(xp[i] * inv);
                qs[(int64_t)r * cols + 32 * b + i] = (int8_t)v;
                if (i < 16) s0 += v; else s1 += v;
            }
            d[(int64_t)r * (cols / 32) + b] = scale;
            s[(int64_t)r * (cols / 16) + 2 * b] = s0;
            s[(int64_t)r * (cols / 16) + 2 * b + 1] = s1;
        }
    }
}

void or_gemv_q4k(const uint8_t* w, int64_t rows, int64_t cols, const int8_t* qs, const float* d,
                 const int32_t* s, double* out) {
    (void)s;
    float y[256];
    for (int64_t r = 0; r < rows; ++r) {
        double acc = 0.0;
        for (int64_t b = 0; b < cols / 256; ++b) {
            or_q4k_dequant_block(w + (r * (cols / 256) + b) * 144, y);
            for (int i = 0; i < 256; ++i) {
                const int64_t k = 256 * b + i;
                acc += (double)y[i] * ((double)qs[k] * (double)d[k / 32]);
            }
        }
        out[r] = acc;
    }
}

void or_kv_gather_paged(or_geom g, const uint16_t* pool, const int32_t* table, int layer, int nb,
                        int64_t n, uint16_t* out) {
    const int64_t kvw = (int64_t)g.nkv * g.hd;
    for (int64_t p = 0; p < n; ++p) {
        const int64_t off = page_base(g, layer, nb, table[p / g.kb]) + (p % g.kb) * kvw;
        memcpy(out + p * kvw, pool + off, sizeof(uint16_t) * (size_t)kvw);
    }
}

void or_cow_copy(or_geom g, uint16_t* pool_k, uint16_t* pool_v, int n_layers, int nb, int src, int dst) {
    /* Engine::cow_guard model.cpp:178-187: for every layer, K and V page src -> dst */
    const size_t per = (size_t)g.kb * (size_t)g.nkv * (size_t)g.hd;
    for (int l = 0; l < n_layers; ++l) {
        memcpy(pool_k + page_base(g, l, nb, dst), pool_k + page_base(g, l, nb, src), per * 2);
        memcpy(pool_v + page_base(g, l, nb, dst), pool_v + page_base(g, l, nb, src), per * 2);
    }
}

/* ======================= attention ======================= */
#define OR_MAXD 256

static inline const uint16_t* key_row(or_geom g, const uint16_t* pool, const int32_t* table,
                                      int layer, int nb, int64_t p, int kvh) {
    const int64_t kvw = (int64_t)g.nkv * g.hd;
    return pool + page_base(g, layer, nb, table[p / g.kb]) + (p % g.kb) * kvw + (int64_t)kvh * g.hd;
}

/* One warp's dot product: lane l accumulates d = l + 32c for c = 0..hd/32-1 with
 * fmaf, then the shuffle-down tree of warp_sum (attn.cu:31-35) reduces to lane 0. */
static float warp_dot(const float* q, const uint16_t* k, int hd) {
    float v[32];
    for (int l = 0; l < 32; ++l) {
        float part = 0.f;
        for (int c = 0; c < hd / 32; ++c) part = fmaf(q[l + 32 * c], or_f16_to_f32(k[l + 32 * c]), part);
        v[l] = part;
    }
    for (int o = 16; o > 0; o >>= 1) {
        float nv[32];
        for (int l = 0; l < 32; ++l) nv[l] = v[l] + ((l + o) < 32 ? v[l + o] : v[l]);
        memcpy(v, nv, sizeof v);
    }
    return v[0];
}

static float attn_scale(int hd) { return hd == 64 ? 0.125f : 0.08838834764831845f; }

/* fa_split_paged_kernel (attn.cu:197-289) for one head over all splits, then
 * fa_combine_kernel (attn.cu:163-191). */
static void decode_head(or_geom g, const float* qh, const uint16_t* pool_k, const uint16_t* pool_v,
                        const int32_t* table, int layer, int nb, int n_keys, int head, float* oh) {
    const int hd = g.hd;
    const int kvh = head / (g.nh / g.nkv);
    const float scale = attn_scale(hd);
    int nsplit = (n_keys + 31) / 32;                 /* attn.cu:503-507 */
    if (nsplit > 32) nsplit = 32;
    if (nsplit < 1) nsplit = 1;
    const int chunk = (n_keys + nsplit - 1) / nsplit;
    float pm[32], pl[32];
    float pacc[32][OR_MAXD];
    for (int sp = 0; sp < nsplit; ++sp) {
        float wm[4], wl[4], wacc[4][OR_MAXD];
        const int q4 = (chunk + 3) >> 2;
        for (int w = 0; w < 4; ++w) {
            const int kv0 = sp * chunk + w * q4;
            int kv1 = kv0 + q4;
            if (kv1 > n_keys) kv1 = n_keys;
            if (kv1 > (sp + 1) * chunk) kv1 = (sp + 1) * chunk;
            float m = -INFINITY, l = 0.f;
            float* acc = wacc[w];
            for (int d = 0; d < hd; ++d) acc[d] = 0.f;
            for (int p = kv0; p < kv1; ++p) {
                const uint16_t* kp = key_row(g, pool_k, table, layer, nb, p, kvh);
                const float qk = warp_dot(qh, kp, hd) * scale;
                const float mn = fmaxf(m, qk);
                const float corr = expf(m - mn);
                const float pr = expf(qk - mn);
                l = fmaf(l, corr, pr);
                const uint16_t* vp = key_row(g, pool_v, table, layer, nb, p, kvh);
                for (int d = 0; d < hd; ++d) acc[d] = fmaf(acc[d], corr, pr * or_f16_to_f32(vp[d]));
                m = mn;
            }
            wm[w] = m;
            wl[w] = l;
        }
        float mm = -INFINITY;
        for (int w = 0; w < 4; ++w) mm = fmaxf(mm, wm[w]);
        float ll = 0.f;
        for (int w = 0; w < 4; ++w) if (wl[w] > 0.f) ll = fmaf(wl[w], expf(wm[w] - mm), ll);
        pm[sp] = mm;
        pl[sp] = ll;
        for (int d = 0; d < hd; ++d) {
            float a = 0.f;
            for (int w = 0; w < 4; ++w) a = fmaf(wacc[w][d], expf(wm[w] - mm), a);
            pacc[sp][d] = a;
        }
    }
    float m = -INFINITY;
    for (int s = 0; s < nsplit; ++s) m = fmaxf(m, pm[s]);
    float l = 0.f;
    for (int s = 0; s < nsplit; ++s) if (pl[s] > 0.f) l = fmaf(pl[s], expf(pm[s] - m), l);
    for (int d = 0; d < hd; ++d) {
        float a = 0.f;
        for (int s = 0; s < nsplit; ++s) a = fmaf(pacc[s][d], expf(pm[s] - m), a);
        oh[d] = (l > 0.f) ? a / l : 0.f;
    }
}

void or_attn_decode_paged(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                          const int32_t* table, int layer, int nb, int n_keys, float* o) {
    for (int h = 0; h < g.nh; ++h)
        decode_head(g, q + (int64_t)h * g.hd, pool_k, pool_v, table, layer, nb, n_keys, h,
                    o + (int64_t)h * g.hd);
}

static void softmax_attn_f64(or_geom g, const float* qh, const uint16_t* pool_k, const uint16_t* pool_v,
                             const int32_t* table, int layer, int nb, int64_t n_keys, int kvh, double* oh) {
    const double scale = (double)attn_scale(g.hd);
    double* sc = (double*)malloc(sizeof(double) * (size_t)(n_keys > 0 ? n_keys : 1));
    double mx = -1e300;
    for (int64_t p = 0; p < n_keys; ++p) {
        const uint16_t* kp = key_row(g, pool_k, table, layer, nb, p, kvh);
        double acc = 0.0;
        for (int d = 0; d < g.hd; ++d) acc += (double)qh[d] * (double)or_f16_to_f32(kp[d]);
        sc[p] = acc * scale;
        if (sc[p] > mx) mx = sc[p];
    }
    double sum = 0.0;
    for (int64_t p = 0; p < n_keys; ++p) { sc[p] = exp(sc[p] - mx); sum += sc[p]; }
    for (int d = 0; d < g.hd; ++d) oh[d] = 0.0;
    for (int64_t p = 0; p < n_keys; ++p) {
        const uint16_t* vp = key_row(g, pool_v, table, layer, nb, p, kvh);
        for (int d = 0; d < g.hd; ++d) oh[d] += sc[p] * (double)or_f16_to_f32(vp[d]);
    }
    for (int d = 0; d < g.hd; ++d) oh[d] = n_keys > 0 ? oh[d] / sum : 0.0;
    free(sc);
}

void or_attn_decode_paged_f64(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                              const int32_t* table, int layer, int nb, int n_keys, double* o) {
    for (int h = 0; h < g.nh; ++h)
        softmax_attn_f64(g, q + (int64_t)h * g.hd, pool_k, pool_v, table, layer, nb, n_keys,
                         h / (g.nh / g.nkv), o + (int64_t)h * g.hd);
}

void or_attn_prefill_paged(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                           const int32_t* table, int layer, int nb, int n_q, int n_past, float* o) {
    /* flash_paged_kernel<false> attn.cu:293-357 */
    const float scale = attn_scale(g.hd);
    float acc[OR_MAXD];
    for (int qi = 0; qi < n_q; ++qi) {
        for (int h = 0; h < g.nh; ++h) {
            const int kvh = h / (g.nh / g.nkv);
            const float* qp = q + ((int64_t)qi * g.nh + h) * g.hd;
            const int64_t pos = (int64_t)n_past + qi;
            float m = -INFINITY, l = 0.f;
            for (int d = 0; d < g.hd; ++d) acc[d] = 0.f;
            for (int64_t p = 0; p <= pos; ++p) {
                const float qk = warp_dot(qp, key_row(g, pool_k, table, layer, nb, p, kvh), g.hd) * scale;
                const float mn = fmaxf(m, qk);
                const float e = expf(m - mn);
                const float pe = expf(qk - mn);
                l = fmaf(l, e, pe);
                const uint16_t* vp = key_row(g, pool_v, table, layer, nb, p, kvh);
                for (int d = 0; d < g.hd; ++d) acc[d] = fmaf(acc[d], e, pe * or_f16_to_f32(vp[d]));
                m = mn;
            }
            float* op = o + ((int64_t)qi * g.nh + h) * g.hd;
            const float inv = 1.f / l;
            for (int d = 0; d < g.hd; ++d) op[d] = acc[d] * inv;
        }
    }
}

void or_attn_prefill_paged_f64(or_geom g, const float* q, const uint16_t* pool_k,
                               const uint16_t* pool_v, const int32_t* table, int layer, int nb,
                               int n_q, int n_past, double* o) {
    for (int qi = 0; qi < n_q; ++qi)
        for (int h = 0; h < g.nh; ++h)
            softmax_attn_f64(g, q + ((int64_t)qi * g.nh + h) * g.hd, pool_k, pool_v, table, layer, nb,
                             (int64_t)n_past + qi + 1, h / (g.nh / g.nkv),
                             o + ((int64_t)qi * g.nh + h) * g.hd);
}

/* ---------------- threaded batch decode (CPU baseline) ---------------- */
typedef struct {
    or_geom g;
    const float* q;
    const uint16_t *pool_k, *pool_v;
    const int32_t* tables;
    int table_stride;
    const int32_t* n_keys;
    int n_sess, layer, nb;
    float* o;
    int next;                 /* shared work counter */
    pthread_mutex_t mu;
} batch_job;

static void* batch_worker(void* arg) {
    batch_job* j = (batch_job*)arg;
    const int units = j->n_sess * j->g.nh;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int u = j->next++;
        pthread_mutex_unlock(&j->mu);
        if (u >= units) break;
        const int s = u / j->g.nh, h = u % j->g.nh;
        const int64_t qo = ((int64_t)s * j->g.nh + h) * j->g.hd;
        decode_head(j->g, j->q + qo, j->pool_k, j->pool_v, j->tables + (int64_t)s * j->table_stride,
                    j->layer, j->nb, j->n_keys[s], h, j->o + qo);
    }
    return NULL;
}

void or_attn_decode_batch(or_geom g, const float* q, const uint16_t* pool_k, const uint16_t* pool_v,
                          const int32_t* tables, int table_stride, const int32_t* n_keys, int n_sess,
                          int layer, int nb, float* o, int n_threads) {
    batch_job j;
    j.g = g; j.q = q; j.pool_k = pool_k; j.pool_v = pool_v; j.tables = tables;
    j.table_stride = table_stride; j.n_keys = n_keys; j.n_sess = n_sess; j.layer = layer; j.nb = nb;
    j.o = o; j.next = 0;
    pthread_mutex_init(&j.mu, NULL);
    if (n_threads < 1) n_threads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)n_threads);
    for (int t = 0; t < n_threads; ++t) pthread_create(&th[t], NULL, batch_worker, &j);
    for (int t = 0; t < n_threads; ++t) pthread_join(th[t], NULL);
    free(th);
    pthread_mutex_destroy(&j.mu);
}
