// abi_consumer.cpp -- a C++ caller of the drop-in, written the way the
// reference's engine drives its kernel layer and session manager
// (src/model.cpp:171-191,282-289, code/session.h:84-180), using only the
// public headers include/hal.h, include/nova_kernel.h and include/nova_graph.h.
//
// One layer of a 1.5B-geometry pool: session A appends 100 tokens with
// launch_kv_store_paged; session B forks A's first 99 tokens (attach_prefix,
// unaligned, so the tail page is shared), runs session_cow over position 99
// and appends its own token 99; both sessions then decode with
// launch_attn_decode_paged, and A's last 20 positions run as a chunked
// prefill through launch_attn_prefill_paged.  Checks: the appended rows read
// back bit-exact, one COW with the donor page untouched and the refcounts of
// the shared and copied pages, and the decode and prefill outputs against an
// f64 softmax computed here, within max-abs 2e-3 / rel 1e-2.
// Exit 0 = pass, 77 = no GPU.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "hal.h"
#include "nova_graph.h"
#include "nova_kernel.h"

namespace {

// fp16 bits of a float that fp16 represents exactly (|x| in [2^-14, 65504] or 0)
uint16_t exact_half(float x) {
    if (x == 0.f) return 0;
    uint32_t u;
    std::memcpy(&u, &x, 4);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const int e = (int)((u >> 23) & 0xff) - 127 + 15;
    return (uint16_t)(sign | ((uint32_t)e << 10) | ((u >> 13) & 0x3ffu));
}
float half_value(uint16_t h) {
    const int e = (h >> 10) & 0x1f, m = h & 0x3ff;
    const float v = e == 0 ? std::ldexp((float)m, -24) : std::ldexp(1.f + m / 1024.f, e - 15);
    return (h & 0x8000) ? -v : v;
}

int fails = 0;
void check(bool ok, const char* what) {
    if (!ok) {
        std::printf("FAIL: %s\n", what);
        ++fails;
    }
}

}  // namespace

int main() {
    if (dev_count() == 0) {
        std::printf("no GPU visible: skipped\n");
        return 77;
    }
    const nova_geometry g = nova_model_geometry();
    const int KVW = g.nkv * g.hd, G = g.nh / g.nkv, layer = 3, n_tok = 100;
    std::printf("library %s: nh %d nkv %d hd %d layers %d\n", g.name, g.nh, g.nkv, g.hd, g.n_layers);

    nova_paged_t pg = nova_paged_new(3, 256);
    nova_kvpool_t pool = nova_paged_pool(pg);
    nova_stream_t st = nova_paged_stream(pg);
    uint16_t* pk = nova_paged_pool_k(pg);
    uint16_t* pv = nova_paged_pool_v(pg);
    const int nb = nova_paged_nb(pg);
    const int a = nova_paged_create_session(pg, 1);
    const int b = nova_paged_create_session(pg, 1);
    check(a >= 0 && b >= 0 && a != b, "two sessions");

    // host K/V rows of A (tokens 0..99) and B's own token 99, exact fp16 values
    std::mt19937 rng(7);
    std::uniform_int_distribution<int> d(-32, 32);
    auto row = [&](std::vector<uint16_t>& out, int n) {
        out.resize((size_t)n * KVW);
        for (auto& x : out) x = exact_half(d(rng) / 16.f);
    };
    std::vector<uint16_t> ka, va, kb1, vb1;
    row(ka, n_tok);
    row(va, n_tok);
    row(kb1, 1);
    row(vb1, 1);
    auto up = [&](const std::vector<uint16_t>& h) {
        void* p = dev_alloc(h.size() * 2);
        dev_upload(p, h.data(), h.size() * 2);
        return static_cast<uint16_t*>(p);
    };
    uint16_t *dka = up(ka), *dva = up(va), *dkb = up(kb1), *dvb = up(vb1);

    // A appends its 100 tokens (one call per token, the decode loop's shape)
    for (int t = 0; t < n_tok; ++t)
        launch_kv_store_paged(pk, pv, nova_paged_table_dev(pg, a), layer, nb, 1, t, dka + (size_t)t * KVW,
                              dva + (size_t)t * KVW, st);
    // B shares A's first 99 tokens; its first append at 99 copies the shared tail page
    nova_paged_attach_prefix(pg, b, a, n_tok - 1);
    const int tail = n_tok / 16;                                    // logical page of token 99
    std::vector<int32_t> tab_a(nova_kvpool_nblocks(pool)), tab_b(tab_a.size());
    nova_kvpool_table(pool, a, tab_a.data(), (int)tab_a.size());
    nova_kvpool_table(pool, b, tab_b.data(), (int)tab_b.size());
    check(tab_b[tail] == tab_a[tail], "tail page shared after attach_prefix");
    check(nova_kvpool_refcnt(pool, tab_a[tail]) == 2, "shared tail page refcount 2");
    nova_paged_session_cow(pg, b, n_tok - 1, 1, st);
    launch_kv_store_paged(pk, pv, nova_paged_table_dev(pg, b), layer, nb, 1, n_tok - 1, dkb, dvb, st);
    dev_stream_sync(st);
    nova_kvpool_table(pool, b, tab_b.data(), (int)tab_b.size());
    check(nova_kvpool_cow_count(pool) == 1, "one COW");
    check(tab_b[tail] != tab_a[tail], "B's tail page is its own after the COW");
    check(nova_kvpool_refcnt(pool, tab_a[tail]) == 1 && nova_kvpool_refcnt(pool, tab_b[tail]) == 1,
          "donor and copy refcount 1");
    check(tab_b[0] == tab_a[0] && nova_kvpool_refcnt(pool, tab_a[0]) == 2, "head pages still shared");

    // read back the layer's pages: A's rows bit-exact, B's rows = A's 0..98 + its own 99
    const size_t page = (size_t)16 * KVW;
    std::vector<uint16_t> hk((size_t)nb * page), hv((size_t)nb * page);
    dev_download(hk.data(), pk + (size_t)layer * nb * page, hk.size() * 2);
    dev_download(hv.data(), pv + (size_t)layer * nb * page, hv.size() * 2);
    auto at = [&](const std::vector<uint16_t>& pool_h, const std::vector<int32_t>& tab, int t) {
        return &pool_h[(size_t)tab[t / 16] * page + (size_t)(t % 16) * KVW];
    };
    bool rows_ok = true;
    for (int t = 0; t < n_tok; ++t) {
        rows_ok &= !std::memcmp(at(hk, tab_a, t), &ka[(size_t)t * KVW], KVW * 2);
        rows_ok &= !std::memcmp(at(hv, tab_a, t), &va[(size_t)t * KVW], KVW * 2);
        const uint16_t* kb_src = t < n_tok - 1 ? &ka[(size_t)t * KVW] : kb1.data();
        const uint16_t* vb_src = t < n_tok - 1 ? &va[(size_t)t * KVW] : vb1.data();
        rows_ok &= !std::memcmp(at(hk, tab_b, t), kb_src, KVW * 2);
        rows_ok &= !std::memcmp(at(hv, tab_b, t), vb_src, KVW * 2);
    }
    check(rows_ok, "appended rows bit-exact, donor page untouched");

    // decode both sessions (reference signature, scratch of NH*32*(HD+2) floats)
    std::vector<float> q((size_t)g.nh * g.hd);
    std::normal_distribution<float> nd(0.f, 1.f);
    for (auto& x : q) x = nd(rng);
    float* dq = static_cast<float*>(dev_alloc(q.size() * 4));
    float* dout = static_cast<float*>(dev_alloc(q.size() * 4));
    float* scratch = static_cast<float*>(dev_alloc((size_t)g.nh * 32 * (g.hd + 2) * 4));
    dev_upload(dq, q.data(), q.size() * 4);
    const double scale = 1.0 / std::sqrt((double)g.hd);
    for (int s : {a, b}) {
        const auto& tab = s == a ? tab_a : tab_b;
        launch_attn_decode_paged(dq, pk, pv, nova_paged_table_dev(pg, s), layer, nb, n_tok, dout, scratch, st);
        dev_stream_sync(st);
        std::vector<float> o(q.size());
        dev_download(o.data(), dout, o.size() * 4);
        double worst = 0.0;
        bool ok = true;
        for (int h = 0; h < g.nh; ++h) {
            const int kvh = h / G;
            std::vector<double> sc(n_tok);
            double mx = -1e300;
            for (int t = 0; t < n_tok; ++t) {
                const uint16_t* kr = at(hk, tab, t) + (size_t)kvh * g.hd;
                double acc = 0.0;
                for (int e = 0; e < g.hd; ++e) acc += (double)q[(size_t)h * g.hd + e] * half_value(kr[e]);
                sc[t] = acc * scale;
                mx = std::fmax(mx, sc[t]);
            }
            double den = 0.0;
            for (auto& x : sc) den += (x = std::exp(x - mx));
            for (int e = 0; e < g.hd; ++e) {
                double num = 0.0;
                for (int t = 0; t < n_tok; ++t) num += sc[t] * half_value(at(hv, tab, t)[(size_t)kvh * g.hd + e]);
                const double ref = num / den, got = o[(size_t)h * g.hd + e];
                const double err = std::fabs(got - ref);
                worst = std::fmax(worst, err);
                ok &= std::isfinite(got) && err <= 2e-3 + 1e-2 * std::fabs(ref);
            }
        }
        std::printf("session %d: decode max |gpu - f64| = %.3e\n", s, worst);
        check(ok, s == a ? "decode of the donor session" : "decode of the forked session");
    }

    // chunked prefill through the reference signature: A's last 20 positions
    // as queries over its own keys, causal (query i sees keys 0..80+i)
    {
        const int n_q = 20, n_past = n_tok - n_q;
        std::vector<float> qs((size_t)n_q * g.nh * g.hd);
        for (auto& x : qs) x = nd(rng);
        float* dqs = static_cast<float*>(dev_alloc(qs.size() * 4));
        float* dos = static_cast<float*>(dev_alloc(qs.size() * 4));
        dev_upload(dqs, qs.data(), qs.size() * 4);
        launch_attn_prefill_paged(dqs, pk, pv, nova_paged_table_dev(pg, a), layer, nb, n_q, n_past, dos, st);
        dev_stream_sync(st);
        std::vector<float> os(qs.size());
        dev_download(os.data(), dos, os.size() * 4);
        double worst = 0.0;
        bool ok = true;
        for (int i = 0; i < n_q; ++i)
            for (int h = 0; h < g.nh; ++h) {
                const int kvh = h / G, n_keys = n_past + i + 1;
                const float* qr = &qs[((size_t)i * g.nh + h) * g.hd];
                std::vector<double> sc(n_keys);
                double mx = -1e300, den = 0.0;
                for (int t = 0; t < n_keys; ++t) {
                    const uint16_t* kr = at(hk, tab_a, t) + (size_t)kvh * g.hd;
                    double acc = 0.0;
                    for (int e = 0; e < g.hd; ++e) acc += (double)qr[e] * half_value(kr[e]);
                    sc[t] = acc * scale;
                    mx = std::fmax(mx, sc[t]);
                }
                for (auto& x : sc) den += (x = std::exp(x - mx));
                for (int e = 0; e < g.hd; ++e) {
                    double num = 0.0;
                    for (int t = 0; t < n_keys; ++t) num += sc[t] * half_value(at(hv, tab_a, t)[(size_t)kvh * g.hd + e]);
                    const double ref = num / den, got = os[((size_t)i * g.nh + h) * g.hd + e];
                    worst = std::fmax(worst, std::fabs(got - ref));
                    ok &= std::isfinite(got) && std::fabs(got - ref) <= 2e-3 + 1e-2 * std::fabs(ref);
                }
            }
        std::printf("prefill of %d queries: max |gpu - f64| = %.3e\n", n_q, worst);
        check(ok, "chunked prefill of the donor session");
        dev_free(dqs);
        dev_free(dos);
    }

    for (void* p : {(void*)dka, (void*)dva, (void*)dkb, (void*)dvb, (void*)dq, (void*)dout, (void*)scratch}) dev_free(p);
    nova_paged_destroy_session(pg, b);
    nova_paged_destroy_session(pg, a);
    nova_paged_delete(pg);
    std::printf(fails ? "abi_consumer: %d check(s) failed\n" : "abi_consumer: PASS\n", fails);
    return fails ? 1 : 0;
}
