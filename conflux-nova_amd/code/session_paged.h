// session_paged.h -- the device-backed paging layer: pool memory, per-session
// block tables on the device, session create/destroy, prefix attach and
// copy-on-write.
//
// Covers the paging parts of the reference's engine and session layer:
//   * pool allocation and geometry views: Engine::load (src/model.cpp:93-96),
//     kv_width/kv_nblocks/kv_nb/kv_span (include/nova/model.h:140-145)
//   * SessionManager::create / destroy paging steps (code/session.h:84-142):
//     acquire a slice, push its table, clear its pages, release on destroy
//   * session_attach / session_attach_prefix / session_cow (code/session.h:156-180)
//   * Engine::cow_guard (src/model.cpp:171-191)
// Differences, all MI355X-motivated:
//   * pools are fp16 and sized by (n_slices, ctx) at run time, from one
//     dev_alloc per pool; at 288 GB per GPU the pool is the dominant tenant
//   * page clears and COW copies are single launches (launch_kv_zero_pages,
//     launch_kv_cow_apply) instead of 2*L memset/memcpy calls per page; the
//     table patch rides in the same launch
//   * cow_batch() applies the COW decisions of many sessions in one launch (the
//     reference decides per session per block and copies each immediately)
//   * create_sessions() / push_tables() serve many sessions at once: one table
//     upload per run of consecutive slice ids (tables are rows of one device
//     array) and one page-clear launch, where the reference uploads and clears
//     per session
// Errors abort, as in the reference: pool exhaustion during COW prints
// "[FATAL] KV pool full during COW" (model.cpp:173), no free slice exits with 3
// (session.h:88,99).
#pragma once
#include <cstdint>
#include <cstdio>
#include <algorithm>
#include <cstdlib>
#include <vector>

#include "graph/kv_pool.h"
#include "hal.h"
#include "nova_kernel.h"

namespace nova {

class PagedKv {
public:
    // n_slices sessions of up to ctx tokens share NB = n_slices * ceil(ctx/16) pages
    void init(int n_slices, int64_t ctx) {
        geo_ = nova_model_geometry();
        pool_.init(n_slices, ctx);
        nb_ = pool_.nb_total();
        const uint64_t per_pool = (uint64_t)geo_.n_layers * (uint64_t)nb_ * (uint64_t)geo_.kv_block *
                                  (uint64_t)geo_.nkv * (uint64_t)geo_.hd * 2ull;
        k_ = static_cast<uint16_t*>(dev_alloc(per_pool));
        v_ = static_cast<uint16_t*>(dev_alloc(per_pool));
        pool_bytes_ = per_pool;
        tables_ = static_cast<int32_t*>(dev_alloc((uint64_t)(nb_ > 0 ? nb_ : 1) * 4ull));
        pool_.set_dev(tables_);
        stream_ = dev_stream_create();
    }

    void destroy() {
        if (stream_) dev_stream_sync(stream_);
        dev_free(k_);
        dev_free(v_);
        dev_free(tables_);
        if (stream_) dev_stream_destroy(stream_);
        k_ = v_ = nullptr;
        tables_ = nullptr;
        stream_ = nullptr;
    }

    // SessionManager::create paging steps: acquire, push table, clear own pages
    KvSlice* create_session(bool clear_pages = true) {
        KvSlice* s = pool_.acquire();
        if (!s) {
            std::fprintf(stderr, "[ERROR] KV page pool has no free slice\n");
            std::exit(3);
        }
        s->k = k_;
        s->v = v_;
        push_table(*s);
        if (clear_pages) {
            std::vector<int32_t> pages(s->table.begin(), s->table.end());
            int32_t* d = static_cast<int32_t*>(dev_alloc(pages.size() * 4));
            dev_upload_async(d, pages.data(), pages.size() * 4, stream_);
            launch_kv_zero_pages(k_, v_, nb_, d, (int)pages.size(), stream_);
            dev_stream_sync(stream_);
            dev_free(d);
        }
        dev_stream_sync(stream_);
        return s;
    }

    void destroy_session(KvSlice* s) { pool_.release(s); }

    // count sessions at once: acquire in order (the ids a serial caller would
    // get), one upload per run of consecutive ids, one clear of all their
    // pages.  Returns the number created; stops early (after the creations so
    // far) with -1 in the remaining ids when the pool runs out of slices.
    int create_sessions(int count, bool clear_pages, int* ids) {
        std::vector<int> got;
        got.reserve((size_t)count);
        for (int j = 0; j < count; ++j) {
            KvSlice* sl = pool_.acquire();
            if (!sl) break;
            sl->k = k_;
            sl->v = v_;
            got.push_back(sl->id);
        }
        for (int j = 0; j < count; ++j) ids[j] = j < (int)got.size() ? got[(size_t)j] : -1;
        push_tables(got.data(), (int)got.size());
        if (clear_pages && !got.empty()) {
            std::vector<int32_t> pages;
            for (int id : got) {
                const KvSlice& sl = *pool_.slice(id);
                pages.insert(pages.end(), sl.table.begin(), sl.table.end());
            }
            int32_t* d = static_cast<int32_t*>(dev_alloc(pages.size() * 4));
            dev_upload_async(d, pages.data(), pages.size() * 4, stream_);
            launch_kv_zero_pages(k_, v_, nb_, d, (int)pages.size(), stream_);
            dev_stream_sync(stream_);
            dev_free(d);
        }
        dev_stream_sync(stream_);
        return (int)got.size();
    }

    // Upload the host tables of several sessions: ids are sorted and each run
    // of consecutive ids goes up as one copy of adjacent device rows.
    void push_tables(const int* ids, int count) {
        if (count <= 0) return;
        std::vector<int> v(ids, ids + count);
        std::sort(v.begin(), v.end());
        v.erase(std::unique(v.begin(), v.end()), v.end());
        const size_t nbk = (size_t)pool_.nblocks();
        size_t j = 0;
        while (j < v.size()) {
            size_t e = j + 1;
            while (e < v.size() && v[e] == v[e - 1] + 1) ++e;
            staging_.resize((e - j) * nbk);
            for (size_t t = j; t < e; ++t) {
                const KvSlice& sl = *pool_.slice(v[t]);
                std::copy(sl.table.begin(), sl.table.end(), staging_.begin() + (t - j) * nbk);
            }
            dev_upload_async(pool_.slice(v[j])->table_dev, staging_.data(), staging_.size() * sizeof(int32_t),
                             stream_);
            dev_stream_sync(stream_);    // staging_ is reused by the next run
            j = e;
        }
    }

    // session_attach (session.h:156-163)
    void attach(KvSlice& dst, const KvSlice& src, int k) {
        pool_.attach(dst, src, k);
        push_table(dst);
        dev_stream_sync(stream_);
    }

    // session_attach_prefix (session.h:173-180)
    void attach_prefix(KvSlice& dst, const KvSlice& src, int64_t n_tokens) {
        pool_.attach_prefix(dst, src, n_tokens);
        push_table(dst);
        dev_stream_sync(stream_);
    }

    // Engine::cow_guard: decide for the page holding pos; copy on the device if needed.
    // Returns the new physical page or -1.
    int cow_guard(KvSlice& s, int64_t pos, nova_stream_t st) {
        nova_cow_op op;
        const int nb = decide(s, pos, &op);
        if (nb >= 0) launch_kv_cow_apply(k_, v_, nb_, tables_, &op, 1, st);
        return nb;
    }

    // session_cow (session.h:166-171): every logical page touched by [pos0, pos0+n)
    void session_cow(KvSlice& s, int64_t pos0, int n, nova_stream_t st) {
        std::vector<nova_cow_op> ops;
        const int b0 = kv_block_index(pos0), b1 = kv_block_index(pos0 + n - 1);
        for (int b = b0; b <= b1; ++b) {
            nova_cow_op op;
            if (decide(s, (int64_t)b * kKvBlockCfg, &op) >= 0) ops.push_back(op);
        }
        if (!ops.empty()) launch_kv_cow_apply(k_, v_, nb_, tables_, ops.data(), (int)ops.size(), st);
    }

    // Many sessions' next writes at once: session i writes [pos0[i], pos0[i]+n[i]).
    // Decisions run in session order (the order a serial caller would use);
    // all copies and table patches then go out as one launch.  Returns the
    // number of pages copied.
    int cow_batch(KvSlice* const* ss, const int64_t* pos0, const int* n, int count, nova_stream_t st) {
        std::vector<nova_cow_op> ops;
        for (int i = 0; i < count; ++i) {
            if (n[i] <= 0) continue;
            const int b0 = kv_block_index(pos0[i]), b1 = kv_block_index(pos0[i] + n[i] - 1);
            for (int b = b0; b <= b1; ++b) {
                nova_cow_op op;
                if (decide(*ss[i], (int64_t)b * kKvBlockCfg, &op) >= 0) ops.push_back(op);
            }
        }
        if (!ops.empty()) launch_kv_cow_apply(k_, v_, nb_, tables_, ops.data(), (int)ops.size(), st);
        return (int)ops.size();
    }

    void push_table(const KvSlice& s) {
        dev_upload_async(s.table_dev, s.table.data(), s.table.size() * sizeof(int32_t), stream_);
    }

    KvPool& pool() { return pool_; }
    uint16_t* k_base() const { return k_; }
    uint16_t* v_base() const { return v_; }
    int32_t* tables() const { return tables_; }
    int nb() const { return nb_; }
    uint64_t pool_bytes() const { return pool_bytes_; }
    nova_stream_t stream() const { return stream_; }

private:
    int decide(KvSlice& s, int64_t pos, nova_cow_op* op) {
        const int nb = pool_.cow_slice(s, pos);
        if (nb == -2) {
            std::fprintf(stderr, "[FATAL] KV pool full during COW\n");
            std::fflush(stderr);
            std::abort();
        }
        if (nb < 0) return -1;
        op->src = s.need_copy_from;
        op->dst = nb;
        op->table_index = (int64_t)s.id * pool_.nblocks() + kv_block_index(pos);
        s.need_copy_from = -1;   // consumed (cow_guard clears it, model.cpp:175-176)
        return nb;
    }

    nova_geometry geo_{};
    KvPool pool_;
    int nb_ = 0;
    uint16_t* k_ = nullptr;
    uint16_t* v_ = nullptr;
    int32_t* tables_ = nullptr;
    uint64_t pool_bytes_ = 0;
    nova_stream_t stream_ = nullptr;
    std::vector<int32_t> staging_;
};

}  // namespace nova
