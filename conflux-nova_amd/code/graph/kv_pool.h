// kv_pool.h -- shared page-pool bookkeeping (host side).
//
// Same API and observable behaviour as the reference's nova::KvPool / KvSlice
// (code/graph/kv_pool.h:56-199): slice stack handing out slice 0 first, an
// identity table per acquired slice, a LIFO free-page stack that starts
// descending (lowest id on top), refcounts clamped at zero, attach /
// attach_prefix sharing, and cow_slice's copy decision.  The observable quirks
// are kept on purpose so block tables, refcounts and the free list stay
// bit-identical to the reference's:
//   * attach/attach_prefix overwrite the destination's own identity pages
//     without freeing them (they keep refcount 1 for good);
//   * attach sets n_past only inside its loop (k == 0 leaves it alone);
//   * need_copy_from/need_copy_blk are one-shot signals the caller clears.
// Differences (not observable through block tables / refcounts / free list):
//   * acquire removes the slice's pages from the free list in one pass instead
//     of one std::find per page (O(free) instead of O(free * pages): at 288 GB
//     of HBM3E a pool holds hundreds of thousands of pages);
//   * slices live in fixed per-id storage, so release() does not move other
//     live KvSlice objects (the reference's vector erase shifts them,
//     kv_pool.h:171-173), and held KvSlice* stay valid;
//   * pool pointers are fp16 (uint16_t bit patterns).
#pragma once
#include <algorithm>
#include <cstdint>
#include <vector>

#include "graph/kv_pool_cfg.h"

namespace nova {

struct KvSlice {
    int need_copy_from = -1;   // one-shot COW source page
    int need_copy_blk = -1;    // one-shot COW destination page
    int id = -1;
    uint16_t* k = nullptr;
    uint16_t* v = nullptr;
    int64_t n_past = 0;
    int nblocks = 0;
    std::vector<int32_t> table;     // logical page -> physical page
    int32_t* table_dev = nullptr;   // device copy of the same table
    bool live = false;
};

class KvPool {
public:
    void init(int n_slices, int64_t ctx) {
        ctx_ = ctx;
        nblocks_ = (int)((ctx + kKvBlockCfg - 1) / kKvBlockCfg);
        slots_.assign((size_t)(n_slices > 0 ? n_slices : 0), KvSlice{});
        order_.clear();
        free_.clear();
        for (int i = n_slices - 1; i >= 0; --i) free_.push_back(i);
        nb_total_ = n_slices * nblocks_;
        refcnt_.assign((size_t)nb_total_, 0);
        free_blocks_.clear();
        free_blocks_.reserve((size_t)nb_total_);
        for (int b = nb_total_ - 1; b >= 0; --b) free_blocks_.push_back(b);
        cow_count_ = 0;
    }

    void set_dev(int32_t* base) { dev_ = base; }
    int32_t* dev() const { return dev_; }

    KvSlice* acquire() {
        if (free_.empty()) return nullptr;
        const int id = free_.back();
        free_.pop_back();
        KvSlice& s = slots_[(size_t)id];
        s = KvSlice{};
        s.id = id;
        s.live = true;
        s.nblocks = nblocks_;
        s.table.resize((size_t)nblocks_);
        for (int b = 0; b < nblocks_; ++b) s.table[(size_t)b] = (int32_t)(id * nblocks_ + b);
        s.table_dev = dev_ ? dev_ + (size_t)id * (size_t)nblocks_ : nullptr;
        order_.push_back(id);
        // claim the identity range: refcount 1 and off the free stack.  One
        // stable pass drops the first occurrence of each claimed page, which is
        // what a std::find + erase per page leaves behind.
        const int lo = id * nblocks_;
        const int hi = std::min(lo + nblocks_, nb_total_);
        if (hi > lo) {
            for (int p = lo; p < hi; ++p) refcnt_[(size_t)p] = 1;
            std::vector<uint8_t> taken((size_t)(hi - lo), 0);
            size_t outp = 0;
            for (size_t k = 0; k < free_blocks_.size(); ++k) {
                const int b = free_blocks_[k];
                if (b >= lo && b < hi && !taken[(size_t)(b - lo)]) {
                    taken[(size_t)(b - lo)] = 1;
                    continue;
                }
                free_blocks_[outp++] = b;
            }
            free_blocks_.resize(outp);
        }
        return &s;
    }

    int alloc_block() {
        if (free_blocks_.empty()) return -1;
        const int b = free_blocks_.back();
        free_blocks_.pop_back();
        refcnt_[(size_t)b] = 1;
        return b;
    }
    void free_block(int b) {
        if (b < 0 || b >= nb_total_) return;
        if (--refcnt_[(size_t)b] <= 0) {
            refcnt_[(size_t)b] = 0;
            free_blocks_.push_back(b);
        }
    }
    void ref_block(int b) {
        if (b >= 0 && b < nb_total_) ++refcnt_[(size_t)b];
    }
    int refcnt(int b) const { return (b >= 0 && b < nb_total_) ? refcnt_[(size_t)b] : 0; }
    int nb_total() const { return nb_total_; }

    void attach(KvSlice& dst, const KvSlice& src, int k) {
        for (int i = 0; i < k; ++i) {
            dst.table[(size_t)i] = src.table[(size_t)i];
            ref_block(src.table[(size_t)i]);
            dst.n_past = (int64_t)k * kKvBlockCfg;
        }
    }

    void attach_prefix(KvSlice& dst, const KvSlice& src, int64_t n_tokens) {
        const int nb = (int)((n_tokens + kKvBlockCfg - 1) / kKvBlockCfg);
        for (int i = 0; i < nb && i < (int)src.table.size(); ++i) {
            dst.table[(size_t)i] = src.table[(size_t)i];
            ref_block(src.table[(size_t)i]);
        }
        dst.n_past = n_tokens;
    }

    int cow_count() const { return cow_count_; }
    int free_blocks() const { return (int)free_blocks_.size(); }
    const std::vector<int>& free_list() const { return free_blocks_; }
    const std::vector<int>& refcnts() const { return refcnt_; }

    // -1: no copy needed; -2: pool exhausted; otherwise the new physical page
    int cow_slice(KvSlice& s, int64_t pos) {
        const int lb = kv_block_index(pos);
        if (lb < 0 || lb >= (int)s.table.size()) return -1;
        const int phys = s.table[(size_t)lb];
        if (refcnt(phys) <= 1) return -1;
        const int nb = alloc_block();
        if (nb < 0) return -2;
        ++cow_count_;
        s.need_copy_from = phys;
        s.need_copy_blk = nb;
        s.table[(size_t)lb] = nb;
        free_block(phys);
        return nb;
    }

    void release(KvSlice* s) {
        if (!s || !s->live) return;
        for (int32_t b : s->table) free_block(b);
        free_.push_back(s->id);
        order_.erase(std::find(order_.begin(), order_.end(), s->id));
        s->live = false;
    }

    int32_t phys_block(const KvSlice& s, int64_t pos) const { return s.table[(size_t)kv_block_index(pos)]; }
    int slot(int64_t pos) const { return kv_slot_index(pos); }

    KvSlice* slice(int id) {
        return (id >= 0 && id < (int)slots_.size() && slots_[(size_t)id].live) ? &slots_[(size_t)id] : nullptr;
    }
    int nblocks() const { return nblocks_; }
    int64_t ctx() const { return ctx_; }
    int used() const { return (int)order_.size(); }
    int free_slices() const { return (int)free_.size(); }

private:
    int64_t ctx_ = 0;
    int nblocks_ = 0;
    int32_t* dev_ = nullptr;
    std::vector<KvSlice> slots_;   // indexed by slice id
    std::vector<int> order_;       // live ids in acquisition order
    std::vector<int> free_;
    std::vector<int> free_blocks_;
    std::vector<int> refcnt_;
    int nb_total_ = 0;
    int cow_count_ = 0;
};

inline KvPool& kv_pool() {
    static KvPool p;
    return p;
}

}  // namespace nova
