// kv_registry.h -- registry of kv_blocks: (prefix, suffix) -> KV range.
// Same behaviour as the reference's nova::BlockRegistry
// (code/graph/kv_registry.h:16-70): put() retires a live entry with the same
// (prefix, suffix) and appends; capacity (default 64) retires the oldest live
// entries first; find() returns the first live match.
#pragma once
#include <cstdint>
#include <cstdio>
#include <vector>

#include "graph/kv_block.h"

namespace nova {

struct KvBlock {
    uint64_t prefix = 0;
    uint64_t suffix = 0;
    int session = -1;
    int turn = 0;
    int64_t pos0 = 0;
    int64_t pos1 = 0;
    bool alive = true;
};

class BlockRegistry {
public:
    void set_capacity(size_t n) { cap_ = n ? n : 1; evict(); }
    size_t capacity() const { return cap_; }

    void put(const KvBlock& b) {
        for (auto& x : v_)
            if (x.alive && x.prefix == b.prefix && x.suffix == b.suffix) { x.alive = false; --live_; }
        v_.push_back(b);
        v_.back().alive = true;
        ++live_;
        evict();
    }

    const KvBlock* find(uint64_t prefix, uint64_t suffix) const {
        for (const auto& x : v_)
            if (x.alive && x.prefix == prefix && x.suffix == suffix) return &x;
        return nullptr;
    }

    int live() const { return (int)live_; }
    int total() const { return (int)v_.size(); }

    void dump() const {
        std::printf("[KV] registry: live=%d total=%d cap=%zu\n", live(), total(), cap_);
        for (const auto& x : v_)
            if (x.alive)
                std::printf("[KV]   %s  session=%d turn=%d kv=[%lld,%lld)\n", kv_block_id(x.prefix, x.suffix).c_str(),
                            x.session, x.turn, (long long)x.pos0, (long long)x.pos1);
    }

private:
    void evict() {
        size_t k = oldest_;
        while (live_ > cap_) {
            while (!v_[k].alive) ++k;
            v_[k].alive = false;
            --live_;
        }
        oldest_ = k;   // entries before k are all retired
    }

    std::vector<KvBlock> v_;
    size_t cap_ = 64;
    size_t live_ = 0;
    size_t oldest_ = 0;
};

inline BlockRegistry& blocks() {
    static BlockRegistry r;
    return r;
}

}  // namespace nova
