// kv_pool_cfg.h -- compile-time page size and position -> (page, slot) split.
// Same constants and helpers as the reference's code/graph/kv_pool_cfg.h:12-33
// (kKvBlock in {8,16,32,64}, default 16; shift/mask addressing).
#pragma once
#include <cstdint>

#ifndef NOVA_KV_BLOCK
#define NOVA_KV_BLOCK 16
#endif

namespace nova {

constexpr int kKvBlockCfg = NOVA_KV_BLOCK;
static_assert(kKvBlockCfg == 8 || kKvBlockCfg == 16 || kKvBlockCfg == 32 || kKvBlockCfg == 64,
              "NOVA_KV_BLOCK must be one of 8 / 16 / 32 / 64");
constexpr int kKvBlockShiftCfg = kKvBlockCfg == 8 ? 3 : kKvBlockCfg == 16 ? 4 : kKvBlockCfg == 32 ? 5 : 6;
constexpr int kKvBlockMaskCfg = kKvBlockCfg - 1;

inline int kv_block_index(int64_t pos) { return (int)(pos >> kKvBlockShiftCfg); }
inline int kv_slot_index(int64_t pos) { return (int)(pos & kKvBlockMaskCfg); }

}  // namespace nova
