// model.h -- compile-time geometry of one library build (gfx950).
//
// The reference welds the model into the binary (include/nova/model/select.h:6-32,
// matrix.h:46-53) and the page size into kv_pool_cfg.h:12-33; this build does the
// same with -DNOVA_MODEL_* and -DNOVA_KV_BLOCK.  Qwen2.5-14B (40/8/128, 48 layers)
// has no ModelSpec in the reference and is added here.
#pragma once
#include <cstdint>

#ifndef NOVA_KV_BLOCK
#define NOVA_KV_BLOCK 16
#endif

namespace nova {

template <int NH_, int NKV_, int HD_, int L_, int THETA_>
struct Geometry {
    static constexpr int NH = NH_, NKV = NKV_, HD = HD_, L = L_;
    static constexpr int kTheta = THETA_;       // RoPE base (matrix.h:46-50: 1e6 for Qwen2.5)
    static constexpr int G = NH / NKV;          // GQA group
    static constexpr int KVW = NKV * HD;        // halves per token per pool
    static_assert(NH % NKV == 0, "GQA heads must divide");
};

#if defined(NOVA_MODEL_QWEN25_7B)
using Model = Geometry<28, 4, 128, 28, 1000000>;
inline constexpr const char* kModelName = "Qwen2.5-7B";
#elif defined(NOVA_MODEL_QWEN25_1P5B)
using Model = Geometry<12, 2, 128, 28, 1000000>;
inline constexpr const char* kModelName = "Qwen2.5-1.5B";
#elif defined(NOVA_MODEL_QWEN25_14B)
using Model = Geometry<40, 8, 128, 48, 1000000>;
inline constexpr const char* kModelName = "Qwen2.5-14B";
#else
#error "no model selected: pass -DNOVA_MODEL_QWEN25_7B, _1P5B or _14B"
#endif

constexpr int kKvBlock = NOVA_KV_BLOCK;
static_assert(kKvBlock == 16, "the gfx950 kernels are tiled for 16-token pages");
constexpr int kKvBlockShift = 4;
constexpr int kKvBlockMask = kKvBlock - 1;
static_assert(Model::HD == 128, "the gfx950 kernels are tiled for head_dim 128");
static_assert(Model::G <= 16, "a GQA group must fit one 16-column MFMA tile");

// reference split bound for the single-session entry point (attn.cu:19; scratch
// NH*32*(HD+2), model.cpp:114)
constexpr int kMaxSplit = 32;
// softmax scale 1/sqrt(128) (attn.cu:21)
constexpr float kScale = 0.08838834764831845f;

}  // namespace nova
