// rope_math.h -- the rotation step shared by every kernel that applies RoPE,
// so that all of them produce the same bits.
//
// NeoX pairs (i, i + HD/2) of the Qwen2 family (reference
// include/nova/arch/traits.h:15-17, src/kernel/rope.cu:21-58):
//   y0 = x0*c - x1*s,  y1 = x0*s + x1*c
// with every product rounded on its own: the products pass through an empty
// asm so that they cannot be contracted into an fma (the library is built
// with -ffp-contract=fast, under which clang ignores the fp-contract pragma).
#pragma once

namespace nova {

__device__ __forceinline__ void rope_rotate(float x0, float x1, float c, float s, float& y0, float& y1) {
    float a0 = x0 * c, a1 = x1 * s, b0 = x0 * s, b1 = x1 * c;
    asm("" : "+v"(a0), "+v"(a1), "+v"(b0), "+v"(b1));
    y0 = a0 - a1;
    y1 = b0 + b1;
}

}  // namespace nova
