// ref_q4k_harness.cpp -- C-ABI harness over the reference's own Q4_K host code
// (include/nova/quant/q4_k.h, compiled unchanged) -- TEST INFRASTRUCTURE.
//
// Exposes dequant_block / half_to_float, and reproduces the known-answer block
// of tests/selftest_q4k.cpp:31-38 (d = 0x2C00, dmin = 0x1A00, scale and nibble
// bytes from std::mt19937(12345)) so the oracle can be checked against it.
#include <cstdint>
#include <cstring>
#include <random>
#include "nova/quant/q4_k.h"

extern "C" {
float ref_q4k_half(uint16_t h) { return nova::half_to_float(h); }
void ref_q4k_dequant_block(const uint8_t* block, float* y) {
    nova::block_q4_K b;
    std::memcpy(&b, block, sizeof b);
    nova::dequant_block(&b, y);
}
void ref_q4k_selftest_block(uint8_t* block) {
    std::mt19937 rng(12345);
    nova::block_q4_K b{};
    b.d = 0x2C00;
    b.dmin = 0x1A00;
    for (int i = 0; i < 12; ++i) b.scales[i] = (uint8_t)(rng() & 0xFF);
    for (int i = 0; i < 128; ++i) b.qs[i] = (uint8_t)(rng() & 0xFF);
    std::memcpy(block, &b, sizeof b);
}
}
