// kv_block.h -- 64-bit kv_block IDs.
//
// Same ID layout as the reference's code/graph/kv_block.h:21-83: every token id
// is written in decimal, the decimal text's bytes become uppercase hex, the hex
// string is cut into 16-digit (64-bit) words with the last word padded with '0'
// on the right, and the words are folded end-to-end (w[i] + w[n-1-i], middle
// word carried when n is odd, wrapping uint64) until one word is left.  The
// empty sequence hashes to 0.  A kv_block is "{ PPPPPPPPPPPPPPPP . SSSSSSSSSSSSSSSS }".
// This implementation folds the digits straight into words without building
// the intermediate hex string.
#pragma once
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

namespace nova {

inline uint64_t kv_hash_ids(const int* ids, size_t n) {
    if (n == 0) return 0;
    std::vector<uint64_t> words;
    words.reserve(n / 2 + 1);
    uint64_t cur = 0;
    int nib = 0;   // hex digits in cur
    auto push_byte = [&](unsigned char ch) {
        for (int half = 0; half < 2; ++half) {
            cur = (cur << 4) | (uint64_t)(half ? (ch & 15) : (ch >> 4));
            if (++nib == 16) { words.push_back(cur); cur = 0; nib = 0; }
        }
    };
    char dec[16];
    for (size_t i = 0; i < n; ++i) {
        const int len = std::snprintf(dec, sizeof dec, "%d", ids[i]);
        for (int j = 0; j < len; ++j) push_byte((unsigned char)dec[j]);
    }
    if (nib) words.push_back(cur << (4 * (16 - nib)));   // right-pad with '0' digits
    size_t m = words.size();
    while (m > 1) {
        const size_t half = m / 2;
        const uint64_t mid = words[half];
        for (size_t i = 0; i < half; ++i) words[i] += words[m - 1 - i];
        if (m & 1) words[half] = mid;
        m = half + (m & 1);
    }
    return words[0];
}

inline uint64_t kv_hash_ids(const std::vector<int>& ids) { return kv_hash_ids(ids.data(), ids.size()); }

inline uint64_t kv_hash_text(const std::string& text) {
    std::vector<int> b(text.begin(), text.end());
    for (auto& x : b) x &= 0xFF;
    return kv_hash_ids(b);
}

inline std::string kv_hash_hex(uint64_t v) {
    char s[17];
    std::snprintf(s, sizeof s, "%016llX", (unsigned long long)v);
    return std::string(s, 16);
}

inline std::string kv_block_id(uint64_t prefix, uint64_t suffix) {
    return "{ " + kv_hash_hex(prefix) + " . " + kv_hash_hex(suffix) + " }";
}

}  // namespace nova
