// Host check of the kernels' bit-plane transforms (csrc/kvszp_bits.h)
// against the stream word layout of the reference encoder
// (cuszp_batched_fixed.cu:320-351): word 0 holds the signs, word 1+p bit
// plane p of |q|, element v at bit (v ^ 7) of the little-endian word.
#include "kvszp_bits.h"

#include <cstdio>
#include <random>

using namespace kvszp;

static uint32_t naive_word(const uint32_t* a, int w) {
    uint32_t out = 0;
    for (int v = 0; v < 32; ++v) {
        const uint32_t bit = (w == 0) ? (a[v] >> 31) : ((a[v] >> (w - 1)) & 1u);
        out |= bit << (v ^ 7);
    }
    return out;
}

int main() {
    std::mt19937 rng(12345);
    long bad = 0, cases = 0;
    for (int it = 0; it < 50000; ++it) {
        const int bits = it % 32;  // magnitudes below 2^bits (bits <= 31)
        uint32_t a[32];
        for (int v = 0; v < 32; ++v) {
            const uint32_t m = bits ? (rng() & ((1u << bits) - 1u)) : 0u;
            const uint32_t s = (rng() & 1u) && m ? 1u : 0u;
            a[v] = m | (s << 31);
        }
        uint32_t words[32];
        pack_block_words(a, words);
        for (int w = 0; w < 32; ++w) bad += words[w] != naive_word(a, w);
        uint32_t back[32];
        unpack_block_words(words, back);
        for (int v = 0; v < 32; ++v) bad += back[v] != a[v];
        ++cases;
    }
    std::printf("cases=%ld mismatches=%ld\n", cases, bad);
    return bad != 0;
}
