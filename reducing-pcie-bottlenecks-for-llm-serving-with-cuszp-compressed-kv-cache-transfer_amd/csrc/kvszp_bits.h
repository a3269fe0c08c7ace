// kvszp_bits.h -- register-level bit-plane transforms of the fixed-mode
// stream, shared by the encoder and decoder kernels.  Pure functions on
// uint32_t arrays so the host test suite can check them with g++.
//
// Stream word layout (reference: cuszp_batched_fixed.cu:320-351): in the
// sign word and in plane word p of a 32-element block, element v sits in
// byte v>>3 at bit 7-(v&7), i.e. at bit (v ^ 7) of the little-endian u32.
//
// Both directions are the same bit-matrix transpose, because a transpose is
// its own inverse:
//   rows-by-element  A[k] = a[k^7]      (a = |q| with the sign in the top bit)
//   rows-by-plane    A[b] = word b      (plane words, sign word last)
// Two widths are provided:
//   * 16-bit fields (rates <= 15): two independent 16x16 matrices share the
//     dword halves.  A[k] = f[k^7] | f[16+(k^7)] << 16 with
//     f = |q| | sign << 15; after the transpose A[b] is plane word b for
//     b < 15 and A[15] is the sign word.  4 stages on 16 dwords.
//   * 32-bit fields (any rate): A[k] = a[k^7] with a = |q| | sign << 31;
//     after the transpose A[b] is plane b (b <= 30) and A[31] the sign word.
#ifndef KVSZP_BITS_H
#define KVSZP_BITS_H

#include <stdint.h>

#if defined(__HIPCC__)
#define KVSZP_HD __host__ __device__ __forceinline__
#else
#define KVSZP_HD static inline
#endif

namespace kvszp {

// Exchange the columns {c : c & j} of x with the columns {c : !(c & j)} of y
// (the block-swap step of a recursive bit-matrix transpose).  `mask` selects
// the columns with (c & j) == 0.
template <int J>
KVSZP_HD void delta_swap(uint32_t& x, uint32_t& y, uint32_t mask) {
    const uint32_t t = ((x >> J) ^ y) & mask;
    y ^= t;
    x ^= t << J;
}

// Transposes rows [0,16) as two independent 16x16 bit matrices (low and high
// dword halves).  Row k, column c  <->  row c, column k within each half.
KVSZP_HD void transpose16x2(uint32_t* a) {
#pragma unroll
    for (int k = 0; k < 8; ++k) delta_swap<8>(a[k], a[k + 8], 0x00FF00FFu);
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if ((k & 4) == 0) delta_swap<4>(a[k], a[k + 4], 0x0F0F0F0Fu);
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if ((k & 2) == 0) delta_swap<2>(a[k], a[k + 2], 0x33333333u);
#pragma unroll
    for (int k = 0; k < 16; ++k)
        if ((k & 1) == 0) delta_swap<1>(a[k], a[k + 1], 0x55555555u);
}

// Transposes a 32x32 bit matrix held in rows [0,32).
KVSZP_HD void transpose32(uint32_t* a) {
#pragma unroll
    for (int k = 0; k < 16; ++k) delta_swap<16>(a[k], a[k + 16], 0x0000FFFFu);
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if ((k & 8) == 0) delta_swap<8>(a[k], a[k + 8], 0x00FF00FFu);
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if ((k & 4) == 0) delta_swap<4>(a[k], a[k + 4], 0x0F0F0F0Fu);
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if ((k & 2) == 0) delta_swap<2>(a[k], a[k + 2], 0x33333333u);
#pragma unroll
    for (int k = 0; k < 32; ++k)
        if ((k & 1) == 0) delta_swap<1>(a[k], a[k + 1], 0x55555555u);
}

// Magnitude-with-sign a = |q| | sign<<31 -> 16-bit field |q| | sign<<15.
// Valid when |q| < 2^15.
KVSZP_HD uint32_t field16(uint32_t a) {
    return (a & 0x7FFFu) | ((a >> 16) & 0x8000u);
}

// Encoder: a[32] (|q| | sign<<31, element order) -> words[0] = sign word,
// words[1 + p] = plane p.
// Narrow form: every |q| < 2^15, 16 words out (planes 0..14).
KVSZP_HD void pack_block_words_narrow(const uint32_t* a, uint32_t* words) {
    uint32_t m[16];
#pragma unroll
    for (int k = 0; k < 16; ++k)
        m[k] = field16(a[k ^ 7]) | (field16(a[16 + (k ^ 7)]) << 16);
    transpose16x2(m);
    words[0] = m[15];
#pragma unroll
    for (int p = 0; p < 15; ++p) words[1 + p] = m[p];
}

// Wide form: any |q| < 2^31, 32 words out (planes 0..30).
KVSZP_HD void pack_block_words_wide(const uint32_t* a, uint32_t* words) {
    uint32_t m[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) m[k] = a[k ^ 7];
    transpose32(m);
    words[0] = m[31];
#pragma unroll
    for (int p = 0; p < 31; ++p) words[1 + p] = m[p];
}

}  // namespace kvszp

#endif  // KVSZP_BITS_H
