// kvszp_bits.h -- register-level bit-plane transforms of the fixed-mode
// stream, shared by the encoder and decoder kernels.  Pure functions on
// uint32_t arrays so the host test suite can check them with g++.
//
// Stream word layout (reference: cuszp_batched_fixed.cu:320-351): a block
// with rate r > 0 is stored as words w_0 .. w_r, where w_0 is the sign word
// and w_{1+p} is bit plane p of |q|.  In every word, element v of the block
// sits in byte v>>3 at bit 7-(v&7), i.e. at bit (v ^ 7) of the
// little-endian u32.
//
// Register layout.  Each element is turned into a 16-bit FIELD and two
// fields share a dword: row k holds element k^7 in the low half and element
// 16+(k^7) in the high half.  A 16x16 bit-matrix transpose of each half
// (transpose16x2) turns "row k = field of one element" into "row b = bit b
// of every field, one bit per element at position v^7" -- i.e. row b IS a
// stream word.  With the field
//     f_lo = ((|q| << 1) | sign) & 0xFFFF
// row 0 is the sign word and row 1+p is plane p, so rows 0..15 are stream
// words w_0..w_15: a block with rate <= 15 is finished in one transpose.  For
// rates 16..31 a second pass with
//     f_hi = (|q| >> 15) & 0xFFFF
// yields planes 15..30 = words w_16..w_31.  The transpose is its own
// inverse, which is how the decoder gets the fields back.
#ifndef KVSZP_BITS_H
#define KVSZP_BITS_H

#include <stdint.h>

#if defined(__HIPCC__)
#define KVSZP_HD __host__ __device__ __forceinline__
#else
#define KVSZP_HD static inline
#endif

namespace kvszp {

// Exchange the columns {c : c & J} of x with the columns {c : !(c & J)} of y
// (the block-swap step of a recursive bit-matrix transpose).  `mask` selects
// the columns with (c & J) == 0.  Written as two bit-selects,
//     x' = (x & mask) | ((y << J) & ~mask),  y' = ((x >> J) & mask) | (y & ~mask),
// two instructions each (shift + one 3-input bit op); for J = 8 each half is
// one byte permute.
template <int J>
KVSZP_HD void delta_swap(uint32_t& x, uint32_t& y, uint32_t mask) {
#if defined(__HIP_DEVICE_COMPILE__)
    if (J == 8) {
        // bytes of (x, y) = (x0 x1 x2 x3, y0 y1 y2 y3), byte 0 lowest:
        // x' = (x0 y0 x2 y2), y' = (x1 y1 x3 y3)
        const uint32_t nx = __builtin_amdgcn_perm(y, x, 0x06020400u);
        const uint32_t ny = __builtin_amdgcn_perm(y, x, 0x07030501u);
        x = nx;
        y = ny;
        return;
    }
    // Each output is one shift and one 3-input bit select (v_bitop3_b32,
    // truth table 0xE4 = S2 ? S0 : S1), written out so the compiler keeps
    // it at two instructions instead of splitting the masks into ANDs.
    {
        const uint32_t nx = __builtin_amdgcn_bitop3_b32(x, y << J, mask, 0xE4);
        const uint32_t ny = __builtin_amdgcn_bitop3_b32(x >> J, y, mask, 0xE4);
        x = nx;
        y = ny;
        return;
    }
#endif
    const uint32_t nx = (x & mask) | ((y << J) & ~mask);
    const uint32_t ny = ((x >> J) & mask) | (y & ~mask);
    x = nx;
    y = ny;
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

// Element held in the low / high half of row k.
KVSZP_HD int row_lo_elem(int k) { return k ^ 7; }
KVSZP_HD int row_hi_elem(int k) { return 16 + (k ^ 7); }

// 16-bit fields of a magnitude m = |q| (< 2^31) and sign s (0/1).
KVSZP_HD uint32_t field_lo(uint32_t m, uint32_t s) { return ((m << 1) | s) & 0xFFFFu; }
KVSZP_HD uint32_t field_hi(uint32_t m) { return (m >> 15) & 0xFFFFu; }

// The whole field 2|q| + sign of the reference quantizer's q
// (cuszp_batched_fixed.cu:10-25: v = fl(x*r), s = !(v >= -0.5),
// t = fl(v + 0.5) or fl(x*r + 0.5), q = cvt.rzi(t) - s) from t alone, for
// |t| < 2^31 (the conversion does not saturate):
//   * the sign test on v equals a test on t.  Two roundings: v >= -0.5 iff
//     t >= 0 (for v in [-1, -0.5) the sum v + 0.5 is exact by Sterbenz, below
//     that t <= -0.5).  Fused: v >= -0.5 iff the exact product p is at least
//     -0.5 - 2^-25 (the rounding midpoint below -0.5, ties to -0.5), iff
//     t >= -2^-25: near -0.5, p (an 8-bit by 24-bit significand product) is
//     a multiple of 2^-33, so no p + 0.5 lies in the half-ulp interval
//     [-2^-25 - 2^-49, -2^-25) where the two tests could disagree.  NaN
//     fails both tests (s = 1).
//   * with c = trunc(|t|) (NaN -> 0): s = 0 gives q = c; s = 1 means t < 0
//     or NaN, q = -c - 1.  So |q| = c + s and the field is 2(c + s) + s.
constexpr float kFusedSignThreshold = 0x1p-25f;
KVSZP_HD bool field_sign(float t, int fused) {
    return fused ? !(t >= -kFusedSignThreshold) : !(t >= 0.0f);
}
KVSZP_HD uint32_t field_from_trunc(uint32_t c, bool s) {
    return (c << 1) + (s ? 3u : 0u);  // = 2(c + s) + s
}

// Reference-free host helpers (used by the host test): a[v] = |q_v| with the
// sign in bit 31, element order.  words[0..31] receive w_0..w_31.
KVSZP_HD void pack_block_words(const uint32_t* a, uint32_t* words) {
    uint32_t m[16];
    for (int k = 0; k < 16; ++k) {
        const uint32_t lo = a[row_lo_elem(k)], hi = a[row_hi_elem(k)];
        m[k] = field_lo(lo & 0x7FFFFFFFu, lo >> 31) |
               (field_lo(hi & 0x7FFFFFFFu, hi >> 31) << 16);
    }
    transpose16x2(m);
    for (int b = 0; b < 16; ++b) words[b] = m[b];
    for (int k = 0; k < 16; ++k) {
        const uint32_t lo = a[row_lo_elem(k)], hi = a[row_hi_elem(k)];
        m[k] = field_hi(lo & 0x7FFFFFFFu) | (field_hi(hi & 0x7FFFFFFFu) << 16);
    }
    transpose16x2(m);
    for (int b = 0; b < 16; ++b) words[16 + b] = m[b];
}

KVSZP_HD void unpack_block_words(const uint32_t* words, uint32_t* a) {
    uint32_t lo[16], hi[16];
    for (int b = 0; b < 16; ++b) {
        lo[b] = words[b];
        hi[b] = words[16 + b];
    }
    transpose16x2(lo);
    transpose16x2(hi);
    for (int k = 0; k < 16; ++k) {
        const uint32_t fl0 = lo[k] & 0xFFFFu, fl1 = lo[k] >> 16;
        const uint32_t fh0 = hi[k] & 0xFFFFu, fh1 = hi[k] >> 16;
        a[row_lo_elem(k)] = ((fl0 >> 1) | (fh0 << 15)) | ((fl0 & 1u) << 31);
        a[row_hi_elem(k)] = ((fl1 >> 1) | (fh1 << 15)) | ((fl1 & 1u) << 31);
    }
}

}  // namespace kvszp

#endif  // KVSZP_BITS_H
