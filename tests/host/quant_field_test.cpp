// Host check of the encoder's whole-field quantizer identity
// (csrc/kvszp_bits.h: field_sign, field_from_trunc) against the CPU
// oracle's restatement of the reference quantizer
// (cuszp_batched_fixed.cu:10-25).  Every BF16 bit pattern x (NaNs and
// infinities included) meets reciprocals spread over 2^-40 .. 2^40 and, per
// negative x, the reciprocals that put x*r next to the sign test's boundary
// -0.5 (two roundings) and -0.5 - 2^-25 (fused), for both quantizer
// variants, wherever the identity's precondition holds: f32 |x|*r < 2^30,
// which the kernel checks for the largest |x| of the job.
#include "kvszp_bits.h"
#include "kvszp_oracle.h"

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>

using namespace kvszp;

static float bits_f32(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

static uint32_t trunc_abs(float t) {  // v_cvt_u32_f32 of |t| below 2^31
    return t != t ? 0u : (uint32_t)std::fabs(t);
}

static uint32_t fast_field(float x, float r, int fused) {
    volatile float v = x * r;  // rounded product (two-roundings variant)
    const float t = fused ? std::fmaf(x, r, 0.5f) : (float)(v + 0.5f);
    return field_from_trunc(trunc_abs(t), field_sign(t, fused));
}

static uint32_t oracle_field(float x, float r, int fused) {
    const int32_t q = kvo_quantize(x, r, fused);
    const uint32_t m = q < 0 ? 0u - (uint32_t)q : (uint32_t)q;
    return 2u * m + (q < 0 ? 1u : 0u);
}

static long cases = 0, bad = 0;

static void check(float x, float r) {
    if (!(r > 0.0f) || std::isinf(r)) return;
    volatile float ax = std::fabs(x) * r;
    if (!(x != x) && !(ax < 0x1p30f)) return;
    for (int fused = 0; fused < 2; ++fused) {
        ++cases;
        const uint32_t a = fast_field(x, r, fused), b = oracle_field(x, r, fused);
        if (a != b && bad++ < 10)
            std::printf("x=%a r=%a fused=%d fast=%u oracle=%u\n", x, r, fused, a, b);
    }
}

int main() {
    std::mt19937 rng(2024);
    std::uniform_real_distribution<float> e(-40.0f, 40.0f);
    float recips[400];
    for (float& r : recips) r = std::ldexp(1.0f + (rng() & 0x7FFFFF) * 0x1p-23f, (int)e(rng));
    for (uint32_t h = 0; h < 65536; ++h) {
        const float x = bits_f32(h << 16);
        for (float r : recips) check(x, r);
        if (!(x < 0.0f) || std::isinf(x)) continue;
        for (const float target : {0.5f, 0.5f + 0x1p-25f}) {
            float r0 = target / -x;
            float lo = r0, hi = r0;
            check(x, r0);
            for (int k = 0; k < 6; ++k) {
                lo = std::nextafter(lo, 0.0f);
                hi = std::nextafter(hi, INFINITY);
                check(x, lo);
                check(x, hi);
            }
        }
    }
    std::printf("cases=%ld mismatches=%ld\n", cases, bad);
    return bad != 0;
}
