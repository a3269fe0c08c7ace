/*
 * kvszp_oracle.c -- TEST INFRASTRUCTURE ONLY (see kvszp_oracle.h).
 *
 * A scalar, one-element-at-a-time restatement of the reference's batched
 * fixed-mode BF16 codec, written from reading
 *   integration/cuszp_wrapper/cuszp_batched_fixed.cu   (kernels, :10-627)
 *   integration/cuszp_wrapper/cuszp_wrapper.cpp         (size/eps rules)
 * It deliberately follows the reference's *semantics*, not its schedule:
 * blocks are visited in natural order and the payload offset is a running
 * sum, which is what the reference's per-warp scan plus decoupled look-back
 * computes (cu:233-299).
 *
 * Build: gcc -O2 -fPIC -shared -ffp-contract=off -fopenmp (no fast-math):
 * every float operation below must round exactly once, in fp32.
 */
#include "kvszp_oracle.h"

#include <float.h>
#include <math.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define KVO_BLOCK 32u
#define KVO_REF_TILE 32768u /* tblock_size(32) * thread_chunk(1024) */

/* cvt.rzi.s32.f32 (cu:21): truncate toward zero, saturate, NaN -> 0. */
static int32_t cvt_rzi_s32_sat(float t) {
    if (t != t) return 0;
    if (t >= 2147483648.0f) return INT32_MAX;
    if (t <= -2147483648.0f) return INT32_MIN;
    return (int32_t)t;
}

/* batch_quantization, cuszp_batched_fixed.cu:10-25.
 *   v = fl(x*recip)               mul.f32           (:17)
 *   s = (v >= -0.5) ? 0 : 1       setp.ge + selp    (:18-19)  NaN -> s = 1
 *   t = fl(v + 0.5)  [or fma]     add.f32           (:20)
 *   c = cvt.rzi.s32.f32(t)                          (:21)
 *   q = c - s  (32-bit wrap)      sub.s32           (:22) */
int32_t kvo_quantize(float x, float recip, int variant) {
    volatile float v = x * recip; /* volatile: keep the product rounded */
    const int32_t s = (v >= -0.5f) ? 0 : 1;
    const float t = (variant == KVO_QUANT_FUSED) ? fmaf(x, recip, 0.5f)
                                                 : v + 0.5f;
    const int32_t c = cvt_rzi_s32_sat(t);
    return (int32_t)((uint32_t)c - (uint32_t)s);
}

void kvo_quantize_array(const float* x, uint64_t n, float recip, int variant,
                        int32_t* q) {
    for (uint64_t i = 0; i < n; ++i) q[i] = kvo_quantize(x[i], recip, variant);
}

/* batch_bit_count, cu:27-31: 32 - clz(v). */
int kvo_bit_count(uint32_t v) {
    int bits = 0;
    while (v) {
        ++bits;
        v >>= 1;
    }
    return bits;
}

/* __bfloat162float: exact widening. */
float kvo_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof(f));
    return f;
}

/* __float2bfloat16_rn: round to nearest, ties to even.  NaN inputs keep
 * their sign and upper payload and are quieted (the decoder only produces a
 * NaN when eb is Inf or NaN; the reference's NaN bit pattern is unpinned). */
uint16_t kvo_f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof(u));
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* selected_bf16_source_index, cu:33-50. */
uint64_t kvo_source_index(uint64_t logical, const int64_t* layer_indices,
                          uint64_t selected_layers, uint64_t source_layers,
                          uint64_t elements_per_layer) {
    if (layer_indices == NULL) return logical;
    const uint64_t per_prefix = selected_layers * elements_per_layer;
    const uint64_t prefix = logical / per_prefix;
    const uint64_t within = logical % per_prefix;
    const uint64_t layer = within / elements_per_layer;
    const uint64_t inner = within % elements_per_layer;
    return (prefix * source_layers + (uint64_t)layer_indices[layer]) *
               elements_per_layer + inner;
}

/* rate_offset, cu:165 and cuszp_wrapper.cpp:534-535. */
uint64_t kvo_header_bytes(uint64_t n) {
    return (n + KVO_REF_TILE - 1) / KVO_REF_TILE * (KVO_REF_TILE / KVO_BLOCK);
}

/* compute_relative_bounds_bf16_kernel, cu:55-133: fminf/fmaxf over the n
 * logical values (NaN never wins), then eb *= fmaxf(max - min, 1e-6f). */
float kvo_relative_bound(const uint16_t* page, uint64_t n,
                         const int64_t* layer_indices, uint64_t selected_layers,
                         uint64_t source_layers, uint64_t elements_per_layer,
                         float eps) {
    float lo = FLT_MAX;
    float hi = -FLT_MAX;
    for (uint64_t i = 0; i < n; ++i) {
        const float x = kvo_bf16_to_f32(page[kvo_source_index(
            i, layer_indices, selected_layers, source_layers,
            elements_per_layer)]);
        lo = fminf(lo, x);
        hi = fmaxf(hi, x);
    }
    const float range = fmaxf(hi - lo, 1e-6f);
    return eps * range;
}

static void put_word(uint8_t* out, uint64_t pos, uint32_t word) {
    /* uchar4 {x,y,z,w} = {w>>24, w>>16, w>>8, w} (cu:321-327). */
    out[pos + 0] = (uint8_t)(word >> 24);
    out[pos + 1] = (uint8_t)(word >> 16);
    out[pos + 2] = (uint8_t)(word >> 8);
    out[pos + 3] = (uint8_t)(word);
}

/* Where the encoder reads logical element i: a BF16 page (through the
 * layer map) or a contiguous fp32 array. */
typedef struct {
    const uint16_t* page;
    const float* f32;
    const int64_t* layer_indices;
    uint64_t sel, src, epl;
} source_t;

static float source_get(const source_t* s, uint64_t i) {
    if (s->f32 != NULL) return s->f32[i];
    return kvo_bf16_to_f32(
        s->page[kvo_source_index(i, s->layer_indices, s->sel, s->src, s->epl)]);
}

/* compress_batch_fixed_bf16_kernel, cu:135-359, one page. */
static uint64_t encode_page(const source_t* in, uint64_t n, float eb,
                            int variant, uint8_t* out) {
    const float recip = 0.5f / eb; /* cu:166 */
    const uint64_t nb = (n + KVO_BLOCK - 1) / KVO_BLOCK;
    const uint64_t header = kvo_header_bytes(n);
    memset(out, 0, header); /* padding [nb, R): never written by the ref */
    uint64_t pos = header;
    for (uint64_t b = 0; b < nb; ++b) {
        uint32_t mag[KVO_BLOCK];
        uint32_t sign = 0;
        uint32_t largest = 0;
        for (uint32_t v = 0; v < KVO_BLOCK; ++v) {
            const uint64_t i = b * KVO_BLOCK + v;
            int32_t q = 0;
            if (i < n) /* cu:200-211: tail elements quantize to 0 */
                q = kvo_quantize(source_get(in, i), recip, variant);
            uint32_t a = (uint32_t)q;
            if (q < 0) { /* cu:212-215 */
                sign |= 1u << (31 - v);
                a = 0u - (uint32_t)q;
            }
            mag[v] = a;
            if (a > largest) largest = a;
        }
        const int rate = kvo_bit_count(largest); /* cu:221-222 */
        out[b] = (uint8_t)rate;                  /* cu:226-229 */
        if (rate == 0) continue;
        put_word(out, pos, sign); /* cu:320-328 */
        pos += 4;
        for (int bit = 0; bit < rate; ++bit) { /* cu:330-354 */
            uint32_t plane = 0;
            for (uint32_t v = 0; v < KVO_BLOCK; ++v)
                plane |= ((mag[v] >> bit) & 1u) << (31 - v);
            put_word(out, pos, plane);
            pos += 4;
        }
    }
    return pos; /* = R + payload, cuszp_wrapper.cpp:534-541 */
}

uint64_t kvo_compress_page(const uint16_t* page, uint64_t n,
                           const int64_t* layer_indices,
                           uint64_t selected_layers, uint64_t source_layers,
                           uint64_t elements_per_layer, float eb, int variant,
                           uint8_t* out) {
    const source_t s = {page, NULL, layer_indices, selected_layers,
                        source_layers, elements_per_layer};
    return encode_page(&s, n, eb, variant, out);
}

/* The fp32 single-page path (CuSZpWrapper::compress / compress_batch_fixed,
 * cuszp_wrapper.cpp:216-429): the same stream over fp32 values.  The
 * reference runs upstream cuSZp's fp32 fixed-mode kernel there, which is not
 * vendored; cuszp_batched_fixed.cu:52-54 states that the batched BF16 layout
 * is that kernel's.  Parity with upstream itself is unpinned. */
uint64_t kvo_compress_page_f32(const float* x, uint64_t n, float eb,
                               int variant, uint8_t* out) {
    const source_t s = {NULL, x, NULL, 0, 0, 0};
    return encode_page(&s, n, eb, variant, out);
}

/* at::aminmax over the whole input (NaN anywhere -> NaN extrema), range =
 * max - min raised to 1e-6f when below it, eb = eps * range
 * (cuszp_wrapper.cpp:249-257 and the std::max form at :371-377). */
float kvo_relative_bound_f32(const float* x, uint64_t n, float eps) {
    float lo = x[0], hi = x[0];
    for (uint64_t i = 0; i < n; ++i) {
        if (x[i] != x[i]) return eps * NAN;
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
    }
    float range = hi - lo;
    if (range < 1e-6f) range = 1e-6f;
    return eps * range;
}

/* Where the decoder puts logical element i. */
typedef struct {
    int kind; /* 0 contiguous, 1 scatter, 2 indexed, 3 contiguous fp32 */
    uint16_t* out;
    uint16_t* const* destinations;
    uint64_t dpp, epd;
    const int64_t* layer_indices;
    uint64_t sel, src, epl;
} sink_t;

static void sink_put(const sink_t* s, uint64_t i, float decoded) {
    if (s->kind == 3) {
        ((float*)(void*)s->out)[i] = decoded;
        return;
    }
    const uint16_t value = kvo_f32_to_bf16_rne(decoded);
    switch (s->kind) {
    case 0: /* decoded + output_index (cu:569-576, 608-620) */
        s->out[i] = value;
        break;
    case 1: /* destination_pages[page*dpp + i/epd][i%epd] (cu:577-606) */
        s->destinations[i / s->epd][i % s->epd] = value;
        break;
    default: /* selected_bf16_source_index into the full page (cu:539-565) */
        s->out[kvo_source_index(i, s->layer_indices, s->sel, s->src,
                                s->epl)] = value;
        break;
    }
}

/* decompress_batch_fixed_bf16_kernel, cu:361-627, one page. */
static int decode_page(const uint8_t* in, uint64_t stream_size, uint64_t n,
                       float eb, int rate0_policy, const sink_t* sink) {
    const uint64_t nb = (n + KVO_BLOCK - 1) / KVO_BLOCK;
    const uint64_t header = kvo_header_bytes(n);
    if (stream_size < header) return -1;
    uint64_t pos = header;
    for (uint64_t b = 0; b < nb; ++b) {
        const int rate = in[b];
        if (rate > 31) return -1;
        if (rate == 0) {
            if (rate0_policy == KVO_RATE0_ZERO)
                for (uint32_t v = 0; v < KVO_BLOCK && b * KVO_BLOCK + v < n; ++v)
                    sink_put(sink, b * KVO_BLOCK + v, 0.0f);
            continue; /* cu:496: nothing written */
        }
        if (pos + 4u + 4u * (uint64_t)rate > stream_size) return -1;
        const uint32_t sign = ((uint32_t)in[pos] << 24) |
                              ((uint32_t)in[pos + 1] << 16) |
                              ((uint32_t)in[pos + 2] << 8) | in[pos + 3];
        pos += 4;
        uint32_t mag[KVO_BLOCK];
        memset(mag, 0, sizeof(mag));
        for (int bit = 0; bit < rate; ++bit) { /* cu:511-522 */
            for (uint32_t v = 0; v < KVO_BLOCK; ++v)
                mag[v] |= (uint32_t)((in[pos + (v >> 3)] >> (7 - (v & 7))) & 1u)
                          << bit;
            pos += 4;
        }
        for (uint32_t v = 0; v < KVO_BLOCK; ++v) {
            const uint64_t i = b * KVO_BLOCK + v;
            if (i >= n) break;
            int32_t q = (int32_t)mag[v];
            if (sign & (1u << (31 - v))) q = (int32_t)(0u - mag[v]); /* :528 */
            const float scaled = (float)q * eb;                       /* :535 */
            const float value = scaled * 2.0f;
            sink_put(sink, i, value); /* BF16 sinks round here (cu:538) */
        }
    }
    return 0;
}

int kvo_decompress_contiguous(const uint8_t* stream, uint64_t stream_size,
                              uint64_t n, float eb, int rate0_policy,
                              uint16_t* out) {
    sink_t s = {0, out, NULL, 0, 0, NULL, 0, 0, 0};
    return decode_page(stream, stream_size, n, eb, rate0_policy, &s);
}

int kvo_decompress_scatter(const uint8_t* stream, uint64_t stream_size,
                           uint64_t n, float eb, int rate0_policy,
                           uint16_t* const* destinations,
                           uint64_t destinations_per_page,
                           uint64_t elements_per_destination) {
    sink_t s = {1, NULL, destinations, destinations_per_page,
                elements_per_destination, NULL, 0, 0, 0};
    return decode_page(stream, stream_size, n, eb, rate0_policy, &s);
}

int kvo_decompress_indexed(const uint8_t* stream, uint64_t stream_size,
                           uint64_t n, float eb, int rate0_policy,
                           uint16_t* destination, const int64_t* layer_indices,
                           uint64_t selected_layers, uint64_t source_layers,
                           uint64_t elements_per_layer) {
    sink_t s = {2, destination, NULL, 0, 0, layer_indices, selected_layers,
                source_layers, elements_per_layer};
    return decode_page(stream, stream_size, n, eb, rate0_policy, &s);
}

/* The fp32 single-page decode (CuSZpWrapper::decompress, fixed mode,
 * cuszp_wrapper.cpp:870-943): y = fl(fl(q * eb) * 2) without the BF16
 * rounding.  Upstream's fp32 decoder is not vendored (parity unpinned);
 * kvo_f32_to_bf16_rne of this output is the BF16 decoders' value. */
int kvo_decompress_f32(const uint8_t* stream, uint64_t stream_size, uint64_t n,
                       float eb, int rate0_policy, float* out) {
    sink_t s = {3, (uint16_t*)(void*)out, NULL, 0, 0, NULL, 0, 0, 0};
    return decode_page(stream, stream_size, n, eb, rate0_policy, &s);
}

/* ---- Lorenzo modes (plain, outlier) of the fp32 single-page API ---------
 *
 * CuSZpWrapper::compress/decompress hand the plain and outlier modes to
 * upstream cuSZp (cuszp_wrapper.cpp:302-313, 922-933; the fp32 decoders at
 * cuszp_fastpath.cu:37-59), whose sources are not vendored
 * (reproducibility/install_cuszp.sh clones them).  What follows is this
 * build's own specification of those modes, after the published cuSZp
 * design (1D Lorenzo prediction inside each 32-value block, then the
 * fixed-length block code); byte parity with upstream is unpinned.
 *
 * Per block: q_v = the fixed-mode quantizer's value (q_v = q_{v-1} past the
 * end of the data), residuals d_0 = q_0, d_v = q_v - q_{v-1} (32-bit wrap).
 * Plain codes c_v = d_v; outlier keeps o = d_0 aside and codes c_0 = 0,
 * c_v = d_v.  With m_v = |c_v| as a 32-bit magnitude (|INT_MIN| = 2^31) the
 * rate r is the bit length of max m_v (0..32).  Header byte: r, with bit 7
 * set in outlier mode when o != 0.  Payload, blocks in order: o as 4 bytes
 * (least significant first) when present, then for r > 0 the sign word and
 * r plane words laid out exactly as in fixed mode.  Decoding: q_{-1} = o
 * (outlier) or 0 (plain), q_v = q_{v-1} + c_v, y_v = fl(fl(q_v * eb) * 2),
 * so both modes decode to the fixed mode's values of the same page. */
static uint64_t encode_page_lorenzo(const float* x, uint64_t n, float eb,
                                    int variant, int mode, uint8_t* out) {
    const float recip = 0.5f / eb;
    const uint64_t nb = (n + KVO_BLOCK - 1) / KVO_BLOCK;
    const uint64_t header = kvo_header_bytes(n);
    memset(out, 0, header);
    uint64_t pos = header;
    for (uint64_t b = 0; b < nb; ++b) {
        uint32_t mag[KVO_BLOCK];
        uint32_t sign = 0, largest = 0, outlier = 0;
        int32_t prev = 0;
        for (uint32_t v = 0; v < KVO_BLOCK; ++v) {
            const uint64_t i = b * KVO_BLOCK + v;
            const int32_t q = i < n ? kvo_quantize(x[i], recip, variant) : prev;
            uint32_t d = (uint32_t)q - (uint32_t)prev;
            prev = q;
            if (mode == KVO_MODE_OUTLIER && v == 0) {
                outlier = d;
                d = 0;
            }
            uint32_t a = d;
            if ((int32_t)d < 0) {
                sign |= 1u << (31 - v);
                a = 0u - d;
            }
            mag[v] = a;
            if (a > largest) largest = a;
        }
        const int rate = kvo_bit_count(largest);
        out[b] = (uint8_t)(rate | (outlier != 0 ? 0x80 : 0));
        if (outlier != 0) {
            for (int k = 0; k < 4; ++k) out[pos + k] = (uint8_t)(outlier >> (8 * k));
            pos += 4;
        }
        if (rate == 0) continue;
        put_word(out, pos, sign);
        pos += 4;
        for (int bit = 0; bit < rate; ++bit) {
            uint32_t plane = 0;
            for (uint32_t v = 0; v < KVO_BLOCK; ++v)
                plane |= ((mag[v] >> bit) & 1u) << (31 - v);
            put_word(out, pos, plane);
            pos += 4;
        }
    }
    return pos;
}

static int decode_page_lorenzo(const uint8_t* in, uint64_t stream_size, uint64_t n,
                               float eb, int mode, int rate0_policy, float* out) {
    const uint64_t nb = (n + KVO_BLOCK - 1) / KVO_BLOCK;
    const uint64_t header = kvo_header_bytes(n);
    if (stream_size < header) return -1;
    uint64_t pos = header;
    for (uint64_t b = 0; b < nb; ++b) {
        const int h = in[b];
        const int has_outlier = mode == KVO_MODE_OUTLIER && (h & 0x80);
        const int rate = mode == KVO_MODE_OUTLIER ? (h & 0x7F) : h;
        if (rate > 32) return -1;
        if (h == 0) {
            if (rate0_policy == KVO_RATE0_ZERO)
                for (uint32_t v = 0; v < KVO_BLOCK && b * KVO_BLOCK + v < n; ++v)
                    out[b * KVO_BLOCK + v] = 0.0f;
            continue;
        }
        const uint64_t bytes =
            (has_outlier ? 4u : 0u) + (rate ? 4u + 4u * (uint64_t)rate : 0u);
        if (pos + bytes > stream_size) return -1;
        uint32_t q = 0;
        if (has_outlier) {
            q = (uint32_t)in[pos] | ((uint32_t)in[pos + 1] << 8) |
                ((uint32_t)in[pos + 2] << 16) | ((uint32_t)in[pos + 3] << 24);
            pos += 4;
        }
        uint32_t sign = 0, mag[KVO_BLOCK];
        memset(mag, 0, sizeof(mag));
        if (rate) {
            sign = ((uint32_t)in[pos] << 24) | ((uint32_t)in[pos + 1] << 16) |
                   ((uint32_t)in[pos + 2] << 8) | in[pos + 3];
            pos += 4;
            for (int bit = 0; bit < rate; ++bit) {
                for (uint32_t v = 0; v < KVO_BLOCK; ++v)
                    mag[v] |= (uint32_t)((in[pos + (v >> 3)] >> (7 - (v & 7))) & 1u)
                              << bit;
                pos += 4;
            }
        }
        for (uint32_t v = 0; v < KVO_BLOCK; ++v) {
            const uint64_t i = b * KVO_BLOCK + v;
            if (i >= n) break;
            const uint32_t c = (sign & (1u << (31 - v))) ? 0u - mag[v] : mag[v];
            q += c;
            const float scaled = (float)(int32_t)q * eb;
            out[i] = scaled * 2.0f;
        }
    }
    return 0;
}

uint64_t kvo_compress_page_f32_mode(const float* x, uint64_t n, float eb,
                                    int variant, int mode, uint8_t* out) {
    if (mode == KVO_MODE_FIXED) return kvo_compress_page_f32(x, n, eb, variant, out);
    return encode_page_lorenzo(x, n, eb, variant, mode, out);
}

int kvo_decompress_f32_mode(const uint8_t* stream, uint64_t stream_size, uint64_t n,
                            float eb, int mode, int rate0_policy, float* out) {
    if (mode == KVO_MODE_FIXED)
        return kvo_decompress_f32(stream, stream_size, n, eb, rate0_policy, out);
    return decode_page_lorenzo(stream, stream_size, n, eb, mode, rate0_policy, out);
}

/* CuSZpWrapper::compress_batch_fixed_bf16[_indexed] (cuszp_wrapper.cpp:
 * 431-681): eps_i = eps[i] > 0 ? eps[i] : default; optional relative bound;
 * size = R + payload. */
int kvo_compress_batch(const uint16_t* const* pages, uint8_t* const* outs,
                       uint64_t batch, uint64_t n,
                       const int64_t* layer_indices, uint64_t selected_layers,
                       uint64_t source_layers, uint64_t elements_per_layer,
                       const float* eps, float default_eps, int relative,
                       int variant, int threads, uint64_t* sizes,
                       float* bounds) {
    int64_t p;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1)
#endif
    for (p = 0; p < (int64_t)batch; ++p) {
        const float e = (eps != NULL && eps[p] > 0.0f) ? eps[p] : default_eps;
        const float eb = relative
            ? kvo_relative_bound(pages[p], n, layer_indices, selected_layers,
                                 source_layers, elements_per_layer, e)
            : e;
        bounds[p] = eb;
        sizes[p] = kvo_compress_page(pages[p], n, layer_indices,
                                     selected_layers, source_layers,
                                     elements_per_layer, eb, variant, outs[p]);
    }
    (void)threads;
    return 0;
}

int kvo_decompress_batch_contiguous(const uint8_t* const* streams,
                                    const uint64_t* sizes, uint64_t batch,
                                    uint64_t n, const float* bounds,
                                    int rate0_policy, int threads,
                                    uint16_t* out) {
    int status = 0;
    int64_t p;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) reduction(|: status)
#endif
    for (p = 0; p < (int64_t)batch; ++p)
        status |= kvo_decompress_contiguous(streams[p], sizes[p], n, bounds[p],
                                            rate0_policy, out + (uint64_t)p * n)
                  ? 1 : 0;
    (void)threads;
    return status ? -1 : 0;
}

/* Indexed restore of a batch (the reference's indexed scatter decode,
 * cu:539-565): page p's segment to destinations[p], pages split across
 * `threads` OpenMP threads (for the CPU baseline). */
int kvo_decompress_batch_indexed(const uint8_t* const* streams,
                                 const uint64_t* sizes, uint64_t batch,
                                 uint64_t n, const float* bounds,
                                 int rate0_policy, int threads,
                                 uint16_t* const* destinations,
                                 const int64_t* layer_indices,
                                 uint64_t selected_layers, uint64_t source_layers,
                                 uint64_t elements_per_layer) {
    int status = 0;
    int64_t p;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) reduction(|: status)
#endif
    for (p = 0; p < (int64_t)batch; ++p)
        status |= kvo_decompress_indexed(streams[p], sizes[p], n, bounds[p],
                                          rate0_policy, destinations[p],
                                          layer_indices, selected_layers,
                                          source_layers, elements_per_layer)
                  ? 1 : 0;
    (void)threads;
    return status ? -1 : 0;
}

/* ---- INT8 host codec --------------------------------------------------
 * vllm_v1_compressed_offload.py:711-724 runs on BF16 tensors, so every torch
 * op result is rounded to BF16:
 *   scale = bf16(bf16(max|x|) / 127), 1 if 0
 *   q = clamp(round_half_even(bf16(x / scale)), -127, 127)
 * and :2090-2123 decodes bf16(float(q) * scale). */
static float bf16_round(float f) { return kvo_bf16_to_f32(kvo_f32_to_bf16_rne(f)); }

float kvo_int8_encode(const uint16_t* page, uint64_t n, int8_t* q) {
    float largest = 0.0f;
    for (uint64_t i = 0; i < n; ++i) {
        const float a = fabsf(kvo_bf16_to_f32(page[i]));
        if (a > largest) largest = a;
    }
    float scale = bf16_round(largest / 127.0f);
    if (scale == 0.0f) scale = 1.0f;
    for (uint64_t i = 0; i < n; ++i) {
        float r = nearbyintf(bf16_round(kvo_bf16_to_f32(page[i]) / scale));
        if (r > 127.0f) r = 127.0f;
        if (r < -127.0f) r = -127.0f;
        q[i] = (int8_t)r;
    }
    return scale;
}

void kvo_int8_decode(const int8_t* q, uint64_t n, float scale, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i)
        out[i] = kvo_f32_to_bf16_rne((float)q[i] * scale);
}
