/*
 * kvszp_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * Scalar CPU restatement of the reference's batched cuSZp fixed-mode BF16
 * KV-page codec (integration/cuszp_wrapper/cuszp_batched_fixed.cu).  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or the timed CPU baseline).  The
 * product path never calls it.
 *
 * BF16 values travel as raw uint16_t bit patterns; the fp32 single-page path
 * takes and returns float arrays.
 */
#ifndef KVSZP_ORACLE_H
#define KVSZP_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Quantizer reading: the reference's inline PTX (cuszp_batched_fixed.cu:17-20)
 * has an unrounded mul.f32/add.f32 pair that ptxas may or may not contract. */
#define KVO_QUANT_TWO_ROUNDINGS 0
#define KVO_QUANT_FUSED 1

/* Rate-0 block policy for the decoders. */
#define KVO_RATE0_SKIP 0 /* reference: block not written (cu:496) */
#define KVO_RATE0_ZERO 1 /* write +0.0 (the decoded value of q = 0) */

int32_t kvo_quantize(float x, float recip, int variant);
void kvo_quantize_array(const float* x, uint64_t n, float recip, int variant,
                        int32_t* q);
int kvo_bit_count(uint32_t v);
float kvo_bf16_to_f32(uint16_t h);
uint16_t kvo_f32_to_bf16_rne(float f);
uint64_t kvo_source_index(uint64_t logical, const int64_t* layer_indices,
                          uint64_t selected_layers, uint64_t source_layers,
                          uint64_t elements_per_layer);

/* Header bytes R = 1024 * ceil(n / 32768). */
uint64_t kvo_header_bytes(uint64_t n);

float kvo_relative_bound(const uint16_t* page, uint64_t n,
                         const int64_t* layer_indices, uint64_t selected_layers,
                         uint64_t source_layers, uint64_t elements_per_layer,
                         float eps);

/* Encodes one page; returns the stream size S.  Header padding is zeroed. */
uint64_t kvo_compress_page(const uint16_t* page, uint64_t n,
                           const int64_t* layer_indices,
                           uint64_t selected_layers, uint64_t source_layers,
                           uint64_t elements_per_layer, float eb, int variant,
                           uint8_t* out);

/* fp32 single-page path (CuSZpWrapper::compress/decompress, fixed mode):
 * the same stream over contiguous fp32 values; bound as at::aminmax. */
float kvo_relative_bound_f32(const float* x, uint64_t n, float eps);
uint64_t kvo_compress_page_f32(const float* x, uint64_t n, float eb,
                               int variant, uint8_t* out);
int kvo_decompress_f32(const uint8_t* stream, uint64_t stream_size, uint64_t n,
                       float eb, int rate0_policy, float* out);

/* Lorenzo modes of the fp32 single-page API (this build's specification of
 * upstream cuSZp's plain and outlier modes; see kvszp_oracle.c).  `mode` is
 * KVO_MODE_*; KVO_MODE_FIXED selects the fixed-mode functions above.  The
 * worst-case stream is R + 136 bytes per block. */
#define KVO_MODE_FIXED 0
#define KVO_MODE_PLAIN 1
#define KVO_MODE_OUTLIER 2
uint64_t kvo_compress_page_f32_mode(const float* x, uint64_t n, float eb,
                                    int variant, int mode, uint8_t* out);
int kvo_decompress_f32_mode(const uint8_t* stream, uint64_t stream_size, uint64_t n,
                            float eb, int mode, int rate0_policy, float* out);

/* Decoders.  Each returns 0 on success, -1 if the stream is malformed
 * (rate > 31 or payload past stream_size). */
int kvo_decompress_contiguous(const uint8_t* stream, uint64_t stream_size,
                              uint64_t n, float eb, int rate0_policy,
                              uint16_t* out);
int kvo_decompress_scatter(const uint8_t* stream, uint64_t stream_size,
                           uint64_t n, float eb, int rate0_policy,
                           uint16_t* const* destinations,
                           uint64_t destinations_per_page,
                           uint64_t elements_per_destination);
int kvo_decompress_indexed(const uint8_t* stream, uint64_t stream_size,
                           uint64_t n, float eb, int rate0_policy,
                           uint16_t* destination, const int64_t* layer_indices,
                           uint64_t selected_layers, uint64_t source_layers,
                           uint64_t elements_per_layer);

/* Batched encoder over page pointers (the reference's per-call semantics:
 * eps_i > 0 ? eps_i : default_eps, optional relative bound).  Pages are
 * split across `threads` OpenMP threads.  Returns 0. */
int kvo_compress_batch(const uint16_t* const* pages, uint8_t* const* outs,
                       uint64_t batch, uint64_t n,
                       const int64_t* layer_indices, uint64_t selected_layers,
                       uint64_t source_layers, uint64_t elements_per_layer,
                       const float* eps, float default_eps, int relative,
                       int variant, int threads, uint64_t* sizes,
                       float* bounds);
int kvo_decompress_batch_contiguous(const uint8_t* const* streams,
                                    const uint64_t* sizes, uint64_t batch,
                                    uint64_t n, const float* bounds,
                                    int rate0_policy, int threads,
                                    uint16_t* out);

int kvo_decompress_batch_indexed(const uint8_t* const* streams,
                                 const uint64_t* sizes, uint64_t batch,
                                 uint64_t n, const float* bounds,
                                 int rate0_policy, int threads,
                                 uint16_t* const* destinations,
                                 const int64_t* layer_indices,
                                 uint64_t selected_layers, uint64_t source_layers,
                                 uint64_t elements_per_layer);

/* INT8 host codec (vllm_v1_compressed_offload.py:711-724, 2090-2123). */
float kvo_int8_encode(const uint16_t* page, uint64_t n, int8_t* q);
void kvo_int8_decode(const int8_t* q, uint64_t n, float scale, uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif
