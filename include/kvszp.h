/*
 * kvszp.h -- C ABI of the MI355X batched fixed-mode BF16 KV-page codec.
 *
 * Drop-in boundary for the reference's pybind11 module `cuszp_wrapper_cpp`
 * (integration/cuszp_wrapper/pybind11_bindings.cpp) and the C++ class behind
 * it (integration/cuszp_wrapper/cuszp_wrapper.h:9-158).  Every entry point
 * takes plain pointers and sizes; no framework types cross this boundary.
 *
 * Conventions shared by all entry points:
 *  - Return value: KVSZP_OK (0) or a negative KVSZP_E* code.  The message of
 *    the last failure on the calling thread is kvszp_last_error().
 *  - Pointer arrays (page lists) live in HOST memory; the pointers in them
 *    are DEVICE addresses.  Layer-index arrays are DEVICE int64 arrays, as in
 *    the reference (a torch cuda int64 tensor).
 *  - `stream` is a hipStream_t (0 = legacy default stream).  Compress entry
 *    points block until sizes are on the host (the reference synchronizes,
 *    cuszp_wrapper.cpp:530); decompress entry points only enqueue
 *    (cuszp_wrapper.cpp:1102-1109).  kvszp_destroy waits for the device.
 *  - A context owns grow-only device workspaces, so one context must not be
 *    used from two host threads or two streams at once (same as the
 *    reference's CuSZpWrapper).
 *  - Compressed streams are byte-exact to the reference fixed-mode layout:
 *    R = 1024*ceil(N/32768) header bytes (one rate byte per 32-element
 *    block, padding written as 0), then per block with rate r > 0 a sign
 *    word and r bit-plane words.  Compressed buffers must be 4-byte aligned
 *    (the reference stores uchar4 words, cuszp_batched_fixed.cu:326).
 */
#ifndef KVSZP_H
#define KVSZP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct kvszp_ctx kvszp_ctx;
typedef void* kvszp_stream_t; /* hipStream_t */

enum {
    KVSZP_OK = 0,
    KVSZP_EINVAL = -1,   /* argument validation failed (reference: false) */
    KVSZP_EHIP = -2,     /* a HIP runtime call failed */
    KVSZP_ENOMEM = -3,   /* workspace allocation failed */
    KVSZP_EDEVICE = -4   /* a kernel reported an error (bad layer index,
                            malformed stream, or a bounded wait expired) */
};

/* Mirrors cuSZp's enums as exposed by pybind11_bindings.cpp:13-28. */
enum { KVSZP_DIM_1D = 0, KVSZP_DIM_2D = 1, KVSZP_DIM_3D = 2 };
enum { KVSZP_MODE_FIXED = 0, KVSZP_MODE_PLAIN = 1, KVSZP_MODE_OUTLIER = 2 };
enum { KVSZP_TYPE_FLOAT = 0, KVSZP_TYPE_DOUBLE = 1 };

/* Quantizer reading of cuszp_batched_fixed.cu:17-20 (mul.f32 then add.f32
 * without rounding modifiers): two roundings (default) or one fused FMA. */
enum { KVSZP_QUANT_TWO_ROUNDINGS = 0, KVSZP_QUANT_FUSED = 1 };
/* Rate-0 blocks on decode: write +0.0 (default) or leave the destination
 * untouched exactly like the reference (cuszp_batched_fixed.cu:496). */
enum { KVSZP_RATE0_SKIP = 0, KVSZP_RATE0_ZERO = 1 };

/* CuSZpWrapper::CompressionConfig, cuszp_wrapper.h:11-17. */
typedef struct kvszp_config {
    float error_bound;      /* default 1e-4 */
    int use_relative_error; /* default 1 */
    int processing_dim;     /* KVSZP_DIM_* (default 1D) */
    int encoding_mode;      /* KVSZP_MODE_* (default PLAIN) */
    int data_type;          /* KVSZP_TYPE_* (default FLOAT) */
} kvszp_config;

/* Replaces CuSZpWrapper(config, device_id), cuszp_wrapper.cpp:23-39. */
int kvszp_create(const kvszp_config* config, int device_id, kvszp_ctx** out);
/* Replaces ~CuSZpWrapper, cuszp_wrapper.cpp:41-66. */
int kvszp_destroy(kvszp_ctx* ctx);
/* Replaces get_config / update_config, cuszp_wrapper.h:126-127. */
int kvszp_get_config(const kvszp_ctx* ctx, kvszp_config* out);
int kvszp_update_config(kvszp_ctx* ctx, const kvszp_config* config);
/* Codec options with no reference counterpart (see the enums above). */
int kvszp_set_options(kvszp_ctx* ctx, int quantizer, int rate0_policy);

/* Replaces CuSZpWrapper::estimate_compressed_buffer_size,
 * cuszp_wrapper.cpp:1319-1321 (2 x bytes; callers pass 4*N). */
size_t kvszp_estimate_compressed_buffer_size(size_t original_size);
/* Header bytes R of a stream of n elements (cuszp_wrapper.cpp:534-535). */
size_t kvszp_header_bytes(size_t num_elements);

/* Replaces CuSZpWrapper::compress_batch_fixed_bf16,
 * cuszp_wrapper.cpp:431-544 (binding pybind11_bindings.cpp:84-101).
 *  inputs[batch]      : device BF16 pages, num_elements each
 *  outputs[batch]     : device byte buffers, capacities[i] bytes each
 *                       (must be >= 8*num_elements, cuszp_wrapper.cpp:449)
 *  eps_overrides      : NULL or [batch]; eps_i > 0 overrides error_bound
 *  sizes_out[batch]   : stream bytes S_i
 *  bounds_out[batch]  : absolute error bound used for page i */
int kvszp_compress_batch_fixed_bf16(
    kvszp_ctx* ctx, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const float* eps_overrides, size_t batch,
    size_t num_elements, kvszp_stream_t stream, uint64_t* sizes_out,
    float* bounds_out);

/* kvszp_compress_batch_fixed_bf16 for callers that cannot allocate memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  Same arguments, checks and
 * results as kvszp_compress_batch_fixed_bf16, but the call allocates
 * nothing: the encoder's device state (look-back and min/max words, job
 * table) lives in one file-scope device array per GPU of about 1.2 MiB,
 * held until the process ends, and its pinned host areas are set up by
 * kvszp_create.  Limits: at most 4096 pages and 65536 tiles of 8192 values
 * (512 Mi values) per call; larger calls fail with KVSZP_EINVAL.  All
 * contexts on a GPU share that array: calls that overlap in time on one GPU
 * (two host threads, or two streams) race and must not be issued. */
int kvszp_compress_batch_fixed_bf16_noalloc(
    kvszp_ctx* ctx, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const float* eps_overrides, size_t batch,
    size_t num_elements, kvszp_stream_t stream, uint64_t* sizes_out,
    float* bounds_out);

/* Replaces CuSZpWrapper::compress_batch_fixed_bf16_indexed,
 * cuszp_wrapper.cpp:548-681 (pybind11_bindings.cpp:104-132).  Page i is
 * read as view(prefix_count, source_layers, elements_per_layer) and the
 * layers in layer_indices[selected_layers] (device int64) are encoded as one
 * logical segment of prefix_count*selected_layers*elements_per_layer values. */
int kvszp_compress_batch_fixed_bf16_indexed(
    kvszp_ctx* ctx, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const int64_t* layer_indices,
    size_t selected_layers, size_t prefix_count, size_t source_layers,
    size_t elements_per_layer, const float* eps_overrides, size_t batch,
    kvszp_stream_t stream, uint64_t* sizes_out, float* bounds_out);

/* Replaces CuSZpWrapper::compress_batch_fixed_bf16_indexed_groups,
 * cuszp_wrapper.cpp:683-868 (pybind11_bindings.cpp:133-163).  Requests are
 * laid out group by group: group g covers the next group_sizes[g] entries of
 * inputs/outputs and uses layer_indices[g] (device int64, selected_layers[g]
 * long).  Up to 16 groups run in ONE kernel launch (the reference launches
 * once per group); more groups take one launch per 16. */
int kvszp_compress_batch_fixed_bf16_indexed_groups(
    kvszp_ctx* ctx, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const int64_t* const* layer_indices,
    const size_t* selected_layers, const size_t* group_sizes,
    size_t num_groups, size_t prefix_count, size_t source_layers,
    size_t elements_per_layer, const float* eps_overrides, size_t batch,
    kvszp_stream_t stream, uint64_t* sizes_out, float* bounds_out);

/* Replaces CuSZpWrapper::decompress_batch_fixed_bf16,
 * cuszp_wrapper.cpp:1034-1110 (pybind11_bindings.cpp:190-207).  Page i is
 * decoded to output + i*num_elements_per_page; output holds
 * output_elements >= batch*num_elements_per_page BF16 values. */
int kvszp_decompress_batch_fixed_bf16(
    kvszp_ctx* ctx, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* output,
    size_t output_elements, size_t num_elements_per_page,
    kvszp_stream_t stream);

/* Replaces CuSZpWrapper::decompress_batch_fixed_bf16_scatter,
 * cuszp_wrapper.cpp:1111-1212 (pybind11_bindings.cpp:208-230).  Logical
 * element e of page i goes to
 *   destinations[i*destinations_per_page + e/elements_per_destination]
 *               [e % elements_per_destination];
 * num_elements_per_page == destinations_per_page*elements_per_destination. */
int kvszp_decompress_batch_fixed_bf16_scatter(
    kvszp_ctx* ctx, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    size_t num_elements_per_page, size_t destinations_per_page,
    size_t elements_per_destination, kvszp_stream_t stream);

/* Replaces CuSZpWrapper::decompress_batch_fixed_bf16_indexed_scatter,
 * cuszp_wrapper.cpp:1214-1313 (pybind11_bindings.cpp:232-256).  Decodes the
 * layer-selected segment straight into the full page destinations[i]
 * (view(prefix_count, source_layers, elements_per_layer)). */
int kvszp_decompress_batch_fixed_bf16_indexed_scatter(
    kvszp_ctx* ctx, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    const int64_t* layer_indices, size_t selected_layers,
    size_t prefix_count, size_t source_layers, size_t elements_per_layer,
    kvszp_stream_t stream);

/* Several calls of kvszp_decompress_batch_fixed_bf16_indexed_scatter in
 * ONE kernel launch: requests are laid out group by group like
 * kvszp_compress_batch_fixed_bf16_indexed_groups (group g covers the next
 * group_sizes[g] entries and uses layer_indices[g], selected_layers[g] long).
 * No reference counterpart: the reference decodes a mixed-bound job with one
 * decompress_batch_fixed_bf16_indexed_scatter call per layer group
 * (vllm_v1_compressed_offload.py:1815-2006); this entry point gives that
 * caller the same result in a single launch. */
int kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups(
    kvszp_ctx* ctx, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    const int64_t* const* layer_indices, const size_t* selected_layers,
    const size_t* group_sizes, size_t num_groups, size_t prefix_count,
    size_t source_layers, size_t elements_per_layer, kvszp_stream_t stream);

/* ---- single-page fp32 API (fixed mode) ----------------------------------
 * The reference serves these with upstream cuSZp's fp32 fixed-mode kernels
 * (cuszp_fastpath.cu:5-64); the stream layout is the batched BF16 one
 * (cuszp_batched_fixed.cu:52-54), so here the same kernels run with fp32
 * loads and stores.  The relative bound is the one these methods compute:
 * at::aminmax over the whole input (a NaN makes the bound NaN), range raised
 * to 1e-6f when below it, eb = eps * range (cuszp_wrapper.cpp:249-257,
 * :371-377).  The *_fixed_f32 entries require MODE_FIXED, DIM_1D,
 * TYPE_FLOAT; kvszp_compress_f32 / kvszp_decompress_f32 /
 * kvszp_decompress_batch_f32 below follow the context's encoding mode.
 * Inputs and outputs are contiguous fp32 arrays, 4-byte aligned. */

/* Replaces CuSZpWrapper::compress (fixed mode), cuszp_wrapper.cpp:216-325
 * (pybind11_bindings.cpp:49-64).  eps_override > 0 overrides error_bound.
 * Blocks until *size_out (stream bytes S) and *bound_out are on the host. */
int kvszp_compress_fixed_f32(kvszp_ctx* ctx, const float* input,
                             size_t num_elements, void* output,
                             uint64_t capacity, float eps_override,
                             kvszp_stream_t stream, uint64_t* size_out,
                             float* bound_out);

/* Replaces CuSZpWrapper::compress_batch_fixed, cuszp_wrapper.cpp:327-429
 * (pybind11_bindings.cpp:65-82): batch pages of num_elements fp32 values in
 * one launch (the reference launches once per page). */
int kvszp_compress_batch_fixed_f32(kvszp_ctx* ctx, const void* const* inputs,
                                   void* const* outputs,
                                   const uint64_t* capacities,
                                   const float* eps_overrides, size_t batch,
                                   size_t num_elements, kvszp_stream_t stream,
                                   uint64_t* sizes_out, float* bounds_out);

/* Replaces CuSZpWrapper::decompress (fixed mode), cuszp_wrapper.cpp:870-943
 * (pybind11_bindings.cpp:164-173): num_elements fp32 values
 * y = fl(fl(q * eb) * 2) to output; enqueue only. */
int kvszp_decompress_fixed_f32(kvszp_ctx* ctx, const void* compressed,
                               uint64_t compressed_size, float* output,
                               size_t num_elements, float error_bound,
                               kvszp_stream_t stream);

/* Replaces CuSZpWrapper::decompress_batch (fixed mode),
 * cuszp_wrapper.cpp:944-1033 (pybind11_bindings.cpp:174-189): page i
 * (num_elements[i] values) to outputs[i], all pages in one launch per run of
 * equal lengths (the reference fans pages out over up to 8 streams). */
int kvszp_decompress_batch_fixed_f32(kvszp_ctx* ctx,
                                     const void* const* compressed,
                                     const uint64_t* sizes,
                                     const float* error_bounds, size_t batch,
                                     void* const* outputs,
                                     const uint64_t* num_elements,
                                     kvszp_stream_t stream);

/* Replaces CuSZpWrapper::compress in every encoding mode,
 * cuszp_wrapper.cpp:216-325 (pybind11_bindings.cpp:49-64): MODE_FIXED as
 * kvszp_compress_fixed_f32; MODE_PLAIN and MODE_OUTLIER (the reference hands
 * them to upstream cuSZp, :302-313) as this library's residual codes: the
 * fixed-length block code over q_v - q_{v-1} inside each 32-value block
 * (outlier: the block's first q kept aside as a 4-byte word).  Their byte
 * layout is this library's own; capacity >= max(8n, R + 136 * blocks). */
int kvszp_compress_f32(kvszp_ctx* ctx, const float* input, size_t num_elements,
                       void* output, uint64_t capacity, float eps_override,
                       kvszp_stream_t stream, uint64_t* size_out, float* bound_out);

/* Replaces CuSZpWrapper::decompress in every encoding mode,
 * cuszp_wrapper.cpp:870-943 (launch_cuszp_decompress_1d_f32 picks the
 * mode's decoder, cuszp_fastpath.cu:26-59); enqueue only. */
int kvszp_decompress_f32(kvszp_ctx* ctx, const void* compressed,
                         uint64_t compressed_size, float* output,
                         size_t num_elements, float error_bound,
                         kvszp_stream_t stream);

/* Replaces CuSZpWrapper::decompress_batch in every encoding mode,
 * cuszp_wrapper.cpp:944-1033; enqueue only. */
int kvszp_decompress_batch_f32(kvszp_ctx* ctx, const void* const* compressed,
                               const uint64_t* sizes, const float* error_bounds,
                               size_t batch, void* const* outputs,
                               const uint64_t* num_elements, kvszp_stream_t stream);

/* ---- packed publication and restore --------------------------------------- */

/* Replaces CompressedPageStore.put_many_packed
 * (vllm_v1_compressed_offload.py:371-447): payload i (any device buffer,
 * sizes[i] bytes, e.g. a stream written by a compress call or a raw page) is
 * placed at offsets_out[i] of `slab`, the offsets being the 8-byte-aligned
 * exclusive scan of the sizes (gaps zeroed); *packed_bytes_out = end of the
 * last payload.  `slab` is normally pinned host memory (hipHostMalloc, torch
 * pin_memory): one gather kernel then writes every payload across the link,
 * which is the device-to-host transfer (the reference concatenates on the
 * device with torch.cat and copies the result).  Device memory works too.
 * Blocks until the slab is complete, like the reference (:429-430). */
int kvszp_pack_streams(kvszp_ctx* ctx, const void* const* payloads,
                       const uint64_t* sizes, size_t count, void* slab,
                       uint64_t slab_capacity, kvszp_stream_t stream,
                       uint64_t* offsets_out, uint64_t* packed_bytes_out);

/* The packed restore of a grouped indexed store
 * (vllm_v1_compressed_offload.py:1618-1711 then :1815-2006): one
 * host-to-device copy of `packed_bytes` from the pinned slab `packed` into
 * the device buffer `staging`, then
 * kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups with stream i at
 * staging + offsets[i].  staging == NULL: no copy and no staging buffer;
 * the decoder reads stream i at packed + offsets[i] across the link itself
 * (256 workgroups, which reach the link's rate).  Enqueue only. */
int kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups_packed(
    kvszp_ctx* ctx, const void* packed, uint64_t packed_bytes, void* staging,
    uint64_t staging_capacity, const uint64_t* offsets, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    const int64_t* const* layer_indices, const size_t* selected_layers,
    const size_t* group_sizes, size_t num_groups, size_t prefix_count,
    size_t source_layers, size_t elements_per_layer, kvszp_stream_t stream);

/* Waits for `stream` and reports any error a kernel of this context flagged
 * since the last check.  Decompress calls only enqueue, so their
 * device-side errors (malformed stream, layer index out of range) surface
 * here; compress calls report only the errors of their own launches.  No
 * reference counterpart: the reference's decoders have no device-side
 * checks. */
int kvszp_synchronize(kvszp_ctx* ctx, kvszp_stream_t stream);

/* Kernel timing.  For the kernel kinds in `kinds` (a mask of KVSZP_TIME_*;
 * 0 disables), every launch of this context carries a pair of HIP events
 * that the launch itself stamps with the kernel's start and end
 * (hipExtLaunchKernelGGL; compress: relative-bound pre-pass, if any, plus
 * encoder; decompress: decoder).  kvszp_drain_timing waits for the events,
 * returns the summed
 * milliseconds and launch counts per kind, and forgets them.  No reference
 * counterpart: the reference times whole stages with synchronize +
 * perf_counter (vllm_v1_compressed_offload.py:2009-2019). */
enum { KVSZP_KERNEL_COMPRESS = 0, KVSZP_KERNEL_DECOMPRESS = 1 };
enum {
    KVSZP_TIME_COMPRESS = 1 << KVSZP_KERNEL_COMPRESS,
    KVSZP_TIME_DECOMPRESS = 1 << KVSZP_KERNEL_DECOMPRESS,
    KVSZP_TIME_ALL = KVSZP_TIME_COMPRESS | KVSZP_TIME_DECOMPRESS
};
int kvszp_enable_timing(kvszp_ctx* ctx, int kinds);
int kvszp_drain_timing(kvszp_ctx* ctx, double* compress_ms, int* compress_count,
                       double* decompress_ms, int* decompress_count);

/* The durations (milliseconds, launch order) of the timed launches of one
 * kernel kind (KVSZP_KERNEL_*) recorded since they were last drained; at
 * most `capacity` are written, *count_out says how many.  Those records are
 * forgotten, records of the other kind are kept.  No reference counterpart. */
int kvszp_timing_durations(kvszp_ctx* ctx, int kind, double* ms_out,
                           int capacity, int* count_out);

/* How many compress calls of this context were encoded a second time, with
 * the schedule that needs no residency (min/max pre-pass, one workgroup per
 * tile), because a launch's time-bounded cross-workgroup wait gave up (the
 * device was shared with other work; KVSZP_WAIT_US sets the bound, default
 * 200 us) or the persistent encoder's staging overflowed.  No reference
 * counterpart: the reference's kernels assume the launch runs alone. */
int kvszp_reencode_count(const kvszp_ctx* ctx, uint64_t* count);

/* Compress calls of this context encoded again after a give-up or a
 * staging overflow (as kvszp_reencode_count), and compress calls that ran
 * the schedule needing no residency from the start because a launch of the
 * context gave up within the previous KVSZP_SAFE_CALLS calls (default 0:
 * every call tries the persistent encoder).  No reference counterpart. */
int kvszp_schedule_counts(const kvszp_ctx* ctx, uint64_t* reencoded, uint64_t* safe_calls);

/* Sets the time bound of the encoders' cross-workgroup waits of this
 * context (microseconds, 0 to 1e6; the default is KVSZP_WAIT_US or 200 us).
 * A wait that outlasts it stops the launch, and the call is encoded again
 * with the schedule that needs no residency (kvszp_reencode_count).  No
 * reference counterpart: the reference's look-back spins without a bound
 * (cuszp_batched_fixed.cu:256-275).  For callers that share the device with
 * long-running kernels, and for tests that force the give-up path. */
int kvszp_set_wait_bound(kvszp_ctx* ctx, double microseconds);

/* Message of the last failed call on this thread ("" if none). */
const char* kvszp_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* KVSZP_H */
