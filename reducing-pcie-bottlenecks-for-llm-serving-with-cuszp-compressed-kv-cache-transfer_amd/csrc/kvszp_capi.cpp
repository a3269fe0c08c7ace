// kvszp_capi.cpp -- host side of the C ABI declared in include/kvszp.h.
//
// Replaces the batched BF16 methods of CuSZpWrapper
// (integration/cuszp_wrapper/cuszp_wrapper.cpp:431-868, 1034-1313).
// Differences in mechanism (not in results):
//  - one launch per call, also for grouped requests (the reference launches
//    once per group, cuszp_wrapper.cpp:795-848);
//  - no per-call memsets: cross-workgroup words carry an epoch tag;
//  - one H2D copy of a packed job table from a pinned staging ring; the
//    encoder writes sizes and bounds straight into pinned host memory (the
//    reference issues one D2H copy per page, cuszp_wrapper.cpp:523-529);
//  - kernels raise a marker in a pinned host control block when they flag an
//    error, so the device error word is copied back only when it is set.
#include "kvszp.h"
#include "kvszp_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

using namespace kvszp;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(KVSZP_EHIP, "%s: %s", what, hipGetErrorString(e));
}

struct DevBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
};

// A pinned buffer the job table is copied from.  `seq` is the launch that
// follows the copy: once that launch has published its sequence number the
// copy has completed and the slot may be rewritten.
struct StagingSlot {
    void* host = nullptr;
    size_t bytes = 0;
    uint32_t seq = 0;
    hipStream_t stream = nullptr;
    bool pending = false;
};

constexpr int kSlots = 4;
constexpr uint32_t kLinkDecodeGrid = 256;  // decoder workgroups reading pinned memory
constexpr size_t kJobBalancedRuns = 1024;   // batches from this size: job-balanced decoder runs
constexpr uint32_t kEpochLimit = (1u << 30) - 2u;
constexpr double kMaxWaitMicros = 1e6;  // longest bound of a cross-workgroup wait
constexpr uint64_t kMaxElements = 1ull << 29;      // per logical segment
constexpr uint64_t kMaxTiles = (1ull << 32) / kThreads - 1;

struct TimingRecord {
    int kind;  // KVSZP_KERNEL_*
    hipEvent_t start, stop;
    double bytes;  // algorithmic bytes of the launch (filled when known)
};

}  // namespace

struct kvszp_ctx {
    kvszp_config config;
    int device = 0;
    int quantizer = KVSZP_QUANT_TWO_ROUNDINGS;
    int rate0 = KVSZP_RATE0_ZERO;
    uint32_t fused_tile_limit = 0;
    bool use_tickets = false;  // KVSZP_TICKETS=1: ticket-ordered tiles
    // Job tables of the persistent kernels that fit an ArgTable travel in
    // the kernel arguments instead of a table copy on the stream
    // (KVSZP_ARG_TABLES=0 turns that off).
    int arg_tables = 3;  // bit 0: stores, bit 1: restores
    // Time bound of the encoders' cross-workgroup waits, in steady-clock
    // ticks (KVSZP_WAIT_US, default 200 us), and how many calls were encoded
    // again after a launch gave up or overflowed.
    uint64_t wait_ticks = 0;
    uint32_t clock_khz = 100000;  // device steady-clock rate
    uint64_t redone = 0;
    // After a launch gave up, the next `safe_after_abort` compress calls use
    // the schedule that needs no residency straight away (KVSZP_SAFE_CALLS,
    // default 0: off).  Measured on MI355X beside a stream of large matrix
    // products, the persistent encoder did not give up and took 0.83 ms per
    // configuration-1 store, the schedule that needs no residency 2.26 ms,
    // so a give-up is not taken as a sign that the next call would give up
    // too.  `safe_left` counts them down.
    uint32_t safe_after_abort = 0;
    uint32_t safe_left = 0;
    uint64_t safe_calls = 0;      // compress calls run on that schedule
    // Epoch tags run from 1 to epoch_limit, then every tagged word is
    // cleared and they start again (KVSZP_EPOCH_LIMIT lowers the limit so
    // that tests can cross the wrap).
    uint32_t epoch_limit = kEpochLimit;
    // Persistent encoder grid (co-resident workgroups); 0 = one workgroup
    // per tile (KVSZP_PERSISTENT=0, or ticket mode).
    uint32_t pipelined_grid = 0;
    // Compute units of the device, and the persistent encoder's first-tile
    // mapping (persistent_slot_cus mode; KVSZP_SLOT_MIX=0/1/2, default 1).
    uint32_t cus = 0;
    int slot_mix = 1;
    uint32_t decompress_grid = 0;   // persistent decoder grid (0 = off)
    // control words: [0] ticket counter, [1] low 32 bits = error word
    unsigned long long* control = nullptr;
    unsigned long long ticket_next = 0;
    uint32_t epoch = 0;
    DevBuf tile_state, tile_minmax, job_minmax, job_flags, tables;
    StagingSlot slots[kSlots];
    int next_slot = 0;
    uint32_t seq = 0;                     // last launch sequence number
    uint32_t* host_ctl = nullptr;         // pinned coherent control block
    void* host_results = nullptr;         // pinned coherent sizes + bounds
    size_t host_results_bytes = 0;
    // No-allocation encoder: the device's scratch array (device address) and
    // pinned host areas of fixed size, all set up by kvszp_create.
    unsigned char* scratch = nullptr;
    CompressJob* noalloc_stage = nullptr;     // kNoAllocMaxJobs job records
    void* noalloc_results = nullptr;          // kNoAllocMaxJobs sizes, bounds, redo marks
    // Optional kernel timing: event pairs recorded on the launch stream for
    // the kernel kinds in the mask (bit KVSZP_KERNEL_*).
    int timing = 0;
    std::vector<TimingRecord> timed;      // recorded, not yet drained
    std::vector<hipEvent_t> spare_events;
};

namespace {

// Device error words: encoder kernels (low half of control word 1) and
// decoder kernels (high half), each with its own host marker.
uint32_t* error_word(kvszp_ctx* c) {
    return reinterpret_cast<uint32_t*>(c->control + 1);
}
uint32_t* decode_error_word(kvszp_ctx* c) {
    return reinterpret_cast<uint32_t*>(c->control + 1) + 1;
}
uint32_t* error_marker(kvszp_ctx* c) { return &c->host_ctl[kHostErrorMarker]; }
uint32_t* decode_error_marker(kvszp_ctx* c) { return &c->host_ctl[kHostDecodeErrorMarker]; }

// Epoch of the last launch of this context whose bounded waits gave up.
unsigned long long* abort_word(kvszp_ctx* c) { return c->control + 2; }

int use_device(kvszp_ctx* c) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (cur != c->device) {
        e = hipSetDevice(c->device);
        if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    }
    return KVSZP_OK;
}

// Grow-only device buffer, a whole number of 256-byte lines.  New memory is
// zeroed when `zero` (epoch-tagged words must never start with a tag that
// could match).
int ensure(DevBuf& b, size_t bytes, bool zero, hipStream_t stream) {
    if (bytes <= b.bytes) return KVSZP_OK;
    const size_t grown = (std::max(bytes, b.bytes + b.bytes / 2) + 255) & ~(size_t)255;
    if (b.ptr) {
        hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        (void)hipFree(b.ptr);
        b.ptr = nullptr;
        b.bytes = 0;
    }
    hipError_t e = hipMalloc(&b.ptr, grown);
    if (e != hipSuccess) {
        b.ptr = nullptr;
        return fail(KVSZP_ENOMEM, "hipMalloc(%zu): %s", grown,
                    hipGetErrorString(e));
    }
    b.bytes = grown;
    if (zero) {
        e = launch_fill_u64(static_cast<unsigned long long*>(b.ptr), grown / 8, stream);
        if (e != hipSuccess) return hip_fail(e, "clearing a new workspace");
    }
    return KVSZP_OK;
}

// Grows the pinned results area.  Only the encoder writes it and every
// compress call waits for its kernel, so no launch still refers to the old
// area when it is freed.
int ensure_host_results(kvszp_ctx* c, size_t bytes) {
    if (bytes <= c->host_results_bytes) return KVSZP_OK;
    if (c->host_results) (void)hipHostFree(c->host_results);
    c->host_results = nullptr;
    c->host_results_bytes = 0;
    const size_t grown = std::max<size_t>(bytes, 4096);
    hipError_t e = hipHostMalloc(&c->host_results, grown, hipHostMallocCoherent);
    if (e != hipSuccess) return fail(KVSZP_ENOMEM, "hipHostMalloc: %s", hipGetErrorString(e));
    std::memset(c->host_results, 0, grown);  // no stale redo marks
    c->host_results_bytes = grown;
    return KVSZP_OK;
}

uint32_t host_seq(const kvszp_ctx* c) {
    return __atomic_load_n(&c->host_ctl[kHostSeq], __ATOMIC_ACQUIRE);
}

// Waits for `stream` to drain.  Polls first (a compress launch lasts tens of
// microseconds, and a blocking wait adds the wake-up latency of the waiting
// thread to every call), then blocks if the stream is still busy after
// kSpinWaitMicros.
constexpr int64_t kSpinWaitMicros = 2000;

hipError_t wait_stream(hipStream_t stream) {
    const auto t0 = std::chrono::steady_clock::now();
    for (;;) {
        const hipError_t e = hipStreamQuery(stream);
        if (e != hipErrorNotReady) return e;
        const auto us = std::chrono::duration_cast<std::chrono::microseconds>(
            std::chrono::steady_clock::now() - t0).count();
        if (us > kSpinWaitMicros) return hipStreamSynchronize(stream);
    }
}

// Copies `bytes` of host data to c->tables through a pinned staging slot;
// `seq` is the sequence number of the launch that will read the table.
int upload_tables(kvszp_ctx* c, const void* data, size_t bytes, uint32_t seq,
                  hipStream_t stream) {
    int rc = ensure(c->tables, bytes, false, stream);
    if (rc) return rc;
    StagingSlot& s = c->slots[c->next_slot];
    c->next_slot = (c->next_slot + 1) % kSlots;
    hipError_t e;
    if (s.pending) {
        // The copy out of this slot may still be queued: wait for it unless
        // the launch behind it has already started.
        if ((int32_t)(host_seq(c) - s.seq) < 0) {
            e = s.stream == stream ? hipStreamSynchronize(stream)
                                   : hipDeviceSynchronize();
            if (e != hipSuccess) return hip_fail(e, "synchronize (staging slot)");
        }
        s.pending = false;
    }
    if (bytes > s.bytes) {
        if (s.host) (void)hipHostFree(s.host);
        s.host = nullptr;
        s.bytes = 0;
        const size_t grown = std::max<size_t>(bytes, 16384);
        e = hipHostMalloc(&s.host, grown, hipHostMallocDefault);
        if (e != hipSuccess)
            return fail(KVSZP_ENOMEM, "hipHostMalloc: %s", hipGetErrorString(e));
        s.bytes = grown;
    }
    std::memcpy(s.host, data, bytes);
    e = hipMemcpyAsync(c->tables.ptr, s.host, bytes, hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(H2D tables)");
    s.seq = seq;
    s.stream = stream;
    s.pending = true;
    return KVSZP_OK;
}

// Next epoch tag.  When the tags run out, every word that holds one is
// cleared before they start again: the look-back, min/max and flag words,
// and the abort word, which holds the epoch of the last launch whose
// bounded waits gave up (left standing, it would make every wait of the
// next launch with that epoch give up without telling the host).  The
// words are cleared by a fill kernel on `stream`, behind every earlier
// launch of the context on it.
int next_epoch(kvszp_ctx* c, hipStream_t stream, uint32_t* epoch) {
    if (c->epoch >= c->epoch_limit) {
        DevBuf* bufs[4] = {&c->tile_state, &c->tile_minmax, &c->job_minmax,
                           &c->job_flags};
        for (DevBuf* b : bufs) {
            if (!b->ptr) continue;
            hipError_t e = launch_fill_u64(static_cast<unsigned long long*>(b->ptr),
                                           b->bytes / 8, stream);
            if (e != hipSuccess) return hip_fail(e, "clearing the epoch words");
        }
        hipError_t e = launch_fill_u64(abort_word(c), 1, stream);
        if (e != hipSuccess) return hip_fail(e, "clearing the abort word");
        c->epoch = 0;
    }
    *epoch = ++c->epoch;
    return KVSZP_OK;
}

int check_fixed_config(const kvszp_ctx* c) {
    // cuszp_wrapper.cpp:439-446: the batched BF16 methods require fixed mode,
    // 1D processing and the float data type.
    if (c->config.processing_dim != KVSZP_DIM_1D ||
        c->config.data_type != KVSZP_TYPE_FLOAT ||
        c->config.encoding_mode != KVSZP_MODE_FIXED)
        return fail(KVSZP_EINVAL,
                    "batched BF16 codec requires MODE_FIXED, DIM_1D, TYPE_FLOAT");
    return KVSZP_OK;
}

// The fp32 single-page methods take every encoding mode
// (cuszp_wrapper.cpp:268-313, 886-939) but only 1D float data.
int check_f32_config(const kvszp_ctx* c) {
    if (c->config.processing_dim != KVSZP_DIM_1D ||
        c->config.data_type != KVSZP_TYPE_FLOAT)
        return fail(KVSZP_EINVAL, "fp32 codec requires DIM_1D, TYPE_FLOAT");
    const int m = c->config.encoding_mode;
    if (m != KVSZP_MODE_FIXED && m != KVSZP_MODE_PLAIN && m != KVSZP_MODE_OUTLIER)
        return fail(KVSZP_EINVAL, "unknown encoding mode %d", m);
    return KVSZP_OK;
}

static_assert(KVSZP_MODE_FIXED == kModeFixed && KVSZP_MODE_PLAIN == kModePlain &&
                  KVSZP_MODE_OUTLIER == kModeOutlier,
              "kernel modes are the C ABI's");

hipEvent_t take_event(kvszp_ctx* c) {
    if (!c->spare_events.empty()) {
        hipEvent_t e = c->spare_events.back();
        c->spare_events.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

// When timing is enabled for `kind`, returns the index of a new record whose
// start/stop events the launch stamps with the kernel's own start and end;
// otherwise -1.
int timing_begin(kvszp_ctx* c, int kind) {
    if (!(c->timing & (1 << kind))) return -1;
    TimingRecord r{kind, take_event(c), take_event(c), 0.0};
    if (!r.start || !r.stop) {
        if (r.start) c->spare_events.push_back(r.start);
        if (r.stop) c->spare_events.push_back(r.stop);
        return -1;
    }
    c->timed.push_back(r);
    return (int)c->timed.size() - 1;
}

hipEvent_t timing_start(kvszp_ctx* c, int rec) {
    return rec < 0 ? nullptr : c->timed[rec].start;
}
hipEvent_t timing_stop(kvszp_ctx* c, int rec) {
    return rec < 0 ? nullptr : c->timed[rec].stop;
}

// Reports (and clears) errors flagged by kernels of this context: those of
// its encoder kernels, and with `decoders` also those of its decoders.  The
// caller has synchronized `stream`, so no kernel of the context is running.
// A device word is read only when a kernel raised its host marker.
int consume_device_error(kvszp_ctx* c, hipStream_t stream, bool decoders = false) {
    uint32_t err = 0;
    for (int side = 0; side < (decoders ? 2 : 1); ++side) {
        uint32_t* marker = side ? decode_error_marker(c) : error_marker(c);
        if (__atomic_load_n(marker, __ATOMIC_ACQUIRE) == 0) continue;
        uint32_t* word = side ? decode_error_word(c) : error_word(c);
        uint32_t bits = 0;
        hipError_t e = hipMemcpyAsync(&bits, word, sizeof(bits), hipMemcpyDeviceToHost,
                                      stream);
        if (e == hipSuccess) e = hipMemsetAsync(word, 0, sizeof(uint32_t), stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_fail(e, "reading the device error word");
        __atomic_store_n(marker, 0u, __ATOMIC_RELEASE);
        err |= bits;
    }
    if (!err) return KVSZP_OK;
    std::string what;
    if (err & kErrSpin) what += " bounded-wait-expired";
    if (err & kErrLayerIndex) what += " layer-index-out-of-range";
    if (err & kErrRate) what += " rate-byte>31";
    if (err & kErrTruncated) what += " payload-past-stream-size";
    return fail(KVSZP_EDEVICE, "kernel reported:%s", what.c_str());
}

int validate_layers(const int64_t* layers, uint64_t sel, uint64_t prefix,
                    uint64_t src, uint64_t epl) {
    // cuszp_wrapper.cpp:562-575.
    if (layers == nullptr || prefix == 0 || src == 0 || epl == 0 || sel == 0 ||
        sel > src)
        return fail(KVSZP_EINVAL,
                    "invalid layer selection (prefix=%llu source_layers=%llu "
                    "elements_per_layer=%llu selected=%llu)",
                    (unsigned long long)prefix, (unsigned long long)src,
                    (unsigned long long)epl, (unsigned long long)sel);
    if (sel * epl > 0xFFFFFFFFull - kTileElems)
        return fail(KVSZP_EINVAL, "selected layers x elements_per_layer too large");
    return KVSZP_OK;
}

// Common compress path: `specs` are the groups, requests laid out group by
// group in inputs/outputs.  `f32`: contiguous fp32 pages (the single-page
// API, cuszp_wrapper.cpp:216-429) instead of BF16 pages.
// `safe`: only the schedule that needs no residency (pre-pass bound, one
// workgroup per tile).  `mode` (fp32 only): kModeFixed, or the plain and
// outlier residual codes of compress_lorenzo_kernel.  `bounds_given`: the
// eps values are the jobs' absolute bounds, worked out already (used as
// they are, also under a relative configuration).
int compress_groups(kvszp_ctx* c, const void* const* inputs,
                    void* const* outputs, const uint64_t* capacities,
                    const float* eps_overrides, size_t batch,
                    const std::vector<GroupSpec>& specs, hipStream_t stream,
                    uint64_t* sizes_out, float* bounds_out, bool f32 = false,
                    bool safe = false, int mode = kModeFixed, bool bounds_given = false) {
    int rc = mode == kModeFixed ? check_fixed_config(c) : check_f32_config(c);
    if (rc) return rc;
    if (batch == 0) return fail(KVSZP_EINVAL, "empty batch");
    if (!inputs || !outputs || !sizes_out || !bounds_out)
        return fail(KVSZP_EINVAL, "null pointer argument");
    if (specs.empty()) return fail(KVSZP_EINVAL, "no groups");
    rc = use_device(c);
    if (rc) return rc;

    const uintptr_t elem_align = f32 ? 3u : 1u;
    std::vector<CompressJob> jobs(batch);
    bool aligned16 = true;
    size_t job = 0;
    for (size_t gi = 0; gi < specs.size(); ++gi) {
        const GroupSpec& s = specs[gi];
        if (s.n == 0 || s.n > kMaxElements)
            return fail(KVSZP_EINVAL, "segment of %llu elements unsupported",
                        (unsigned long long)s.n);
        if (f32 && s.layers) return fail(KVSZP_EINVAL, "fp32 pages take no layer map");
        if (s.layers && (s.epl % 8) != 0) aligned16 = false;
        // cuszp_wrapper.cpp:449-450 asks for capacity >= estimate(4n) = 8n.
        // That does not cover the header of tiny segments (R = 1024 bytes for
        // n < 128), so the worst-case stream R + 128 * nb is required too
        // (R + 136 * nb in the residual modes: outlier word, sign, 32 planes).
        const uint64_t per_block = mode == kModeFixed ? 128ull : 136ull;
        const uint64_t worst = header_bytes_of(s.n) + per_block * ((s.n + 31) / 32);
        const uint64_t need = std::max<uint64_t>(8ull * s.n, worst);
        for (uint32_t k = 0; k < s.jobs; ++k, ++job) {
            if (job >= batch) return fail(KVSZP_EINVAL, "group sizes exceed batch");
            const uintptr_t in = (uintptr_t)inputs[job];
            const uintptr_t out = (uintptr_t)outputs[job];
            if (!in || !out) return fail(KVSZP_EINVAL, "null page pointer %zu", job);
            if (in & elem_align)
                return fail(KVSZP_EINVAL, "input %zu not %u-byte aligned", job,
                            (unsigned)elem_align + 1u);
            if (out & 3u)
                return fail(KVSZP_EINVAL, "compressed buffer %zu not 4-byte aligned", job);
            if (capacities && capacities[job] < need)
                return fail(KVSZP_EINVAL,
                            "compressed buffer %zu holds %llu bytes, needs %llu", job,
                            (unsigned long long)capacities[job],
                            (unsigned long long)need);
            if (in & 15u) aligned16 = false;
            const float e = bounds_given ? eps_overrides[job]
                            : (eps_overrides && eps_overrides[job] > 0.0f)
                                ? eps_overrides[job]
                                : c->config.error_bound;  // cuszp_wrapper.cpp:473-479
            jobs[job].in = reinterpret_cast<const uint16_t*>(in);
            jobs[job].out = reinterpret_cast<uint8_t*>(out);
            jobs[job].eps = e;
            jobs[job].reserved = 0;
        }
    }
    if (job != batch) return fail(KVSZP_EINVAL, "group sizes do not cover the batch");
    const std::vector<Chunk> chunks = split_chunks(specs);
    uint64_t max_tiles = 0;
    for (const Chunk& ch : chunks) {
        if (ch.tiles == 0 || ch.tiles > kMaxTiles)
            return fail(KVSZP_EINVAL, "batch too large for one launch");
        max_tiles = std::max(max_tiles, ch.tiles);
    }

    const bool relative = c->config.use_relative_error != 0 && !bounds_given;
    // Workspaces.
    if ((rc = ensure(c->tile_state, max_tiles * 8, true, stream)) ||
        (rc = ensure(c->tile_minmax, max_tiles * 8, true, stream)) ||
        (rc = ensure(c->job_minmax, batch * 16, true, stream)) ||
        (rc = ensure(c->job_flags, batch * 4, true, stream)) ||
        (rc = ensure_host_results(c, batch * 12)))
        return rc;
    const uint32_t seq = ++c->seq;
    // Small calls pass the job table in the kernel arguments (no upload), and
    // so do persistent-encoder launches whose table fits an ArgTable.  The
    // table is uploaded, once, for every other launch: from the start, or
    // when a launch is encoded again with the schedule that needs no
    // residency.
    const bool inline_jobs = batch <= (size_t)kInlineJobs;
    const size_t table_bytes = batch * sizeof(CompressJob);
    const bool arg_table = !inline_jobs && (c->arg_tables & 1) && table_bytes <= kArgTableBytes;
    bool uploaded = false;
    auto need_table = [&]() -> int {
        if (inline_jobs || uploaded) return KVSZP_OK;
        uploaded = true;
        return upload_tables(c, jobs.data(), table_bytes, seq, stream);
    };
    if (!arg_table && (rc = need_table())) return rc;

    uint32_t* host_sizes = reinterpret_cast<uint32_t*>(c->host_results);
    float* host_bounds = reinterpret_cast<float*>(host_sizes + batch);
    uint32_t* host_redo = host_sizes + 2 * batch;

    // One launch per chunk (normally one); all share the call's sequence
    // number and table, each has its own epoch (the look-back and min/max
    // words are reused from launch to launch).  `safe`: the schedule that
    // needs no residency (pre-pass bound, one workgroup per tile, untimed
    // look-back on earlier workgroups); otherwise the fused bound and the
    // persistent encoder where they apply, with time-bounded waits.
    std::vector<char> redo_candidate(chunks.size(), 0);
    std::vector<size_t> chunk_first_job(chunks.size(), 0);
    for (size_t k = 1; k < chunks.size(); ++k) {
        chunk_first_job[k] = chunk_first_job[k - 1];
        for (size_t gi = chunks[k - 1].g0; gi < chunks[k - 1].g1; ++gi)
            chunk_first_job[k] += specs[gi].jobs;
    }
    auto launch_chunk = [&](size_t k, bool safe, bool timed) -> int {
        const Chunk& ch = chunks[k];
        CompressParams p;
        std::memset(&p, 0, sizeof(p));
        p.num_groups = fill_groups(p.groups, specs, ch, chunk_first_job[k]);
        int bound_mode = kBoundAbsolute;
        if (relative)
            bound_mode = (!safe && !f32 && ch.max_tiles_per_job <= c->fused_tile_limit)
                             ? kBoundFused : kBoundPrepass;
        // Persistent encoder (whole, aligned, single-layer blocks only); its
        // waits are cycle-free while a job's tiles number at most the grid
        // (half of it here, for margin) and all its workgroups are resident.
        const bool persistent = !safe && !f32 && bound_mode != kBoundPrepass &&
                                c->pipelined_grid != 0 && ch.whole_blocks && aligned16 &&
                                ch.max_tiles_per_job <= c->pipelined_grid / 2;
        const bool use_arg = persistent && arg_table;
        if (!use_arg) {
            const int r = need_table();
            if (r) return r;
        }
        // The uploaded table, read only after the upload (which may have
        // grown the buffer); ArgTable and inline launches read no table.
        const CompressJob* djobs =
            uploaded ? reinterpret_cast<const CompressJob*>(c->tables.ptr) : nullptr;
        uint32_t epoch;
        int r = next_epoch(c, stream, &epoch);
        if (r) return r;
        const int rec = timed ? timing_begin(c, KVSZP_KERNEL_COMPRESS) : -1;
        hipError_t e;
        if (bound_mode == kBoundPrepass) {
            MinMaxParams m;
            std::memset(&m, 0, sizeof(m));
            m.jobs = djobs;
            m.num_jobs = (uint32_t)batch;
            if (inline_jobs) {
                m.jobs_inline = 1;
                std::memcpy(m.inline_jobs, jobs.data(), batch * sizeof(CompressJob));
            }
            m.job_minmax = reinterpret_cast<unsigned long long*>(c->job_minmax.ptr);
            m.error = error_word(c);
            m.error_marker = error_marker(c);
            m.host_ctl = c->host_ctl;
            m.seq = seq;
            m.epoch = epoch;
            m.num_groups = p.num_groups;
            m.input_f32 = f32 ? 1 : 0;
            std::memcpy(m.groups, p.groups, sizeof(m.groups));
            e = launch_minmax(m, (uint32_t)ch.tiles, stream, timing_start(c, rec));
            if (e != hipSuccess) return hip_fail(e, "minmax launch");
        }
        p.jobs = djobs;
        p.num_jobs = (uint32_t)batch;
        if (inline_jobs) {
            p.jobs_inline = 1;
            std::memcpy(p.inline_jobs, jobs.data(), batch * sizeof(CompressJob));
        }
        p.tile_state = reinterpret_cast<unsigned long long*>(c->tile_state.ptr);
        p.tile_minmax = reinterpret_cast<unsigned long long*>(c->tile_minmax.ptr);
        p.job_minmax = reinterpret_cast<const unsigned long long*>(c->job_minmax.ptr);
        p.host_sizes = host_sizes;
        p.host_bounds = host_bounds;
        p.host_redo = host_redo;
        p.job_flags = reinterpret_cast<uint32_t*>(c->job_flags.ptr);
        p.error = error_word(c);
        p.error_marker = error_marker(c);
        p.host_ctl = c->host_ctl;
        p.seq = seq;
        p.ticket = c->use_tickets ? c->control : nullptr;
        p.ticket_base = c->ticket_next;
        p.epoch = epoch;
        p.total_tiles = (uint32_t)ch.tiles;
        p.bound_mode = bound_mode;
        p.quantizer = c->quantizer;
        p.aligned16 = aligned16 ? 1 : 0;
        p.input_f32 = f32 ? 1 : 0;
        p.mode = f32 ? mode : kModeFixed;
        if (use_arg) p.jobs_inline = 2;
        if (persistent || bound_mode == kBoundFused) {
            p.abort_word = abort_word(c);
            p.wait_ticks = c->wait_ticks;
        }
        redo_candidate[k] = p.abort_word != nullptr;
        if (persistent) {
            p.ticket = nullptr;
            const uint32_t grid = (uint32_t)std::min<uint64_t>(ch.tiles, c->pipelined_grid);
            p.slot_cus = persistent_slot_cus(ch.tiles, grid, c->cus, c->slot_mix);
            e = launch_compress_pipelined(p, grid, stream, timing_start(c, rec),
                                          timing_stop(c, rec), use_arg ? jobs.data() : nullptr,
                                          use_arg ? table_bytes : 0);
        } else {
            e = launch_compress(p, stream,
                                bound_mode == kBoundPrepass ? nullptr : timing_start(c, rec),
                                timing_stop(c, rec));
        }
        if (e != hipSuccess) return hip_fail(e, "compress launch");
        c->ticket_next += ch.tiles;
        return KVSZP_OK;
    };
    // A recent give-up on this context: the schedule that needs no residency
    // for this call too (the device is likely still shared).
    bool schedule_safe = safe;
    if (!safe && !f32 && c->safe_left > 0) {
        c->safe_left -= 1;
        c->safe_calls += 1;
        schedule_safe = true;
    }
    for (size_t k = 0; k < chunks.size(); ++k)
        if ((rc = launch_chunk(k, schedule_safe, true))) return rc;

    // The encoder wrote sizes and bounds into pinned host memory; wait for it,
    // since callers need the sizes on the host (cuszp_wrapper.cpp:520-532).
    hipError_t e = wait_stream(stream);
    if (e != hipSuccess) return hip_fail(e, "waiting for the encoder");
    if (__atomic_load_n(&c->host_ctl[kHostAbort], __ATOMIC_ACQUIRE) == seq) {
        // A bounded wait gave up (the device was shared): encode those
        // launches again with the schedule that needs no residency, under
        // fresh epochs.
        for (size_t k = 0; k < chunks.size(); ++k)
            if (redo_candidate[k] && (rc = launch_chunk(k, true, false))) return rc;
        e = wait_stream(stream);
        if (e != hipSuccess) return hip_fail(e, "waiting for the encoder");
        c->redone += 1;
        c->safe_left = c->safe_after_abort;
    }
    rc = consume_device_error(c, stream);
    if (rc) return rc;
    for (size_t i = 0; i < batch; ++i) {
        sizes_out[i] = host_sizes[i];
        bounds_out[i] = relative ? host_bounds[i] : jobs[i].eps;
    }
    if (__atomic_load_n(&c->host_ctl[kHostOverflow], __ATOMIC_ACQUIRE) == seq) {
        // Jobs whose staged payload overflowed in the persistent encoder
        // (rates near 31 throughout): those jobs again, one workgroup per tile.
        std::vector<const void*> in;
        std::vector<void*> out;
        std::vector<uint64_t> cap;
        std::vector<float> eps;
        std::vector<size_t> where;
        std::vector<GroupSpec> sub;
        size_t j = 0;
        for (size_t gi = 0; gi < specs.size(); ++gi) {
            // the marked jobs of a group form one group of the new call
            bool open = false;
            for (uint32_t k = 0; k < specs[gi].jobs; ++k, ++j) {
                if (host_redo[j] != seq) continue;
                if (!open) {
                    sub.push_back(specs[gi]);
                    sub.back().jobs = 0;
                    open = true;
                }
                sub.back().jobs += 1;
                in.push_back(inputs[j]);
                out.push_back(outputs[j]);
                cap.push_back(capacities ? capacities[j] : ~0ull);
                // the bound the launch worked out for the job (its first
                // tile wrote it), so that the new launch needs no pre-pass
                eps.push_back(bounds_out[j]);
                where.push_back(j);
            }
        }
        if (!where.empty()) {
            std::vector<uint64_t> sz(where.size());
            std::vector<float> eb(where.size());
            rc = compress_groups(c, in.data(), out.data(), cap.data(), eps.data(),
                                 where.size(), sub, stream, sz.data(), eb.data(), f32, true,
                                 mode, true);
            if (rc) return rc;
            for (size_t k = 0; k < where.size(); ++k) {
                sizes_out[where[k]] = sz[k];
                bounds_out[where[k]] = eb[k];
            }
            c->redone += 1;
        }
    }
    return KVSZP_OK;
}

// Common decompress path: `specs` are the groups, requests laid out group by
// group (one launch per kMaxGroups groups).  `f32`: fp32 values into
// contiguous per-job outputs (kDstLinear).
int decompress_groups(kvszp_ctx* c, const void* const* compressed,
                      const uint64_t* sizes, const float* bounds, size_t batch,
                      const std::vector<GroupSpec>& specs, int dst_kind,
                      const std::vector<uint16_t*>& dst_base,
                      const std::vector<uint16_t*>& dest_table, uint64_t dpp,
                      uint64_t epd, bool aligned16, hipStream_t stream,
                      bool f32 = false, uint32_t grid_cap = 0, int mode = kModeFixed) {
    int rc = use_device(c);
    if (rc) return rc;
    if (specs.empty()) return fail(KVSZP_EINVAL, "no groups");
    std::vector<DecompressJob> jobs(batch);
    size_t job = 0;
    for (size_t gi = 0; gi < specs.size(); ++gi) {
        const GroupSpec& spec = specs[gi];
        if (spec.n == 0 || spec.n > kMaxElements)
            return fail(KVSZP_EINVAL, "segment of %llu elements unsupported",
                        (unsigned long long)spec.n);
        const uint32_t R = header_bytes_of(spec.n);
        for (uint32_t k = 0; k < spec.jobs; ++k, ++job) {
            if (job >= batch) return fail(KVSZP_EINVAL, "group sizes exceed batch");
            const size_t i = job;
            const uintptr_t in = (uintptr_t)compressed[i];
            // cuszp_wrapper.cpp:1077: a zero size is rejected.  A stream shorter
            // than its own header cannot be decoded either.
            if (!in || sizes[i] == 0)
                return fail(KVSZP_EINVAL, "invalid compressed page %zu", i);
            if (sizes[i] < R)
                return fail(KVSZP_EINVAL, "stream %zu (%llu bytes) shorter than its "
                            "%u-byte header", i, (unsigned long long)sizes[i], R);
            if (sizes[i] > 0xFFFFFFFFull)
                return fail(KVSZP_EINVAL, "stream %zu too large", i);
            if (in & 3u)
                return fail(KVSZP_EINVAL, "compressed buffer %zu not 4-byte aligned", i);
            jobs[i].in = reinterpret_cast<const uint8_t*>(in);
            jobs[i].dst = dst_kind == kDstMulti ? nullptr : dst_base[i];
            jobs[i].eb = bounds[i];
            jobs[i].size = (uint32_t)sizes[i];
        }
    }
    if (job != batch) return fail(KVSZP_EINVAL, "group sizes do not cover the batch");
    const std::vector<Chunk> chunks = split_chunks(specs);
    uint64_t max_tiles = 0;
    for (const Chunk& ch : chunks) {
        if (ch.tiles > kMaxTiles) return fail(KVSZP_EINVAL, "batch too large for one launch");
        max_tiles = std::max(max_tiles, ch.tiles);
    }

    // Large single-launch batches: persistent-decoder runs balanced job by
    // job (each job weighs its BF16 output plus its payload, spread evenly
    // over its tiles), so that pages of very different rates (all-zero,
    // constant, heavy-tailed) do not leave some workgroups with several
    // times the bytes of others.  Smaller batches keep the per-group
    // weights: their table copy stays small.
    std::vector<uint32_t> runs;
    // The persistent decoder walks runs of tiles; a launch with at most one
    // tile per resident workgroup (and no grid cap) gains nothing from runs
    // and decodes one workgroup per tile instead, each tile finding its
    // offset by look-back rather than by summing the header words of all the
    // job's earlier tiles (config 0, two jobs of 128 tiles: the decoder
    // 9.3-9.9 us against 10.2-10.7 us).
    auto persistent_for = [&](uint64_t tiles) {
        return c->decompress_grid != 0 && !f32 && (grid_cap != 0 || tiles > c->decompress_grid);
    };
    const bool persistent = chunks.size() == 1 && persistent_for(chunks[0].tiles);
    if (persistent && batch >= kJobBalancedRuns && chunks[0].tiles > 0) {
        uint32_t grid = (uint32_t)std::min<uint64_t>(chunks[0].tiles, c->decompress_grid);
        if (grid_cap) grid = std::min(grid, grid_cap);
        runs = job_balanced_runs(specs, sizes, batch, chunks[0].tiles, grid);
    }

    // Packed table: jobs, then (kDstMulti) the destination pointers, then
    // the run starts.
    const size_t jobs_bytes = (batch * sizeof(DecompressJob) + 255) & ~(size_t)255;
    const size_t dests_bytes = dest_table.size() * sizeof(uint16_t*);
    const size_t runs_off = (jobs_bytes + dests_bytes + 15) & ~(size_t)15;
    if ((rc = ensure(c->tile_state, max_tiles * 8, true, stream))) return rc;
    const uint32_t seq = ++c->seq;
    // Small calls without a destination table or run starts pass their job
    // table in the kernel arguments (no upload), and so does a persistent
    // launch whose job table (no destination table, no run starts) fits an
    // ArgTable.  Only the other calls build and upload the packed table.
    const bool inline_jobs =
        batch <= (size_t)kInlineJobs && dest_table.empty() && runs.empty();
    const size_t job_bytes = batch * sizeof(DecompressJob);
    const bool arg_table = !inline_jobs && (c->arg_tables & 2) && persistent &&
                           dest_table.empty() && runs.empty() && job_bytes <= kArgTableBytes;
    if (!inline_jobs && !arg_table) {
        std::vector<char> table(runs.empty() ? jobs_bytes + dests_bytes
                                             : runs_off + runs.size() * sizeof(uint32_t));
        std::memcpy(table.data(), jobs.data(), batch * sizeof(DecompressJob));
        if (!dest_table.empty())
            std::memcpy(table.data() + jobs_bytes, dest_table.data(), dests_bytes);
        if (!runs.empty())
            std::memcpy(table.data() + runs_off, runs.data(), runs.size() * sizeof(uint32_t));
        if ((rc = upload_tables(c, table.data(), table.size(), seq, stream))) return rc;
    }

    size_t first_job = 0;
    for (const Chunk& ch : chunks) {
        DecompressParams p;
        std::memset(&p, 0, sizeof(p));
        p.num_groups = fill_groups(p.groups, specs, ch, first_job);
        // Persistent decoder: per-group tile weights (BF16 output plus the
        // group's average payload per tile), so that workgroups holding tiles
        // of a high-rate group get fewer of them.  Kernel arguments only: the
        // table keeps its size.
        p.total_weight = group_tile_weights(p.groups, p.num_groups, specs, ch, sizes,
                                            p.weight_before, p.tile_weight);
        for (size_t gi = ch.g0; gi < ch.g1; ++gi) first_job += specs[gi].jobs;
        if (ch.tiles == 0) continue;
        uint32_t epoch;
        if ((rc = next_epoch(c, stream, &epoch))) return rc;
        p.jobs = reinterpret_cast<const DecompressJob*>(c->tables.ptr);
        p.num_jobs = (uint32_t)batch;
        if (inline_jobs) {
            p.jobs_inline = 1;
            std::memcpy(p.inline_jobs, jobs.data(), batch * sizeof(DecompressJob));
        } else if (arg_table) {
            p.jobs_inline = 2;
        }
        p.dests = reinterpret_cast<uint16_t* const*>(
            reinterpret_cast<char*>(c->tables.ptr) + jobs_bytes);
        if (!runs.empty())
            p.run_starts = reinterpret_cast<const uint32_t*>(
                reinterpret_cast<char*>(c->tables.ptr) + runs_off);
        p.tile_state = reinterpret_cast<unsigned long long*>(c->tile_state.ptr);
        p.error = decode_error_word(c);
        p.error_marker = decode_error_marker(c);
        p.host_ctl = c->host_ctl;
        p.seq = seq;
        p.ticket = c->use_tickets ? c->control : nullptr;
        p.ticket_base = c->ticket_next;
        p.epoch = epoch;
        p.total_tiles = (uint32_t)ch.tiles;
        p.dst_kind = dst_kind;
        p.rate0_zero = c->rate0 == KVSZP_RATE0_ZERO ? 1 : 0;
        p.aligned16 = aligned16 ? 1 : 0;
        p.output_f32 = f32 ? 1 : 0;
        p.mode = f32 ? mode : kModeFixed;
        p.dests_per_page = dpp;
        p.elements_per_dest = epd;
        const int rec = timing_begin(c, KVSZP_KERNEL_DECOMPRESS);
        hipError_t e;
        if (persistent_for(ch.tiles)) {
            p.ticket = nullptr;
            uint32_t grid = (uint32_t)std::min<uint64_t>(ch.tiles, c->decompress_grid);
            if (grid_cap) grid = std::min(grid, grid_cap);
            if (!runs.empty() && runs.size() != (size_t)grid + 1)
                return fail(KVSZP_EINVAL, "decoder run table for %zu workgroups, launch of %u",
                            runs.size() - 1, grid);
            e = launch_decompress_persistent(p, grid, stream, timing_start(c, rec),
                                             timing_stop(c, rec),
                                             arg_table ? jobs.data() : nullptr,
                                             arg_table ? job_bytes : 0);
        } else {
            e = launch_decompress(p, stream, timing_start(c, rec), timing_stop(c, rec));
        }
        if (e != hipSuccess) return hip_fail(e, "decompress launch");
        c->ticket_next += ch.tiles;
    }
    return KVSZP_OK;
}

}  // namespace

extern "C" {

int kvszp_create(const kvszp_config* config, int device_id, kvszp_ctx** out) {
    if (!out) return fail(KVSZP_EINVAL, "null output handle");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device_id < 0 || device_id >= count)
        return fail(KVSZP_EINVAL, "device %d not present (%d devices)", device_id, count);
    e = hipSetDevice(device_id);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    kvszp_ctx* c = new kvszp_ctx();
    if (config) {
        c->config = *config;
    } else {  // CompressionConfig defaults, cuszp_wrapper.h:11-17
        c->config.error_bound = 1e-4f;
        c->config.use_relative_error = 1;
        c->config.processing_dim = KVSZP_DIM_1D;
        c->config.encoding_mode = KVSZP_MODE_PLAIN;
        c->config.data_type = KVSZP_TYPE_FLOAT;
    }
    c->device = device_id;
    {
        const char* env = std::getenv("KVSZP_TICKETS");
        c->use_tickets = env && env[0] == '1';
        const char* at = std::getenv("KVSZP_ARG_TABLES");
        c->arg_tables = at ? std::atoi(at) & 3 : 3;
        int khz = 0;
        if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device_id) !=
                hipSuccess || khz <= 0)
            khz = 100000;  // the steady counter of gfx9 parts runs at 100 MHz
        c->clock_khz = (uint32_t)khz;
        const char* us = std::getenv("KVSZP_WAIT_US");
        const double wait_us = us ? std::atof(us) : 200.0;
        c->wait_ticks = (uint64_t)(std::min(kMaxWaitMicros, std::max(0.0, wait_us)) * khz /
                                   1000.0);
        if (const char* sc = std::getenv("KVSZP_SAFE_CALLS")) {
            const long v = std::atol(sc);
            c->safe_after_abort = (uint32_t)std::max(0L, std::min(v, 1L << 20));
        }
        if (const char* lim = std::getenv("KVSZP_EPOCH_LIMIT")) {
            const long v = std::atol(lim);
            if (v >= 2) c->epoch_limit = (uint32_t)std::min<long>(v, kEpochLimit);
        }
    }
    e = hipMalloc(&c->control, 64);
    if (e == hipSuccess) e = hipMemset(c->control, 0, 64);
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&c->host_ctl),
                          kHostCtlWords * sizeof(uint32_t), hipHostMallocCoherent);
    if (e == hipSuccess) std::memset(c->host_ctl, 0, kHostCtlWords * sizeof(uint32_t));
    if (e != hipSuccess) {
        kvszp_destroy(c);
        return hip_fail(e, "context setup");
    }
    // No-allocation entry point: the device's scratch array and the pinned
    // areas its calls use, so that those calls allocate nothing.
    {
        void* sp = nullptr;
        e = scratch_address(device_id, &sp);
        if (e == hipSuccess)
            e = hipHostMalloc(reinterpret_cast<void**>(&c->noalloc_stage),
                              sizeof(CompressJob) * kNoAllocMaxJobs, hipHostMallocDefault);
        if (e == hipSuccess)
            e = hipHostMalloc(&c->noalloc_results, 12ull * kNoAllocMaxJobs,
                              hipHostMallocCoherent);
        if (e == hipSuccess) std::memset(c->noalloc_results, 0, 12ull * kNoAllocMaxJobs);
        if (e != hipSuccess) {
            kvszp_destroy(c);
            return hip_fail(e, "scratch setup");
        }
        c->scratch = static_cast<unsigned char*>(sp);
    }
    // Tiles of one job wait for each other in the fused relative-bound
    // exchange, so a job may use it only if all its tiles fit on the device
    // at once with a wide margin.
    const int resident = compress_resident_workgroups(device_id, false);
    c->fused_tile_limit = (uint32_t)std::min(kThreads, std::max(0, resident / 4));
    {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_id) ==
                hipSuccess && cus > 0)
            c->cus = (uint32_t)cus;
        if (const char* mix = std::getenv("KVSZP_SLOT_MIX"))
            c->slot_mix = mix[0] == '0' ? 0 : mix[0] == '2' ? 2 : 1;
        const char* env = std::getenv("KVSZP_PERSISTENT");
        const bool off = (env && env[0] == '0') || c->use_tickets;
        c->pipelined_grid =
            off ? 0u : (uint32_t)std::max(0, compress_resident_workgroups(device_id, true));
        c->decompress_grid =
            off ? 0u : (uint32_t)std::max(0, decompress_resident_workgroups(device_id));
    }
    if (const char* dbg = std::getenv("KVSZP_DEBUG"); dbg && dbg[0] == '1')
        std::fprintf(stderr, "kvszp: device %d resident encoder workgroups %d, "
                     "fused tile limit %u, persistent grids %u / %u\n", device_id,
                     resident, c->fused_tile_limit, c->pipelined_grid,
                     c->decompress_grid);
    *out = c;
    return KVSZP_OK;
}

int kvszp_destroy(kvszp_ctx* c) {
    if (!c) return KVSZP_OK;
    (void)hipSetDevice(c->device);
    // Launches of this context may still be queued or running; they read the
    // staging slots and write the host control block.
    if (c->seq != 0) (void)hipDeviceSynchronize();
    for (auto& s : c->slots)
        if (s.host) (void)hipHostFree(s.host);
    for (auto& r : c->timed) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    for (hipEvent_t ev : c->spare_events) (void)hipEventDestroy(ev);
    DevBuf* bufs[5] = {&c->tile_state, &c->tile_minmax, &c->job_minmax,
                       &c->job_flags, &c->tables};
    for (DevBuf* b : bufs)
        if (b->ptr) (void)hipFree(b->ptr);
    if (c->control) (void)hipFree(c->control);
    if (c->host_results) (void)hipHostFree(c->host_results);
    if (c->host_ctl) (void)hipHostFree(c->host_ctl);
    if (c->noalloc_stage) (void)hipHostFree(c->noalloc_stage);
    if (c->noalloc_results) (void)hipHostFree(c->noalloc_results);
    delete c;
    return KVSZP_OK;
}

int kvszp_get_config(const kvszp_ctx* c, kvszp_config* out) {
    if (!c || !out) return fail(KVSZP_EINVAL, "null argument");
    *out = c->config;
    return KVSZP_OK;
}

int kvszp_update_config(kvszp_ctx* c, const kvszp_config* config) {
    if (!c || !config) return fail(KVSZP_EINVAL, "null argument");
    c->config = *config;
    return KVSZP_OK;
}

int kvszp_set_options(kvszp_ctx* c, int quantizer, int rate0_policy) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (quantizer != KVSZP_QUANT_TWO_ROUNDINGS && quantizer != KVSZP_QUANT_FUSED)
        return fail(KVSZP_EINVAL, "unknown quantizer %d", quantizer);
    if (rate0_policy != KVSZP_RATE0_SKIP && rate0_policy != KVSZP_RATE0_ZERO)
        return fail(KVSZP_EINVAL, "unknown rate-0 policy %d", rate0_policy);
    c->quantizer = quantizer;
    c->rate0 = rate0_policy;
    return KVSZP_OK;
}

int kvszp_set_wait_bound(kvszp_ctx* c, double microseconds) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (!(microseconds >= 0.0 && microseconds <= kMaxWaitMicros))
        return fail(KVSZP_EINVAL, "wait bound %g us outside [0, %g]", microseconds,
                    kMaxWaitMicros);
    c->wait_ticks = (uint64_t)(microseconds * c->clock_khz / 1000.0);
    return KVSZP_OK;
}

size_t kvszp_estimate_compressed_buffer_size(size_t original_size) {
    return original_size * 2;
}

size_t kvszp_header_bytes(size_t num_elements) { return header_bytes_of(num_elements); }

int kvszp_compress_batch_fixed_bf16(kvszp_ctx* c, const void* const* inputs,
                                    void* const* outputs,
                                    const uint64_t* capacities,
                                    const float* eps_overrides, size_t batch,
                                    size_t num_elements, kvszp_stream_t stream,
                                    uint64_t* sizes_out, float* bounds_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    std::vector<GroupSpec> specs(1);
    specs[0] = GroupSpec{num_elements, nullptr, 0, 0, 0, (uint32_t)batch};
    return compress_groups(c, inputs, outputs, capacities, eps_overrides, batch,
                           specs, (hipStream_t)stream, sizes_out, bounds_out);
}

// Epoch tags of the words in each device's scratch array.  All contexts on
// a device share the array, so the tags come from one counter per device:
// no two calls on a device use the same tag, and a wrap clears the tagged
// words first.
static std::mutex g_scratch_epoch_mutex;
static uint32_t g_scratch_epoch[64];

static int scratch_epoch(kvszp_ctx* c, hipStream_t stream, uint32_t* epoch) {
    std::lock_guard<std::mutex> lock(g_scratch_epoch_mutex);
    uint32_t& cur = g_scratch_epoch[c->device];
    if (cur >= c->epoch_limit) {
        // Every tagged word: look-back, min/max, flags and the abort word.
        hipError_t e = launch_fill_u64(reinterpret_cast<unsigned long long*>(c->scratch),
                                       kScratchJobs / 8, stream);
        if (e == hipSuccess)
            e = launch_fill_u64(reinterpret_cast<unsigned long long*>(c->scratch +
                                                                     kScratchJobFlags),
                                (kScratchBytes - kScratchJobFlags) / 8, stream);
        if (e != hipSuccess) return hip_fail(e, "clearing the scratch words");
        cur = 0;
    }
    *epoch = ++cur;
    return KVSZP_OK;
}

int kvszp_compress_batch_fixed_bf16_noalloc(
    kvszp_ctx* c, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const float* eps_overrides, size_t batch,
    size_t num_elements, kvszp_stream_t stream_handle, uint64_t* sizes_out,
    float* bounds_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    hipStream_t stream = (hipStream_t)stream_handle;
    int rc = check_fixed_config(c);
    if (rc) return rc;
    if (batch == 0) return fail(KVSZP_EINVAL, "empty batch");
    if (!inputs || !outputs || !sizes_out || !bounds_out)
        return fail(KVSZP_EINVAL, "null pointer argument");
    const uint64_t n = num_elements;
    if (n == 0 || n > kMaxElements)
        return fail(KVSZP_EINVAL, "segment of %llu elements unsupported",
                    (unsigned long long)n);
    const uint32_t tiles_per_job = (uint32_t)((n + kTileElems - 1) / kTileElems);
    if (batch > kNoAllocMaxJobs || (uint64_t)tiles_per_job * batch > kNoAllocMaxTiles)
        return fail(KVSZP_EINVAL,
                    "no-allocation compress takes at most %u pages and %u tiles of "
                    "8192 values per call (got %zu pages, %llu tiles)",
                    kNoAllocMaxJobs, kNoAllocMaxTiles, batch,
                    (unsigned long long)tiles_per_job * batch);
    rc = use_device(c);
    if (rc) return rc;
    const uint64_t need = std::max<uint64_t>(8ull * n, header_bytes_of(n) + 128ull * ((n + 31) / 32));
    bool aligned16 = true;
    for (size_t i = 0; i < batch; ++i) {
        const uintptr_t in = (uintptr_t)inputs[i], out = (uintptr_t)outputs[i];
        if (!in || !out) return fail(KVSZP_EINVAL, "null page pointer %zu", i);
        if (in & 1u) return fail(KVSZP_EINVAL, "input %zu not 2-byte aligned", i);
        if (out & 3u) return fail(KVSZP_EINVAL, "compressed buffer %zu not 4-byte aligned", i);
        if (capacities && capacities[i] < need)
            return fail(KVSZP_EINVAL, "compressed buffer %zu holds %llu bytes, needs %llu", i,
                        (unsigned long long)capacities[i], (unsigned long long)need);
        if (in & 15u) aligned16 = false;
        CompressJob& j = c->noalloc_stage[i];
        j.in = reinterpret_cast<const uint16_t*>(in);
        j.out = reinterpret_cast<uint8_t*>(out);
        j.eps = (eps_overrides && eps_overrides[i] > 0.0f) ? eps_overrides[i]
                                                          : c->config.error_bound;
        j.reserved = 0;
    }
    // The previous call on this context waited for its kernels, so the
    // staging records are free; the copy goes into the scratch job table.
    CompressJob* djobs = reinterpret_cast<CompressJob*>(c->scratch + kScratchJobs);
    // Small calls pass the job table in the kernel arguments instead.
    const bool inline_jobs = batch <= (size_t)kInlineJobs;
    hipError_t e = hipSuccess;
    if (!inline_jobs) {
        e = hipMemcpyAsync(djobs, c->noalloc_stage, batch * sizeof(CompressJob),
                           hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(H2D job table)");
    }
    uint32_t epoch;
    if ((rc = scratch_epoch(c, stream, &epoch))) return rc;

    const bool relative = c->config.use_relative_error != 0;
    const bool whole_blocks = (n % kBlockElems) == 0;
    const uint32_t seq = ++c->seq;
    CompressParams p;
    std::memset(&p, 0, sizeof(p));
    Group& g = p.groups[0];
    g.n = n;
    g.first_job = 0;
    g.first_tile = 0;
    g.tiles_per_job = tiles_per_job;
    g.header_bytes = header_bytes_of(n);
    set_group_divisors(g);
    p.num_groups = 1;
    // After a recent give-up, the schedule that needs no residency at once.
    const bool schedule_safe = c->safe_left > 0;
    if (schedule_safe) {
        c->safe_left -= 1;
        c->safe_calls += 1;
    }
    const int bound_mode =
        !relative ? kBoundAbsolute
                  : (!schedule_safe && tiles_per_job <= c->fused_tile_limit ? kBoundFused
                                                                            : kBoundPrepass);
    uint32_t* host_sizes = reinterpret_cast<uint32_t*>(c->noalloc_results);
    float* host_bounds = reinterpret_cast<float*>(host_sizes + kNoAllocMaxJobs);
    uint32_t* host_redo = host_sizes + 2 * kNoAllocMaxJobs;
    unsigned long long* words = reinterpret_cast<unsigned long long*>(c->scratch);
    if (bound_mode == kBoundPrepass) {
        MinMaxParams m;
        std::memset(&m, 0, sizeof(m));
        m.jobs = djobs;
        m.num_jobs = (uint32_t)batch;
        if (inline_jobs) {
            m.jobs_inline = 1;
            std::memcpy(m.inline_jobs, c->noalloc_stage, batch * sizeof(CompressJob));
        }
        m.job_minmax = words + kScratchJobMinMax / 8;
        m.error = error_word(c);
        m.error_marker = error_marker(c);
        m.host_ctl = c->host_ctl;
        m.seq = seq;
        m.epoch = epoch;
        m.num_groups = 1;
        m.groups[0] = g;
        e = launch_minmax(m, tiles_per_job * (uint32_t)batch, stream, nullptr);
        if (e != hipSuccess) return hip_fail(e, "minmax launch");
    }
    p.jobs = djobs;
    p.num_jobs = (uint32_t)batch;
    if (inline_jobs) {
        p.jobs_inline = 1;
        std::memcpy(p.inline_jobs, c->noalloc_stage, batch * sizeof(CompressJob));
    }
    p.tile_state = words + kScratchTileState / 8;
    p.tile_minmax = words + kScratchTileMinMax / 8;
    p.job_minmax = words + kScratchJobMinMax / 8;
    p.host_sizes = host_sizes;
    p.host_bounds = host_bounds;
    p.host_redo = host_redo;
    p.job_flags = reinterpret_cast<uint32_t*>(c->scratch + kScratchJobFlags);
    p.error = error_word(c);
    p.error_marker = error_marker(c);
    p.host_ctl = c->host_ctl;
    p.seq = seq;
    p.epoch = epoch;
    p.total_tiles = tiles_per_job * (uint32_t)batch;
    p.bound_mode = bound_mode;
    p.quantizer = c->quantizer;
    p.aligned16 = aligned16 ? 1 : 0;
    const bool persistent = !schedule_safe && bound_mode != kBoundPrepass &&
                            c->pipelined_grid != 0 && whole_blocks && aligned16 &&
                            tiles_per_job <= c->pipelined_grid / 2;
    if (persistent || bound_mode == kBoundFused) {
        p.abort_word = words + kScratchAbort / 8;
        p.wait_ticks = c->wait_ticks;
    }
    if (persistent) {
        const uint32_t grid = (uint32_t)std::min<uint64_t>(p.total_tiles, c->pipelined_grid);
        p.slot_cus = persistent_slot_cus(p.total_tiles, grid, c->cus, c->slot_mix);
        e = launch_compress_pipelined(p, grid, stream, nullptr, nullptr);
    } else
        e = launch_compress(p, stream, nullptr, nullptr);
    if (e != hipSuccess) return hip_fail(e, "compress launch");
    e = wait_stream(stream);
    if (e != hipSuccess) return hip_fail(e, "waiting for the encoder");
    const bool gave_up = p.abort_word != nullptr &&
                         __atomic_load_n(&c->host_ctl[kHostAbort], __ATOMIC_ACQUIRE) == seq;
    if (gave_up) c->safe_left = c->safe_after_abort;
    if (p.abort_word != nullptr &&
        (gave_up || __atomic_load_n(&c->host_ctl[kHostOverflow], __ATOMIC_ACQUIRE) == seq)) {
        // Staging overflow, or a bounded wait gave up: the schedule that
        // needs no residency (pre-pass bound, one workgroup per tile).
        if ((rc = scratch_epoch(c, stream, &epoch))) return rc;
        p.epoch = epoch;
        p.abort_word = nullptr;
        if (relative) {
            p.bound_mode = kBoundPrepass;
            MinMaxParams m;
            std::memset(&m, 0, sizeof(m));
            m.jobs = djobs;
            m.num_jobs = (uint32_t)batch;
            if (inline_jobs) {
                m.jobs_inline = 1;
                std::memcpy(m.inline_jobs, c->noalloc_stage, batch * sizeof(CompressJob));
            }
            m.job_minmax = words + kScratchJobMinMax / 8;
            m.error = error_word(c);
            m.error_marker = error_marker(c);
            m.host_ctl = c->host_ctl;
            m.seq = seq;
            m.epoch = epoch;
            m.num_groups = 1;
            m.groups[0] = g;
            e = launch_minmax(m, p.total_tiles, stream, nullptr);
            if (e != hipSuccess) return hip_fail(e, "minmax launch");
        }
        e = launch_compress(p, stream, nullptr, nullptr);
        if (e != hipSuccess) return hip_fail(e, "compress launch");
        e = wait_stream(stream);
        if (e != hipSuccess) return hip_fail(e, "waiting for the encoder");
        c->redone += 1;
    }
    rc = consume_device_error(c, stream);
    if (rc) return rc;
    for (size_t i = 0; i < batch; ++i) {
        sizes_out[i] = host_sizes[i];
        bounds_out[i] = relative ? host_bounds[i] : c->noalloc_stage[i].eps;
    }
    return KVSZP_OK;
}

int kvszp_compress_batch_fixed_bf16_indexed(
    kvszp_ctx* c, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const int64_t* layer_indices,
    size_t selected_layers, size_t prefix_count, size_t source_layers,
    size_t elements_per_layer, const float* eps_overrides, size_t batch,
    kvszp_stream_t stream, uint64_t* sizes_out, float* bounds_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    int rc = validate_layers(layer_indices, selected_layers, prefix_count,
                             source_layers, elements_per_layer);
    if (rc) return rc;
    std::vector<GroupSpec> specs(1);
    specs[0] = GroupSpec{(uint64_t)prefix_count * selected_layers * elements_per_layer,
                         layer_indices, selected_layers, source_layers,
                         elements_per_layer, (uint32_t)batch};
    return compress_groups(c, inputs, outputs, capacities, eps_overrides, batch,
                           specs, (hipStream_t)stream, sizes_out, bounds_out);
}

int kvszp_compress_batch_fixed_bf16_indexed_groups(
    kvszp_ctx* c, const void* const* inputs, void* const* outputs,
    const uint64_t* capacities, const int64_t* const* layer_indices,
    const size_t* selected_layers, const size_t* group_sizes,
    size_t num_groups, size_t prefix_count, size_t source_layers,
    size_t elements_per_layer, const float* eps_overrides, size_t batch,
    kvszp_stream_t stream, uint64_t* sizes_out, float* bounds_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (num_groups == 0 || !layer_indices || !selected_layers || !group_sizes)
        return fail(KVSZP_EINVAL, "empty group list");
    std::vector<GroupSpec> specs;
    uint64_t covered = 0;
    for (size_t gi = 0; gi < num_groups; ++gi) {
        // cuszp_wrapper.cpp:717-743.
        if (group_sizes[gi] == 0)
            return fail(KVSZP_EINVAL, "group %zu is empty", gi);
        int rc = validate_layers(layer_indices[gi], selected_layers[gi],
                                 prefix_count, source_layers, elements_per_layer);
        if (rc) return rc;
        specs.push_back(GroupSpec{
            (uint64_t)prefix_count * selected_layers[gi] * elements_per_layer,
            layer_indices[gi], selected_layers[gi], source_layers,
            elements_per_layer, (uint32_t)group_sizes[gi]});
        covered += group_sizes[gi];
    }
    if (covered != batch)
        return fail(KVSZP_EINVAL, "group sizes sum to %llu, batch is %zu",
                    (unsigned long long)covered, batch);
    return compress_groups(c, inputs, outputs, capacities, eps_overrides, batch,
                           specs, (hipStream_t)stream, sizes_out, bounds_out);
}

int kvszp_decompress_batch_fixed_bf16(kvszp_ctx* c, const void* const* compressed,
                                      const uint64_t* sizes,
                                      const float* error_bounds, size_t batch,
                                      void* output, size_t output_elements,
                                      size_t num_elements_per_page,
                                      kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;  // cuszp_wrapper.cpp:1042
    int rc = check_fixed_config(c);
    if (rc) return rc;
    if (!compressed || !sizes || !error_bounds || !output ||
        num_elements_per_page == 0 ||
        output_elements < batch * num_elements_per_page)
        return fail(KVSZP_EINVAL, "invalid fixed BF16 batch metadata");
    if ((uintptr_t)output & 1u) return fail(KVSZP_EINVAL, "output not 2-byte aligned");
    std::vector<uint16_t*> base(batch);
    for (size_t i = 0; i < batch; ++i)
        base[i] = reinterpret_cast<uint16_t*>(output) + i * num_elements_per_page;
    const bool aligned16 =
        ((uintptr_t)output & 15u) == 0 && (num_elements_per_page % 8) == 0;
    const std::vector<GroupSpec> spec{
        GroupSpec{num_elements_per_page, nullptr, 0, 0, 0, (uint32_t)batch}};
    return decompress_groups(c, compressed, sizes, error_bounds, batch, spec,
                             kDstLinear, base, {}, 0, 0, aligned16,
                             (hipStream_t)stream);
}

int kvszp_decompress_batch_fixed_bf16_scatter(
    kvszp_ctx* c, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    size_t num_elements_per_page, size_t destinations_per_page,
    size_t elements_per_destination, kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;  // cuszp_wrapper.cpp:1121
    int rc = check_fixed_config(c);
    if (rc) return rc;
    // cuszp_wrapper.cpp:1123-1133.
    if (!compressed || !sizes || !error_bounds || !destinations ||
        destinations_per_page == 0 || elements_per_destination == 0 ||
        num_elements_per_page != destinations_per_page * elements_per_destination)
        return fail(KVSZP_EINVAL, "invalid direct-scatter metadata");
    const size_t count = batch * destinations_per_page;
    std::vector<uint16_t*> dests(count);
    bool aligned16 = true;
    for (size_t i = 0; i < count; ++i) {
        const uintptr_t d = (uintptr_t)destinations[i];
        if (!d || (d & 1u))
            return fail(KVSZP_EINVAL, "invalid BF16 direct-scatter destination %zu", i);
        if (d & 15u) aligned16 = false;
        dests[i] = reinterpret_cast<uint16_t*>(d);
    }
    const std::vector<GroupSpec> spec{
        GroupSpec{num_elements_per_page, nullptr, 0, 0, 0, (uint32_t)batch}};
    if (destinations_per_page == 1) {
        // One destination per page: straight 16-byte stores into the page
        // (cu:383-386, 566-576).
        return decompress_groups(c, compressed, sizes, error_bounds, batch, spec,
                                 kDstLinear, dests, {}, 0, 0,
                                 aligned16 && (num_elements_per_page % 8) == 0,
                                 (hipStream_t)stream);
    }
    return decompress_groups(c, compressed, sizes, error_bounds, batch, spec,
                             kDstMulti, {}, dests, destinations_per_page,
                             elements_per_destination, false, (hipStream_t)stream);
}

int kvszp_decompress_batch_fixed_bf16_indexed_scatter(
    kvszp_ctx* c, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    const int64_t* layer_indices, size_t selected_layers, size_t prefix_count,
    size_t source_layers, size_t elements_per_layer, kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;  // cuszp_wrapper.cpp:1227
    int rc = check_fixed_config(c);
    if (rc) return rc;
    rc = validate_layers(layer_indices, selected_layers, prefix_count,
                         source_layers, elements_per_layer);
    if (rc) return rc;
    if (!compressed || !sizes || !error_bounds || !destinations)
        return fail(KVSZP_EINVAL, "null pointer argument");
    std::vector<uint16_t*> dests(batch);
    for (size_t i = 0; i < batch; ++i) {
        const uintptr_t d = (uintptr_t)destinations[i];
        if (!d || (d & 1u))
            return fail(KVSZP_EINVAL, "invalid BF16 destination page %zu", i);
        dests[i] = reinterpret_cast<uint16_t*>(d);
    }
    const std::vector<GroupSpec> spec{
        GroupSpec{(uint64_t)prefix_count * selected_layers * elements_per_layer,
                  layer_indices, selected_layers, source_layers, elements_per_layer,
                  (uint32_t)batch}};
    return decompress_groups(c, compressed, sizes, error_bounds, batch, spec,
                             kDstIndexed, dests, {}, 0, 0, false,
                             (hipStream_t)stream);
}

int kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups(
    kvszp_ctx* c, const void* const* compressed, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    const int64_t* const* layer_indices, const size_t* selected_layers,
    const size_t* group_sizes, size_t num_groups, size_t prefix_count,
    size_t source_layers, size_t elements_per_layer, kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;
    int rc = check_fixed_config(c);
    if (rc) return rc;
    if (!compressed || !sizes || !error_bounds || !destinations)
        return fail(KVSZP_EINVAL, "null pointer argument");
    if (num_groups == 0 || !layer_indices || !selected_layers || !group_sizes)
        return fail(KVSZP_EINVAL, "empty group list");
    std::vector<GroupSpec> specs;
    uint64_t covered = 0;
    for (size_t gi = 0; gi < num_groups; ++gi) {
        if (group_sizes[gi] == 0)
            return fail(KVSZP_EINVAL, "group %zu is empty", gi);
        rc = validate_layers(layer_indices[gi], selected_layers[gi], prefix_count,
                             source_layers, elements_per_layer);
        if (rc) return rc;
        specs.push_back(GroupSpec{
            (uint64_t)prefix_count * selected_layers[gi] * elements_per_layer,
            layer_indices[gi], selected_layers[gi], source_layers,
            elements_per_layer, (uint32_t)group_sizes[gi]});
        covered += group_sizes[gi];
    }
    if (covered != batch)
        return fail(KVSZP_EINVAL, "group sizes sum to %llu, batch is %zu",
                    (unsigned long long)covered, batch);
    std::vector<uint16_t*> dests(batch);
    for (size_t i = 0; i < batch; ++i) {
        const uintptr_t d = (uintptr_t)destinations[i];
        if (!d || (d & 1u))
            return fail(KVSZP_EINVAL, "invalid BF16 destination page %zu", i);
        dests[i] = reinterpret_cast<uint16_t*>(d);
    }
    return decompress_groups(c, compressed, sizes, error_bounds, batch, specs,
                             kDstIndexed, dests, {}, 0, 0, false,
                             (hipStream_t)stream);
}

int kvszp_compress_fixed_f32(kvszp_ctx* c, const float* input, size_t num_elements,
                             void* output, uint64_t capacity, float eps_override,
                             kvszp_stream_t stream, uint64_t* size_out,
                             float* bound_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (num_elements == 0) return fail(KVSZP_EINVAL, "empty input");
    const void* in = input;
    void* out = output;
    const float eps = eps_override;  // <= 0: config.error_bound (cpp:241)
    std::vector<GroupSpec> specs{GroupSpec{num_elements, nullptr, 0, 0, 0, 1}};
    return compress_groups(c, &in, &out, &capacity, &eps, 1, specs,
                           (hipStream_t)stream, size_out, bound_out, true);
}

int kvszp_compress_batch_fixed_f32(kvszp_ctx* c, const void* const* inputs,
                                   void* const* outputs, const uint64_t* capacities,
                                   const float* eps_overrides, size_t batch,
                                   size_t num_elements, kvszp_stream_t stream,
                                   uint64_t* sizes_out, float* bounds_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    std::vector<GroupSpec> specs{
        GroupSpec{num_elements, nullptr, 0, 0, 0, (uint32_t)batch}};
    return compress_groups(c, inputs, outputs, capacities, eps_overrides, batch,
                           specs, (hipStream_t)stream, sizes_out, bounds_out, true);
}

// Contiguous fp32 outputs, one per request, grouped by equal length;
// `any_mode`: the context's encoding mode, else fixed mode only.
static int decompress_f32(kvszp_ctx* c, const void* const* compressed,
                          const uint64_t* sizes, const float* error_bounds,
                          size_t batch, void* const* outputs,
                          const uint64_t* num_elements, hipStream_t stream,
                          bool any_mode = false) {
    int rc = any_mode ? check_f32_config(c) : check_fixed_config(c);
    if (rc) return rc;
    if (!compressed || !sizes || !error_bounds || !outputs || !num_elements)
        return fail(KVSZP_EINVAL, "null pointer argument");
    std::vector<GroupSpec> specs;
    std::vector<uint16_t*> base(batch);
    bool aligned16 = true;
    for (size_t i = 0; i < batch; ++i) {
        const uintptr_t d = (uintptr_t)outputs[i];
        if (!d || (d & 3u)) return fail(KVSZP_EINVAL, "invalid fp32 output %zu", i);
        if (num_elements[i] == 0) return fail(KVSZP_EINVAL, "empty output %zu", i);
        if (d & 15u) aligned16 = false;
        base[i] = reinterpret_cast<uint16_t*>(d);
        if (specs.empty() || specs.back().n != num_elements[i])
            specs.push_back(GroupSpec{num_elements[i], nullptr, 0, 0, 0, 0});
        specs.back().jobs += 1;
    }
    return decompress_groups(c, compressed, sizes, error_bounds, batch, specs,
                             kDstLinear, base, {}, 0, 0, aligned16, stream, true, 0,
                             any_mode ? c->config.encoding_mode : kModeFixed);
}

int kvszp_decompress_fixed_f32(kvszp_ctx* c, const void* compressed,
                               uint64_t compressed_size, float* output,
                               size_t num_elements, float error_bound,
                               kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    void* out = output;
    const uint64_t n = num_elements;
    return decompress_f32(c, &compressed, &compressed_size, &error_bound, 1, &out, &n,
                          (hipStream_t)stream);
}

int kvszp_decompress_batch_fixed_f32(kvszp_ctx* c, const void* const* compressed,
                                     const uint64_t* sizes, const float* error_bounds,
                                     size_t batch, void* const* outputs,
                                     const uint64_t* num_elements,
                                     kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;  // cuszp_wrapper.cpp:950
    return decompress_f32(c, compressed, sizes, error_bounds, batch, outputs,
                          num_elements, (hipStream_t)stream);
}

int kvszp_compress_f32(kvszp_ctx* c, const float* input, size_t num_elements,
                       void* output, uint64_t capacity, float eps_override,
                       kvszp_stream_t stream, uint64_t* size_out, float* bound_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    int rc = check_f32_config(c);
    if (rc) return rc;
    if (num_elements == 0) return fail(KVSZP_EINVAL, "empty input");
    const void* in = input;
    void* out = output;
    const float eps = eps_override;  // <= 0: config.error_bound (cpp:241)
    std::vector<GroupSpec> specs{GroupSpec{num_elements, nullptr, 0, 0, 0, 1}};
    return compress_groups(c, &in, &out, &capacity, &eps, 1, specs,
                           (hipStream_t)stream, size_out, bound_out, true, false,
                           c->config.encoding_mode);
}

int kvszp_decompress_f32(kvszp_ctx* c, const void* compressed, uint64_t compressed_size,
                         float* output, size_t num_elements, float error_bound,
                         kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    void* out = output;
    const uint64_t n = num_elements;
    return decompress_f32(c, &compressed, &compressed_size, &error_bound, 1, &out, &n,
                          (hipStream_t)stream, true);
}

int kvszp_decompress_batch_f32(kvszp_ctx* c, const void* const* compressed,
                               const uint64_t* sizes, const float* error_bounds,
                               size_t batch, void* const* outputs,
                               const uint64_t* num_elements, kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;  // cuszp_wrapper.cpp:950
    return decompress_f32(c, compressed, sizes, error_bounds, batch, outputs,
                          num_elements, (hipStream_t)stream, true);
}

int kvszp_pack_streams(kvszp_ctx* c, const void* const* payloads, const uint64_t* sizes,
                       size_t count, void* slab, uint64_t slab_capacity,
                       kvszp_stream_t stream_handle, uint64_t* offsets_out,
                       uint64_t* packed_bytes_out) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    hipStream_t stream = (hipStream_t)stream_handle;
    if (count == 0) return fail(KVSZP_EINVAL, "nothing to pack");
    if (!payloads || !sizes || !slab || !offsets_out || !packed_bytes_out)
        return fail(KVSZP_EINVAL, "null pointer argument");
    int rc = use_device(c);
    if (rc) return rc;
    // vllm_v1_compressed_offload.py:385-392: start = align8(end of the
    // previous payload); the slab ends with the last payload.  Each payload
    // becomes pieces of at most kPackPiece bytes; the last piece of a
    // payload zeroes the gap to the next one.
    std::vector<PackJob> jobs;
    jobs.reserve(count);
    uint64_t end = 0;
    for (size_t i = 0; i < count; ++i) {
        if (sizes[i] && !payloads[i]) return fail(KVSZP_EINVAL, "null payload %zu", i);
        const uint64_t start = (end + 7) & ~7ull;
        if (sizes[i] && !jobs.empty())  // the gap behind the last piece written
            jobs.back().pad = start - (jobs.back().dst_off + jobs.back().size);
        const uint8_t* src = static_cast<const uint8_t*>(payloads[i]);
        for (uint64_t off = 0; off < sizes[i]; off += kPackPiece)
            jobs.push_back(PackJob{src + off, start + off,
                                   std::min<uint64_t>(kPackPiece, sizes[i] - off), 0});
        offsets_out[i] = start;
        end = start + sizes[i];
    }
    if (jobs.empty()) {  // nothing but empty payloads
        *packed_bytes_out = end;
        return KVSZP_OK;
    }
    if (end > slab_capacity)
        return fail(KVSZP_EINVAL, "slab holds %llu bytes, the packed payloads %llu",
                    (unsigned long long)slab_capacity, (unsigned long long)end);
    *packed_bytes_out = end;
    const uint32_t seq = ++c->seq;
    if ((rc = upload_tables(c, jobs.data(), jobs.size() * sizeof(PackJob), seq, stream)))
        return rc;
    PackParams p;
    p.jobs = reinterpret_cast<const PackJob*>(c->tables.ptr);
    p.dst = static_cast<uint8_t*>(slab);
    p.count = (uint32_t)jobs.size();
    p.host_ctl = c->host_ctl;
    p.seq = seq;
    // Writes into pinned host memory run at the link's rate from a few dozen
    // workgroups; more only take CUs from other work.
    const uint32_t grid = (uint32_t)std::min<size_t>(jobs.size(), 128);
    hipError_t e = launch_pack(p, grid, stream);
    if (e != hipSuccess) return hip_fail(e, "pack launch");
    // The slab is complete when the call returns (the reference synchronizes
    // after its device-to-host copy, :429-430).
    e = wait_stream(stream);
    if (e != hipSuccess) return hip_fail(e, "waiting for the pack");
    return KVSZP_OK;
}

int kvszp_decompress_batch_fixed_bf16_indexed_scatter_groups_packed(
    kvszp_ctx* c, const void* packed, uint64_t packed_bytes, void* staging,
    uint64_t staging_capacity, const uint64_t* offsets, const uint64_t* sizes,
    const float* error_bounds, size_t batch, void* const* destinations,
    const int64_t* const* layer_indices, const size_t* selected_layers,
    const size_t* group_sizes, size_t num_groups, size_t prefix_count,
    size_t source_layers, size_t elements_per_layer, kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (batch == 0) return KVSZP_OK;
    if (!packed || !offsets || !sizes || !error_bounds || !destinations)
        return fail(KVSZP_EINVAL, "null pointer argument");
    if (staging && packed_bytes > staging_capacity)
        return fail(KVSZP_EINVAL, "staging holds %llu bytes, the slab %llu",
                    (unsigned long long)staging_capacity, (unsigned long long)packed_bytes);
    if (num_groups == 0 || !layer_indices || !selected_layers || !group_sizes)
        return fail(KVSZP_EINVAL, "empty group list");
    int rc = check_fixed_config(c);
    if (rc) return rc;
    const uint8_t* base = static_cast<const uint8_t*>(staging ? staging : packed);
    std::vector<const void*> streams(batch);
    for (size_t i = 0; i < batch; ++i) {
        if (offsets[i] > packed_bytes || sizes[i] > packed_bytes - offsets[i])
            return fail(KVSZP_EINVAL, "payload %zu lies outside the slab", i);
        streams[i] = base + offsets[i];
    }
    std::vector<GroupSpec> specs;
    uint64_t covered = 0;
    for (size_t gi = 0; gi < num_groups; ++gi) {
        if (group_sizes[gi] == 0) return fail(KVSZP_EINVAL, "group %zu is empty", gi);
        rc = validate_layers(layer_indices[gi], selected_layers[gi], prefix_count,
                             source_layers, elements_per_layer);
        if (rc) return rc;
        specs.push_back(GroupSpec{
            (uint64_t)prefix_count * selected_layers[gi] * elements_per_layer,
            layer_indices[gi], selected_layers[gi], source_layers, elements_per_layer,
            (uint32_t)group_sizes[gi]});
        covered += group_sizes[gi];
    }
    if (covered != batch)
        return fail(KVSZP_EINVAL, "group sizes sum to %llu, batch is %zu",
                    (unsigned long long)covered, batch);
    std::vector<uint16_t*> dests(batch);
    for (size_t i = 0; i < batch; ++i) {
        const uintptr_t d = (uintptr_t)destinations[i];
        if (!d || (d & 1u)) return fail(KVSZP_EINVAL, "invalid BF16 destination page %zu", i);
        dests[i] = reinterpret_cast<uint16_t*>(d);
    }
    if ((rc = use_device(c))) return rc;
    uint32_t grid_cap = 0;
    if (staging) {
        // vllm_v1_compressed_offload.py:1648-1676: one host-to-device copy of
        // the packed slab, then decode from it.
        hipError_t e = hipMemcpyAsync(staging, packed, packed_bytes, hipMemcpyHostToDevice,
                                      (hipStream_t)stream);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(H2D packed slab)");
    } else {
        // The decoder reads the streams across the link itself: kernel reads
        // of pinned memory run at the link's rate from a few hundred
        // workgroups, so a small grid does it and leaves the CUs to others.
        grid_cap = kLinkDecodeGrid;
    }
    return decompress_groups(c, streams.data(), sizes, error_bounds, batch, specs,
                             kDstIndexed, dests, {}, 0, 0, false, (hipStream_t)stream,
                             false, grid_cap);
}

int kvszp_synchronize(kvszp_ctx* c, kvszp_stream_t stream) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    int rc = use_device(c);
    if (rc) return rc;
    hipError_t e = hipStreamSynchronize((hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    return consume_device_error(c, (hipStream_t)stream, true);
}

int kvszp_enable_timing(kvszp_ctx* c, int kinds) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    if (kinds & ~KVSZP_TIME_ALL) return fail(KVSZP_EINVAL, "unknown timing mask %d", kinds);
    c->timing = kinds;
    return KVSZP_OK;
}

int kvszp_drain_timing(kvszp_ctx* c, double* compress_ms, int* compress_count,
                       double* decompress_ms, int* decompress_count) {
    if (!c) return fail(KVSZP_EINVAL, "null context");
    double ms[2] = {0.0, 0.0};
    int count[2] = {0, 0};
    int rc = KVSZP_OK;
    for (auto& r : c->timed) {
        float t = 0.0f;
        hipError_t e = hipEventSynchronize(r.stop);
        if (e == hipSuccess) e = hipEventElapsedTime(&t, r.start, r.stop);
        if (e != hipSuccess) {
            rc = hip_fail(e, "timing events");
        } else if (r.kind == KVSZP_KERNEL_COMPRESS || r.kind == KVSZP_KERNEL_DECOMPRESS) {
            ms[r.kind] += t;
            count[r.kind] += 1;
        }
        c->spare_events.push_back(r.start);
        c->spare_events.push_back(r.stop);
    }
    c->timed.clear();
    if (compress_ms) *compress_ms = ms[KVSZP_KERNEL_COMPRESS];
    if (compress_count) *compress_count = count[KVSZP_KERNEL_COMPRESS];
    if (decompress_ms) *decompress_ms = ms[KVSZP_KERNEL_DECOMPRESS];
    if (decompress_count) *decompress_count = count[KVSZP_KERNEL_DECOMPRESS];
    return rc;
}

int kvszp_timing_durations(kvszp_ctx* c, int kind, double* ms_out, int capacity,
                           int* count_out) {
    if (!c || !count_out || (capacity > 0 && !ms_out))
        return fail(KVSZP_EINVAL, "null argument");
    if (kind != KVSZP_KERNEL_COMPRESS && kind != KVSZP_KERNEL_DECOMPRESS)
        return fail(KVSZP_EINVAL, "unknown kernel kind %d", kind);
    int rc = KVSZP_OK, n = 0;
    std::vector<TimingRecord> keep;
    for (auto& r : c->timed) {
        if (r.kind != kind) {
            keep.push_back(r);
            continue;
        }
        float t = 0.0f;
        hipError_t e = hipEventSynchronize(r.stop);
        if (e == hipSuccess) e = hipEventElapsedTime(&t, r.start, r.stop);
        if (e != hipSuccess) rc = hip_fail(e, "timing events");
        else if (n < capacity) ms_out[n++] = t;
        c->spare_events.push_back(r.start);
        c->spare_events.push_back(r.stop);
    }
    c->timed.swap(keep);
    *count_out = n;
    return rc;
}

int kvszp_reencode_count(const kvszp_ctx* c, uint64_t* count) {
    if (!c || !count) return fail(KVSZP_EINVAL, "null argument");
    *count = c->redone;
    return KVSZP_OK;
}

int kvszp_schedule_counts(const kvszp_ctx* c, uint64_t* reencoded, uint64_t* safe_calls) {
    if (!c || !reencoded || !safe_calls) return fail(KVSZP_EINVAL, "null argument");
    *reencoded = c->redone;
    *safe_calls = c->safe_calls;
    return KVSZP_OK;
}

const char* kvszp_last_error(void) { return g_last_error.c_str(); }

}  // extern "C"
