// kvszp_internal.h -- launch descriptors shared by the HIP kernels
// (kvszp_kernels.hip) and the host C-ABI (kvszp_capi.cpp).  Groups, jobs,
// tiles and their numbering: kvszp_plan.h.
//
// Schedules.  By default the one-workgroup-per-tile kernels take tile =
// blockIdx.x; their only cross-workgroup waits are on tiles of lower
// blockIdx.x, which the in-order dispatcher has started (KVSZP_TICKETS=1
// takes tile numbers from a counter instead and turns the persistent
// kernels off).  The persistent kernels launch the co-resident number of
// workgroups and walk tiles b, b + G, ...: the decoder's never wait on each
// other; the encoder's waits are bounded in time, and a launch whose wait
// gave up is encoded again by the one-workgroup-per-tile schedule.
#ifndef KVSZP_INTERNAL_H
#define KVSZP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kvszp_plan.h"

namespace kvszp {

constexpr int kThreads = kTileBlocks;               // one thread per block
// Calls of at most this many jobs pass their job table in the kernel
// arguments (no table upload before the launch).
constexpr int kInlineJobs = 16;
// Job tables of up to kArgTableBytes (`jobs_inline` 2): the persistent
// kernels' *_argtable_kernel variants take an ArgTable as a second kernel
// argument, so the records travel with the launch, right behind the
// parameter block at arg_table_offset<Params>() in the kernel-argument
// segment.  The launch then needs no table copy on the stream before it.
constexpr size_t kArgTableBytes = 14336;
struct alignas(16) ArgTable {
    unsigned char bytes[kArgTableBytes];
};
template <class Params>
constexpr size_t arg_table_offset() {
    return (sizeof(Params) + alignof(ArgTable) - 1) & ~(alignof(ArgTable) - 1);
}
constexpr uint32_t kSpinLimit = 1u << 20;           // bounded waits (~1 s)

// Device-side error bits (OR-ed into the context's error word).
enum : uint32_t {
    kErrSpin = 1u,         // a bounded wait expired
    kErrLayerIndex = 2u,   // a layer index outside [0, source_layers)
    kErrRate = 4u,         // a header byte above its mode's limit
    kErrTruncated = 8u,    // payload past the declared stream size
};

// Encoding modes of the fp32 single-page API (the values of KVSZP_MODE_*):
// the fixed-length block code over the quantized values, or over their
// residuals inside each 32-value block (plain), with the block's first value
// kept aside as a 4-byte word (outlier).
enum : int { kModeFixed = 0, kModePlain = 1, kModeOutlier = 2 };

// How the relative error bound is obtained.
enum : int {
    kBoundAbsolute = 0,    // eb = job eps
    kBoundFused = 1,       // per-job min/max exchanged inside the kernel
    kBoundPrepass = 2,     // per-job min/max from a preceding reduction
};

// Decoder destination kinds.
enum : int {
    kDstLinear = 0,        // element e -> dst + e
    kDstMulti = 1,         // element e -> dests[job*dpp + e/epd] + e%epd
    kDstIndexed = 2,       // element e -> dst + layer-mapped index
};

// Host control block: pinned, coherent host memory that kernels write with
// plain system-scope stores and the host reads after (or while) the stream
// runs.  Word kHostErrorMarker becomes nonzero once an encoder kernel
// (min/max pre-pass, encoders) flagged an error, kHostDecodeErrorMarker once
// a decoder did; the bits themselves accumulate in one device error word
// per side, so that a compress call reports only what its own launches
// found, not the errors of restores enqueued before it.  Word kHostSeq holds
// the sequence number of the last launch that started, which tells the host
// that the table copy queued before it has completed.
constexpr int kHostErrorMarker = 0;
constexpr int kHostSeq = 1;
constexpr int kHostOverflow = 2;  // seq of a launch with jobs to encode again
constexpr int kHostAbort = 3;     // seq of an encode whose bounded waits gave up
constexpr int kHostDecodeErrorMarker = 4;
constexpr int kHostCtlWords = 16;

struct CompressJob {
    const uint16_t* in;         // BF16 page (full page when indexed)
    uint8_t* out;               // stream buffer, 4-byte aligned
    float eps;                  // eps (relative) or eb (absolute)
    uint32_t reserved;
};

struct DecompressJob {
    const uint8_t* in;          // stream, 4-byte aligned
    uint16_t* dst;              // destination base (kDstLinear/kDstIndexed)
    float eb;                   // absolute error bound
    uint32_t size;              // declared stream bytes (read bound)
};

struct CompressParams {
    const CompressJob* jobs;
    unsigned long long* tile_state;   // look-back words, one per tile
    unsigned long long* tile_minmax;  // fused min/max words, one per tile
    const unsigned long long* job_minmax;  // pre-pass words, two per job
    uint32_t* host_sizes;             // out (pinned host): stream bytes per job
    float* host_bounds;               // out (pinned host): absolute bound per job
    uint32_t* host_redo;              // out (pinned host): seq = encode the job again
    uint32_t* job_flags;              // device, one per job: epoch = job marked
    uint32_t* error;                  // device error word (kErr* bits)
    uint32_t* error_marker;           // its marker in the host control block
    uint32_t* host_ctl;               // pinned host control words, see above
    uint32_t seq;                     // launch sequence number
    unsigned long long* ticket;
    unsigned long long ticket_base;
    uint32_t epoch;
    uint32_t total_tiles;
    int num_groups;
    int bound_mode;
    int quantizer;                    // 0 two roundings, 1 fused
    int aligned16;                    // every input page is 16-byte aligned
    int input_f32;                    // pages hold fp32 values (not BF16)
    int mode;                         // fp32 pages: kModeFixed/Plain/Outlier
    // Persistent encoder: the C of persistent_first_tile (0: workgroup b
    // starts at tile b).
    uint32_t slot_cus;
    // Time-bounded waits (persistent encoder, fused bound exchange): a wait
    // longer than wait_ticks of the steady clock stores the launch's epoch
    // in *abort_word and seq in host_ctl[kHostAbort], and every wait of the
    // launch then gives up; the host encodes the call again with the
    // pre-pass schedule.  nullptr: waits bounded by kSpinLimit polls only.
    unsigned long long* abort_word;
    uint64_t wait_ticks;
    Group groups[kMaxGroups];
    uint32_t num_jobs;                // job records in the table (jobs or inline_jobs)
    int jobs_inline;                  // 1: inline_jobs; 2: the ArgTable; 0: *jobs
    CompressJob inline_jobs[kInlineJobs];
};

struct MinMaxParams {
    const CompressJob* jobs;
    unsigned long long* job_minmax;   // two words per job: max key, ~min key
    uint32_t* error;
    uint32_t* error_marker;
    uint32_t* host_ctl;
    uint32_t seq;
    uint32_t epoch;
    int num_groups;
    int input_f32;                    // fp32 pages: 32-bit keys, NaN marked
    Group groups[kMaxGroups];         // first_tile is the first chunk
    uint32_t num_jobs;                // job records in the table (jobs or inline_jobs)
    int jobs_inline;                  // 1: the jobs are inline_jobs, not *jobs
    CompressJob inline_jobs[kInlineJobs];
};

struct DecompressParams {
    const DecompressJob* jobs;
    uint16_t* const* dests;           // kDstMulti destination table
    unsigned long long* tile_state;
    uint32_t* error;
    uint32_t* error_marker;
    uint32_t* host_ctl;
    uint32_t seq;
    unsigned long long* ticket;
    unsigned long long ticket_base;
    uint32_t epoch;
    uint32_t total_tiles;
    int num_groups;
    int dst_kind;
    int rate0_zero;                   // 1: write +0.0 for rate-0 blocks
    int aligned16;                    // every destination base 16B aligned
    int output_f32;                   // write fp32 values (kDstLinear only)
    int mode;                         // fp32 streams: kModeFixed/Plain/Outlier
    uint64_t dests_per_page;
    uint64_t elements_per_dest;
    // Persistent decoder runs balanced by bytes moved: each tile of group
    // g weighs tile_weight[g] (its BF16 output plus the group's average
    // payload per tile), weight_before[g] is the weight of the tiles before
    // the group, total_weight that of all tiles; 0 = equal tile counts.
    // run_starts (gridDim.x + 1 tile numbers, or null) overrides them with
    // runs balanced job by job.
    const uint32_t* run_starts;
    uint64_t total_weight;
    uint64_t weight_before[kMaxGroups];
    uint32_t tile_weight[kMaxGroups];
    Group groups[kMaxGroups];
    uint32_t num_jobs;                // job records in the table (jobs or inline_jobs)
    int jobs_inline;                  // 1: inline_jobs; 2: the ArgTable; 0: *jobs
    DecompressJob inline_jobs[kInlineJobs];
};

// Packed publication: every payload i (src, size bytes) goes to
// dst + dst_off, dst_off an 8-byte-aligned exclusive scan of the sizes; the
// gap up to the next payload is zeroed.  dst may be pinned host memory.
// Payloads are cut into pieces of at most kPackPiece bytes (one PackJob
// each), so that any mix of payload sizes spreads over the grid.
constexpr uint64_t kPackPiece = 64 * 1024;
struct PackJob {
    const uint8_t* src;
    uint64_t dst_off;
    uint64_t size;
    uint64_t pad;                     // zero bytes written after the piece
};

struct PackParams {
    const PackJob* jobs;
    uint8_t* dst;
    uint32_t count;
    uint32_t* host_ctl;
    uint32_t seq;
};

hipError_t launch_pack(const PackParams& p, uint32_t grid, hipStream_t stream);

// Device memory of the no-allocation encoder entry point
// (kvszp_compress_batch_fixed_bf16_noalloc): one file-scope array per device
// holding, at these byte offsets, the look-back words, the min/max words,
// the pre-pass words and the job table of one call.
constexpr uint32_t kNoAllocMaxJobs = 4096;
constexpr uint32_t kNoAllocMaxTiles = 65536;   // 512 Mi values per call
constexpr size_t kScratchTileState = 0;
constexpr size_t kScratchTileMinMax = kScratchTileState + 8ull * kNoAllocMaxTiles;
constexpr size_t kScratchJobMinMax = kScratchTileMinMax + 8ull * kNoAllocMaxTiles;
constexpr size_t kScratchJobs = kScratchJobMinMax + 16ull * kNoAllocMaxJobs;
constexpr size_t kScratchJobFlags = kScratchJobs + sizeof(CompressJob) * kNoAllocMaxJobs;
constexpr size_t kScratchAbort = kScratchJobFlags + 4ull * kNoAllocMaxJobs;
constexpr size_t kScratchBytes = kScratchAbort + 256;

// Device address of this device's scratch array: looked up once per device
// (hipGetSymbolAddress with the device current) and kept.
hipError_t scratch_address(int device, void** out);
// Zeroes `count` 64-bit words (a fill kernel, not a memset node).
hipError_t launch_fill_u64(unsigned long long* words, size_t count, hipStream_t stream);

// Launchers (kvszp_kernels.hip).  Return hipGetLastError() of the launch.
// Non-null events are stamped with the kernel's start / end.
hipError_t launch_compress(const CompressParams& p, hipStream_t stream,
                           hipEvent_t start, hipEvent_t stop);
// Persistent encoder: `grid` workgroups (all co-resident) walk the tiles.
// With p.jobs_inline == 2 the `table_bytes` bytes at `table` (the job
// records) go into the kernel arguments.
hipError_t launch_compress_pipelined(const CompressParams& p, uint32_t grid,
                                     hipStream_t stream, hipEvent_t start,
                                     hipEvent_t stop, const void* table = nullptr,
                                     size_t table_bytes = 0);
hipError_t launch_minmax(const MinMaxParams& p, uint32_t grid,
                         hipStream_t stream, hipEvent_t start);
hipError_t launch_decompress(const DecompressParams& p, hipStream_t stream,
                             hipEvent_t start, hipEvent_t stop);
// Persistent decoder: `grid` workgroups each decode a run of consecutive
// tiles; it has no cross-workgroup waits.
hipError_t launch_decompress_persistent(const DecompressParams& p, uint32_t grid,
                                       hipStream_t stream, hipEvent_t start,
                                       hipEvent_t stop, const void* table = nullptr,
                                       size_t table_bytes = 0);
int decompress_resident_workgroups(int device);
// Maximum co-resident workgroups of an encoder kernel on this device.
int compress_resident_workgroups(int device, bool pipelined);

}  // namespace kvszp

#endif  // KVSZP_INTERNAL_H
