// kvszp_kernels.hip -- gfx950 kernels of the batched fixed-mode BF16
// KV-page codec.
//
// Reference semantics: integration/cuszp_wrapper/cuszp_batched_fixed.cu
//   quantizer            :10-25   -> quantize(), build_rows_signhi()
//   rate                 :27-31   -> rate_from_keys(), rate_by_quantizing(),
//                                    OR of |q| (compress_kernel)
//   layer gather         :33-50   -> LayerCursor / map_index()
//   relative bound       :55-133  -> fused min/max exchange (compress) or
//                                    minmax_kernel (pre-pass)
//   encoder              :135-359 -> compress_persistent_kernel, compress_kernel
//   decoder              :361-627 -> decompress_persistent_kernel,
//                                    decompress_kernel
//
// Schedule (not the reference's): tiles of 256 blocks.  The one-workgroup-
// per-tile kernels use 256 threads, ONE THREAD PER 32-ELEMENT BLOCK; the
// persistent encoder uses two waves with two blocks per thread, the
// persistent decoder four waves with one, each walking many tiles.  A thread
// loads its blocks with 16-byte loads, quantizes in registers, and builds the
// sign and plane words with a register bit-matrix transpose (kvszp_bits.h)
// instead of the reference's per-bit loops.  Block offsets come from a workgroup scan plus a
// decoupled look-back across the tiles of a job.  Cross-workgroup state is a
// single 64-bit word per tile holding {epoch tag, status, value}, read and
// written with relaxed agent-scope atomics (these bypass the per-XCD L2), so
// no fence and no per-call memset is needed: stale words carry an older
// epoch and never match.
#include "kvszp_internal.h"
#include "kvszp_bits.h"

#include <float.h>

#include <hip/hip_ext.h>

#include <algorithm>
#include <cstring>
#include <mutex>
#include <type_traits>

#pragma clang fp contract(off)

namespace kvszp {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
// Global-address-space views (global_* instead of flat_* instructions).
typedef __attribute__((address_space(1))) uint32_t g_u32;
typedef __attribute__((address_space(1))) u32x4 g_u32x4;
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef __attribute__((address_space(1))) u32x4_a4 g_u32x4_a4;

template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T* to_global(T* p) {
    return (__attribute__((address_space(1))) T*)p;
}

// Read-only views of the per-call tables (job entries): the constant
// address space lets a wave-uniform entry come through the scalar cache.
template <typename T>
__device__ __forceinline__ T load_const(const T* table, uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
    return ((const __attribute__((address_space(4))) T*)table)[i];
#else
    return table[i];  // host pass only parses this
#endif
}

// Record i of the ArgTable behind the parameter block in the kernel-argument
// segment (only kernels launched with an ArgTable argument get
// jobs_inline == 2 from the host).
template <typename T, class Params>
__device__ __forceinline__ T arg_table_record(uint32_t i) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef const __attribute__((address_space(4))) unsigned char k_u8;
    k_u8* k = (k_u8*)__builtin_amdgcn_kernarg_segment_ptr();
    return ((const __attribute__((address_space(4))) T*)(k + arg_table_offset<Params>()))[i];
#else
    return T{};  // host pass only parses this
#endif
}

// Job record i of a launch: from the kernel arguments for calls of at most
// kInlineJobs jobs or for ArgTable launches, else from the uploaded table
// (`jobs_inline` is uniform, so these are scalar branches).
template <class Params>
__device__ __forceinline__ auto job_at(const Params& p, uint32_t i) {
    typedef typename std::remove_cv<
        typename std::remove_reference<decltype(p.inline_jobs[0])>::type>::type Job;
    if (p.jobs_inline == 2) return arg_table_record<Job, Params>(i);
    return p.jobs_inline ? p.inline_jobs[i] : load_const(p.jobs, i);
}

// ---- cross-workgroup primitives -------------------------------------------

__device__ __forceinline__ unsigned long long load_relaxed(
    const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_relaxed(unsigned long long* p,
                                              unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Error reporting: the bits accumulate in the device word `e`; the host
// control block gets a nonzero marker so the host learns of the error
// without copying the device word back on every call.
__device__ __forceinline__ void flag_error(uint32_t* e, uint32_t* marker,
                                           uint32_t bits) {
    __hip_atomic_fetch_or(e, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(marker, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Time bound of a wait of the persistent encoder or of the fused bound
// exchange (CompressParams::abort_word).  A wait that lasts longer than
// `ticks` of the steady clock gives up and marks the launch: the epoch goes
// to *word and the sequence number to the host control block, and every
// other wait of the launch gives up as soon as it reads the mark.  The host
// then encodes the call again with the pre-pass schedule, whose only wait
// (the look-back) is on workgroups that started earlier.  word == nullptr:
// the wait is bounded by kSpinLimit polls and reports kErrSpin instead.
struct WaitBound {
    unsigned long long* word;
    uint32_t* host_ctl;
    uint32_t seq, epoch;
    uint64_t ticks;
};

__device__ __forceinline__ WaitBound wait_bound(unsigned long long* word, uint32_t* host_ctl,
                                                uint32_t seq, uint32_t epoch, uint64_t ticks) {
    WaitBound b;
    b.word = word;
    b.host_ctl = host_ctl;
    b.seq = seq;
    b.epoch = epoch;
    b.ticks = ticks;
    return b;
}

// One poll of a bounded wait: true when the caller must give up.
// `deadline` is 0 before the first poll of the wait, `spins` counts the
// polls.  The clock is read on every poll (a scalar read, no memory
// traffic); the launch's mark only on every 32nd: all spinning waves read
// that one word, and reading it on every poll makes it a hot spot that slows
// every wait of the launch.
__device__ __forceinline__ bool wait_gives_up(const WaitBound& b, uint64_t& deadline,
                                              uint32_t spins) {
    const uint64_t now = (uint64_t)wall_clock64();
    if (deadline == 0) deadline = now + b.ticks + 1;
    if (now >= deadline) {
        store_relaxed(b.word, (unsigned long long)b.epoch);
        __hip_atomic_store(&b.host_ctl[kHostAbort], b.seq, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        return true;
    }
    return (spins & 31u) == 31u && (uint32_t)load_relaxed(b.word) == b.epoch;
}

// The first workgroup of a launch records the launch's sequence number in
// the host control block: once it is visible, every copy queued on the
// stream before this launch has completed.
__device__ __forceinline__ void publish_seq(uint32_t* host_ctl, uint32_t seq) {
    if (blockIdx.x == 0 && threadIdx.x == 0)
        __hip_atomic_store(&host_ctl[kHostSeq], seq, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

// Tile number of this workgroup.  With a ticket counter the number is the
// order in which workgroups started, so every tile a workgroup waits for has
// already started.  Without one it is blockIdx.x, which relies on the
// dispatcher starting workgroups in index order (one atomic per tile on a
// single address serializes at the memory side, so this is the fast mode).
__device__ __forceinline__ uint32_t take_ticket(unsigned long long* ticket,
                                                unsigned long long base) {
    if (ticket == nullptr) return blockIdx.x;
    return (uint32_t)(__hip_atomic_fetch_add(ticket, 1ull, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT) -
                      base);
}

// ---- wave / workgroup reductions ------------------------------------------

// Wave64 scans and reductions on DPP: row_shr:1,2,4,8 scan each row of 16
// lanes, then row_bcast:15 and row_bcast:31 carry row totals into the rows
// above.  A lane with no source lane keeps `identity`.  All 64 lanes must be
// active.
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114,
              kDppRowShr8 = 0x118, kDppRowBcast15 = 0x142,
              kDppRowBcast31 = 0x143;

template <int kCtrl, int kRowMask>
__device__ __forceinline__ uint32_t dpp_move(uint32_t identity, uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)v, kCtrl,
                                                 kRowMask, 0xF, false);
}

template <class Op>
__device__ __forceinline__ uint32_t wave_scan(uint32_t v, uint32_t identity,
                                              Op op) {
    v = op(v, dpp_move<kDppRowShr1, 0xF>(identity, v));
    v = op(v, dpp_move<kDppRowShr2, 0xF>(identity, v));
    v = op(v, dpp_move<kDppRowShr4, 0xF>(identity, v));
    v = op(v, dpp_move<kDppRowShr8, 0xF>(identity, v));
    v = op(v, dpp_move<kDppRowBcast15, 0xA>(identity, v));
    v = op(v, dpp_move<kDppRowBcast31, 0xC>(identity, v));
    return v;
}

struct OpAdd {
    __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; }
};
struct OpMax {
    __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; }
};
struct OpMin {
    __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; }
};

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
    return __builtin_amdgcn_readlane(wave_scan(v, 0u, OpAdd()), 63);
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
    return __builtin_amdgcn_readlane(wave_scan(v, 0u, OpMax()), 63);
}

__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
    return __builtin_amdgcn_readlane(wave_scan(v, 0xFFFFFFFFu, OpMin()), 63);
}

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v, int) {
    return wave_scan(v, 0u, OpAdd());
}

// ---- quantizer and BF16 helpers -------------------------------------------

// cvt.rzi.s32.f32 of the reference: truncate, saturate, NaN -> 0; this is
// exactly v_cvt_i32_f32.  Inline asm keeps the compiler from treating the
// out-of-range conversion as undefined.
__device__ __forceinline__ int32_t cvt_rzi_sat(float t) {
    int32_t c;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(c) : "v"(t));
    return c;
}

// batch_quantization, cuszp_batched_fixed.cu:10-25.
template <int kQuant>
__device__ __forceinline__ int32_t quantize(float x, float recip) {
    const float v = x * recip;
    const uint32_t s = (v >= -0.5f) ? 0u : 1u;
    const float t = kQuant ? __builtin_fmaf(x, recip, 0.5f) : v + 0.5f;
    return (int32_t)((uint32_t)cvt_rzi_sat(t) - s);
}

// trunc(|t|) as an unsigned integer, NaN -> 0 (v_cvt_u32_f32 with the abs
// modifier; the callers keep |t| below 2^31).
__device__ __forceinline__ uint32_t cvt_abs_u32(float t) {
    uint32_t c;
    asm("v_cvt_u32_f32 %0, |%1|" : "=v"(c) : "v"(t));
    return c;
}

__device__ __forceinline__ float bf16_lo(uint32_t d) {
    return __uint_as_float(d << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t d) {
    return __uint_as_float(d & 0xFFFF0000u);
}

// BF16 order key of a non-NaN value: monotone in the value.
__device__ __forceinline__ uint32_t bf16_key(float x) {
    const uint32_t h = __float_as_uint(x) >> 16;
    return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ float key_value(uint32_t k) {
    const uint32_t h = (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
    return __uint_as_float(h << 16);
}
// Sentinels for "no non-NaN value seen": they decode to the reference's
// initial FLT_MAX / -FLT_MAX (cu:72-73), which no BF16 value equals.
constexpr uint32_t kKeyEmptyMin = 0xFFFFu;
constexpr uint32_t kKeyEmptyMax = 0x0000u;

__device__ __forceinline__ float min_key_value(uint32_t k) {
    return k == kKeyEmptyMin ? FLT_MAX : key_value(k);
}
__device__ __forceinline__ float max_key_value(uint32_t k) {
    return k == kKeyEmptyMax ? -FLT_MAX : key_value(k);
}

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// Order keys (kKeyEmpty* when none) of the smallest and largest non-NaN
// values among the first `count` values of a block, d[] holding BF16 pairs
// (fminf/fmaxf skip NaN, cu:78-79).  A full block is done two values per
// instruction on packed 16-bit keys; NaN keys fall outside [key(-inf),
// key(+inf)] = [0x007F, 0xFF80], so a block holding a NaN (or a partial
// block) is redone value by value.
__device__ __forceinline__ void block_key_minmax(const uint32_t* d,
                                                 uint32_t count,
                                                 uint32_t& kmin,
                                                 uint32_t& kmax) {
    if (count == kBlockElems) {
        u16x2 mn = {0xFFFFu, 0xFFFFu}, mx = {0u, 0u};
#pragma unroll
        for (int i = 0; i < kBlockElems / 2; ++i) {
            // key = sign ? ~h : h | 0x8000, for both halves at once
            const uint32_t neg = __builtin_bit_cast(
                uint32_t, __builtin_bit_cast(s16x2, d[i]) >> (short)15);
            const u16x2 k = __builtin_bit_cast(u16x2, d[i] ^ (neg | 0x80008000u));
            mn = __builtin_elementwise_min(mn, k);
            mx = __builtin_elementwise_max(mx, k);
        }
        kmin = mn.x < mn.y ? mn.x : mn.y;
        kmax = mx.x > mx.y ? mx.x : mx.y;
        if (kmin >= 0x007Fu && kmax <= 0xFF80u) return;
    }
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (uint32_t v = 0; v < count; ++v) {
        const float x = (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
        lo = fminf(lo, x);
        hi = fmaxf(hi, x);
    }
    kmin = lo == FLT_MAX ? kKeyEmptyMin : bf16_key(lo);
    kmax = hi == -FLT_MAX ? kKeyEmptyMax : bf16_key(hi);
}

// eb = eps * fmaxf(max - min, 1e-6f), cu:128-131.
__device__ __forceinline__ float relative_bound(float eps, uint32_t kmin,
                                                uint32_t kmax) {
    const float range = fmaxf(max_key_value(kmax) - min_key_value(kmin), 1e-6f);
    return eps * range;
}

// fp32 order keys: key32 = sign ? ~bits : bits | 0x80000000 for a non-NaN
// value (monotone in the value); kKey32Nan marks "a NaN was seen" in the
// max word (it exceeds key32(+inf) = 0xFF800000).
constexpr uint32_t kKey32Nan = 0xFFFFFFFFu;
__device__ __forceinline__ uint32_t key32(float x) {
    const uint32_t u = __float_as_uint(x);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key32_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The fp32 single-page bound of cuszp_wrapper.cpp:249-257 and :371-377:
// at::aminmax over the page (a NaN anywhere makes min and max NaN), then
// range = max - min, raised to 1e-6f when below it, eb = eps * range.
__device__ __forceinline__ float relative_bound_f32(float eps, uint32_t kmin,
                                                    uint32_t kmax) {
    if (kmax == kKey32Nan) return __uint_as_float(0x7FC00000u);
    float range = key32_value(kmax) - key32_value(kmin);
    if (range < 1e-6f) range = 1e-6f;
    return eps * range;
}

// ---- layer-index gather ----------------------------------------------------

// selected_bf16_source_index (cu:33-50) for an arbitrary logical index.
__device__ uint64_t map_index(uint64_t i, const int64_t* layers,
                              uint64_t sel, uint64_t src, uint64_t epl,
                              uint32_t* bad) {
    const uint64_t per_prefix = sel * epl;
    const uint64_t prefix = i / per_prefix;
    const uint64_t within = i - prefix * per_prefix;
    const uint64_t layer = within / epl;
    const uint64_t inner = within - layer * epl;
    int64_t l = to_global(layers)[layer];
    if (l < 0 || (uint64_t)l >= src) {
        *bad = 1;
        l = 0;
    }
    return (prefix * src + (uint64_t)l) * epl + inner;
}

// The layer map evaluated for the first element of this thread's block:
// the tile start is decomposed once per workgroup (64-bit, uniform) and each
// thread only adds its 32-bit offset.
struct LayerCursor {
    uint64_t src_index;  // source index of the block's first element
    bool contiguous;     // the 32 elements stay inside one layer
};

__device__ __forceinline__ LayerCursor layer_cursor(
    const Group& g, uint64_t tile_first_elem, uint32_t elem_in_tile,
    uint32_t* bad) {
    const uint64_t per_prefix = g.selected_layers * g.elements_per_layer;
    const uint64_t t_prefix = tile_first_elem / per_prefix;
    const uint32_t t_within = (uint32_t)(tile_first_elem - t_prefix * per_prefix);
    const uint32_t pp = (uint32_t)per_prefix;
    const uint32_t epl = (uint32_t)g.elements_per_layer;
    uint32_t w = t_within + elem_in_tile;
    const uint32_t padv = w / pp;
    w -= padv * pp;
    const uint32_t layer = w / epl;
    const uint32_t inner = w - layer * epl;
    int64_t l = to_global(g.layers)[layer];
    if (l < 0 || (uint64_t)l >= g.source_layers) {
        *bad = 1;
        l = 0;
    }
    LayerCursor c;
    c.src_index = ((t_prefix + padv) * g.source_layers + (uint64_t)l) *
                      g.elements_per_layer + inner;
    c.contiguous = inner + kBlockElems <= epl;
    return c;
}

// Loads the 32 BF16 values of a block as 16 packed pairs; elements at or
// past `count` are loaded as 0 (the caller masks them anyway).
__device__ __forceinline__ void load_block(
    const Group& g, const uint16_t* in, uint64_t tile_first_elem,
    uint32_t elem_in_tile, uint32_t count, bool aligned16, uint32_t* d,
    uint32_t* bad) {
    const uint64_t e0 = tile_first_elem + elem_in_tile;
    uint64_t src = e0;
    bool contiguous = true;
    if (g.layers != nullptr) {
        const LayerCursor c = layer_cursor(g, tile_first_elem, elem_in_tile, bad);
        src = c.src_index;
        contiguous = c.contiguous;
    }
    if (count == kBlockElems && contiguous && aligned16) {
        const g_u32x4* p = (const g_u32x4*)to_global(in + src);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4 v = p[i];
            d[4 * i + 0] = v.x;
            d[4 * i + 1] = v.y;
            d[4 * i + 2] = v.z;
            d[4 * i + 3] = v.w;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) d[i] = 0;
    for (uint32_t v = 0; v < count; ++v) {
        uint64_t s = src + v;
        if (!contiguous)
            s = map_index(e0 + v, g.layers, g.selected_layers, g.source_layers,
                          g.elements_per_layer, bad);
        const uint32_t h = to_global(in)[s];
        d[v >> 1] |= (v & 1) ? (h << 16) : h;
    }
}

// Wave-cooperative load of the wave's 64 blocks when they are consecutive
// in memory (wave_src = source of the wave's first block, 16-byte aligned):
// four coalesced 1 KiB loads straight into LDS, then every lane reads its
// own 64-byte block.  In load i, lane l fetches 16-byte chunk
// 64i + 4(l%16) + l/16 of the wave's 4 KiB; global_load_lds puts lane l's
// chunk at LDS slot 64i + l, so chunk c of block b sits at slot
// 64(b/16) + (b%16) + 16c and the per-lane reads are bank-conflict free.
__device__ __forceinline__ void wave_load_blocks(const uint16_t* wave_src,
                                                 uint32_t* lds_wave, uint32_t* d) {
    const int lane = threadIdx.x & 63;
    const uint32_t chunk = 4u * (lane & 15) + (lane >> 4);
    const char* src = reinterpret_cast<const char*>(wave_src) + 16u * chunk;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(src + 1024 * i),
            (__attribute__((address_space(3))) void*)(lds_wave + 256 * i), 16, 0, 0);
    __builtin_amdgcn_s_waitcnt(0);  // vmcnt(0): the LDS writes have landed
    const u32x4* slots = reinterpret_cast<const u32x4*>(lds_wave);
    const uint32_t base = 64u * (lane >> 4) + (lane & 15);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const u32x4 v = slots[base + 16u * c];
        d[4 * c + 0] = v.x;
        d[4 * c + 1] = v.y;
        d[4 * c + 2] = v.z;
        d[4 * c + 3] = v.w;
    }
}

// Loads this thread's block; whole waves whose 64 blocks are consecutive,
// full and 16-byte aligned take the coalesced LDS path.
__device__ __forceinline__ void load_block_wave(
    const Group& g, const uint16_t* in, uint64_t tile_first_elem,
    uint32_t elem_in_tile, uint32_t count, bool aligned16, uint32_t* d,
    uint32_t* bad, uint32_t* lds_wave) {
    uint64_t src = tile_first_elem + elem_in_tile;
    bool contiguous = true;
    if (g.layers != nullptr) {
        const LayerCursor c = layer_cursor(g, tile_first_elem, elem_in_tile, bad);
        src = c.src_index;
        contiguous = c.contiguous;
    }
    const int lane = threadIdx.x & 63;
    const uint64_t src0 = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(src >> 32)) << 32) |
                          __builtin_amdgcn_readfirstlane((uint32_t)src);
    const bool fast = count == kBlockElems && contiguous && aligned16 &&
                      src == src0 + (uint64_t)kBlockElems * lane;
    if (__ballot(!fast) == 0ull) {
        wave_load_blocks(in + src0, lds_wave, d);
        return;
    }
    load_block(g, in, tile_first_elem, elem_in_tile, count, aligned16, d, bad);
}

// The 32 fp32 values of a block starting at element e0 of a contiguous page
// (values at or past `count` read as 0): eight 16-byte loads when the block
// is whole and the page 16-byte aligned, else one value at a time.
__device__ __forceinline__ void load_block_f32(const float* in, uint64_t e0,
                                               uint32_t count, bool aligned16,
                                               uint32_t* d) {
    if (count == kBlockElems && aligned16) {
        const g_u32x4* p = (const g_u32x4*)to_global(in + e0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const u32x4 v = p[i];
            d[4 * i + 0] = v.x;
            d[4 * i + 1] = v.y;
            d[4 * i + 2] = v.z;
            d[4 * i + 3] = v.w;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kBlockElems; ++i) d[i] = 0;
    const __attribute__((address_space(1))) uint32_t* g =
        (const __attribute__((address_space(1))) uint32_t*)(in + e0);
    for (uint32_t v = 0; v < count; ++v) d[v] = g[v];
}

// ---- workgroup scan + decoupled look-back ---------------------------------

struct TileScan {
    uint32_t exclusive;  // bytes of earlier blocks in this tile
    uint32_t total;      // bytes of the whole tile
};

__device__ __forceinline__ TileScan tile_scan(uint32_t bytes, int tid,
                                              uint32_t* s_wave) {
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const uint32_t incl = wave_inclusive_scan(bytes, lane);
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    uint32_t base = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        const uint32_t s = s_wave[w];
        base += (w < wave) ? s : 0u;
        total += s;
    }
    TileScan r;
    r.exclusive = base + incl - bytes;
    r.total = total;
    return r;
}

// Payload bytes announced by one header dword (four rate bytes r):
// sum of (r ? 4 + 4r : 0) = 4 * (sum of r + number of nonzero r).
__device__ __forceinline__ uint32_t header_word_bytes(uint32_t w) {
    const uint32_t sum = __builtin_amdgcn_sad_u8(w, 0u, 0u);
    const uint32_t nz = (((w & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | w) & 0x80808080u;
    return 4u * (sum + (uint32_t)__builtin_popcount(nz));
}

// Decoupled look-back over the tiles of one job.  Tile state words carry
// an epoch tag: epoch*4+1 = aggregate (this tile's bytes), epoch*4+2 =
// inclusive prefix (bytes of this and all earlier tiles of the job).
//
// lookback_publish: lane 0 publishes the tile's aggregate (tile 0 its
// inclusive prefix right away).
__device__ __forceinline__ void lookback_publish(unsigned long long* state,
                                                 uint32_t t, uint32_t tile,
                                                 uint32_t total, uint32_t epoch) {
    if (__lane_id() != 0) return;
    const uint32_t tag = epoch * 4u + (tile == 0 ? 2u : 1u);
    store_relaxed(&state[t], ((unsigned long long)tag << 32) | total);
}

// lookback_wait: executed by one full wave after lookback_publish.  Walks
// back over earlier tiles of the job 64 at a time until it meets one whose
// inclusive prefix is published, publishes this tile's inclusive prefix and
// returns the exclusive one (bytes of earlier tiles of the job).
// lookback_first_addr: the word of the first window lookback_wait reads in
// this lane (lanes outside the window get t's own word, which is ignored),
// for a caller that issues that read early, ahead of other memory traffic.
__device__ __forceinline__ const unsigned long long* lookback_first_addr(
    const unsigned long long* state, uint32_t t, uint32_t tile) {
    const uint32_t lane = __lane_id();
    return (tile != 0 && lane < (tile < 64u ? tile : 64u)) ? &state[t - 1 - lane] : &state[t];
}

// `bound` (optional): a time-bounded wait; when it gives up, *gave_up is
// set, nothing is published and the result is meaningless.
__device__ uint32_t lookback_wait(unsigned long long* state, uint32_t t,
                                  uint32_t tile, uint32_t total, uint32_t epoch,
                                  uint32_t* err, uint32_t* err_marker,
                                  bool have_first = false, unsigned long long first = 0,
                                  const WaitBound* bound = nullptr,
                                  bool* gave_up = nullptr) {
    if (tile == 0) return 0;
    const int lane = __lane_id();
    const uint32_t tag_agg = epoch * 4u + 1u;
    const uint32_t tag_inc = epoch * 4u + 2u;
    uint32_t acc = 0;
    uint32_t remaining = tile;   // earlier tiles of this job
    uint32_t pos = t - 1;        // tile read by lane 0
    const bool timed = bound != nullptr && bound->word != nullptr;
    uint64_t deadline = 0;
    for (;;) {
        const uint32_t nwin = remaining < 64u ? remaining : 64u;
        const bool in_win = (uint32_t)lane < nwin;
        const unsigned long long win_mask =
            nwin == 64u ? ~0ull : ((1ull << nwin) - 1ull);
        unsigned long long w = 0, need = 0, incl = 0;
        for (uint32_t spins = 0;; ++spins) {
            if (have_first) {  // the caller's early read of this window
                w = first;
                have_first = false;
            } else {
                w = in_win ? load_relaxed(&state[pos - lane]) : 0ull;
            }
            const uint32_t tag = (uint32_t)(w >> 32);
            incl = __ballot(in_win && tag == tag_inc);
            const unsigned long long ready =
                __ballot(in_win && (tag == tag_inc || tag == tag_agg));
            need = incl ? (((incl & (~incl + 1ull)) << 1) - 1ull) : win_mask;
            if ((ready & need) == need) break;
            if (timed) {
                if (__builtin_amdgcn_readfirstlane(wait_gives_up(*bound, deadline, spins) ? 1 : 0)) {
                    *gave_up = true;
                    return 0;
                }
            } else if (spins >= kSpinLimit) {
                if (lane == 0) flag_error(err, err_marker, kErrSpin);
                need &= ready;
                incl = 1;  // stop walking
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        acc += wave_sum(((need >> lane) & 1ull) ? (uint32_t)w : 0u);
        if (incl || remaining <= 64u) break;
        remaining -= 64u;
        pos -= 64u;
    }
    if (lane == 0)
        store_relaxed(&state[t],
                      ((unsigned long long)tag_inc << 32) | (acc + total));
    return acc;
}

// Both halves back to back (one full wave).
__device__ __forceinline__ uint32_t lookback(unsigned long long* state,
                                             uint32_t t, uint32_t tile,
                                             uint32_t total, uint32_t epoch,
                                             uint32_t* err, uint32_t* err_marker,
                                             const WaitBound* bound = nullptr,
                                             bool* gave_up = nullptr) {
    lookback_publish(state, t, tile, total, epoch);
    return lookback_wait(state, t, tile, total, epoch, err, err_marker, false, 0, bound,
                         gave_up);
}

// Finds the group of tile t (groups are few and ordered by first_tile).
// Unrolled over the kernel-argument table so the lookups are independent
// scalar loads rather than a dependent chain.
__device__ __forceinline__ int find_group(const Group* groups, int num_groups,
                                          uint32_t t) {
    int g = 0;
#pragma unroll
    for (int i = 1; i < kMaxGroups; ++i)
        if (i < num_groups && t >= groups[i].first_tile) g = i;
    return g;
}

// Wave-uniform tile number.  Ticket mode broadcasts thread 0's ticket through
// LDS (one barrier); otherwise the tile is blockIdx.x with no barrier.
__device__ __forceinline__ uint32_t tile_number(unsigned long long* ticket,
                                                unsigned long long base,
                                                uint32_t* s_tile) {
    if (ticket == nullptr) return blockIdx.x;
    if (threadIdx.x == 0) *s_tile = take_ticket(ticket, base);
    __syncthreads();
    return __builtin_amdgcn_readfirstlane(*s_tile);
}

// ---- stream word I/O --------------------------------------------------------
// A block's payload is `count` consecutive 4-byte-aligned words.  Lanes move
// them as 16-byte groups (unaligned 128-bit accesses) plus single words for
// the tail; `cmax` is the wave-uniform maximum count, so groups no lane needs
// are skipped without divergence.  Nothing outside [0, count) is touched.
// Plain (cached) accesses on purpose: the L2 merges the lanes' partial
// writes of a tile's contiguous payload into full lines, while non-temporal
// stores reach HBM as partial-line writes (measured: ~4x the stream bytes).
template <int kWords>
__device__ __forceinline__ void store_words(uint32_t* dst, const uint32_t* w,
                                            uint32_t count, uint32_t cmax) {
    g_u32* d = to_global(dst);
#pragma unroll
    for (int j = 0; j < kWords / 4; ++j) {
        if ((uint32_t)(4 * j) < cmax) {
            if (count >= (uint32_t)(4 * j + 4)) {
                u32x4 v;
                v.x = w[4 * j + 0];
                v.y = w[4 * j + 1];
                v.z = w[4 * j + 2];
                v.w = w[4 * j + 3];
                *(g_u32x4_a4*)(d + 4 * j) = v;
            } else {
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    if (count > (uint32_t)(4 * j + i))
                        d[4 * j + i] = w[4 * j + i];
            }
        }
    }
}

template <int kWords>
__device__ __forceinline__ void load_words(const uint32_t* src, uint32_t* w,
                                           uint32_t count, uint32_t cmax) {
    const g_u32* s = to_global(const_cast<uint32_t*>(src));
#pragma unroll
    for (int j = 0; j < kWords / 4; ++j) {
        w[4 * j + 0] = w[4 * j + 1] = w[4 * j + 2] = w[4 * j + 3] = 0;
        if ((uint32_t)(4 * j) < cmax) {
            if (count >= (uint32_t)(4 * j + 4)) {
                const u32x4 v = *(const g_u32x4_a4*)(s + 4 * j);
                w[4 * j + 0] = v.x;
                w[4 * j + 1] = v.y;
                w[4 * j + 2] = v.z;
                w[4 * j + 3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    if (count > (uint32_t)(4 * j + i))
                        w[4 * j + i] = s[4 * j + i];
            }
        }
    }
}

// Value v of a block: 16 packed BF16 pairs (kIn = 0) or 32 fp32 words
// (kIn = 1).
template <int kIn>
__device__ __forceinline__ float elem_value(const uint32_t* d, int v) {
    if (kIn) return __uint_as_float(d[v]);
    return (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
}

// Quantized element v of a block; elements at or past `count` quantize to 0
// (cu:200-211).
template <int kQuant, bool kFull, int kIn = 0>
__device__ __forceinline__ int32_t quant_elem(const uint32_t* d, int v,
                                              uint32_t count, float recip) {
    const int32_t q = quantize<kQuant>(elem_value<kIn>(d, v), recip);
    return (kFull || (uint32_t)v < count) ? q : 0;
}

__device__ __forceinline__ uint32_t magnitude(int32_t q) {
    return (uint32_t)(q < 0 ? -q : q);  // q > INT_MIN always (cu:212-215)
}

// Rows of low fields ((|q| << 1) | sign) and the OR of all |q| (the rate is
// its bit length, cu:221-222).
template <int kQuant, bool kFull, int kIn = 0>
__device__ __forceinline__ void build_rows_lo(const uint32_t* d, uint32_t count,
                                              float recip, uint32_t* P,
                                              uint32_t& orv) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int32_t q0 = quant_elem<kQuant, kFull, kIn>(d, row_lo_elem(k), count, recip);
        const int32_t q1 = quant_elem<kQuant, kFull, kIn>(d, row_hi_elem(k), count, recip);
        const uint32_t m0 = magnitude(q0), m1 = magnitude(q1);
        orv |= m0 | m1;
        P[k] = field_lo(m0, (uint32_t)q0 >> 31) | (field_lo(m1, (uint32_t)q1 >> 31) << 16);
    }
}

// build_rows_lo for a full block, one row after the other: each row's
// reciprocal passes through an empty asm that takes the previous row as an
// input, so the scheduler cannot start all 32 conversions at once (which
// would hold ~2x the registers inside the persistent encoder's loop).
template <int kQuant>
__device__ __forceinline__ void build_rows_lo_chained(const uint32_t* d, float recip,
                                                      uint32_t* P, uint32_t& orv) {
    uint32_t prev = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        float r = recip;
        asm volatile("" : "+v"(r) : "v"(prev));
        const int32_t q0 = quant_elem<kQuant, true>(d, row_lo_elem(k), kBlockElems, r);
        const int32_t q1 = quant_elem<kQuant, true>(d, row_hi_elem(k), kBlockElems, r);
        const uint32_t m0 = magnitude(q0), m1 = magnitude(q1);
        orv |= m0 | m1;
        P[k] = field_lo(m0, (uint32_t)q0 >> 31) | (field_lo(m1, (uint32_t)q1 >> 31) << 16);
        prev = P[k];
    }
}

template <int kQuant>
__device__ __forceinline__ void build_rows_hi_chained(const uint32_t* d, float recip,
                                                      uint32_t* P) {
    uint32_t prev = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        float r = recip;
        asm volatile("" : "+v"(r) : "v"(prev));
        const uint32_t m0 = magnitude(quant_elem<kQuant, true>(d, row_lo_elem(k), kBlockElems, r));
        const uint32_t m1 = magnitude(quant_elem<kQuant, true>(d, row_hi_elem(k), kBlockElems, r));
        P[k] = field_hi(m0) | (field_hi(m1) << 16);
        prev = P[k];
    }
}

// Rows of high fields (|q| >> 15), for rates above 15.
template <int kQuant, bool kFull, int kIn = 0>
__device__ __forceinline__ void build_rows_hi(const uint32_t* d, uint32_t count,
                                              float recip, uint32_t* P) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t m0 = magnitude(quant_elem<kQuant, kFull, kIn>(d, row_lo_elem(k), count, recip));
        const uint32_t m1 = magnitude(quant_elem<kQuant, kFull, kIn>(d, row_hi_elem(k), count, recip));
        P[k] = field_hi(m0) | (field_hi(m1) << 16);
    }
}

// ---- encoder ---------------------------------------------------------------

// kIn = 0: BF16 pages (any bound mode, layer maps); kIn = 1: contiguous
// fp32 pages (absolute or pre-pass bound), the single-page fp32 API.
template <int kQuant, int kIn>
__global__ __launch_bounds__(kThreads) void compress_kernel(CompressParams p) {
    __shared__ uint32_t s_tile;
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_min[kThreads / 64];
    __shared__ uint32_t s_max[kThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_abort;
    __shared__ uint8_t s_rate[kTileBlocks];
    __shared__ __attribute__((aligned(16))) uint32_t s_stage[kThreads / 64][1024];  // 4 KiB per wave

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    publish_seq(p.host_ctl, p.seq);
    const WaitBound bound = wait_bound(p.abort_word, p.host_ctl, p.seq, p.epoch, p.wait_ticks);
    if (tid == 0) s_abort = 0;
    const uint32_t t = tile_number(p.ticket, p.ticket_base, &s_tile);
    if (t >= p.total_tiles) {  // tickets of another launch: never index past
        if (tid == 0) flag_error(p.error, p.error_marker, kErrSpin);
        return;
    }
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];

    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = __builtin_amdgcn_readfirstlane(local / g.tiles_per_job);
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const CompressJob J = job_at(p, job);
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t tile_first = (uint64_t)tile * kTileElems;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;

    uint32_t bad = 0;
    uint32_t d[kIn ? kBlockElems : kBlockElems / 2];
    if constexpr (kIn)
        load_block_f32(reinterpret_cast<const float*>(J.in), e0, count,
                       p.aligned16 != 0, d);
    else
        load_block_wave(g, J.in, tile_first, (uint32_t)tid * kBlockElems, count,
                        p.aligned16 != 0, d, &bad, &s_stage[wave][0]);

    float eb = J.eps;
    if constexpr (kIn) {
        if (p.bound_mode != kBoundAbsolute) {  // pre-pass words (32-bit keys)
            const unsigned long long wmax = p.job_minmax[2 * job];
            const unsigned long long wmin = p.job_minmax[2 * job + 1];
            if ((uint32_t)(wmax >> 32) != p.epoch || (uint32_t)(wmin >> 32) != p.epoch)
                bad |= 2;
            eb = relative_bound_f32(J.eps, 0xFFFFFFFFu - (uint32_t)wmin, (uint32_t)wmax);
        }
    } else if (p.bound_mode != kBoundAbsolute) {
        uint32_t kmin, kmax;
        if (p.bound_mode == kBoundFused) {
            block_key_minmax(d, count, kmin, kmax);
            kmin = wave_min(kmin);
            kmax = wave_max(kmax);
            if (lane == 0) {
                s_min[wave] = kmin;
                s_max[wave] = kmax;
            }
            __syncthreads();
            if (tid == 0) {
#pragma unroll
                for (int w = 1; w < kThreads / 64; ++w) {
                    kmin = s_min[w] < kmin ? s_min[w] : kmin;
                    kmax = s_max[w] > kmax ? s_max[w] : kmax;
                }
                store_relaxed(&p.tile_minmax[t],
                              ((unsigned long long)p.epoch << 32) |
                                  (kmin << 16) | kmax);
            }
            // Exchange with every tile of this job (host guarantees
            // tiles_per_job <= kThreads and that they can be co-resident).
            kmin = kKeyEmptyMin;
            kmax = kKeyEmptyMax;
            if ((uint32_t)tid < g.tiles_per_job) {
                const unsigned long long* slot = &p.tile_minmax[t - tile + tid];
                unsigned long long w = load_relaxed(slot);
                uint64_t deadline = 0;
                for (uint32_t spins = 0; (uint32_t)(w >> 32) != p.epoch; ++spins) {
                    if (bound.word != nullptr) {
                        if (wait_gives_up(bound, deadline, spins)) {
                            s_abort = 1;
                            break;
                        }
                    } else if (spins >= kSpinLimit) {
                        flag_error(p.error, p.error_marker, kErrSpin);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                    w = load_relaxed(slot);
                }
                kmin = (uint32_t)(w >> 16) & 0xFFFFu;
                kmax = (uint32_t)w & 0xFFFFu;
            }
            kmin = wave_min(kmin);
            kmax = wave_max(kmax);
            __syncthreads();  // s_min/s_max reuse
            if (s_abort) return;  // the launch gave up; the host encodes again
            if (lane == 0) {
                s_min[wave] = kmin;
                s_max[wave] = kmax;
            }
            __syncthreads();
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) {
                kmin = s_min[w] < kmin ? s_min[w] : kmin;
                kmax = s_max[w] > kmax ? s_max[w] : kmax;
            }
        } else {
            const unsigned long long wmax = p.job_minmax[2 * job];
            const unsigned long long wmin = p.job_minmax[2 * job + 1];
            if ((uint32_t)(wmax >> 32) != p.epoch ||
                (uint32_t)(wmin >> 32) != p.epoch)
                bad |= 2;  // reported as a spin error below
            kmax = (uint32_t)wmax & 0xFFFFu;
            kmin = 0xFFFFu - ((uint32_t)wmin & 0xFFFFu);
        }
        eb = relative_bound(J.eps, kmin, kmax);
    }
    const float recip = 0.5f / eb;  // cu:166, IEEE division

    // Quantize (cu:180-231) into the row layout of kvszp_bits.h: P[k] holds
    // the low fields ((|q| << 1) | sign) of elements k^7 and 16+(k^7).
    uint32_t P[16];
    uint32_t orv = 0;
    if (count == kBlockElems)
        build_rows_lo<kQuant, true, kIn>(d, count, recip, P, orv);
    else
        build_rows_lo<kQuant, false, kIn>(d, count, recip, P, orv);
    const uint32_t rate = orv ? 32u - (uint32_t)__builtin_clz(orv) : 0u;
    const uint32_t bytes = rate ? 4u + 4u * rate : 0u;
    s_rate[tid] = (uint8_t)rate;

    const TileScan sc = tile_scan(bytes, tid, s_wave);  // has __syncthreads

    // Header bytes of this tile (cu:226-229); the last tile also zeroes the
    // padding up to R, which the reference leaves unwritten.
    const uint32_t R = g.header_bytes;
    if (tid < kTileBlocks / 4) {
        const uint32_t word = (uint32_t)s_rate[4 * tid] |
                              ((uint32_t)s_rate[4 * tid + 1] << 8) |
                              ((uint32_t)s_rate[4 * tid + 2] << 16) |
                              ((uint32_t)s_rate[4 * tid + 3] << 24);
        *to_global(reinterpret_cast<uint32_t*>(J.out + tile * kTileBlocks + 4 * tid)) = word;
    }
    const bool last_tile = tile + 1 == g.tiles_per_job;
    if (last_tile) {
        for (uint32_t off = (tile + 1) * kTileBlocks + 4u * tid; off < R;
             off += 4u * kThreads)
            *to_global(reinterpret_cast<uint32_t*>(J.out + off)) = 0u;
    }

    if (wave == 0) {
        bool gave_up = false;
        const uint32_t prefix = lookback(p.tile_state, t, tile, sc.total, p.epoch, p.error,
                                         p.error_marker, &bound, &gave_up);
        if (gave_up && lane == 0) s_abort = 1;
        if (lane == 0) {
            s_prefix = prefix;
            if (last_tile)
                __hip_atomic_store(&p.host_sizes[job], R + prefix + sc.total,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (tile == 0)
                __hip_atomic_store(&p.host_bounds[job], eb, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (bad & 1) flag_error(p.error, p.error_marker, kErrLayerIndex);
    if (bad & 2) flag_error(p.error, p.error_marker, kErrSpin);
    __syncthreads();
    if (s_abort) return;

    // Payload (cu:302-358): sign word, then `rate` plane words.
    const uint32_t rmax = wave_max(rate);
    if (rmax == 0) return;
    uint32_t* dst = reinterpret_cast<uint32_t*>(J.out + R + s_prefix + sc.exclusive);
    const uint32_t count_words = rate ? rate + 1u : 0u;
    transpose16x2(P);  // rows 0..15 = words w_0..w_15
    store_words<16>(dst, P, count_words < 16u ? count_words : 16u,
                    rmax < 15u ? rmax + 1u : 16u);
    if (rmax >= 16u) {
        // Planes 15..30 (rates 16..31): high fields, a second transpose.
        // Rare, so the block is re-read instead of kept in registers.
        uint32_t bad2 = 0;
        if constexpr (kIn)
            load_block_f32(reinterpret_cast<const float*>(J.in), e0, count,
                           p.aligned16 != 0, d);
        else
            load_block(g, J.in, tile_first, (uint32_t)tid * kBlockElems, count,
                       p.aligned16 != 0, d, &bad2);
        if (count == kBlockElems)
            build_rows_hi<kQuant, true, kIn>(d, count, recip, P);
        else
            build_rows_hi<kQuant, false, kIn>(d, count, recip, P);
        transpose16x2(P);
        store_words<16>(dst + 16, P, count_words > 16u ? count_words - 16u : 0u,
                        rmax - 15u);
    }
}

// ---- Lorenzo modes (plain, outlier) of the fp32 single-page API -------------
//
// The reference hands these modes to upstream cuSZp (cuszp_wrapper.cpp:
// 302-313, 922-933; decoders launched at cuszp_fastpath.cu:37-59), which is
// not vendored.  This is the build's own specification of them, after the
// published cuSZp design (1D Lorenzo prediction inside each 32-value block,
// then the fixed-length block code):
//   q_v      the fixed-mode quantizer's value; past the end of the data a
//            block repeats its last q (residual 0)
//   d_0 = q_0, d_v = q_v - q_{v-1}   (32-bit wrap-around)
//   plain    codes c_v = d_v;  outlier keeps o = d_0 aside, c_0 = 0
//   rate r   bit length of max |c_v| as a 32-bit magnitude (0..32: the
//            magnitude of INT_MIN is 2^31)
//   header   one byte per block: r, plus bit 7 in outlier mode when o != 0
//   payload  per block: o (4 bytes, only when its bit is set), then for r > 0
//            the sign word and r plane words as in fixed mode (w_32 is plane
//            31, bit 31 of the magnitudes)
//   decode   q_{-1} = o (outlier) or 0, q_v = q_{v-1} + c_v,
//            y_v = fl(fl(q_v * eb) * 2)
// Both modes decode to the fixed mode's values of the same page; byte parity
// with upstream cuSZp is unpinned.

// Residual words of one block, in place of its 32 fp32 words; returns the OR
// of their magnitudes and the outlier word (0 in plain mode).
template <int kQuant, int kMode>
__device__ __forceinline__ uint32_t lorenzo_residuals(uint32_t* d, uint32_t count,
                                                      float recip, uint32_t& outlier) {
    int32_t prev = 0;
    uint32_t orv = 0;
    outlier = 0;
#pragma unroll
    for (int v = 0; v < kBlockElems; ++v) {
        const int32_t q =
            (uint32_t)v < count ? quantize<kQuant>(__uint_as_float(d[v]), recip) : prev;
        uint32_t c = (uint32_t)q - (uint32_t)prev;
        prev = q;
        if (kMode == kModeOutlier && v == 0) {
            outlier = c;
            c = 0;
        }
        d[v] = c;
        orv |= (int32_t)c < 0 ? 0u - c : c;
    }
    return orv;
}

__device__ __forceinline__ uint32_t residual_magnitude(uint32_t c) {
    return (int32_t)c < 0 ? 0u - c : c;
}

// Rows of the residuals' low fields ((m << 1) | sign), high fields m >> 15
// (bits 15..30), and the plane-31 word, in the row layout of kvszp_bits.h.
__device__ __forceinline__ void residual_rows_lo(const uint32_t* c, uint32_t* P) {
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const uint32_t a = c[row_lo_elem(k)], b = c[row_hi_elem(k)];
        P[k] = field_lo(residual_magnitude(a), a >> 31) |
               (field_lo(residual_magnitude(b), b >> 31) << 16);
    }
}

__device__ __forceinline__ void residual_rows_hi(const uint32_t* c, uint32_t* P) {
#pragma unroll
    for (int k = 0; k < 16; ++k)
        P[k] = field_hi(residual_magnitude(c[row_lo_elem(k)])) |
               (field_hi(residual_magnitude(c[row_hi_elem(k)])) << 16);
}

__device__ __forceinline__ uint32_t residual_plane31(const uint32_t* c) {
    uint32_t w = 0;
#pragma unroll
    for (int v = 0; v < kBlockElems; ++v)
        w |= (residual_magnitude(c[v]) >> 31) << (v ^ 7);
    return w;
}

// One workgroup per tile, one block per thread, contiguous fp32 pages with
// an absolute or pre-pass bound (the schedule of compress_kernel).
template <int kQuant, int kMode>
__global__ __launch_bounds__(kThreads) void compress_lorenzo_kernel(CompressParams p) {
    __shared__ uint32_t s_tile;
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_abort;
    __shared__ uint8_t s_hdr[kTileBlocks];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    publish_seq(p.host_ctl, p.seq);
    const WaitBound bound = wait_bound(p.abort_word, p.host_ctl, p.seq, p.epoch, p.wait_ticks);
    if (tid == 0) s_abort = 0;
    const uint32_t t = tile_number(p.ticket, p.ticket_base, &s_tile);
    if (t >= p.total_tiles) {
        if (tid == 0) flag_error(p.error, p.error_marker, kErrSpin);
        return;
    }
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];
    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = __builtin_amdgcn_readfirstlane(local / g.tiles_per_job);
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const CompressJob J = job_at(p, job);
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;

    uint32_t d[kBlockElems];
    load_block_f32(reinterpret_cast<const float*>(J.in), e0, count, p.aligned16 != 0, d);
    float eb = J.eps;
    uint32_t bad = 0;
    if (p.bound_mode != kBoundAbsolute) {  // pre-pass words (32-bit keys)
        const unsigned long long wmax = p.job_minmax[2 * job];
        const unsigned long long wmin = p.job_minmax[2 * job + 1];
        if ((uint32_t)(wmax >> 32) != p.epoch || (uint32_t)(wmin >> 32) != p.epoch) bad = 1;
        eb = relative_bound_f32(J.eps, 0xFFFFFFFFu - (uint32_t)wmin, (uint32_t)wmax);
    }
    const float recip = 0.5f / eb;  // IEEE division, as in fixed mode

    uint32_t outlier;
    const uint32_t orv = lorenzo_residuals<kQuant, kMode>(d, count, recip, outlier);
    const uint32_t rate = orv ? 32u - (uint32_t)__builtin_clz(orv) : 0u;
    const bool has_o = kMode == kModeOutlier && outlier != 0;
    const uint32_t bytes = (has_o ? 4u : 0u) + (rate ? 4u + 4u * rate : 0u);
    s_hdr[tid] = (uint8_t)(rate | (has_o ? 0x80u : 0u));

    const TileScan sc = tile_scan(bytes, tid, s_wave);  // has __syncthreads

    const uint32_t R = g.header_bytes;
    if (tid < kTileBlocks / 4) {
        const uint32_t word = (uint32_t)s_hdr[4 * tid] | ((uint32_t)s_hdr[4 * tid + 1] << 8) |
                              ((uint32_t)s_hdr[4 * tid + 2] << 16) |
                              ((uint32_t)s_hdr[4 * tid + 3] << 24);
        *to_global(reinterpret_cast<uint32_t*>(J.out + tile * kTileBlocks + 4 * tid)) = word;
    }
    const bool last_tile = tile + 1 == g.tiles_per_job;
    if (last_tile) {
        for (uint32_t off = (tile + 1) * kTileBlocks + 4u * tid; off < R;
             off += 4u * kThreads)
            *to_global(reinterpret_cast<uint32_t*>(J.out + off)) = 0u;
    }
    if (wave == 0) {
        bool gave_up = false;
        const uint32_t prefix = lookback(p.tile_state, t, tile, sc.total, p.epoch, p.error,
                                         p.error_marker, &bound, &gave_up);
        if (gave_up && lane == 0) s_abort = 1;
        if (lane == 0) {
            s_prefix = prefix;
            if (last_tile)
                __hip_atomic_store(&p.host_sizes[job], R + prefix + sc.total,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (tile == 0)
                __hip_atomic_store(&p.host_bounds[job], eb, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    if (bad) flag_error(p.error, p.error_marker, kErrSpin);
    __syncthreads();
    if (s_abort) return;

    uint32_t* dst = reinterpret_cast<uint32_t*>(J.out + R + s_prefix + sc.exclusive);
    if (has_o) *to_global(dst) = outlier;
    dst += has_o ? 1 : 0;
    const uint32_t rmax = wave_max(rate);
    if (rmax == 0) return;
    const uint32_t count_words = rate ? rate + 1u : 0u;
    uint32_t P[16];
    residual_rows_lo(d, P);
    transpose16x2(P);  // rows 0..15 = words w_0..w_15
    store_words<16>(dst, P, count_words < 16u ? count_words : 16u,
                    rmax < 15u ? rmax + 1u : 16u);
    if (rmax >= 16u) {
        residual_rows_hi(d, P);
        transpose16x2(P);  // words w_16..w_31
        store_words<16>(dst + 16, P, count_words > 16u ? count_words - 16u : 0u,
                        rmax - 15u);
        if (rate == 32u) *to_global(dst + 32) = residual_plane31(d);
    }
}

// ---- persistent encoder ----------------------------------------------------
//
// For launches whose blocks are all whole, inside one layer and 16-byte
// aligned (every segment length and layer length a multiple of 32 values,
// every page 16-byte aligned) -- the shape of KV pages.  Workgroup w encodes
// tiles w, w + G, w + 2G, ... (G = gridDim.x, at most the number of
// co-resident workgroups), one 32-value block per thread held in registers
// together with the block's min/max keys.  Per tile t:
//   a. exchange: min/max over all tiles of t's job -> bound, reciprocal
//   b. rates: while every |x * recip| of a block stays below 2^30 and the block
//      holds no NaN, the quantizer (cu:10-25) is monotone in x, so the
//      block's largest |q| -- its rate (cu:221-222) -- is that of its smallest
//      or largest value: two quantizations per block.  Tile scan, header
//      bytes (cu:226-229) and t's aggregate follow before any quantizing.
//   d. look-back -> t's payload offset
//   c. the next tile (loaded into registers one iteration ago) -> its block
//      keys and min/max, published
//   e. quantize t into 16-bit fields, transpose to stream words, stage the
//      wave's payload in LDS and write it with coalesced 16-byte stores
//   f. the next tile becomes current; its successor starts loading
// Wait-for order: the exchange of t needs the min/max of t's job, the
// look-back of t the aggregates of t's predecessors.  Following what a wait
// depends on always reaches a strictly earlier tile within at most two steps
// once a job has at most G/2 tiles (a publish that depends on a wait is the
// min/max of tile u + G, behind the look-back of u; tiles u + G and u are in
// different jobs), so with all G workgroups resident no cycle of waits
// exists.  All waits are bounded.

// threadIdx.x behind an empty asm: values derived from it inside the tile
// loop are recomputed each iteration instead of being hoisted out of the
// loop and held in registers for its whole length.
__device__ __forceinline__ int loop_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Per-tile uniform context.
struct TileCtx {
    uint32_t t;     // tile number in the launch
    int gi;         // group
    uint32_t job;   // job index
    uint32_t tile;  // tile within the job
};

// The job record of a tile, read where it is needed (scalar loads through
// the constant cache) rather than carried across the tile loop in scalar
// registers.
__device__ __forceinline__ CompressJob job_of(const CompressParams& p, const TileCtx& c) {
    return job_at(p, c.job);
}

// Group lookup from first-tile numbers kept in LDS (a loop over kernel
// arguments would keep all of them in scalar registers across the tile loop).
__device__ __forceinline__ TileCtx tile_ctx(const CompressParams& p, uint32_t t,
                                            const uint32_t* s_gfirst) {
    const TilePlace pl = place_tile(p.groups, s_gfirst, p.num_groups, t);
    TileCtx c;
    c.t = t;
    c.gi = pl.gi;
    c.job = pl.job;
    c.tile = pl.tile;
    return c;
}

// Whether this thread's block exists (all existing blocks are whole here).
__device__ __forceinline__ bool block_exists(const Group& g, uint32_t tile, int tid) {
    return (tile * kTileBlocks + (uint32_t)tid) * kBlockElems < (uint32_t)g.n;
}

// Source element of this thread's block.  A wave's 64 blocks inside one
// layer are placed with wave-uniform (scalar) arithmetic and one scalar load
// of the layer map; otherwise each lane maps its own block.  Element indices
// of a segment are below 2^29.
__device__ __forceinline__ uint64_t enc_block_source(const Group& g, uint32_t tile,
                                                     int wave, int lane, uint32_t* bad) {
    constexpr uint32_t kRun = 64u * kBlockElems;
    const uint32_t E = tile * (uint32_t)kTileElems + (uint32_t)wave * kRun;
    if (g.layers == nullptr) return E + (uint32_t)lane * kBlockElems;
    const uint32_t epl = (uint32_t)g.elements_per_layer;
    const uint32_t per_prefix = (uint32_t)g.selected_layers * epl;
    const uint32_t pre = divide(E, g.prefix_div);
    const uint32_t within = E - pre * per_prefix;
    const uint32_t layer = divide(within, g.layer_div);
    const uint32_t inner = within - layer * epl;
    if (inner + kRun <= epl) {
        int64_t l = load_const(g.layers, layer);
        if (l < 0 || (uint64_t)l >= g.source_layers) {
            *bad = 1;
            l = 0;
        }
        return ((uint64_t)pre * g.source_layers + (uint64_t)l) * epl + inner +
               (uint32_t)lane * kBlockElems;
    }
    return layer_cursor(g, (uint64_t)tile * kTileElems,
                        ((uint32_t)wave * 64u + (uint32_t)lane) * kBlockElems, bad)
        .src_index;
}

// Sixteen zero words, the source of blocks that do not exist: every lane
// then loads unconditionally.  (Loads under a branch make the compiler wait
// for all outstanding memory operations at the next use of any earlier
// load, which would tie the persistent encoder's polls to its prefetch.)
__device__ __attribute__((aligned(16))) uint32_t g_zero_block[kBlockElems / 2];

// This thread's block (zeros when it does not exist, or when `live` is
// false): four 16-byte loads.  A layer index outside [0, source_layers) is
// reported at once (the block is then read from layer 0).
__device__ __forceinline__ void load_block_regs(const CompressParams& p, const TileCtx& c,
                                                const Group& g, int wave, int lane,
                                                uint32_t* d, bool live = true) {
    const bool ex = live && block_exists(g, c.tile, wave * 64 + lane);
    uint32_t bad = 0;
    const uint64_t off = ex ? enc_block_source(g, c.tile, wave, lane, &bad) : 0;
    if (bad) flag_error(p.error, p.error_marker, kErrLayerIndex);
    const g_u32x4* src = ex ? (const g_u32x4*)to_global(job_of(p, c).in + off)
                            : (const g_u32x4*)to_global(&g_zero_block[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 v = src[i];
        d[4 * i + 0] = v.x;
        d[4 * i + 1] = v.y;
        d[4 * i + 2] = v.z;
        d[4 * i + 3] = v.w;
    }
}

// Source of a tile's blocks for one wave, worked out ahead of the loads: when
// the wave's 64 blocks are consecutive in memory, `base` is its first block
// (wave-uniform) and lane l reads base + 32 l; otherwise base is null and
// each lane maps its own block when loading.
struct WaveSource {
    const uint16_t* base;
};

__device__ __forceinline__ WaveSource wave_source(const CompressParams& p, const TileCtx& c,
                                                  const Group& g, int wave) {
    constexpr uint32_t kRun = 64u * kBlockElems;
    WaveSource s;
    const uint16_t* in = job_of(p, c).in;
    const uint32_t E = c.tile * (uint32_t)kTileElems + (uint32_t)wave * kRun;
    if (g.layers == nullptr) {
        s.base = in + E;
        return s;
    }
    const uint32_t epl = (uint32_t)g.elements_per_layer;
    const uint32_t per_prefix = (uint32_t)g.selected_layers * epl;
    const uint32_t pre = divide(E, g.prefix_div);
    const uint32_t within = E - pre * per_prefix;
    const uint32_t layer = divide(within, g.layer_div);
    const uint32_t inner = within - layer * epl;
    const int64_t l = load_const(g.layers, layer);
    s.base = (inner + kRun <= epl && l >= 0 && (uint64_t)l < g.source_layers)
                 ? in + ((uint64_t)pre * g.source_layers + (uint64_t)l) * epl + inner
                 : nullptr;
    return s;
}

// This thread's block from a WaveSource (zeros when it does not exist, or
// when `live` is false).
__device__ __forceinline__ void load_block_from(const CompressParams& p, const TileCtx& c,
                                                const Group& g, WaveSource s, int wave,
                                                int lane, uint32_t* d, bool live) {
    if (s.base == nullptr) {
        load_block_regs(p, c, g, wave, lane, d, live);
        return;
    }
    const bool ex = live && block_exists(g, c.tile, wave * 64 + lane);
    const g_u32x4* src = ex ? (const g_u32x4*)to_global(s.base + (uint32_t)lane * kBlockElems)
                            : (const g_u32x4*)to_global(&g_zero_block[0]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 v = src[i];
        d[4 * i + 0] = v.x;
        d[4 * i + 1] = v.y;
        d[4 * i + 2] = v.z;
        d[4 * i + 3] = v.w;
    }
}

// Block keys packed as (min key << 16) | max key, plus whether the block
// holds a NaN (fminf/fmaxf skip NaN, cu:78-79; the quantizer does not).
//
// Fast case on the raw BF16 patterns: read as signed 16-bit numbers, the
// patterns with the sign bit clear order by value and lie above all others;
// read as unsigned numbers, the patterns with the sign bit set lie above all
// others and order by magnitude.  So in a block holding both kinds, the
// signed maximum is its largest value and the unsigned maximum its smallest
// (two packed operations per pair of values).  NaN patterns exceed every
// other pattern of their sign (0x7F81.. and 0xFF81..) and are caught by the
// range checks; blocks of one sign, or with a NaN, take the general path.
__device__ __forceinline__ uint32_t block_keys(const uint32_t* d, bool exists,
                                               uint32_t& nan) {
    nan = 0;
    if (!exists) return (kKeyEmptyMin << 16) | kKeyEmptyMax;
    s16x2 smax = {(short)-32768, (short)-32768};
    u16x2 umax = {0u, 0u};
#pragma unroll
    for (int i = 0; i < kBlockElems / 2; ++i) {
        smax = __builtin_elementwise_max(smax, __builtin_bit_cast(s16x2, d[i]));
        umax = __builtin_elementwise_max(umax, __builtin_bit_cast(u16x2, d[i]));
    }
    const int32_t hs = smax.x > smax.y ? smax.x : smax.y;
    const uint32_t hu = umax.x > umax.y ? umax.x : umax.y;
    if (hs >= 0 && hs <= 0x7F80 && hu >= 0x8000u && hu <= 0xFF80u)
        return ((~hu & 0xFFFFu) << 16) | ((uint32_t)hs | 0x8000u);
    u16x2 mn = {0xFFFFu, 0xFFFFu}, mx = {0u, 0u};
    for (int i = 0; i < kBlockElems / 2; ++i) {
        // key = sign ? ~h : h | 0x8000, for both halves at once
        const uint32_t neg = __builtin_bit_cast(
            uint32_t, __builtin_bit_cast(s16x2, d[i]) >> (short)15);
        const u16x2 k = __builtin_bit_cast(u16x2, d[i] ^ (neg | 0x80008000u));
        mn = __builtin_elementwise_min(mn, k);
        mx = __builtin_elementwise_max(mx, k);
    }
    uint32_t kmin = mn.x < mn.y ? mn.x : mn.y;
    uint32_t kmax = mx.x > mx.y ? mx.x : mx.y;
    if (!(kmin >= 0x007Fu && kmax <= 0xFF80u)) {
        // NaN keys fall outside [key(-inf), key(+inf)]: redo value by value.
        nan = 1;
        float lo = FLT_MAX, hi = -FLT_MAX;
        for (int v = 0; v < kBlockElems; ++v) {
            const float x = (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
            lo = fminf(lo, x);
            hi = fmaxf(hi, x);
        }
        kmin = lo == FLT_MAX ? kKeyEmptyMin : bf16_key(lo);
        kmax = hi == -FLT_MAX ? kKeyEmptyMax : bf16_key(hi);
    }
    return (kmin << 16) | kmax;
}

// Keys of -inf (min) and +inf (max), kept as the keys of a block holding a
// NaN: they mark the block so that its wave takes the exact quantizer.
constexpr uint32_t kNanRateKeys = (0x007Fu << 16) | 0xFF80u;

// Rate of a block from its keys, for a block whose values all satisfy
// |x * recip| <= kFastLimit and that holds no NaN: the quantizer is monotone
// there, so the largest |q| is that of the block's smallest or largest value.
template <int kQuant>
__device__ __forceinline__ uint32_t rate_from_keys(uint32_t keys, float recip) {
    const uint32_t m = max(magnitude(quantize<kQuant>(key_value(keys >> 16), recip)),
                           magnitude(quantize<kQuant>(key_value(keys & 0xFFFFu), recip)));
    return m ? 32u - (uint32_t)__builtin_clz(m) : 0u;
}

// Rate of a block by quantizing every value (NaN, saturation, wrap).  Each
// value's reciprocal passes through an empty asm that takes the running OR
// as an input, so the values are done one after the other (this rare path
// then needs few registers).
template <int kQuant>
__device__ __forceinline__ uint32_t rate_by_quantizing(const uint32_t* d, float recip) {
    uint32_t orv = 0;
#pragma unroll
    for (int v = 0; v < kBlockElems; ++v) {
        float r = recip;
        asm volatile("" : "+v"(r) : "v"(orv));
        orv |= magnitude(quant_elem<kQuant, true>(d, v, kBlockElems, r));
    }
    return orv ? 32u - (uint32_t)__builtin_clz(orv) : 0u;
}

// a * b + c for a, b < 2^24 as one instruction (the compiler otherwise
// expands s * 0x8001 for a 0/1 value s into an arithmetic shift and an AND).
__device__ __forceinline__ uint32_t mad_u24(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t d;
    asm("v_mad_u32_u24 %0, %1, %2, %3" : "=v"(d) : "v"(a), "s"(b), "v"(c));
    return d;
}

// Rows of 16-bit fields (sign << 15) | |q| for a block whose |q| < 2^15 and
// whose |t| < 2^31 (the identity stated at field_sign in kvszp_bits.h): row
// k holds elements k^7 (low half) and 16+(k^7) (high half).  After
// transpose16x2, rows 0..14 are planes 0..14 (stream words w_1..w_15) and
// row 15 is the sign word w_0.  The two-roundings sign test t < 0 is t's
// sign bit (t is never -0.0: v + 0.5 = 0 rounds to +0.0; the caller excludes
// NaN).  Rows are chained through the block's words (an empty asm) so the
// scheduler does not start all 32 conversions at once.
template <int kQuant>
__device__ __forceinline__ void build_rows_signhi(uint32_t* d, float recip, uint32_t* P) {
    constexpr uint32_t kSignHi = 0x8001u;
    uint32_t prev = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int e0 = row_lo_elem(k), e1 = row_hi_elem(k);
        asm volatile("" : "+v"(d[e0 >> 1]), "+v"(d[e1 >> 1]) : "v"(prev));
        const float x0 = (e0 & 1) ? bf16_hi(d[e0 >> 1]) : bf16_lo(d[e0 >> 1]);
        const float x1 = (e1 & 1) ? bf16_hi(d[e1 >> 1]) : bf16_lo(d[e1 >> 1]);
        uint32_t f[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float x = h ? x1 : x0;
            const float t = kQuant ? __builtin_fmaf(x, recip, 0.5f) : x * recip + 0.5f;
            const uint32_t c = cvt_abs_u32(t);
            const uint32_t s = kQuant ? (field_sign(t, 1) ? 1u : 0u)
                                      : __float_as_uint(t) >> 31;
            f[h] = mad_u24(s, kSignHi, c);  // (c + s) | (s << 15)
        }
        P[k] = __builtin_amdgcn_perm(f[1], f[0], 0x05040100u);  // low halves
        prev = P[k];
    }
}

// Tile-level facts of the tile whose payload waits in the staging words.
struct PendingTile {
    uint32_t t, tile, job, total, R, last, first;
    float eb;
    uint8_t* out;
};

// The pending tile's prefix into LDS and, for the first / last tile of its
// job, the job's bound / size into host memory (one lane).
__device__ __forceinline__ void pending_results(const CompressParams& p, const PendingTile& q,
                                                uint32_t pf, uint32_t* s_prefix) {
    *s_prefix = pf;
    if (q.last)
        __hip_atomic_store(&p.host_sizes[q.job], q.R + pf + q.total, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    if (q.first)
        __hip_atomic_store(&p.host_bounds[q.job], q.eb, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
}

// ---- persistent encoder --------------------------------------------------------
// Two waves per workgroup and two blocks per thread: lane l of wave w holds
// blocks 128w + l and 128w + 64 + l of the tile (its 64-block runs 2w and
// 2w + 1).  The per-tile work that does not grow with the block count (bound
// exchange, scan, look-back, tile bookkeeping) is then shared by 128 blocks
// per wave.
constexpr int kEncThreads = 128;
constexpr int kEncWaves = kEncThreads / 64;
constexpr int kEncStageWords = 2 * 64 * 16 + 16;  // 128 blocks of <= 16 words

// Launches whose jobs have at most this many tiles run the persistent
// encoder that does the look-back of the staged tile beside the bound
// exchange, before the first barrier (two barriers per tile); longer jobs run
// the one that does it after the tile scan, behind a third barrier.  A
// look-back that waits before the first barrier holds back the tile's
// aggregate, which the look-backs of the job's later tiles need; over long
// jobs those delays add up (measured on MI355X: launches of 7- and 21-tile
// jobs 2.5 % faster with the early look-back, of 28-tile jobs 1.3 % slower,
// of 56-tile jobs 7 % slower).
constexpr uint32_t kEarlyLookbackTiles = 24;

// Largest fl(|x| * recip) for which every value of a job quantizes to a
// sign-high field: |t| <= 32766.5 gives |q| = c + s <= 32767 < 2^15 (for
// either quantizer; fl and fma round monotonically).
constexpr float kFastLimit = 32766.0f;

// Wave 0: the min/max keys over all tiles of the job (lane i polls tiles
// i, i + 64, ...; all lanes end together).

// `probe` (when `have_probe`) is an earlier read of lane's first word.
// Returns true (on every lane) when a bounded wait gave up.
__device__ __forceinline__ bool job_keys(const CompressParams& p, uint32_t first_t,
                                         uint32_t tiles, int lane, uint32_t& kmin,
                                         uint32_t& kmax, bool have_probe,
                                         unsigned long long probe, const WaitBound& bound) {
    kmin = kKeyEmptyMin;
    kmax = kKeyEmptyMax;
    bool gave_up = false;
    for (uint32_t i = (uint32_t)lane; i < tiles; i += 64u) {
        const unsigned long long* slot = &p.tile_minmax[first_t + i];
        unsigned long long w = have_probe && i < 64u ? probe : load_relaxed(slot);
        have_probe = false;
        uint64_t deadline = 0;
        for (uint32_t spins = 0; (uint32_t)(w >> 32) != p.epoch; ++spins) {
            if (bound.word != nullptr) {
                if (wait_gives_up(bound, deadline, spins)) {
                    gave_up = true;
                    break;
                }
            } else if (spins >= kSpinLimit) {
                flag_error(p.error, p.error_marker, kErrSpin);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            w = load_relaxed(slot);
        }
        if (gave_up) break;
        const uint32_t lo = (uint32_t)(w >> 16) & 0xFFFFu, hi = (uint32_t)w & 0xFFFFu;
        kmin = lo < kmin ? lo : kmin;
        kmax = hi > kmax ? hi : kmax;
    }
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    return __ballot(gave_up) != 0ull;
}

// A tile's min/max keys out (one barrier): both waves reduce their lanes'
// keys, thread 0 combines and publishes the epoch-tagged word.
__device__ __forceinline__ void publish_keys2(const CompressParams& p, uint32_t t,
                                              uint32_t kmin, uint32_t kmax,
                                              uint32_t* s_min, uint32_t* s_max,
                                              int wave, int lane) {
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    if (lane == 0) {
        s_min[wave] = kmin;
        s_max[wave] = kmax;
    }
    __syncthreads();
    if (wave == 0 && lane == 0) {
        kmin = s_min[1] < kmin ? s_min[1] : kmin;
        kmax = s_max[1] > kmax ? s_max[1] : kmax;
        store_relaxed(&p.tile_minmax[t],
                      ((unsigned long long)p.epoch << 32) | (kmin << 16) | kmax);
    }
}

// A wave's payload staged in LDS: the block is words [off, off + count) of
// the wave's payload.  The stream words are the transposed rows P:
// w_j = P[j] (kSignHi false), or w_0 = P[15] and w_j = P[j - 1] (sign-high
// rows).  Words are written from the highest index down: a lane's unused
// slots (index >= count) only ever fall on words of later blocks, which are
// written afterwards, or past the payload end, so `stage` needs room for
// the payload plus 16 words.
template <bool kSignHi>
__device__ __forceinline__ void stage_payload(const uint32_t* P, uint32_t count,
                                              uint32_t off, uint32_t cmax,
                                              uint32_t* stage) {
    __asm__ volatile("" ::: "memory");
    if (count) {
        uint32_t* s = stage + off;
#pragma unroll
        for (int j = 15; j >= 0; --j)
            if ((uint32_t)j < cmax) s[j] = kSignHi ? P[(j + 15) & 15] : P[j];
    }
    __asm__ volatile("" ::: "memory");
}

// Writes a wave's staged payload (`words` words) to `dst` (4-byte aligned):
// lane l moves words 4l .. 4l + 3 of every 256-word chunk with one 16-byte
// LDS read and one 16-byte store (each store instruction covers 1 KiB of
// contiguous stream), then lanes 0..2 the last words.
__device__ __forceinline__ void copy_payload(uint32_t* dst, uint32_t words,
                                             const uint32_t* stage, int lane) {
    __builtin_amdgcn_wave_barrier();
    __asm__ volatile("" ::: "memory");
    g_u32* d = to_global(dst);
    const uint32_t quads = words >> 2;
    for (uint32_t q = (uint32_t)lane; q < quads; q += 64u)
        *(g_u32x4_a4*)(d + 4u * q) = *(const u32x4*)(stage + 4u * q);
    const uint32_t tail = 4u * quads + (uint32_t)lane;
    if (tail < words) d[tail] = stage[tail];
    __builtin_amdgcn_wave_barrier();
    __asm__ volatile("" ::: "memory");  // before the words are reused
}

// Writes the payload of a wave whose blocks all hold one value, quantized to
// q != 0 (`words` words to `dst`, 4-byte aligned): every block is the same
// rate + 1 words (cu:302-358), the sign word and planes 0 .. rate - 1 of |q|,
// each word all ones or all zeros.  Lane l writes words 4l .. 4l + 3 of every
// 256-word chunk, as copy_payload does, with no staging.
__device__ __forceinline__ void fill_uniform_payload(uint32_t* dst, uint32_t words,
                                                     int32_t q, int lane) {
    const uint32_t m = magnitude(q);
    const uint32_t period = 33u - (uint32_t)__builtin_clz(m);  // rate + 1
    const uint32_t sign = q < 0 ? ~0u : 0u;
    g_u32* d = to_global(dst);
    const uint32_t quads = words >> 2;
    for (uint32_t qd = (uint32_t)lane; qd < quads; qd += 64u) {
        uint32_t j = (4u * qd) % period, w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = j == 0 ? sign : 0u - ((m >> (j - 1u)) & 1u);
            j = j + 1u == period ? 0u : j + 1u;
        }
        u32x4 v;
        v.x = w[0];
        v.y = w[1];
        v.z = w[2];
        v.w = w[3];
        *(g_u32x4_a4*)(d + 4u * qd) = v;
    }
    const uint32_t tail = 4u * quads + (uint32_t)lane;
    if (tail < words) {
        const uint32_t j = tail % period;
        d[tail] = j == 0 ? sign : 0u - ((m >> (j - 1u)) & 1u);
    }
}

// Words 16 .. count - 1 of a block (rates above 15), exactly (no slot past
// `count` is written: the low words of later blocks are already in place).
__device__ __forceinline__ void stage_high_words(const uint32_t* P, uint32_t count,
                                                 uint32_t off, uint32_t* stage) {
    __asm__ volatile("" ::: "memory");
    uint32_t* s = stage + off + 16;
#pragma unroll
    for (int j = 0; j < 16; ++j)
        if ((uint32_t)j + 16u < count) s[j] = P[j];
    __asm__ volatile("" ::: "memory");
}

// Three waves per SIMD (at most 168 VGPRs, no scratch).
//
// Per tile: the next tile starts loading; (c) its keys; (a) wave 0 gathers
// the job's min/max and works out the bound while wave 1 finishes the
// look-back of the tile staged one iteration earlier (kEarly; one barrier
// hands both over); the next tile's keys out; (b) rates, the wave scans, the
// tile scan (second barrier), header and aggregate out; without kEarly the
// look-back here, behind a third barrier; (d) the staged tile's payload out;
// (e) per 64-block half of each wave: rows and staging.
//
// Deferred stores: a tile's payload is staged in LDS at wave-relative
// offsets and written out one iteration later, after the tile's look-back,
// which by then normally finds its predecessors' prefixes published and does
// not wait.  Staging needs only the wave's own offsets, so each half is
// staged as soon as its rows exist and no more than one half's rows are held.
//
// Wait order with deferral: give the iteration that holds tile t rank t.
// Its waits are the exchange of t (before its first barrier) and the
// look-back of t - G (before its first barrier with kEarly, after its second
// without).  The exchange needs the min/max of the tiles u of t's
// job, published after the first barrier of the iteration holding u - G
// (rank u - G < t, as a job has fewer than G tiles; for u = t the prologue
// or the previous iteration of this workgroup).  The look-back of t - G
// needs the aggregates of tiles x < t - G, published after the second
// barrier of iteration x (rank x < t).  Earlier iterations of the same
// workgroup have ranks t - G, t - 2G, ...  Every wait depends only on
// iterations of lower rank: no cycle while all G workgroups are resident.
// The flush after the loop (the last tile's look-back) waits on lower ranks
// too.
//
// Without full residency (another kernel holds CUs, or a second encoder
// launch shares the device) a wait can depend on a workgroup that has not
// started and cannot start while the started ones spin.  Every wait here is
// therefore bounded in time (WaitBound): the first one to outlast the bound
// marks the launch, every other wait gives up on reading the mark, all
// workgroups leave at their next barrier, and the host encodes the call
// again with the pre-pass schedule (no residency assumption).  Normal waits
// last microseconds; the bound is hundreds, so the mark costs nothing when
// the device is not contended.
template <int kQuant, bool kEarly>
__device__ __forceinline__ void compress_persistent(const CompressParams& p) {
    __shared__ uint32_t s_wave[2][kEncWaves];
    __shared__ uint32_t s_min[kEncWaves], s_max[kEncWaves];
    __shared__ float s_bnd[2][2];      // by tile parity: eb, recip
    __shared__ uint32_t s_fast[2];     // by tile parity: job on the fast path
    __shared__ uint32_t s_prefix[3];   // by tile parity; [2] for the last tile
    __shared__ uint32_t s_gfirst[kMaxGroups];
    __shared__ uint8_t s_rate[2][kTileBlocks];
    __shared__ PendingTile s_pend[2];  // by the parity of the tile it holds
    // staged: wave offset, words (bit 31: the payload is one block repeated,
    // not staged), that block's q
    __shared__ uint32_t s_pwave[kEncWaves][3];
    __shared__ uint32_t s_abort;       // a bounded wait of this launch gave up
    __shared__ __attribute__((aligned(16))) uint32_t s_stage[kEncWaves][kEncStageWords];

    publish_seq(p.host_ctl, p.seq);
    if ((int)threadIdx.x < p.num_groups) s_gfirst[threadIdx.x] = p.groups[threadIdx.x].first_tile;
    if (threadIdx.x == 0) s_abort = 0;
    __syncthreads();
    const uint32_t G = gridDim.x;
    const bool fused = p.bound_mode == kBoundFused;
    const WaitBound bound = wait_bound(p.abort_word, p.host_ctl, p.seq, p.epoch, p.wait_ticks);
    bool pending = false;  // a tile's payload waits in the staging words
    bool aborted = false;  // stop: the host encodes this launch again

    // Prologue: the first tile and its keys (published).
    TileCtx cur = tile_ctx(p, persistent_first_tile(blockIdx.x, G, p.slot_cus), s_gfirst);
    uint32_t D0[16], D1[16], N0[16], N1[16];
    // Keys of the current tile's blocks: the published keys, except that a
    // block holding a NaN keeps the keys of -inf and +inf (kNanRateKeys),
    // which keeps its wave off the fast path.
    uint32_t keys0, keys1;
    bool has_next;
    TileCtx nxt;
    {
        const int tid = loop_tid();
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const Group& g = p.groups[cur.gi];
        // ArgTable launches: the job records were written by the host just
        // before the launch and sit in no cache.  Workgroups 0-7 (one on
        // each XCD) read one word of every 64-byte line of the table before
        // their first tile, so that the record reads of the other
        // workgroups' later tiles hit their XCD's L2.
        uint32_t touch0 = 0, touch1 = 0;
        if (p.jobs_inline == 2 && blockIdx.x < 8u) {
            const uint32_t lines = (p.num_jobs * (uint32_t)sizeof(CompressJob) + 63u) / 64u;
            typedef const __attribute__((address_space(4))) unsigned char k_u8;
            k_u8* k = (k_u8*)__builtin_amdgcn_kernarg_segment_ptr() +
                      arg_table_offset<CompressParams>();
            const uint32_t i0 = (uint32_t)tid, i1 = (uint32_t)tid + kEncThreads;
            touch0 = *(const __attribute__((address_space(1))) uint32_t*)(k + 64u * (i0 < lines ? i0 : 0u));
            touch1 = *(const __attribute__((address_space(1))) uint32_t*)(k + 64u * (i1 < lines ? i1 : 0u));
        }
        load_block_regs(p, cur, g, 2 * wave, lane, D0);
        load_block_regs(p, cur, g, 2 * wave + 1, lane, D1);
        uint32_t nan0, nan1;
        keys0 = block_keys(D0, block_exists(g, cur.tile, 128 * wave + lane), nan0);
        keys1 = block_keys(D1, block_exists(g, cur.tile, 128 * wave + 64 + lane), nan1);
        if (fused)
            publish_keys2(p, cur.t, min(keys0 >> 16, keys1 >> 16),
                          max(keys0 & 0xFFFFu, keys1 & 0xFFFFu), s_min, s_max, wave, lane);
        if (nan0) keys0 = kNanRateKeys;
        if (nan1) keys1 = kNanRateKeys;
        has_next = cur.t + G < p.total_tiles;
        if (has_next) nxt = tile_ctx(p, cur.t + G, s_gfirst);
        __asm__ volatile("" ::"v"(touch0), "v"(touch1));  // older than the tile's loads
        __syncthreads();  // thread 0 has read s_min/s_max before c. rewrites them
    }

    // One tile.  X holds this tile's values; the next tile is loaded into Y
    // (whose values were used up in the previous iteration), and the next
    // call swaps the roles (no copies).
    uint32_t parity = 0;
    auto iteration = [&](uint32_t (&X0)[16], uint32_t (&X1)[16], uint32_t (&Y0)[16],
                         uint32_t (&Y1)[16]) -> bool {
        const int tid = loop_tid();
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const Group& g = p.groups[cur.gi];
        const uint32_t blk0 = 128u * (uint32_t)wave + (uint32_t)lane;

        // First reads of the waits (wave 0: the job's min/max words for a.;
        // wave 1: the pending tile's first look-back window), then the next
        // tile's loads: loads and stores retire in order, so reads issued
        // after the loads would wait for them, while these wait only for
        // themselves.  The next tile's values are needed at c.  Every path
        // issues one read and then eight loads, unconditionally (from a
        // harmless address or the zero block where there is nothing to
        // read), so the wait for the read counts only the read.
        const unsigned long long* paddr = &p.tile_state[cur.t];
        if (wave == 0) {
            if (fused)
                paddr = &p.tile_minmax[cur.t - cur.tile +
                                       min((uint32_t)lane, g.tiles_per_job - 1u)];
        } else if (pending) {
            const PendingTile& q = s_pend[parity ^ 1u];
            paddr = lookback_first_addr(p.tile_state, q.t, q.tile);
        }
        const unsigned long long probe = load_relaxed(paddr);
        {
            // Without a next tile the loads read the zero block (values
            // unused), so that the loads are the same on every path.
            const TileCtx& lc = has_next ? nxt : cur;
            const Group& gl = p.groups[lc.gi];
            load_block_from(p, lc, gl, wave_source(p, lc, gl, 2 * wave), 2 * wave, lane, Y0,
                            has_next);
            load_block_from(p, lc, gl, wave_source(p, lc, gl, 2 * wave + 1), 2 * wave + 1,
                            lane, Y1, has_next);
        }

        // c. the next tile's keys, while the reads above are in flight; each
        // wave's min/max goes to LDS now and the tile's word out after a.'s
        // barrier, early in the iteration, so that the exchanges of the next
        // iteration, here and in the other workgroups holding tiles of its
        // job, do not wait for it.
        uint32_t nkeys0 = 0, nkeys1 = 0, nnan0 = 0, nnan1 = 0;
        if (has_next) {
            const Group& gn = p.groups[nxt.gi];
            nkeys0 = block_keys(Y0, block_exists(gn, nxt.tile, (int)blk0), nnan0);
            nkeys1 = block_keys(Y1, block_exists(gn, nxt.tile, (int)blk0 + 64), nnan1);
            if (fused) {
                const uint32_t kmin = wave_min(min(nkeys0 >> 16, nkeys1 >> 16));
                const uint32_t kmax = wave_max(max(nkeys0 & 0xFFFFu, nkeys1 & 0xFFFFu));
                if (lane == 0) {
                    s_min[wave] = kmin;
                    s_max[wave] = kmax;
                }
            }
        }

        // a. wave 0: the bound (one barrier hands it over; thread 0 then
        // publishes the next tile's min/max).
        if (wave == 0) {
            const float eps = job_of(p, cur).eps;
            float eb = eps;
            uint32_t fast = 0;
            if (fused) {
                uint32_t kmin, kmax;
                if (job_keys(p, cur.t - cur.tile, g.tiles_per_job, lane, kmin, kmax, true, probe,
                             bound) && lane == 0)
                    s_abort = 1;
                eb = relative_bound(eps, kmin, kmax);
                const float jabs = fmaxf(fabsf(min_key_value(kmin)), fabsf(max_key_value(kmax)));
                fast = jabs * (0.5f / eb) <= kFastLimit ? 1u : 0u;
            }
            if (lane == 0) {
                s_bnd[parity][0] = eb;
                s_bnd[parity][1] = 0.5f / eb;  // cu:166, IEEE division
                s_fast[parity] = fast;
            }
        } else if (kEarly && pending) {
            // wave 1 meanwhile: the pending tile's look-back (its first read
            // went out with the loads; its predecessors published their
            // aggregates early in the previous iteration).  The same barrier
            // hands the prefix over.
            const PendingTile& q = s_pend[parity ^ 1u];
            bool gave_up = false;
            const uint32_t pf = lookback_wait(p.tile_state, q.t, q.tile, q.total,
                                              p.epoch, p.error, p.error_marker, true, probe,
                                              &bound, &gave_up);
            if (gave_up && lane == 0) s_abort = 1;
            if (lane == 0) pending_results(p, q, pf, &s_prefix[parity]);
        }
        __syncthreads();
        if (s_abort) {
            aborted = true;
            return false;
        }
        if (has_next) {
            if (fused && tid == 0) {
                const uint32_t kmin = min(s_min[0], s_min[1]), kmax = max(s_max[0], s_max[1]);
                store_relaxed(&p.tile_minmax[nxt.t],
                              ((unsigned long long)p.epoch << 32) | (kmin << 16) | kmax);
            }
            if (nnan0) nkeys0 = kNanRateKeys;
            if (nnan1) nkeys1 = kNanRateKeys;
        }

        // b. rates (cu:212-231) and the wave's offsets.  Fast path when no
        // block of the wave holds a NaN and every |x * recip| is at most
        // kFastLimit (known for the whole job from its min/max, or else from
        // the keys): the quantizer is monotone there, so a block's largest
        // |q| is at its smallest or largest value and the rate comes from
        // the keys alone.  Otherwise every value is quantized.
        const float eb = s_bnd[parity][0];
        const float recip = s_bnd[parity][1];
        const bool ex0 = block_exists(g, cur.tile, (int)blk0);
        const bool ex1 = block_exists(g, cur.tile, (int)blk0 + 64);
        bool fast_w = false;
        if (__ballot(keys0 == kNanRateKeys || keys1 == kNanRateKeys) == 0ull) {
            if (s_fast[parity] != 0) {
                fast_w = true;
            } else {
                const float bmax0 = fmaxf(fabsf(key_value(keys0 >> 16)), fabsf(key_value(keys0 & 0xFFFFu)));
                const float bmax1 = fmaxf(fabsf(key_value(keys1 >> 16)), fabsf(key_value(keys1 & 0xFFFFu)));
                const bool ok = (!ex0 || bmax0 * recip <= kFastLimit) &&
                                (!ex1 || bmax1 * recip <= kFastLimit);
                fast_w = __ballot(!ok) == 0ull;
            }
        }
        uint32_t rate0 = 0, rate1 = 0;
        if (fast_w) {
            if (ex0) rate0 = rate_from_keys<kQuant>(keys0, recip);
            if (ex1) rate1 = rate_from_keys<kQuant>(keys1, recip);
        } else {
            // Only existing blocks: an absent block holds zeros, and 0 * recip
            // is NaN (rate 1) when recip is infinite (eb below 0.5 / FLT_MAX).
            if (ex0) rate0 = rate_by_quantizing<kQuant>(X0, recip);
            if (ex1) rate1 = rate_by_quantizing<kQuant>(X1, recip);
        }
        const uint32_t bytes0 = rate0 ? 4u + 4u * rate0 : 0u;
        const uint32_t bytes1 = rate1 ? 4u + 4u * rate1 : 0u;
        const uint32_t incl0 = wave_inclusive_scan(bytes0, lane);
        const uint32_t incl1 = wave_inclusive_scan(bytes1, lane);
        const uint32_t half0 = (uint32_t)__builtin_amdgcn_readlane((int)incl0, 63);
        const uint32_t half1 = (uint32_t)__builtin_amdgcn_readlane((int)incl1, 63);
        const uint32_t rmax0 = wave_max(rate0), rmax1 = wave_max(rate1);
        const uint32_t wave_bytes = half0 + half1;
        s_rate[parity][blk0] = (uint8_t)rate0;
        s_rate[parity][blk0 + 64] = (uint8_t)rate1;
        // Staging slot of each block: word offset in the wave's payload (low
        // half) and word count (high half).
        const uint32_t slot0 = ((incl0 - bytes0) >> 2) | ((rate0 ? rate0 + 1u : 0u) << 16);
        const uint32_t slot1 = ((half0 + incl1 - bytes1) >> 2) | ((rate1 ? rate1 + 1u : 0u) << 16);

        // Tile scan (the barrier), header bytes (padding zeroed by the last
        // tile), aggregate out -- before the rows, so that the look-backs of
        // the tiles after this one find it early.
        if (lane == 0) s_wave[parity][wave] = wave_bytes;
        __syncthreads();
        const uint32_t wb0 = s_wave[parity][0];
        const uint32_t total = wb0 + s_wave[parity][1];
        const uint32_t wave_off = wave ? wb0 : 0u;
        const uint32_t R = g.header_bytes;
        if (tid < kTileBlocks / 4) {
            const uint8_t* r = s_rate[parity];
            const uint32_t word = (uint32_t)r[4 * tid] | ((uint32_t)r[4 * tid + 1] << 8) |
                                  ((uint32_t)r[4 * tid + 2] << 16) |
                                  ((uint32_t)r[4 * tid + 3] << 24);
            *to_global(reinterpret_cast<uint32_t*>(job_of(p, cur).out + cur.tile * kTileBlocks + 4 * tid)) = word;
        }
        const bool last_tile = cur.tile + 1 == g.tiles_per_job;
        if (last_tile) {
            for (uint32_t off = (cur.tile + 1) * kTileBlocks + 4u * tid; off < R;
                 off += 4u * kEncThreads)
                *to_global(reinterpret_cast<uint32_t*>(job_of(p, cur).out + off)) = 0u;
        }
        if (wave == 0) lookback_publish(p.tile_state, cur.t, cur.tile, total, p.epoch);

        // Long jobs: the pending tile's look-back here, after this tile's
        // aggregate is out (wave 1); one more barrier hands the prefix over.
        if (!kEarly && pending) {
            if (wave == 1) {
                const PendingTile& q = s_pend[parity ^ 1u];
                bool gave_up = false;
                const uint32_t pf = lookback_wait(p.tile_state, q.t, q.tile, q.total,
                                                  p.epoch, p.error, p.error_marker, true, probe,
                                                  &bound, &gave_up);
                if (gave_up && lane == 0) s_abort = 1;
                if (lane == 0) pending_results(p, q, pf, &s_prefix[parity]);
            }
            __syncthreads();
            if (s_abort) {
                aborted = true;
                return false;
            }
        }

        // d. the pending tile's payload out (frees the staging words)
        if (pending) {
            const PendingTile& q = s_pend[parity ^ 1u];
            const uint32_t woff = s_pwave[wave][0], words = s_pwave[wave][1];
            if (words) {
                uint32_t* dst = reinterpret_cast<uint32_t*>(q.out + q.R + s_prefix[parity] + woff);
                if (words >> 31)
                    fill_uniform_payload(dst, words & 0x7FFFFFFFu, (int32_t)s_pwave[wave][2],
                                         lane);
                else
                    copy_payload(dst, words, &s_stage[wave][0], lane);
            }
        }

        // e. rows (cu:180-231) and staging (cu:302-358: sign word, then
        // `rate` plane words).  Fast path: sign-high rows (sign << 15) | |q|,
        // whose transpose gives planes 0..14 then the sign word; otherwise
        // the exact quantizer's low fields ((|q| << 1) | sign) & 0xFFFF,
        // whose transpose gives words 0..15 in stream order, and for rates
        // above 15 the high fields |q| >> 15 (words 16..31), staged exactly.
        // A wave whose payload would not fit the staging words (rates far
        // above 15 throughout) stages nothing.  When all its blocks hold one
        // value (every block's min and max keys are the same key: no NaN, no
        // absent block), as on a constant page under a relative bound, its
        // payload is that value's block repeated, written at d. from q alone.
        // Otherwise it marks its job; the host encodes the marked jobs again
        // with the one-workgroup-per-tile kernel.  Sizes, bounds and every
        // other job of this launch come out normally.
        // Only the first wave to mark a job writes host memory: the marks of
        // every wave of a saturated page would be a stream of small writes
        // across the link, most of them to one word.
        const bool overflow = (wave_bytes >> 2) + 16u > (uint32_t)kEncStageWords;
        bool uniform = false;
        if (overflow) {
            const uint32_t ukey = __builtin_amdgcn_readfirstlane(keys0);
            uniform = (ukey >> 16) == (ukey & 0xFFFFu) &&
                      __ballot(keys0 != ukey || keys1 != ukey) == 0ull;
            if (uniform && lane == 0)
                s_pwave[wave][2] =
                    (uint32_t)quantize<kQuant>(key_value(ukey & 0xFFFFu), recip);
        }
        if (overflow && !uniform) {
            if (lane == 0 &&
                __hip_atomic_exchange(&p.job_flags[cur.job], p.epoch, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) != p.epoch) {
                __hip_atomic_store(&p.host_redo[cur.job], p.seq, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(&p.host_ctl[kHostOverflow], p.seq, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
            }
        } else if (!overflow) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t (&X)[16] = h ? X1 : X0;
                const uint32_t rmax = h ? rmax1 : rmax0;
                const uint32_t slot = h ? slot1 : slot0;
                const uint32_t off = slot & 0xFFFFu, count = slot >> 16;
                if (rmax == 0) continue;
                uint32_t P[16];
                const uint32_t cmax = rmax < 15u ? rmax + 1u : 16u;
                if (fast_w) {
                    build_rows_signhi<kQuant>(X, recip, P);
                    transpose16x2(P);
                    stage_payload<true>(P, count, off, cmax, &s_stage[wave][0]);
                } else {
                    uint32_t orv = 0;
                    build_rows_lo_chained<kQuant>(X, recip, P, orv);
                    transpose16x2(P);
                    stage_payload<false>(P, count < 16u ? count : 16u, off, cmax,
                                         &s_stage[wave][0]);
                    if (rmax > 15u) {
                        build_rows_hi_chained<kQuant>(X, recip, P);
                        transpose16x2(P);
                        stage_high_words(P, count, off, &s_stage[wave][0]);
                    }
                }
            }
        }
        if (lane == 0) {
            s_pwave[wave][0] = wave_off;
            s_pwave[wave][1] = !overflow ? wave_bytes >> 2
                               : uniform ? (wave_bytes >> 2) | 0x80000000u : 0u;
        }
        // Written by the wave that reads it first (wave 1's look-back in the
        // next iteration, or the flush below); wave 0 reads it only after the
        // next barrier.
        if (tid == 64) {
            PendingTile q;
            q.t = cur.t;
            q.tile = cur.tile;
            q.job = cur.job;
            q.total = total;
            q.R = R;
            q.last = last_tile;
            q.first = cur.tile == 0;
            q.eb = eb;
            q.out = job_of(p, cur).out;
            s_pend[parity] = q;
        }
        pending = true;

        // f. advance
        if (!has_next) return false;
        cur = nxt;
        keys0 = nkeys0;
        keys1 = nkeys1;
        has_next = cur.t + G < p.total_tiles;
        if (has_next) nxt = tile_ctx(p, cur.t + G, s_gfirst);
        return true;
    };
    for (;;) {
        if (!iteration(D0, D1, N0, N1)) break;
        parity ^= 1u;
        if (!iteration(N0, N1, D0, D1)) break;
        parity ^= 1u;
    }
    // The last staged payload.
    if (pending && !aborted) {
        const int tid = loop_tid();
        const int lane = tid & 63;
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        if (wave == 1) {
            const PendingTile& q = s_pend[parity];
            bool gave_up = false;
            const uint32_t pf = lookback_wait(p.tile_state, q.t, q.tile, q.total,
                                              p.epoch, p.error, p.error_marker, false, 0,
                                              &bound, &gave_up);
            if (gave_up && lane == 0) s_abort = 1;
            if (lane == 0) pending_results(p, q, pf, &s_prefix[2]);
        }
        __syncthreads();
        if (s_abort) return;
        const PendingTile& q = s_pend[parity];
        const uint32_t woff = s_pwave[wave][0], words = s_pwave[wave][1];
        if (words) {
            uint32_t* dst = reinterpret_cast<uint32_t*>(q.out + q.R + s_prefix[2] + woff);
            if (words >> 31)
                fill_uniform_payload(dst, words & 0x7FFFFFFFu, (int32_t)s_pwave[wave][2], lane);
            else
                copy_payload(dst, words, &s_stage[wave][0], lane);
        }
    }
}

template <int kQuant, bool kEarly>
__global__ __launch_bounds__(kEncThreads)
__attribute__((amdgpu_waves_per_eu(3, 3))) void compress_persistent_kernel(CompressParams p) {
    compress_persistent<kQuant, kEarly>(p);
}

// The same with the job records in the kernel arguments (jobs_inline == 2).
template <int kQuant, bool kEarly>
__global__ __launch_bounds__(kEncThreads)
__attribute__((amdgpu_waves_per_eu(3, 3))) void compress_persistent_argtable_kernel(
    CompressParams p, ArgTable) {
    compress_persistent<kQuant, kEarly>(p);
}

// ---- relative-bound pre-pass (jobs too long for the fused exchange) -------

// kIn = 0: BF16 pages, 16-bit keys, NaN ignored (cu:78-79).  kIn = 1:
// contiguous fp32 pages, 32-bit keys, a NaN marks the max word (at::aminmax
// propagates NaN, cuszp_wrapper.cpp:253).
template <int kIn>
__global__ __launch_bounds__(kThreads) void minmax_kernel(MinMaxParams p) {
    __shared__ uint32_t s_min[kThreads / 64];
    __shared__ uint32_t s_max[kThreads / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    publish_seq(p.host_ctl, p.seq);
    const uint32_t t = blockIdx.x;
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];
    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = local / g.tiles_per_job;
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const CompressJob J = job_at(p, job);
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;
    uint32_t bad = 0;
    uint32_t kmin, kmax;
    if constexpr (kIn) {
        uint32_t d[kBlockElems];
        load_block_f32(reinterpret_cast<const float*>(J.in), e0, count,
                       ((uintptr_t)J.in & 15u) == 0, d);
        kmin = 0xFFFFFFFFu;
        kmax = 0u;
        for (uint32_t v = 0; v < count; ++v) {
            const float x = __uint_as_float(d[v]);
            const uint32_t k = x != x ? kKey32Nan : key32(x);
            kmax = k > kmax ? k : kmax;
            if (x == x) kmin = k < kmin ? k : kmin;
        }
    } else {
        uint32_t d[16];
        load_block(g, J.in, (uint64_t)tile * kTileElems, (uint32_t)tid * kBlockElems,
                   count, false, d, &bad);
        block_key_minmax(d, count, kmin, kmax);
    }
    kmin = wave_min(kmin);
    kmax = wave_max(kmax);
    if (lane == 0) {
        s_min[wave] = kmin;
        s_max[wave] = kmax;
    }
    __syncthreads();
    if (tid == 0) {
#pragma unroll
        for (int w = 1; w < kThreads / 64; ++w) {
            kmin = s_min[w] < kmin ? s_min[w] : kmin;
            kmax = s_max[w] > kmax ? s_max[w] : kmax;
        }
        const unsigned long long tag = (unsigned long long)p.epoch << 32;
        __hip_atomic_fetch_max(&p.job_minmax[2 * job], tag | kmax,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint32_t key_max = kIn ? 0xFFFFFFFFu : 0xFFFFu;
        __hip_atomic_fetch_max(&p.job_minmax[2 * job + 1],
                               tag | (key_max - kmin), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    if (bad) flag_error(p.error, p.error_marker, kErrLayerIndex);
}

// ---- decoder ---------------------------------------------------------------

// Restored values are stored non-temporally (the `nt` policy: no lasting
// allocation in L2 and the MALL).  The codec never reads them again, and a
// restore writes far more than it reads (BF16 pages vs compressed streams):
// left as dirty lines in the 256 MiB MALL, they are written back while the
// next kernel runs and take HBM bandwidth from it (on the config-1 step the
// following store's encoder ran 58 us instead of 53 us).
__device__ __forceinline__ void store_streaming(g_u32x4* p, const u32x4& v) {
    __builtin_nontemporal_store(v, p);
}

// Writes the 32 decoded BF16 values of one block (16 packed pairs).
__device__ __forceinline__ void store_block(uint16_t* dst, const uint32_t* out,
                                            uint32_t count, bool aligned16) {
    if (count == kBlockElems && aligned16) {
        g_u32x4* p = (g_u32x4*)to_global(dst);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4 v;
            v.x = out[4 * i + 0];
            v.y = out[4 * i + 1];
            v.z = out[4 * i + 2];
            v.w = out[4 * i + 3];
            store_streaming(&p[i], v);
        }
        return;
    }
    __attribute__((address_space(1))) uint16_t* g = to_global(dst);
    for (uint32_t v = 0; v < count; ++v)
        g[v] = (uint16_t)((v & 1) ? (out[v >> 1] >> 16) : (out[v >> 1] & 0xFFFFu));
}

// Decodes one block payload (count words at src) into 16 packed BF16 pairs
// (cu:496-538): words -> fields by the transpose, then
// y = bf16_rne((float(q) * eb) * 2).  kWide: rates above 15, whose planes
// 15..30 come from a second transpose of words 16..31.
//
// The wide path parks the high fields in LDS (`park`, one column per thread)
// so that only one set of 16 rows is held in registers at a time.
template <bool kWide, bool kEb2>
__device__ __forceinline__ void decode_words(const uint32_t* src,
                                             uint32_t count_words, uint32_t rmax,
                                             float eb, uint32_t rate, uint32_t* out,
                                             uint32_t (*park)[kThreads]) {
    const int tid = threadIdx.x;
    const float eb2 = eb * 2.0f;
    if (!kWide && kEb2) {
        // Rates <= 15: the sign word and planes 0..14 make 16 rows.  Fed to
        // the transpose as rows 15, 0, 1, .., 14 (words w_0, w_1, .., w_15),
        // they give each element the 16-bit field (sign << 15) | |q|, so q
        // fits int16 and both halves of a row are turned into q at once with
        // packed 16-bit operations: q = (|q| ^ -sign) - (-sign), where -sign
        // is the field shifted right arithmetically by 15.  A zero-rate block
        // has all words 0, so q = 0 and y = +0.0 (eb2 is finite here).
        uint32_t W[16], L[16];
        load_words<16>(src, W, count_words < 16u ? count_words : 16u,
                       rmax < 15u ? rmax + 1u : 16u);
#pragma unroll
        for (int b = 0; b < 16; ++b) L[b] = W[(b + 1) & 15];
        transpose16x2(L);  // L[k]: fields of elements k^7 (low), 16+(k^7) (high)
        // Rows k0 = (2j)^7 and k1 = (2j+1)^7 hold elements 2j, 2j+1 (low
        // halves -> out[j]) and 16+2j, 17+2j (high halves -> out[j + 8]).
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k0 = (2 * j) ^ 7, k1 = (2 * j + 1) ^ 7;
            uint32_t Q[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t f = L[h ? k1 : k0];
                const uint32_t ns = __builtin_bit_cast(
                    uint32_t, __builtin_bit_cast(s16x2, f) >> (short)15);
                Q[h] = __builtin_bit_cast(
                    uint32_t, (u16x2)(__builtin_bit_cast(u16x2, (f & 0x7FFF7FFFu) ^ ns) -
                                      __builtin_bit_cast(u16x2, ns)));
            }
            f32x2 y;
            y.x = (float)(int32_t)(int16_t)(Q[0] & 0xFFFFu) * eb2;
            y.y = (float)(int32_t)(int16_t)(Q[1] & 0xFFFFu) * eb2;
            out[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(y, bf16x2));
            y.x = (float)((int32_t)Q[0] >> 16) * eb2;
            y.y = (float)((int32_t)Q[1] >> 16) * eb2;
            out[j + 8] = __builtin_bit_cast(uint32_t, __builtin_convertvector(y, bf16x2));
        }
        return;
    }
    if (kWide) {
        uint32_t H[16];
        load_words<16>(src + 16, H, count_words > 16u ? count_words - 16u : 0u,
                       rmax - 15u);
        transpose16x2(H);  // H[k]: |q| >> 15 of elements k^7, 16+(k^7)
#pragma unroll
        for (int k = 0; k < 16; ++k) park[k][tid] = H[k];
        // Keep the compiler from forwarding the parked rows in registers.
        __asm__ volatile("" ::: "memory");
    }
    uint32_t L[16];
    load_words<16>(src, L, count_words < 16u ? count_words : 16u,
                   rmax < 15u ? rmax + 1u : 16u);
    transpose16x2(L);  // L[k]: low fields ((|q| << 1) | sign) & 0xFFFF
    // out[i] holds elements 2i and 2i+1.  Rows k0, k1 feed both out[j]
    // (low halves) and out[j + 8] (high halves), so they are consumed
    // together.
#pragma unroll
    for (int n = 0; n < 16; ++n) {
        const int i = (n >> 1) + ((n & 1) ? 8 : 0);
        const int v0 = 2 * i, v1 = 2 * i + 1;
        const int k0 = (v0 & 15) ^ 7, k1 = (v1 & 15) ^ 7;
        const int sh0 = v0 < 16 ? 0 : 16, sh1 = v1 < 16 ? 0 : 16;
        const uint32_t lo0 = (L[k0] >> sh0) & 0xFFFFu, lo1 = (L[k1] >> sh1) & 0xFFFFu;
        uint32_t m0 = lo0 >> 1, m1 = lo1 >> 1;
        if (kWide) {
            m0 |= ((park[k0][tid] >> sh0) & 0xFFFFu) << 15;
            m1 |= ((park[k1][tid] >> sh1) & 0xFFFFu) << 15;
        }
        // q = sign ? -m : m as (m ^ -sign) + sign
        const uint32_t s0 = lo0 & 1u, s1 = lo1 & 1u;
        const int32_t q0 = (int32_t)((m0 ^ (0u - s0)) + s0);
        const int32_t q1 = (int32_t)((m1 ^ (0u - s1)) + s1);
        f32x2 y;
        if (kEb2) {
            // fl(fl(q*eb)*2) == fl(q*(2eb)) while FLT_MIN <= eb <= FLT_MAX/2:
            // scaling by 2 commutes with rounding for normal results, and
            // every nonzero |q*eb| >= eb is normal.
            y.x = (float)q0 * eb2;
            y.y = (float)q1 * eb2;
        } else {
            y.x = ((float)q0 * eb) * 2.0f;
            y.y = ((float)q1 * eb) * 2.0f;
        }
        out[i] = rate ? __builtin_bit_cast(uint32_t, __builtin_convertvector(y, bf16x2)) : 0u;
    }
}

// One block: stream words at `base` -> 16 packed BF16 pairs (zeros when the
// whole wave has rate 0).
__device__ __forceinline__ void decode_block(const uint8_t* in, uint64_t base,
                                             uint32_t rate, uint32_t rmax, float eb,
                                             uint32_t* out,
                                             uint32_t (*park)[kThreads]) {
    if (rmax == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = 0;
        return;
    }
    const uint32_t* src = reinterpret_cast<const uint32_t*>(in + base);
    const uint32_t count_words = rate ? rate + 1u : 0u;
    const bool eb2_ok = eb >= FLT_MIN && eb <= FLT_MAX / 2;  // uniform
    if (rmax <= 15u) {
        if (eb2_ok)
            decode_words<false, true>(src, count_words, rmax, eb, rate, out, park);
        else
            decode_words<false, false>(src, count_words, rmax, eb, rate, out, park);
    } else {
        if (eb2_ok)
            decode_words<true, true>(src, count_words, rmax, eb, rate, out, park);
        else
            decode_words<true, false>(src, count_words, rmax, eb, rate, out, park);
    }
}

// One block of stream words -> 32 fp32 values y = fl(fl(q * eb) * 2)
// (cu:535-538 without the BF16 rounding; zeros where rate is 0): the low
// fields ((|q| << 1) | sign) of words 0..15 and, for rates above 15, the
// high fields |q| >> 15 of words 16..31, both by the transpose.
__device__ __forceinline__ void decode_block_f32(const uint8_t* in, uint64_t base,
                                                 uint32_t rate, uint32_t rmax,
                                                 float eb, uint32_t* out) {
    if (rmax == 0) {
#pragma unroll
        for (int i = 0; i < kBlockElems; ++i) out[i] = 0;
        return;
    }
    const uint32_t* src = reinterpret_cast<const uint32_t*>(in + base);
    const uint32_t count_words = rate ? rate + 1u : 0u;
    uint32_t L[16], H[16];
    load_words<16>(src, L, count_words < 16u ? count_words : 16u,
                   rmax < 15u ? rmax + 1u : 16u);
    transpose16x2(L);
    if (rmax > 15u) {
        load_words<16>(src + 16, H, count_words > 16u ? count_words - 16u : 0u,
                       rmax - 15u);
        transpose16x2(H);
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) H[k] = 0;
    }
    const bool eb2_ok = eb >= FLT_MIN && eb <= FLT_MAX / 2;  // uniform
    const float eb2 = eb * 2.0f;
#pragma unroll
    for (int v = 0; v < kBlockElems; ++v) {
        const int k = (v & 15) ^ 7, sh = v < 16 ? 0 : 16;
        const uint32_t lo = (L[k] >> sh) & 0xFFFFu;
        const uint32_t m = (lo >> 1) | (((H[k] >> sh) & 0xFFFFu) << 15);
        const uint32_t sg = lo & 1u;
        const int32_t q = (int32_t)((m ^ (0u - sg)) + sg);
        // fl(fl(q*eb)*2) == fl(q*(2eb)) for FLT_MIN <= eb <= FLT_MAX/2
        const float y = eb2_ok ? (float)q * eb2 : ((float)q * eb) * 2.0f;
        out[v] = rate ? __float_as_uint(y) : 0u;
    }
}

// Writes 32 decoded fp32 values (eight 16-byte stores when whole and
// aligned, else value by value).
__device__ __forceinline__ void store_block_f32(float* dst, const uint32_t* out,
                                                uint32_t count) {
    if (count == kBlockElems && ((uintptr_t)dst & 15u) == 0) {
        g_u32x4* p = (g_u32x4*)to_global(reinterpret_cast<uint32_t*>(dst));
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            u32x4 v;
            v.x = out[4 * i + 0];
            v.y = out[4 * i + 1];
            v.z = out[4 * i + 2];
            v.w = out[4 * i + 3];
            store_streaming(&p[i], v);
        }
        return;
    }
    g_u32* g = to_global(reinterpret_cast<uint32_t*>(dst));
    for (uint32_t v = 0; v < count; ++v) g[v] = out[v];
}

// Destination of this thread's decoded block when its `count` values go to
// one contiguous run (cu:539-606: contiguous page, multi-destination split,
// or layer-indexed position in the full page); nullptr when they do not (or
// the layer index is bad, which sets `badl`).
template <int kDst>
__device__ __forceinline__ uint16_t* block_dst(const DecompressParams& p,
                                               const Group& g, const DecompressJob& J,
                                               uint32_t job, uint32_t tile, int tid,
                                               uint64_t e0, uint32_t count,
                                               uint32_t& badl) {
    if (kDst == kDstLinear) return J.dst + e0;
    if (kDst == kDstMulti) {
        const uint64_t epd = p.elements_per_dest;
        const uint64_t di = e0 / epd;
        const uint64_t off = e0 - di * epd;
        if (off + count > epd) return nullptr;
        return p.dests[(uint64_t)job * p.dests_per_page + di] + off;
    }
    const LayerCursor c = layer_cursor(g, (uint64_t)tile * kTileElems,
                                       (uint32_t)tid * kBlockElems, &badl);
    return (c.contiguous && !badl) ? J.dst + c.src_index : nullptr;
}

// Value by value, for a block that straddles destinations or layers.
template <int kDst>
__device__ __forceinline__ void store_elementwise(const DecompressParams& p,
                                                  const Group& g, const DecompressJob& J,
                                                  uint32_t job, uint64_t e0,
                                                  uint32_t count, const uint32_t* out,
                                                  uint32_t& badl) {
    for (uint32_t v = 0; v < count; ++v) {
        const uint16_t y = (uint16_t)((v & 1) ? (out[v >> 1] >> 16) : (out[v >> 1] & 0xFFFFu));
        const uint64_t e = e0 + v;
        if (kDst == kDstMulti) {
            const uint64_t epd = p.elements_per_dest;
            const uint64_t dv = e / epd;
            to_global(p.dests[(uint64_t)job * p.dests_per_page + dv])[e - dv * epd] = y;
        } else if (kDst == kDstIndexed) {
            const uint64_t s = map_index(e, g.layers, g.selected_layers,
                                         g.source_layers, g.elements_per_layer, &badl);
            if (badl) break;
            to_global(J.dst)[s] = y;
        } else {
            to_global(J.dst)[e] = y;
        }
    }
}

// Each lane writes its own decoded block (cu:539-606).
template <int kDst>
__device__ __forceinline__ void store_block_lane(const DecompressParams& p,
                                                 const Group& g, const DecompressJob& J,
                                                 uint32_t job, uint32_t tile, int tid,
                                                 uint64_t e0, uint32_t count,
                                                 const uint32_t* out, uint32_t& err) {
    uint32_t badl = 0;
    uint16_t* dst = block_dst<kDst>(p, g, J, job, tile, tid, e0, count, badl);
    if (dst != nullptr)
        store_block(dst, out, count, ((uintptr_t)dst & 15u) == 0);
    else
        store_elementwise<kDst>(p, g, J, job, e0, count, out, badl);
    if (badl) err |= kErrLayerIndex;
}

// Destination of the 2048 values of wave `wave` of a tile when they are 64
// whole blocks landing on one contiguous, 16-byte-aligned run; nullptr
// otherwise (then each lane stores its own block).  Wave-uniform: scalar
// arithmetic (every index here is below 2^29, the largest segment).
template <int kDst>
__device__ __forceinline__ uint16_t* wave_run_dst(const DecompressParams& p,
                                                  const Group& g, const DecompressJob& J,
                                                  uint32_t job, uint32_t tile, int wave) {
    constexpr uint32_t kRun = 64u * kBlockElems;
    const uint32_t E = tile * (uint32_t)kTileElems + (uint32_t)wave * kRun;
    if ((uint64_t)E + kRun > g.n) return nullptr;
    uint16_t* d;
    if (kDst == kDstLinear) {
        if (!p.aligned16) return nullptr;
        d = J.dst + E;
    } else if (kDst == kDstMulti) {
        const uint32_t epd = (uint32_t)p.elements_per_dest;
        const uint32_t di = E / epd, off = E - di * epd;
        if (off + kRun > epd) return nullptr;
        d = load_const(p.dests, (uint32_t)(job * p.dests_per_page + di)) + off;
    } else {
        const uint32_t epl = (uint32_t)g.elements_per_layer;
        const uint32_t per_prefix = (uint32_t)g.selected_layers * epl;
        const uint32_t pre = divide(E, g.prefix_div);
        const uint32_t within = E - pre * per_prefix;
        const uint32_t layer = divide(within, g.layer_div);
        const uint32_t inner = within - layer * epl;
        if (inner + kRun > epl) return nullptr;
        const int64_t l = load_const(g.layers, layer);
        if (l < 0 || (uint64_t)l >= g.source_layers) return nullptr;
        d = J.dst + (((uint64_t)pre * g.source_layers + (uint64_t)l) * epl + inner);
    }
    return ((uintptr_t)d & 15u) ? nullptr : d;
}

// Writes the wave's 64 decoded blocks to `run` as four fully coalesced 1 KiB
// stores through the wave's own LDS cells `stage` (lane-strided 64-byte
// stores reach only about half the write bandwidth of coalesced ones on
// MI355X).  Staging layout: 16-byte slot j of the wave is the 4 dwords at
// stage[(j >> 4) * kThreads + 4 * (j & 15)] (the wave's 64-dword column
// range of row j >> 4); chunk q (dwords 4q..4q+3) of block b is kept in slot
// 64q + (b ^ 4q), which keeps both the per-block writes and the coalesced
// reads free of bank conflicts.
__device__ __forceinline__ void store_wave_run(uint16_t* run, const uint32_t* out,
                                               uint32_t* stage, int lane) {
    __asm__ volatile("" ::: "memory");  // after any parked-row reads
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t j = 64u * q + ((uint32_t)lane ^ (4u * q));
        u32x4 v;
        v.x = out[4 * q + 0];
        v.y = out[4 * q + 1];
        v.z = out[4 * q + 2];
        v.w = out[4 * q + 3];
        *reinterpret_cast<u32x4*>(stage + (j >> 4) * kThreads + 4u * (j & 15u)) = v;
    }
    __builtin_amdgcn_wave_barrier();
    __asm__ volatile("" ::: "memory");
    g_u32x4* d = (g_u32x4*)to_global(reinterpret_cast<uint32_t*>(run));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t b = 16u * i + ((uint32_t)lane >> 2), q = (uint32_t)lane & 3u;
        const uint32_t j = 64u * q + (b ^ (4u * q));
        store_streaming(&d[64 * i + lane],
                        *reinterpret_cast<const u32x4*>(stage + (j >> 4) * kThreads +
                                                        4u * (j & 15u)));
    }
    __builtin_amdgcn_wave_barrier();
    __asm__ volatile("" ::: "memory");  // before the cells are reused
}

// Writes the decoded blocks of the wave.  Every lane of the wave calls it;
// `run` is wave_run_dst's result, `write` whether this lane's block is
// written (rate-0 blocks are skipped under the reference's policy).
template <int kDst>
__device__ __forceinline__ void store_decoded(const DecompressParams& p,
                                              const Group& g, const DecompressJob& J,
                                              uint32_t job, uint32_t tile, int tid,
                                              uint64_t e0, uint32_t count, bool write,
                                              uint16_t* run, const uint32_t* out,
                                              uint32_t* stage, uint32_t& err) {
    if (run != nullptr && __ballot(!write) == 0ull) {
        store_wave_run(run, out, stage, tid & 63);
        return;
    }
    if (write) store_block_lane<kDst>(p, g, J, job, tile, tid, e0, count, out, err);
}

// kOut = 0: BF16 values to any destination kind; kOut = 1: fp32 values to
// contiguous per-job outputs (the single-page fp32 API).
template <int kDst, int kOut>
__global__ __launch_bounds__(kThreads) void decompress_kernel(
    DecompressParams p) {
    __shared__ uint32_t s_tile;
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_hdr[kTileBlocks / 4];
    __shared__ uint32_t s_park[16][kThreads];  // wide-rate decode scratch

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    publish_seq(p.host_ctl, p.seq);
    const uint32_t t = tile_number(p.ticket, p.ticket_base, &s_tile);
    if (t >= p.total_tiles) {
        if (tid == 0) flag_error(p.error, p.error_marker, kErrSpin);
        return;
    }
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];
    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = __builtin_amdgcn_readfirstlane(local / g.tiles_per_job);
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const DecompressJob J = job_at(p, job);
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;
    const uint32_t R = g.header_bytes;

    // Rate bytes of this tile (cu:410-418); padding bytes are masked.
    if (tid < kTileBlocks / 4)
        s_hdr[tid] = *to_global(reinterpret_cast<const uint32_t*>(J.in + tile * kTileBlocks + 4 * tid));
    __syncthreads();
    uint32_t rate = count ? (s_hdr[tid >> 2] >> (8 * (tid & 3))) & 0xFFu : 0u;
    uint32_t err = 0;
    if (rate > 31u) {
        err |= kErrRate;
        rate = 0;
    }
    const uint32_t bytes = rate ? 4u + 4u * rate : 0u;
    // Offset of this tile's payload in the job's stream: decoupled look-back
    // over the earlier tiles of the job (tile 0 publishes right away).
    const TileScan sc = tile_scan(bytes, tid, s_wave);  // has __syncthreads
    if (wave == 0) {
        const uint32_t pf = lookback(p.tile_state, t, tile, sc.total,
                                     p.epoch, p.error, p.error_marker);
        if (lane == 0) s_prefix = pf;
    }
    __syncthreads();
    const uint64_t base = (uint64_t)R + s_prefix + sc.exclusive;
    if (rate && base + bytes > J.size) {
        err |= kErrTruncated;
        rate = 0;
    }

    // Unpack (cu:496-538): stream words back to fields, then values
    // y = bf16_rne((float(q) * eb) * 2) (cu:535-538).
    const uint32_t rmax = wave_max(rate);
    if constexpr (kOut) {
        uint32_t out[kBlockElems];
        decode_block_f32(J.in, base, rate, rmax, J.eb, out);
        if (count != 0 && (rate != 0 || p.rate0_zero))
            store_block_f32(reinterpret_cast<float*>(J.dst) + e0, out, count);
    } else {
        uint32_t out[16];
        decode_block(J.in, base, rate, rmax, J.eb, out, s_park);
        store_decoded<kDst>(p, g, J, job, tile, tid, e0, count,
                            count != 0 && (rate != 0 || p.rate0_zero),
                            wave_run_dst<kDst>(p, g, J, job, tile, wave), out,
                            &s_park[0][64 * wave], err);
    }
    if (err) flag_error(p.error, p.error_marker, err);
}

// Decoder of the Lorenzo modes (specification above compress_lorenzo_kernel):
// one workgroup per tile, one block per thread, fp32 values into contiguous
// per-job outputs.
template <int kMode>
__global__ __launch_bounds__(kThreads) void decompress_lorenzo_kernel(DecompressParams p) {
    __shared__ uint32_t s_tile;
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_hdr[kTileBlocks / 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    publish_seq(p.host_ctl, p.seq);
    const uint32_t t = tile_number(p.ticket, p.ticket_base, &s_tile);
    if (t >= p.total_tiles) {
        if (tid == 0) flag_error(p.error, p.error_marker, kErrSpin);
        return;
    }
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];
    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = __builtin_amdgcn_readfirstlane(local / g.tiles_per_job);
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const DecompressJob J = job_at(p, job);
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;
    const uint32_t R = g.header_bytes;

    if (tid < kTileBlocks / 4)
        s_hdr[tid] = *to_global(reinterpret_cast<const uint32_t*>(J.in + tile * kTileBlocks + 4 * tid));
    __syncthreads();
    uint32_t hdr = count ? (s_hdr[tid >> 2] >> (8 * (tid & 3))) & 0xFFu : 0u;
    uint32_t err = 0;
    bool has_o = kMode == kModeOutlier && (hdr & 0x80u) != 0;
    uint32_t rate = kMode == kModeOutlier ? hdr & 0x7Fu : hdr;
    if (rate > 32u) {
        err |= kErrRate;
        hdr = rate = 0;
        has_o = false;
    }
    const uint32_t bytes = (has_o ? 4u : 0u) + (rate ? 4u + 4u * rate : 0u);
    const TileScan sc = tile_scan(bytes, tid, s_wave);  // has __syncthreads
    if (wave == 0) {
        const uint32_t pf = lookback(p.tile_state, t, tile, sc.total, p.epoch, p.error,
                                     p.error_marker);
        if (lane == 0) s_prefix = pf;
    }
    __syncthreads();
    const uint64_t base = (uint64_t)R + s_prefix + sc.exclusive;
    if (bytes && base + bytes > J.size) {
        err |= kErrTruncated;
        hdr = rate = 0;
        has_o = false;
    }

    const uint32_t* src = reinterpret_cast<const uint32_t*>(J.in + base);
    uint32_t q = has_o ? *to_global(const_cast<uint32_t*>(src)) : 0u;
    src += has_o ? 1 : 0;
    const uint32_t rmax = wave_max(rate);
    const uint32_t count_words = rate ? rate + 1u : 0u;
    uint32_t L[16], H[16];
    uint32_t w32 = 0;
    load_words<16>(src, L, count_words < 16u ? count_words : 16u,
                   rmax < 15u ? rmax + 1u : 16u);
    transpose16x2(L);
    if (rmax > 15u) {
        load_words<16>(src + 16, H, count_words > 16u ? count_words - 16u : 0u, rmax - 15u);
        transpose16x2(H);
        if (rate == 32u) w32 = *to_global(const_cast<uint32_t*>(src + 32));
    } else {
#pragma unroll
        for (int k = 0; k < 16; ++k) H[k] = 0;
    }
    const bool eb2_ok = J.eb >= FLT_MIN && J.eb <= FLT_MAX / 2;
    const float eb2 = J.eb * 2.0f;
    uint32_t out[kBlockElems];
#pragma unroll
    for (int v = 0; v < kBlockElems; ++v) {
        const int k = (v & 15) ^ 7, sh = v < 16 ? 0 : 16;
        const uint32_t lo = (L[k] >> sh) & 0xFFFFu;
        const uint32_t m = (lo >> 1) | (((H[k] >> sh) & 0xFFFFu) << 15) |
                           (((w32 >> (v ^ 7)) & 1u) << 31);
        const uint32_t sg = lo & 1u;
        q += (m ^ (0u - sg)) + sg;
        // fl(fl(q*eb)*2) == fl(q*(2eb)) for FLT_MIN <= eb <= FLT_MAX/2
        const float y = eb2_ok ? (float)(int32_t)q * eb2 : ((float)(int32_t)q * J.eb) * 2.0f;
        // A block with header byte 0 is +0.0, as a rate-0 block of the fixed
        // code, also where eb is infinite or NaN (0 * eb would be NaN).
        out[v] = hdr ? __float_as_uint(y) : 0u;
    }
    if (count != 0 && (hdr != 0 || p.rate0_zero))
        store_block_f32(reinterpret_cast<float*>(J.dst) + e0, out, count);
    if (err) flag_error(p.error, p.error_marker, err);
}

// ---- persistent decoder ----------------------------------------------------
//
// Workgroup w decodes the consecutive tiles [w*T/G, (w+1)*T/G) of the launch
// (T tiles over all groups and jobs, G = gridDim.x).  A tile's payload
// offset is the running sum of the payload bytes of the earlier tiles of its
// job: the first tile of a workgroup's run adds up the rate bytes of the
// earlier tiles' headers once (cu:410-470 re-derives offsets from the header
// too), every following tile adds the previous tile's total, and a tile 0
// starts from 0.  No workgroup waits for another, for any job length.  The
// next tile's rate bytes are requested before the current tile is decoded
// and have arrived before its stores are issued (stores count in the same
// in-order memory counter, so a wait placed after them would also wait for
// the stores).

struct DecTile {
    int gi;         // group
    uint32_t job;   // job index
    uint32_t tile;  // tile within the job
};

__device__ __forceinline__ DecTile dec_tile(const DecompressParams& p, uint32_t t,
                                            const uint32_t* s_gfirst) {
    const TilePlace pl = place_tile(p.groups, s_gfirst, p.num_groups, t);
    DecTile c;
    c.gi = pl.gi;
    c.job = pl.job;
    c.tile = pl.tile;
    return c;
}

// This thread's word of a tile's rate bytes (threads < 64).
__device__ __forceinline__ uint32_t tile_header_word(const uint8_t* in, uint32_t tile,
                                                     int tid) {
    return tid < kTileBlocks / 4
               ? to_global(reinterpret_cast<const uint32_t*>(in))[tile * (kTileBlocks / 4) + tid]
               : 0u;
}

// Payload bytes of the tiles [0, tile) of a job, from their rate bytes
// (whole workgroup, one barrier; s_red holds one word per wave).  A thread
// reads its words 16 at a time with all 16 loads in flight (a loop of one
// load per iteration waits out one memory round trip per word, e.g. 32 for
// the last tile of a 128-tile job); indices past the header read word 0 and
// count nothing, so every load is unconditional.
__device__ __forceinline__ uint32_t header_prefix(const uint8_t* in, uint32_t tile,
                                                  int tid, uint32_t* s_red) {
    constexpr int kBatch = 16;
    const g_u32* hw = to_global(reinterpret_cast<const uint32_t*>(in));
    const uint32_t words = tile * (kTileBlocks / 4);
    uint32_t part = 0;
    for (uint32_t base = (uint32_t)tid; base < words; base += kBatch * kThreads) {
        uint32_t v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
            const uint32_t i = base + (uint32_t)k * kThreads;
            v[k] = hw[i < words ? i : 0u];
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k)
            if (base + (uint32_t)k * kThreads < words) part += header_word_bytes(v[k]);
    }
    part = wave_sum(part);
    if ((tid & 63) == 0) s_red[tid >> 6] = part;
    __syncthreads();
    uint32_t total = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) total += s_red[w];
    return total;
}

// First tile of workgroup b's run out of G: the host's per-workgroup run
// table, or the run balanced by the per-group tile weights.
__device__ __forceinline__ uint32_t run_start(const DecompressParams& p, uint32_t b,
                                              uint32_t G) {
    if (p.run_starts != nullptr) return load_const(p.run_starts, b < G ? b : G);
    return weighted_run_start(p.groups, p.num_groups, p.total_tiles, p.total_weight,
                              p.weight_before, p.tile_weight, b, G);
}

template <int kDst>
__device__ __forceinline__ void decompress_persistent(const DecompressParams& p) {
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_red[kThreads / 64];
    __shared__ uint32_t s_hdr[kTileBlocks / 4];
    __shared__ uint32_t s_gfirst[kMaxGroups];
    __shared__ uint32_t s_park[16][kThreads];  // wide-rate scratch, store staging

    publish_seq(p.host_ctl, p.seq);
    if ((int)threadIdx.x < p.num_groups) s_gfirst[threadIdx.x] = p.groups[threadIdx.x].first_tile;
    __syncthreads();
    const uint32_t G = gridDim.x;
    const uint32_t t_begin = run_start(p, blockIdx.x, G);
    const uint32_t t_end = run_start(p, blockIdx.x + 1, G);
    if (t_begin >= t_end) return;  // whole workgroup
    uint32_t err = 0;

    DecTile cur = dec_tile(p, t_begin, s_gfirst);
    uint32_t prefix = 0;
    uint32_t hw;
    {
        const int tid = (int)threadIdx.x;
        const uint8_t* in = job_at(p, cur.job).in;
        if (cur.tile != 0) prefix = header_prefix(in, cur.tile, tid, s_red);
        hw = tile_header_word(in, cur.tile, tid);
    }
    for (uint32_t t = t_begin;;) {
        const int tid = loop_tid();
        const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const Group& g = p.groups[cur.gi];
        const DecompressJob J = job_at(p, cur.job);
        // Segments hold fewer than 2^29 values: 32-bit element indices.
        const uint32_t n = (uint32_t)g.n;
        const uint32_t e0 = (cur.tile * kTileBlocks + (uint32_t)tid) * kBlockElems;
        const uint32_t count = e0 < n ? (n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;

        // Rates (cu:410-418; padding bytes masked), tile scan, offsets.
        if (tid < kTileBlocks / 4) s_hdr[tid] = hw;
        __syncthreads();
        uint32_t rate = count ? (s_hdr[tid >> 2] >> (8 * (tid & 3))) & 0xFFu : 0u;
        if (rate > 31u) {
            err |= kErrRate;
            rate = 0;
        }
        const uint32_t bytes = rate ? 4u + 4u * rate : 0u;
        const TileScan sc = tile_scan(bytes, tid, s_wave);  // has __syncthreads
        const uint64_t base = (uint64_t)g.header_bytes + prefix + sc.exclusive;
        if (rate && base + bytes > J.size) {
            err |= kErrTruncated;
            rate = 0;
        }

        // Ask for the next tile's rate bytes, then decode this tile.
        const bool has_next = t + 1 < t_end;
        DecTile nxt = cur;
        if (has_next) {
            nxt = dec_tile(p, t + 1, s_gfirst);
            hw = tile_header_word(job_at(p, nxt.job).in, nxt.tile, tid);
        }
        const uint32_t rmax = wave_max(rate);
        uint16_t* run = wave_run_dst<kDst>(p, g, J, cur.job, cur.tile, wave);
        uint32_t out[16];
        decode_block(J.in, base, rate, rmax, J.eb, out, s_park);
        __asm__ volatile("" ::"v"(hw));  // arrived before the stores are issued
        store_decoded<kDst>(p, g, J, cur.job, cur.tile, tid, e0, count,
                            count != 0 && (rate != 0 || p.rate0_zero), run, out,
                            &s_park[0][64 * wave], err);
        if (!has_next) break;
        prefix = nxt.tile == 0 ? 0u : prefix + sc.total;
        cur = nxt;
        ++t;
    }
    if (err) flag_error(p.error, p.error_marker, err);
}

template <int kDst>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_num_sgpr(74), amdgpu_waves_per_eu(8, 8))) void decompress_persistent_kernel(
    DecompressParams p) {
    decompress_persistent<kDst>(p);
}

// The same with the job records in the kernel arguments (jobs_inline == 2).
template <int kDst>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_num_sgpr(74), amdgpu_waves_per_eu(8, 8))) void
decompress_persistent_argtable_kernel(DecompressParams p, ArgTable) {
    decompress_persistent<kDst>(p);
}

// ---- packed publication ------------------------------------------------------
// Workgroup b copies payloads b, b + G, ... to their packed offsets: 8-byte
// lanes when source and destination allow it (a wave moves 512 contiguous
// bytes per instruction), else 4-byte or single-byte lanes, then zeroes the
// alignment gap behind the payload.  The destination is normally pinned host
// memory, so the copy is the device-to-host transfer itself.
__global__ __launch_bounds__(256) void pack_kernel(PackParams p) {
    publish_seq(p.host_ctl, p.seq);
    for (uint32_t j = blockIdx.x; j < p.count; j += gridDim.x) {
        const PackJob J = load_const(p.jobs, j);
        const uint8_t* src = J.src;
        uint8_t* dst = p.dst + J.dst_off;
        const uint64_t n = J.size;
        const uintptr_t mis = (uintptr_t)src | (uintptr_t)dst;
        uint64_t done = 0;
        if ((mis & 7u) == 0) {
            typedef __attribute__((address_space(1))) unsigned long long g_u64;
            const g_u64* s8 = (const g_u64*)src;
            g_u64* d8 = (g_u64*)dst;
            const uint64_t words = n >> 3;
            for (uint64_t i = threadIdx.x; i < words; i += blockDim.x) d8[i] = s8[i];
            done = words << 3;
        } else if ((mis & 3u) == 0) {
            const g_u32* s4 = (const g_u32*)src;
            g_u32* d4 = (g_u32*)dst;
            const uint64_t words = n >> 2;
            for (uint64_t i = threadIdx.x; i < words; i += blockDim.x) d4[i] = s4[i];
            done = words << 2;
        }
        typedef __attribute__((address_space(1))) uint8_t g_u8;
        const g_u8* s1 = (const g_u8*)src;
        g_u8* d1 = (g_u8*)dst;
        for (uint64_t i = done + threadIdx.x; i < n; i += blockDim.x) d1[i] = s1[i];
        if (threadIdx.x < J.pad) d1[n + threadIdx.x] = 0;
    }
}

__global__ void fill_u64_kernel(unsigned long long* words, size_t count) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        words[i] = 0ull;
}

}  // namespace

// ---- no-allocation scratch ---------------------------------------------------
// The device memory of kvszp_compress_batch_fixed_bf16_noalloc (layout in
// kvszp_internal.h).  Zero when the code object loads; every GPU holds its
// own copy until the process ends.  Host code never uses the array's name
// as an address: the kernels get the per-device pointer below.
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices];
}  // namespace

hipError_t scratch_address(int device, void** out) {
    if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        int current = -1;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != device && (e = hipSetDevice(device)) != hipSuccess) return e;
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (current != device) (void)hipSetDevice(current);
        if (e != hipSuccess) return e;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

hipError_t launch_pack(const PackParams& p, uint32_t grid, hipStream_t stream) {
    hipLaunchKernelGGL(pack_kernel, dim3(grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_fill_u64(unsigned long long* words, size_t count, hipStream_t stream) {
    const uint32_t grid = (uint32_t)std::min<size_t>((count + 255) / 256, 1024);
    hipLaunchKernelGGL(fill_u64_kernel, dim3(grid), dim3(256), 0, stream, words, count);
    return hipGetLastError();
}

// Launchers.  With timing events, hipExtLaunchKernelGGL stamps them with
// the kernel's own start and end (no separate marker packets).
template <class... Args>
static void launch_block(void (*kernel)(Args...), uint32_t grid, uint32_t block,
                         hipStream_t stream, hipEvent_t start, hipEvent_t stop,
                         Args... args) {
    if (start || stop)
        hipExtLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, stream,
                              start, stop, 0, args...);
    else
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(block), 0, stream, args...);
}

// Job records a kernel of these parameters can read (0 when the table it is
// told to read cannot hold them).  `table_bytes`: the bytes of job records
// an ArgTable launch carries (0 for every other launch, whose kernels have
// no ArgTable argument).
template <class Params>
static uint32_t readable_jobs(const Params& p, size_t table_bytes = 0) {
    const uint64_t need = (uint64_t)p.num_jobs * sizeof(p.inline_jobs[0]);
    switch (p.jobs_inline) {
    case 0:
        return p.jobs != nullptr ? p.num_jobs : 0u;
    case 1:
        return p.num_jobs <= (uint32_t)kInlineJobs ? p.num_jobs : 0u;
    case 2:
        return need <= table_bytes && table_bytes <= kArgTableBytes ? p.num_jobs : 0u;
    default:
        return 0u;
    }
}

// Launches a kernel of parameters (Params, ArgTable) whose ArgTable starts
// with the `table_bytes` bytes at `table` (the rest is never read).
template <class Params>
static hipError_t launch_argtable(void (*kernel)(Params, ArgTable), uint32_t grid,
                                  uint32_t block, hipStream_t stream, hipEvent_t start,
                                  hipEvent_t stop, const Params& p, const void* table,
                                  size_t table_bytes) {
    static thread_local ArgTable t;
    if (table == nullptr || table_bytes > kArgTableBytes) return hipErrorInvalidValue;
    std::memcpy(t.bytes, table, table_bytes);
    void* args[] = {const_cast<Params*>(&p), &t};
    if (start || stop)
        return hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), dim3(grid),
                                  dim3(block), args, 0, stream, start, stop, 0);
    return hipLaunchKernel(reinterpret_cast<const void*>(kernel), dim3(grid), dim3(block),
                           args, 0, stream);
}

template <class... Args>
static void launch(void (*kernel)(Args...), uint32_t grid, hipStream_t stream,
                   hipEvent_t start, hipEvent_t stop, Args... args) {
    launch_block(kernel, grid, kThreads, stream, start, stop, args...);
}

hipError_t launch_compress(const CompressParams& p, hipStream_t stream,
                           hipEvent_t start, hipEvent_t stop) {
    if (!tile_plan_ok(p.groups, p.num_groups, p.total_tiles, p.total_tiles, false,
                      readable_jobs(p)))
        return hipErrorInvalidValue;
    if (p.input_f32 && p.mode != kModeFixed) {
        if (p.mode == kModePlain) {
            if (p.quantizer)
                launch(compress_lorenzo_kernel<1, kModePlain>, p.total_tiles, stream, start, stop, p);
            else
                launch(compress_lorenzo_kernel<0, kModePlain>, p.total_tiles, stream, start, stop, p);
        } else if (p.quantizer) {
            launch(compress_lorenzo_kernel<1, kModeOutlier>, p.total_tiles, stream, start, stop, p);
        } else {
            launch(compress_lorenzo_kernel<0, kModeOutlier>, p.total_tiles, stream, start, stop, p);
        }
    } else if (p.input_f32) {
        if (p.quantizer)
            launch(compress_kernel<1, 1>, p.total_tiles, stream, start, stop, p);
        else
            launch(compress_kernel<0, 1>, p.total_tiles, stream, start, stop, p);
    } else if (p.quantizer) {
        launch(compress_kernel<1, 0>, p.total_tiles, stream, start, stop, p);
    } else {
        launch(compress_kernel<0, 0>, p.total_tiles, stream, start, stop, p);
    }
    return hipGetLastError();
}

hipError_t launch_compress_pipelined(const CompressParams& p, uint32_t grid,
                                     hipStream_t stream, hipEvent_t start,
                                     hipEvent_t stop, const void* table,
                                     size_t table_bytes) {
    const bool arg = p.jobs_inline == 2;
    if (!tile_plan_ok(p.groups, p.num_groups, p.total_tiles, grid, true,
                      readable_jobs(p, arg ? table_bytes : 0)))
        return hipErrorInvalidValue;
    uint32_t longest = 0;
    for (int i = 0; i < p.num_groups; ++i) longest = std::max(longest, p.groups[i].tiles_per_job);
    if (arg) {
        void (*k)(CompressParams, ArgTable) =
            longest <= kEarlyLookbackTiles
                ? (p.quantizer ? compress_persistent_argtable_kernel<1, true>
                               : compress_persistent_argtable_kernel<0, true>)
                : (p.quantizer ? compress_persistent_argtable_kernel<1, false>
                               : compress_persistent_argtable_kernel<0, false>);
        return launch_argtable(k, grid, kEncThreads, stream, start, stop, p, table,
                               table_bytes);
    }
    if (longest <= kEarlyLookbackTiles) {
        if (p.quantizer)
            launch_block(compress_persistent_kernel<1, true>, grid, kEncThreads, stream, start,
                         stop, p);
        else
            launch_block(compress_persistent_kernel<0, true>, grid, kEncThreads, stream, start,
                         stop, p);
    } else {
        if (p.quantizer)
            launch_block(compress_persistent_kernel<1, false>, grid, kEncThreads, stream, start,
                         stop, p);
        else
            launch_block(compress_persistent_kernel<0, false>, grid, kEncThreads, stream, start,
                         stop, p);
    }
    return hipGetLastError();
}

hipError_t launch_minmax(const MinMaxParams& p, uint32_t grid,
                         hipStream_t stream, hipEvent_t start) {
    if (!tile_plan_ok(p.groups, p.num_groups, grid, grid, false, readable_jobs(p)))  // a workgroup per tile
        return hipErrorInvalidValue;
    if (p.input_f32)
        launch(minmax_kernel<1>, grid, stream, start, nullptr, p);
    else
        launch(minmax_kernel<0>, grid, stream, start, nullptr, p);
    return hipGetLastError();
}

hipError_t launch_decompress_persistent(const DecompressParams& p, uint32_t grid,
                                       hipStream_t stream, hipEvent_t start,
                                       hipEvent_t stop, const void* table,
                                       size_t table_bytes) {
    const bool arg = p.jobs_inline == 2;
    if (!tile_plan_ok(p.groups, p.num_groups, p.total_tiles, grid, true,
                      readable_jobs(p, arg ? table_bytes : 0)))
        return hipErrorInvalidValue;
    if (arg) {
        void (*k)(DecompressParams, ArgTable) =
            p.dst_kind == kDstMulti     ? decompress_persistent_argtable_kernel<kDstMulti>
            : p.dst_kind == kDstIndexed ? decompress_persistent_argtable_kernel<kDstIndexed>
                                        : decompress_persistent_argtable_kernel<kDstLinear>;
        return launch_argtable(k, grid, kThreads, stream, start, stop, p, table, table_bytes);
    }
    switch (p.dst_kind) {
    case kDstMulti:
        launch(decompress_persistent_kernel<kDstMulti>, grid, stream, start, stop, p);
        break;
    case kDstIndexed:
        launch(decompress_persistent_kernel<kDstIndexed>, grid, stream, start, stop, p);
        break;
    default:
        launch(decompress_persistent_kernel<kDstLinear>, grid, stream, start, stop, p);
        break;
    }
    return hipGetLastError();
}

int decompress_resident_workgroups(int device) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(decompress_persistent_kernel<kDstIndexed>),
            kThreads, 0) != hipSuccess)
        per_cu = 1;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return per_cu;
    return per_cu * prop.multiProcessorCount;
}

hipError_t launch_decompress(const DecompressParams& p, hipStream_t stream,
                             hipEvent_t start, hipEvent_t stop) {
    if (!tile_plan_ok(p.groups, p.num_groups, p.total_tiles, p.total_tiles, false,
                      readable_jobs(p)))
        return hipErrorInvalidValue;
    if (p.output_f32) {
        if (p.mode == kModePlain)
            launch(decompress_lorenzo_kernel<kModePlain>, p.total_tiles, stream, start, stop, p);
        else if (p.mode == kModeOutlier)
            launch(decompress_lorenzo_kernel<kModeOutlier>, p.total_tiles, stream, start, stop, p);
        else
            launch(decompress_kernel<kDstLinear, 1>, p.total_tiles, stream, start, stop, p);
        return hipGetLastError();
    }
    switch (p.dst_kind) {
    case kDstMulti:
        launch(decompress_kernel<kDstMulti, 0>, p.total_tiles, stream, start, stop, p);
        break;
    case kDstIndexed:
        launch(decompress_kernel<kDstIndexed, 0>, p.total_tiles, stream, start, stop, p);
        break;
    default:
        launch(decompress_kernel<kDstLinear, 0>, p.total_tiles, stream, start, stop, p);
        break;
    }
    return hipGetLastError();
}

int compress_resident_workgroups(int device, bool pipelined) {
    int per_cu = 0;
    const void* fn = pipelined
        ? reinterpret_cast<const void*>(compress_persistent_kernel<0, true>)
        : reinterpret_cast<const void*>(compress_kernel<0, 0>);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, fn, pipelined ? kEncThreads : kThreads, 0) != hipSuccess)
        per_cu = 1;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return per_cu;
    return per_cu * prop.multiProcessorCount;
}

}  // namespace kvszp
