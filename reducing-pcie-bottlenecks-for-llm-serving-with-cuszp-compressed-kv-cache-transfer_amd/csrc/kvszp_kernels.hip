// kvszp_kernels.hip -- gfx950 kernels of the batched fixed-mode BF16
// KV-page codec.
//
// Reference semantics: integration/cuszp_wrapper/cuszp_batched_fixed.cu
//   quantizer            :10-25   -> quantize()
//   rate                 :27-31   -> block_rate()
//   layer gather         :33-50   -> LayerCursor / map_index()
//   relative bound       :55-133  -> fused min/max exchange (compress) or
//                                    minmax_kernel (pre-pass)
//   encoder              :135-359 -> compress_kernel
//   decoder              :361-627 -> decompress_kernel
//
// Schedule (not the reference's): one workgroup of 256 threads per tile of
// 256 blocks, ONE THREAD PER 32-ELEMENT BLOCK.  A thread loads its block with
// four 16-byte loads, quantizes in registers, and builds the sign and plane
// words with a register bit-matrix transpose (kvszp_bits.h) instead of the
// reference's per-bit loops.  Block offsets come from a workgroup scan plus a
// decoupled look-back across the tiles of a job.  Cross-workgroup state is a
// single 64-bit word per tile holding {epoch tag, status, value}, read and
// written with relaxed agent-scope atomics (these bypass the per-XCD L2), so
// no fence and no per-call memset is needed: stale words carry an older
// epoch and never match.
#include "kvszp_internal.h"
#include "kvszp_bits.h"

#include <float.h>

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

// ---- cross-workgroup primitives -------------------------------------------

__device__ __forceinline__ unsigned long long load_relaxed(
    const unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void store_relaxed(unsigned long long* p,
                                              unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void flag_error(uint32_t* e, uint32_t bits) {
    __hip_atomic_fetch_or(e, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const uint32_t o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_min(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const uint32_t o = __shfl_xor(v, d, 64);
        v = o < v ? o : v;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v,
                                                        int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    return v;
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

// eb = eps * fmaxf(max - min, 1e-6f), cu:128-131.
__device__ __forceinline__ float relative_bound(float eps, uint32_t kmin,
                                                uint32_t kmax) {
    const float range = fmaxf(max_key_value(kmax) - min_key_value(kmin), 1e-6f);
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
            const u32x4 v = __builtin_nontemporal_load(p + i);
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

// Executed by one full wave.  Publishes this tile's aggregate, walks back
// over earlier tiles of the same job 64 at a time until it meets one whose
// inclusive prefix is published, and publishes its own inclusive prefix.
// Returns the exclusive prefix (bytes of earlier tiles of the job).
__device__ uint32_t lookback(unsigned long long* state, uint32_t t,
                             uint32_t tile, uint32_t total, uint32_t epoch,
                             uint32_t* err) {
    const int lane = __lane_id();
    const uint32_t tag_agg = epoch * 4u + 1u;
    const uint32_t tag_inc = epoch * 4u + 2u;
    if (tile == 0) {
        if (lane == 0)
            store_relaxed(&state[t],
                          ((unsigned long long)tag_inc << 32) | total);
        return 0;
    }
    if (lane == 0)
        store_relaxed(&state[t], ((unsigned long long)tag_agg << 32) | total);
    uint32_t acc = 0;
    uint32_t remaining = tile;   // earlier tiles of this job
    uint32_t pos = t - 1;        // tile read by lane 0
    for (;;) {
        const uint32_t nwin = remaining < 64u ? remaining : 64u;
        const bool in_win = (uint32_t)lane < nwin;
        const unsigned long long win_mask =
            nwin == 64u ? ~0ull : ((1ull << nwin) - 1ull);
        unsigned long long w = 0, need = 0, incl = 0;
        for (uint32_t spins = 0;; ++spins) {
            w = in_win ? load_relaxed(&state[pos - lane]) : 0ull;
            const uint32_t tag = (uint32_t)(w >> 32);
            incl = __ballot(in_win && tag == tag_inc);
            const unsigned long long ready =
                __ballot(in_win && (tag == tag_inc || tag == tag_agg));
            need = incl ? (((incl & (~incl + 1ull)) << 1) - 1ull) : win_mask;
            if ((ready & need) == need) break;
            if (spins >= kSpinLimit) {
                if (lane == 0) flag_error(err, kErrSpin);
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

// Finds the group of tile t (groups are few and ordered by first_tile).
__device__ __forceinline__ int find_group(const Group* groups, int num_groups,
                                          uint32_t t) {
    int g = 0;
    for (int i = 1; i < num_groups; ++i)
        if (t >= groups[i].first_tile) g = i;
    return g;
}

// ---- stream word I/O --------------------------------------------------------
// A block's payload is `count` consecutive 4-byte-aligned words.  Lanes move
// them as 16-byte groups (unaligned 128-bit accesses) plus single words for
// the tail; `cmax` is the wave-uniform maximum count, so groups no lane needs
// are skipped without divergence.  Nothing outside [0, count) is touched.
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
                __builtin_nontemporal_store(v, (g_u32x4_a4*)(d + 4 * j));
            } else {
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    if (count > (uint32_t)(4 * j + i))
                        __builtin_nontemporal_store(w[4 * j + i], d + 4 * j + i);
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
                const u32x4 v = __builtin_nontemporal_load((const g_u32x4_a4*)(s + 4 * j));
                w[4 * j + 0] = v.x;
                w[4 * j + 1] = v.y;
                w[4 * j + 2] = v.z;
                w[4 * j + 3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 3; ++i)
                    if (count > (uint32_t)(4 * j + i))
                        w[4 * j + i] = __builtin_nontemporal_load(s + 4 * j + i);
            }
        }
    }
}

// ---- encoder ---------------------------------------------------------------

template <int kQuant>
__global__ __launch_bounds__(kThreads) void compress_kernel(CompressParams p) {
    __shared__ uint32_t s_tile;
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_min[kThreads / 64];
    __shared__ uint32_t s_max[kThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ uint8_t s_rate[kTileBlocks];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (tid == 0) s_tile = take_ticket(p.ticket, p.ticket_base);
    __syncthreads();
    const uint32_t t = s_tile;
    if (t >= p.total_tiles) {  // tickets of another launch: never index past
        if (tid == 0) flag_error(p.error, kErrSpin);
        return;
    }
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];

    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = local / g.tiles_per_job;
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const CompressJob J = p.jobs[job];
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t tile_first = (uint64_t)tile * kTileElems;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;

    uint32_t bad = 0;
    uint32_t d[16];
    load_block(g, J.in, tile_first, (uint32_t)tid * kBlockElems, count,
               p.aligned16 != 0, d, &bad);

    float eb = J.eps;
    if (p.bound_mode != kBoundAbsolute) {
        uint32_t kmin, kmax;
        if (p.bound_mode == kBoundFused) {
            // min/max of this thread's values (fminf/fmaxf skip NaN, cu:78-79)
            float lo = FLT_MAX, hi = -FLT_MAX;
            for (uint32_t v = 0; v < count; ++v) {
                const float x = (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
                lo = fminf(lo, x);
                hi = fmaxf(hi, x);
            }
            kmin = lo == FLT_MAX ? kKeyEmptyMin : bf16_key(lo);
            kmax = hi == -FLT_MAX ? kKeyEmptyMax : bf16_key(hi);
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
                for (uint32_t spins = 0; (uint32_t)(w >> 32) != p.epoch; ++spins) {
                    if (spins >= kSpinLimit) {
                        flag_error(p.error, kErrSpin);
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

    // Quantize (cu:180-231): a[v] = |q| | sign << 31.
    uint32_t a[32];
    uint32_t orv = 0;
    if (count == kBlockElems) {
#pragma unroll
        for (int v = 0; v < 32; ++v) {
            const float x = (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
            const int32_t q = quantize<kQuant>(x, recip);
            const uint32_t m = (uint32_t)(q < 0 ? -q : q);
            orv |= m;
            a[v] = m | ((uint32_t)q & 0x80000000u);
        }
    } else {
#pragma unroll
        for (int v = 0; v < 32; ++v) {
            const float x = (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
            int32_t q = quantize<kQuant>(x, recip);
            q = (uint32_t)v < count ? q : 0;
            const uint32_t m = (uint32_t)(q < 0 ? -q : q);
            orv |= m;
            a[v] = m | ((uint32_t)q & 0x80000000u);
        }
    }
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
        const uint32_t prefix =
            lookback(p.tile_state, t, tile, sc.total, p.epoch, p.error);
        if (lane == 0) {
            s_prefix = prefix;
            if (last_tile) p.job_size[job] = R + prefix + sc.total;
            if (tile == 0) p.job_eb[job] = eb;
        }
    }
    if (bad & 1) flag_error(p.error, kErrLayerIndex);
    if (bad & 2) flag_error(p.error, kErrSpin);
    __syncthreads();

    // Payload (cu:302-358): sign word, then `rate` plane words.
    const uint32_t rmax = wave_max(rate);
    if (rmax == 0) return;
    uint32_t* dst = reinterpret_cast<uint32_t*>(J.out + R + s_prefix + sc.exclusive);
    const uint32_t count_words = rate ? rate + 1u : 0u;
    if (rmax <= 15u) {
        uint32_t words[16];
        pack_block_words_narrow(a, words);
        store_words<16>(dst, words, count_words, rmax + 1u);
    } else {
        uint32_t words[32];
        pack_block_words_wide(a, words);
        store_words<32>(dst, words, count_words, rmax + 1u);
    }
}

// ---- relative-bound pre-pass (jobs too long for the fused exchange) -------

__global__ __launch_bounds__(kThreads) void minmax_kernel(MinMaxParams p) {
    __shared__ uint32_t s_min[kThreads / 64];
    __shared__ uint32_t s_max[kThreads / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const uint32_t t = blockIdx.x;
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];
    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = local / g.tiles_per_job;
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const CompressJob J = p.jobs[job];
    const uint64_t n = g.n;
    const uint32_t nb = (uint32_t)((n + kBlockElems - 1) / kBlockElems);
    const uint32_t b = tile * kTileBlocks + tid;
    const uint64_t e0 = (uint64_t)b * kBlockElems;
    const uint32_t count =
        b < nb ? (uint32_t)(n - e0 < kBlockElems ? n - e0 : kBlockElems) : 0u;
    uint32_t bad = 0;
    uint32_t d[16];
    load_block(g, J.in, (uint64_t)tile * kTileElems, (uint32_t)tid * kBlockElems,
               count, false, d, &bad);
    float lo = FLT_MAX, hi = -FLT_MAX;
    for (uint32_t v = 0; v < count; ++v) {
        const float x = (v & 1) ? bf16_hi(d[v >> 1]) : bf16_lo(d[v >> 1]);
        lo = fminf(lo, x);
        hi = fmaxf(hi, x);
    }
    uint32_t kmin = lo == FLT_MAX ? kKeyEmptyMin : bf16_key(lo);
    uint32_t kmax = hi == -FLT_MAX ? kKeyEmptyMax : bf16_key(hi);
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
        __hip_atomic_fetch_max(&p.job_minmax[2 * job + 1],
                               tag | (0xFFFFu - kmin), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    if (bad) flag_error(p.error, kErrLayerIndex);
}

// ---- decoder ---------------------------------------------------------------

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
            __builtin_nontemporal_store(v, p + i);
        }
        return;
    }
    __attribute__((address_space(1))) uint16_t* g = to_global(dst);
    for (uint32_t v = 0; v < count; ++v)
        g[v] = (uint16_t)((v & 1) ? (out[v >> 1] >> 16) : (out[v >> 1] & 0xFFFFu));
}

template <int kDst>
__global__ __launch_bounds__(kThreads) void decompress_kernel(
    DecompressParams p) {
    __shared__ uint32_t s_tile;
    __shared__ uint32_t s_wave[kThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ uint32_t s_hdr[kTileBlocks / 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (tid == 0) s_tile = take_ticket(p.ticket, p.ticket_base);
    __syncthreads();
    const uint32_t t = s_tile;
    if (t >= p.total_tiles) {
        if (tid == 0) flag_error(p.error, kErrSpin);
        return;
    }
    const Group& g = p.groups[find_group(p.groups, p.num_groups, t)];
    const uint32_t local = t - g.first_tile;
    const uint32_t job_in_group = local / g.tiles_per_job;
    const uint32_t tile = local - job_in_group * g.tiles_per_job;
    const uint32_t job = g.first_job + job_in_group;
    const DecompressJob J = p.jobs[job];
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
    const TileScan sc = tile_scan(bytes, tid, s_wave);
    if (wave == 0) {
        const uint32_t prefix =
            lookback(p.tile_state, t, tile, sc.total, p.epoch, p.error);
        if (lane == 0) s_prefix = prefix;
    }
    __syncthreads();
    const uint64_t base = (uint64_t)R + s_prefix + sc.exclusive;
    if (rate && base + bytes > J.size) {
        err |= kErrTruncated;
        rate = 0;
    }

    // Unpack (cu:496-538): rows-by-plane -> rows-by-element.
    const uint32_t rmax = wave_max(rate);
    uint32_t out[16];
    if (rmax == 0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = 0;
    } else {
        const uint32_t* src = reinterpret_cast<const uint32_t*>(J.in + base);
        const uint32_t count_words = rate ? rate + 1u : 0u;
        uint32_t m[32];
        const float eb = J.eb;
        if (rmax <= 15u) {
            uint32_t w[16];
            load_words<16>(src, w, count_words, rmax + 1u);
#pragma unroll
            for (int i = 0; i < 15; ++i) m[i] = w[1 + i];
            m[15] = w[0];
            transpose16x2(m);
#pragma unroll
            for (int v = 0; v < 32; v += 2) {
                const uint32_t f0 = v < 16 ? (m[v ^ 7] & 0xFFFFu) : (m[(v - 16) ^ 7] >> 16);
                const uint32_t f1 = (v + 1) < 16 ? (m[(v + 1) ^ 7] & 0xFFFFu)
                                                 : (m[(v + 1 - 16) ^ 7] >> 16);
                const int32_t q0 = (f0 & 0x8000u) ? -(int32_t)(f0 & 0x7FFFu) : (int32_t)(f0 & 0x7FFFu);
                const int32_t q1 = (f1 & 0x8000u) ? -(int32_t)(f1 & 0x7FFFu) : (int32_t)(f1 & 0x7FFFu);
                f32x2 y;
                y.x = ((float)q0 * eb) * 2.0f;
                y.y = ((float)q1 * eb) * 2.0f;
                const bf16x2 h = __builtin_convertvector(y, bf16x2);
                out[v >> 1] = __builtin_bit_cast(uint32_t, h);
            }
        } else {
            uint32_t w[32];
            load_words<32>(src, w, count_words, rmax + 1u);
#pragma unroll
            for (int i = 0; i < 31; ++i) m[i] = w[1 + i];
            m[31] = w[0];
            transpose32(m);
#pragma unroll
            for (int v = 0; v < 32; v += 2) {
                const uint32_t a0 = m[v ^ 7], a1 = m[(v + 1) ^ 7];
                const int32_t q0 = (a0 >> 31) ? -(int32_t)(a0 & 0x7FFFFFFFu) : (int32_t)(a0 & 0x7FFFFFFFu);
                const int32_t q1 = (a1 >> 31) ? -(int32_t)(a1 & 0x7FFFFFFFu) : (int32_t)(a1 & 0x7FFFFFFFu);
                f32x2 y;
                y.x = ((float)q0 * eb) * 2.0f;
                y.y = ((float)q1 * eb) * 2.0f;
                const bf16x2 h = __builtin_convertvector(y, bf16x2);
                out[v >> 1] = __builtin_bit_cast(uint32_t, h);
            }
        }
        if (rate == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) out[i] = 0;
        }
    }

    if (count && (rate != 0 || p.rate0_zero)) {
        if (kDst == kDstLinear) {
            store_block(J.dst + e0, out, count, p.aligned16 != 0);
        } else if (kDst == kDstMulti) {
            const uint64_t epd = p.elements_per_dest;
            const uint64_t di = e0 / epd;
            const uint64_t off = e0 - di * epd;
            if (off + count <= epd) {
                uint16_t* dst = p.dests[(uint64_t)job * p.dests_per_page + di] + off;
                store_block(dst, out, count,
                            ((uintptr_t)dst & 15u) == 0);
            } else {
                for (uint32_t v = 0; v < count; ++v) {
                    const uint64_t e = e0 + v;
                    const uint64_t dv = e / epd;
                    uint16_t* dst = p.dests[(uint64_t)job * p.dests_per_page + dv];
                    to_global(dst)[e - dv * epd] = (uint16_t)((v & 1) ? (out[v >> 1] >> 16)
                                                           : (out[v >> 1] & 0xFFFFu));
                }
            }
        } else {
            uint32_t badl = 0;
            const LayerCursor c = layer_cursor(g, (uint64_t)tile * kTileElems,
                                               (uint32_t)tid * kBlockElems, &badl);
            if (c.contiguous && !badl) {
                uint16_t* dst = J.dst + c.src_index;
                store_block(dst, out, count, ((uintptr_t)dst & 15u) == 0);
            } else {
                for (uint32_t v = 0; v < count; ++v) {
                    const uint64_t s = map_index(e0 + v, g.layers, g.selected_layers,
                                                 g.source_layers,
                                                 g.elements_per_layer, &badl);
                    if (badl) break;
                    to_global(J.dst)[s] = (uint16_t)((v & 1) ? (out[v >> 1] >> 16)
                                                  : (out[v >> 1] & 0xFFFFu));
                }
            }
            if (badl) err |= kErrLayerIndex;
        }
    }
    if (err) flag_error(p.error, err);
}

}  // namespace

hipError_t launch_compress(const CompressParams& p, hipStream_t stream) {
    if (p.quantizer)
        hipLaunchKernelGGL(compress_kernel<1>, dim3(p.total_tiles), dim3(kThreads),
                           0, stream, p);
    else
        hipLaunchKernelGGL(compress_kernel<0>, dim3(p.total_tiles), dim3(kThreads),
                           0, stream, p);
    return hipGetLastError();
}

hipError_t launch_minmax(const MinMaxParams& p, uint32_t grid,
                         hipStream_t stream) {
    hipLaunchKernelGGL(minmax_kernel, dim3(grid), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_decompress(const DecompressParams& p, hipStream_t stream) {
    switch (p.dst_kind) {
    case kDstMulti:
        hipLaunchKernelGGL(decompress_kernel<kDstMulti>, dim3(p.total_tiles),
                           dim3(kThreads), 0, stream, p);
        break;
    case kDstIndexed:
        hipLaunchKernelGGL(decompress_kernel<kDstIndexed>, dim3(p.total_tiles),
                           dim3(kThreads), 0, stream, p);
        break;
    default:
        hipLaunchKernelGGL(decompress_kernel<kDstLinear>, dim3(p.total_tiles),
                           dim3(kThreads), 0, stream, p);
        break;
    }
    return hipGetLastError();
}

int compress_resident_workgroups(int device) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(compress_kernel<0>),
            kThreads, 0) != hipSuccess)
        per_cu = 1;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return per_cu;
    return per_cu * prop.multiProcessorCount;
}

}  // namespace kvszp
