// kvszp_plan.h -- the tile plan of a launch: how a call's requests become
// groups, jobs and tiles, which group, job and tile of the job a tile number
// stands for, and where each workgroup of the persistent decoder starts.
// Shared by the kernels (the device lookups), the host C-ABI (which builds
// the plan) and a host test that walks every tile of random plans with
// bounds checks.  No HIP headers: the host parts build with g++ alone.
//
// A "job" is one logical segment to encode or decode (one page, or the
// layer-selected part of one page).  Jobs with the same geometry form a
// "group".  Every job is cut into tiles of kTileBlocks fixed-rate blocks;
// tiles are numbered group by group, job by job, so the tiles of a job are
// consecutive.  A launch holds at most kMaxGroups groups (the records are
// kernel arguments); the host splits larger calls into several launches.
#ifndef KVSZP_PLAN_H
#define KVSZP_PLAN_H

#include <stdint.h>

#if defined(__HIPCC__)
#define KVSZP_PLAN_FN __host__ __device__ __forceinline__
#else
#define KVSZP_PLAN_FN static inline
#endif

// A value every lane of a wave holds alike, moved to a scalar register on
// the device (so that what it indexes is read with scalar loads).
#if defined(__HIP_DEVICE_COMPILE__)
#define KVSZP_UNIFORM(x) __builtin_amdgcn_readfirstlane(x)
#else
#define KVSZP_UNIFORM(x) (x)
#endif

#include <algorithm>
#include <vector>

namespace kvszp {

constexpr int kBlockElems = 32;                     // fixed-rate block
constexpr int kTileBlocks = 256;                    // blocks per tile
constexpr int kTileElems = kTileBlocks * kBlockElems;
constexpr int kRefTileElems = 32768;                // header granularity
constexpr int kMaxGroups = 16;

// Division by a launch constant d (1 <= d < 2^32) of an index below 2^29
// (segments hold at most 2^29 values, so every element, tile and job index
// of a launch qualifies) as one multiply and one shift: with
// l = ceil(log2 d) and m = ceil(2^(29+l) / d), floor(n m / 2^(29+l)) =
// floor(n / d) for every n < 2^29, because 2^(29+l) <= m d <= 2^(29+l) + 2^l
// (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, Theorem 4.2).  The kernels divide by a job's
// tile count and by its layer geometry on every tile; the generic 32-bit
// division is a sequence of some twenty instructions.
struct Divisor {
    uint32_t mul;
    uint32_t shift;
};

KVSZP_PLAN_FN uint32_t divide(uint32_t n, Divisor d) {
    return (uint32_t)(((uint64_t)n * d.mul) >> d.shift);
}

struct Group {
    uint64_t n;                 // logical elements per job
    const int64_t* layers;      // device layer map, nullptr = contiguous
    uint64_t selected_layers;
    uint64_t source_layers;
    uint64_t elements_per_layer;
    uint32_t first_job;
    uint32_t first_tile;
    uint32_t tiles_per_job;
    uint32_t header_bytes;      // R = 1024 * ceil(n / 32768)
    Divisor tiles_per_job_div;  // by tiles_per_job
    Divisor layer_div;          // by elements_per_layer (layer maps only)
    Divisor prefix_div;         // by selected_layers * elements_per_layer (layer maps only)
};

// Group, job and tile within the job of one tile of a launch.
struct TilePlace {
    int gi;
    uint32_t job;
    uint32_t tile;
};

// The group of tile t: the last group whose first tile is at most t
// (first_tiles[i] = groups[i].first_tile, ascending from 0).
KVSZP_PLAN_FN int group_of_tile(const uint32_t* first_tiles, int num_groups, uint32_t t) {
    int gi = 0;
    for (int i = 1; i < num_groups; ++i)
        if (t >= first_tiles[i]) gi = i;
    return gi;
}

// Tile t's place, its group found in first_tiles.
KVSZP_PLAN_FN TilePlace place_tile(const Group* groups, const uint32_t* first_tiles,
                                   int num_groups, uint32_t t) {
    TilePlace c;
    c.gi = KVSZP_UNIFORM(group_of_tile(first_tiles, num_groups, t));
    const Group& g = groups[c.gi];
    const uint32_t local = t - g.first_tile;
    const uint32_t jig = KVSZP_UNIFORM(divide(local, g.tiles_per_job_div));
    c.tile = local - jig * g.tiles_per_job;
    c.job = g.first_job + jig;
    return c;
}

// First tile of the persistent decoder's workgroup b out of G when tiles
// are weighed by group: each tile of group g weighs tile_weight[g],
// weight_before[g] is the weight of the tiles before the group and
// total_weight that of all tiles (0: equal tile counts).  Run b starts
// where the cumulative weight reaches b/G of the total (rounded up):
// nondecreasing in b, 0 at b = 0 and total_tiles at b = G, so the runs
// tile [0, total_tiles) exactly.
//
// The quotients are taken in double precision: every wave works out two run
// starts before its first tile, and a 64-bit integer division is a long
// scalar sequence (four per wave held back the first tiles of the
// workgroups issued last).  Rounding is monotone, so the starts stay
// nondecreasing whatever the sizes (the products are exact anyway for a
// resident grid, b < 2^12, and total_weight < 2^40: at most 2^24 tiles of
// weight below 2^16), and a workgroup and its successor compute the same
// value for the boundary they share.
KVSZP_PLAN_FN uint32_t weighted_run_start(const Group* groups, int num_groups,
                                          uint32_t total_tiles, uint64_t total_weight,
                                          const uint64_t* weight_before,
                                          const uint32_t* tile_weight, uint32_t b,
                                          uint32_t G) {
    if (b >= G) return total_tiles;
    if (total_weight == 0)
        return (uint32_t)((double)b * (double)total_tiles / (double)G);
    const uint64_t target = (uint64_t)((double)b * (double)total_weight / (double)G);
    int g = 0;
    for (int k = 1; k < num_groups; ++k)
        if (weight_before[k] <= target) g = k;
    const uint32_t first = groups[g].first_tile;
    const uint32_t tiles =
        (g + 1 < num_groups ? groups[g + 1].first_tile : total_tiles) - first;
    const double i = __builtin_ceil((double)(target - weight_before[g]) / (double)tile_weight[g]);
    return first + (i < (double)tiles ? (uint32_t)i : tiles);
}

// ---- host: building and checking a plan ------------------------------------

// Header bytes of a segment of n values: one rate byte per block, for whole
// 32768-value units (rate_offset, cuszp_batched_fixed.cu:165).
inline uint32_t header_bytes_of(uint64_t n) {
    return (uint32_t)((n + kRefTileElems - 1) / kRefTileElems *
                      (kRefTileElems / kBlockElems));
}

inline uint32_t tiles_per_job_of(uint64_t n) {
    return (uint32_t)((n + kTileElems - 1) / kTileElems);
}

// The multiplier and shift of `divide` for d (1 <= d < 2^32; 0 gives a
// divisor that tile_plan_ok rejects).
inline Divisor divisor_of(uint32_t d) {
    if (d == 0) return Divisor{0, 0};
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint32_t shift = 29 + l;
    return Divisor{(uint32_t)(((1ull << shift) + d - 1) / d), shift};
}

inline bool same_divisor(Divisor a, Divisor b) { return a.mul == b.mul && a.shift == b.shift; }

// The divisors of a group's record from its geometry.
inline void set_group_divisors(Group& g) {
    g.tiles_per_job_div = divisor_of(g.tiles_per_job);
    g.layer_div = g.layers ? divisor_of((uint32_t)g.elements_per_layer) : Divisor{0, 0};
    g.prefix_div = g.layers ? divisor_of((uint32_t)(g.selected_layers * g.elements_per_layer))
                            : Divisor{0, 0};
}

// One group of a call as the caller describes it: n values per job (layer
// map `layers` selecting `sel` of `src` layers of `epl` values, or
// contiguous), `jobs` requests.
struct GroupSpec {
    uint64_t n;
    const int64_t* layers;
    uint64_t sel, src, epl;
    uint32_t jobs;
};

// One launch's share of a call: groups [g0, g1) of the call's specs, with
// job numbers global to the call and tile numbers local to the launch.
struct Chunk {
    size_t g0, g1;
    uint64_t tiles;
    uint32_t max_tiles_per_job;
    bool whole_blocks;  // every block whole and inside one layer
};

// Splits `specs` into launches of at most kMaxGroups groups (the group
// records travel as kernel arguments).  The reference takes any number of
// groups (cuszp_wrapper.cpp:683-868, one launch per group).
inline std::vector<Chunk> split_chunks(const std::vector<GroupSpec>& specs) {
    std::vector<Chunk> chunks;
    for (size_t g0 = 0; g0 < specs.size(); g0 += kMaxGroups) {
        Chunk ch{g0, std::min(specs.size(), g0 + (size_t)kMaxGroups), 0, 0, true};
        for (size_t gi = ch.g0; gi < ch.g1; ++gi) {
            const GroupSpec& s = specs[gi];
            const uint32_t tpj = tiles_per_job_of(s.n);
            ch.tiles += (uint64_t)tpj * s.jobs;
            ch.max_tiles_per_job = std::max(ch.max_tiles_per_job, tpj);
            if ((s.n % kBlockElems) != 0 || (s.layers && (s.epl % kBlockElems) != 0))
                ch.whole_blocks = false;
        }
        chunks.push_back(ch);
    }
    return chunks;
}

// Group records of one chunk; `first_job` is the call-wide job number of
// the chunk's first request.  Returns the number of groups.
inline int fill_groups(Group* groups, const std::vector<GroupSpec>& specs, const Chunk& ch,
                       size_t first_job) {
    uint64_t tiles = 0;
    size_t job = first_job;
    for (size_t gi = ch.g0; gi < ch.g1; ++gi) {
        const GroupSpec& s = specs[gi];
        Group& g = groups[gi - ch.g0];
        g.n = s.n;
        g.layers = s.layers;
        g.selected_layers = s.sel;
        g.source_layers = s.src;
        g.elements_per_layer = s.epl;
        g.first_job = (uint32_t)job;
        g.first_tile = (uint32_t)tiles;
        g.tiles_per_job = tiles_per_job_of(s.n);
        g.header_bytes = header_bytes_of(s.n);
        set_group_divisors(g);
        tiles += (uint64_t)g.tiles_per_job * s.jobs;
        job += s.jobs;
    }
    return (int)(ch.g1 - ch.g0);
}

// First tile of workgroup b of a persistent encoder launch of G workgroups;
// the workgroup then takes tiles f, f + G, f + 2G, ... below the tile count.
// C = 0: f = b.  C = the compute units (G = S * C, S workgroups per unit):
// workgroup s * C + r, the s-th workgroup the dispatcher places on unit r,
// starts at f = r * S + s, so that each unit holds S consecutive tiles of a
// round (mostly tiles of one job) instead of tiles C apart.  Either way the
// first tiles are a permutation of 0 .. G - 1 and each workgroup's tiles
// step by G, which is all the encoder's wait order relies on.
KVSZP_PLAN_FN uint32_t persistent_first_tile(uint32_t b, uint32_t G, uint32_t C) {
    if (C == 0) return b;
    const uint32_t s = b / C;
    return (b - s * C) * (G / C) + s;
}

// The C of persistent_first_tile for a launch of `tiles` tiles on `grid`
// workgroups over `cus` compute units.  mode 0: never; 2: whenever the grid
// is a whole number (at least 2) of workgroups per unit; 1: only for
// launches of at least kSlotMixRounds rounds of the grid.  Measured on
// MI355X: the encoder of launches of 75-340 rounds (jobs of 28-64 tiles)
// 1-7 % faster with consecutive tiles on one unit, a launch of 4.7 rounds
// (Qwen2.5-1.5B 4K, jobs of 7 and 21 tiles) 13 % slower: the partial last
// round then falls on every unit's youngest workgroups too, which the
// issue arbiter serves last, instead of on the oldest slots only.
constexpr uint64_t kSlotMixRounds = 16;

inline uint32_t persistent_slot_cus(uint64_t tiles, uint32_t grid, uint32_t cus, int mode) {
    if (mode == 0 || cus == 0 || grid % cus != 0 || grid / cus < 2) return 0;
    if (mode == 1 && tiles < kSlotMixRounds * (uint64_t)grid) return 0;
    return cus;
}

// The plan every tile loop indexes by: groups in launch order from tile 0,
// each a whole number (at least one) of jobs numbered on from the previous
// group's, together exactly `total_tiles`, all of them among the
// `table_jobs` job records the kernel can read; and a grid of at least one
// workgroup and, for the persistent kernels (a workgroup's first tile is its
// own index), at most `total_tiles`.  The launchers check it before every
// launch, so that no kernel indexes job records, layer maps or look-back
// words past a plan that does not add up.
inline bool tile_plan_ok(const Group* groups, int num_groups, uint32_t total_tiles,
                         uint32_t grid, bool persistent, uint32_t table_jobs) {
    if (num_groups < 1 || num_groups > kMaxGroups || total_tiles == 0 || grid == 0) return false;
    if (persistent && grid > total_tiles) return false;
    if (groups[0].first_tile != 0) return false;
    for (int i = 0; i < num_groups; ++i) {
        const Group& g = groups[i];
        const uint32_t end = i + 1 < num_groups ? groups[i + 1].first_tile : total_tiles;
        if (end <= g.first_tile || g.tiles_per_job == 0 || g.n == 0) return false;
        if (tiles_per_job_of(g.n) != g.tiles_per_job) return false;
        if (!same_divisor(g.tiles_per_job_div, divisor_of(g.tiles_per_job))) return false;
        if (g.layers &&
            (g.elements_per_layer == 0 ||
             g.selected_layers * g.elements_per_layer > 0xFFFFFFFFull ||
             !same_divisor(g.layer_div, divisor_of((uint32_t)g.elements_per_layer)) ||
             !same_divisor(g.prefix_div,
                           divisor_of((uint32_t)(g.selected_layers * g.elements_per_layer)))))
            return false;
        const uint32_t tiles = end - g.first_tile;
        if (tiles % g.tiles_per_job != 0) return false;
        const uint64_t jobs_end = (uint64_t)g.first_job + tiles / g.tiles_per_job;
        if (jobs_end > table_jobs) return false;
        if (i + 1 < num_groups && groups[i + 1].first_job != jobs_end) return false;
    }
    return true;
}

// Per-group tile weights of the persistent decoder (weighted_run_start):
// a tile of group g weighs its BF16 output plus the group's average payload
// per tile, from the stream sizes of the chunk's jobs (sizes[j] for the
// call-wide job j, at least the group's header).  Returns total_weight.
inline uint64_t group_tile_weights(const Group* groups, int num_groups,
                                   const std::vector<GroupSpec>& specs, const Chunk& ch,
                                   const uint64_t* sizes, uint64_t* weight_before,
                                   uint32_t* tile_weight) {
    uint64_t before = 0;
    size_t j = groups[0].first_job;
    for (int k = 0; k < num_groups; ++k) {
        const GroupSpec& spec = specs[ch.g0 + (size_t)k];
        const Group& g = groups[k];
        uint64_t payload = 0;
        for (uint32_t i = 0; i < spec.jobs; ++i, ++j) payload += sizes[j] - g.header_bytes;
        const uint64_t tiles = (uint64_t)g.tiles_per_job * spec.jobs;
        // Callers reject empty groups; the guard keeps the division defined.
        const uint64_t w = tiles ? (2 * spec.n * spec.jobs + payload + tiles / 2) / tiles : 1;
        tile_weight[k] = (uint32_t)std::max<uint64_t>(w, 1);
        weight_before[k] = before;
        before += tiles * tile_weight[k];
    }
    return before;
}

// Run starts of the persistent decoder balanced job by job, for a call that
// is one launch: each job weighs its BF16 output plus its payload, spread
// evenly over its tiles; run b starts where the cumulative weight reaches
// b/grid of the total.  grid + 1 entries, nondecreasing, from 0 to the
// launch's tile count.
inline std::vector<uint32_t> job_balanced_runs(const std::vector<GroupSpec>& specs,
                                               const uint64_t* sizes, size_t batch,
                                               uint64_t total_tiles, uint32_t grid) {
    std::vector<uint64_t> bytes(batch);
    std::vector<uint32_t> tiles_of(batch);
    uint64_t total = 0;
    size_t j = 0;
    for (const GroupSpec& spec : specs) {
        const uint32_t R = header_bytes_of(spec.n);
        const uint32_t tpj = tiles_per_job_of(spec.n);
        for (uint32_t k = 0; k < spec.jobs; ++k, ++j) {
            bytes[j] = 2 * spec.n + (sizes[j] - R);
            tiles_of[j] = tpj;
            total += bytes[j];
        }
    }
    std::vector<uint32_t> runs((size_t)grid + 1);
    size_t jj = 0;
    uint64_t before = 0;
    uint64_t tile_before = 0;
    for (uint32_t b = 0; b < grid; ++b) {
        const uint64_t target = (uint64_t)((unsigned __int128)b * total / grid);
        while (jj < batch && before + bytes[jj] <= target) {
            before += bytes[jj];
            tile_before += tiles_of[jj];
            ++jj;
        }
        if (jj == batch) {
            runs[b] = (uint32_t)total_tiles;
        } else {
            const uint64_t i = (uint64_t)(((unsigned __int128)(target - before) * tiles_of[jj] +
                                           bytes[jj] - 1) / bytes[jj]);
            runs[b] = (uint32_t)(tile_before + std::min<uint64_t>(i, tiles_of[jj]));
        }
    }
    runs[grid] = (uint32_t)total_tiles;
    return runs;
}

}  // namespace kvszp

#endif  // KVSZP_PLAN_H
