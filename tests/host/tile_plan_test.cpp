// Host walk of the tile plan (csrc/kvszp_plan.h), with bounds checks.
// Random calls are split into launches and group records by the C-ABI's own
// functions (split_chunks, fill_groups), and every tile of every launch is
// placed by the kernels' own lookup (place_tile): each tile must land on a
// group, job and tile of the job inside the launch's tables, every (job,
// tile) exactly once, and tile numbers must run job by job.  The launch
// check (tile_plan_ok) must accept these plans at every grid the library
// uses and reject plans that do not add up.  The persistent decoder's run
// starts (per-group weights and per-job runs) must tile [0, tiles) in order.
//
// Launches smaller than the persistent grid (a 3-tile launch of n = 32
// pages, grid = 3) are among the cases; tiles at or past the launch's tile
// count, which no kernel places, map to job records past the launch's last
// job, which the test shows for that case.
//
// Prints "mismatches=0" when every check holds.
#include "kvszp_plan.h"

#include <cstdio>
#include <random>
#include <vector>

using namespace kvszp;

static long g_bad = 0;

#define CHECK(cond, ...)                                  \
    do {                                                  \
        if (!(cond)) {                                    \
            if (g_bad < 20) {                             \
                std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
                std::printf(__VA_ARGS__);                 \
                std::printf("\n");                        \
            }                                             \
            ++g_bad;                                      \
        }                                                 \
    } while (0)

static const uint64_t kSizes[] = {1, 31, 32, 33, 1000, 8191, 8192, 8193, 16384, 32768,
                                  32769, 65536, 131072, 229376, 1048576};

static void check_runs(const std::vector<uint32_t>& starts, uint32_t total, const char* what) {
    CHECK(starts.front() == 0, "%s: first run starts at %u", what, starts.front());
    CHECK(starts.back() == total, "%s: last run ends at %u, not %u", what, starts.back(), total);
    for (size_t b = 1; b < starts.size(); ++b)
        CHECK(starts[b - 1] <= starts[b] && starts[b] <= total,
              "%s: run %zu starts at %u after %u (tiles %u)", what, b, starts[b],
              starts[b - 1], total);
}

// One launch: placement, plan checks, decoder runs.
static void check_launch(const std::vector<GroupSpec>& specs, const Chunk& ch,
                         size_t first_job, const std::vector<uint64_t>& sizes,
                         long* tiles_checked) {
    const uint32_t table_jobs = (uint32_t)sizes.size();  // the call's job records
    Group groups[kMaxGroups];
    const int ng = fill_groups(groups, specs, ch, first_job);
    const uint32_t total = (uint32_t)ch.tiles;
    uint32_t first_tiles[kMaxGroups];
    size_t jobs = 0;
    for (int i = 0; i < ng; ++i) {
        first_tiles[i] = groups[i].first_tile;
        jobs += specs[ch.g0 + (size_t)i].jobs;
    }
    CHECK(ng >= 1 && ng <= kMaxGroups, "groups %d", ng);
    CHECK(groups[0].first_job == first_job, "first job %u, not %zu", groups[0].first_job,
          first_job);

    // The launch check at the grids the library uses.
    CHECK(tile_plan_ok(groups, ng, total, total, false, table_jobs),
          "plan rejected (one tile per workgroup)");
    for (uint32_t G : {1u, 2u, 3u, 7u, 256u, 1536u, 2048u, total}) {
        const uint32_t grid = G < total ? G : total;
        CHECK(tile_plan_ok(groups, ng, total, grid, true, table_jobs), "plan rejected at grid %u",
              grid);
    }
    CHECK(!tile_plan_ok(groups, ng, total, total + 1, true, table_jobs),
          "grid past the tiles accepted");
    CHECK(!tile_plan_ok(groups, ng, total, total, false, (uint32_t)(first_job + jobs - 1)),
          "plan past the job table accepted");

    // Placement: in bounds, a bijection onto (job, tile), job by job.
    std::vector<uint32_t> job_first_tile(jobs + 1, 0);
    {
        uint32_t t = 0;
        size_t j = 0;
        for (int i = 0; i < ng; ++i)
            for (uint32_t k = 0; k < specs[ch.g0 + (size_t)i].jobs; ++k, ++j) {
                job_first_tile[j] = t;
                t += groups[i].tiles_per_job;
            }
        job_first_tile[jobs] = t;
        CHECK(t == total, "tiles of the groups %u, launch %u", t, total);
    }
    std::vector<uint8_t> seen(total, 0);
    for (uint32_t t = 0; t < total; ++t) {
        const TilePlace pl = place_tile(groups, first_tiles, ng, t);
        if (pl.gi < 0 || pl.gi >= ng) {
            CHECK(false, "tile %u: group %d of %d", t, pl.gi, ng);
            continue;
        }
        const Group& g = groups[pl.gi];
        const uint32_t end = pl.gi + 1 < ng ? groups[pl.gi + 1].first_tile : total;
        const uint32_t g_jobs = specs[ch.g0 + (size_t)pl.gi].jobs;
        CHECK(t >= g.first_tile && t < end, "tile %u outside group %d [%u, %u)", t, pl.gi,
              g.first_tile, end);
        CHECK(pl.job >= g.first_job && pl.job < g.first_job + g_jobs,
              "tile %u: job %u outside group %d's jobs [%u, %u)", t, pl.job, pl.gi,
              g.first_job, g.first_job + g_jobs);
        CHECK(pl.job >= first_job && pl.job < first_job + jobs,
              "tile %u: job %u outside the launch's jobs [%zu, %zu)", t, pl.job, first_job,
              first_job + jobs);
        CHECK(pl.tile < g.tiles_per_job, "tile %u: tile %u of %u", t, pl.tile, g.tiles_per_job);
        CHECK((uint64_t)pl.tile * kTileElems < g.n, "tile %u holds no value of its job", t);
        const size_t lj = pl.job - first_job;
        if (lj < jobs) {
            CHECK(job_first_tile[lj] + pl.tile == t, "tile %u placed at job %u tile %u", t,
                  pl.job, pl.tile);
            seen[job_first_tile[lj] + pl.tile] += 1;
        }
        ++*tiles_checked;
    }
    for (uint32_t t = 0; t < total; ++t) CHECK(seen[t] == 1, "tile %u placed %u times", t, seen[t]);

    // Tiles past the launch are never placed by a kernel (every tile loop
    // stops at total_tiles); placed anyway, they land on job records past the
    // launch's last job.
    for (uint32_t t = total; t < total + 3; ++t) {
        const TilePlace pl = place_tile(groups, first_tiles, ng, t);
        CHECK(pl.job >= first_job + jobs, "tile %u past the launch maps into it (job %u)", t,
              pl.job);
    }

    // Persistent decoder: per-group weights and per-job runs.
    uint64_t weight_before[kMaxGroups];
    uint32_t tile_weight[kMaxGroups];
    const uint64_t total_weight =
        group_tile_weights(groups, ng, specs, ch, sizes.data(), weight_before, tile_weight);
    CHECK(total_weight > 0, "no weight");
    for (uint32_t G : {1u, 3u, 256u, 2048u}) {
        const uint32_t grid = G < total ? G : total;
        for (uint64_t tw : {total_weight, (uint64_t)0}) {
            std::vector<uint32_t> starts(grid + 1);
            for (uint32_t b = 0; b <= grid; ++b)
                starts[b] = weighted_run_start(groups, ng, total, tw, weight_before, tile_weight,
                                               b, grid);
            check_runs(starts, total, tw ? "weighted runs" : "equal runs");
        }
    }
}

int main() {
    std::mt19937_64 rng(20260301);
    long launches = 0, tiles_checked = 0;

    // The faulted variant's launch: three one-tile jobs (n = 32), grid 3.
    {
        std::vector<GroupSpec> specs{GroupSpec{32, nullptr, 0, 0, 0, 3}};
        const std::vector<Chunk> chunks = split_chunks(specs);
        CHECK(chunks.size() == 1 && chunks[0].tiles == 3, "3-tile launch");
        std::vector<uint64_t> sizes(3, header_bytes_of(32) + 8);
        check_launch(specs, chunks[0], 0, sizes, &tiles_checked);
        Group groups[kMaxGroups];
        fill_groups(groups, specs, chunks[0], 0);
        const uint32_t first_tiles[1] = {0};
        // A lane per future tile t + k*G (G = 3) reads job record t + k*G.
        for (uint32_t t = 3; t < 3 + 64; ++t)
            CHECK(place_tile(groups, first_tiles, 1, t).job == t, "tile %u", t);
        ++launches;
    }

    for (int trial = 0; trial < 4000; ++trial) {
        const int ngroups = 1 + (int)(rng() % (trial % 5 == 0 ? 40 : 6));
        std::vector<GroupSpec> specs;
        uint64_t tiles = 0;
        for (int g = 0; g < ngroups; ++g) {
            uint64_t n = kSizes[rng() % (sizeof(kSizes) / sizeof(kSizes[0]))];
            if (rng() % 4 == 0) n = 1 + rng() % (1u << 21);
            const uint32_t jobs = 1 + (uint32_t)(rng() % (rng() % 8 == 0 ? 300 : 12));
            if (rng() % 3 == 0) {
                // a layer-mapped group: sel of src layers of epl values, n = prefix x sel x epl
                static const int64_t kMap[1] = {0};
                const uint64_t epl = 32u * (1u + rng() % 512u), sel = 1u + rng() % 8u;
                const uint64_t prefix = 1u + rng() % 2u;
                n = prefix * sel * epl;
                specs.push_back(GroupSpec{n, kMap, sel, sel + rng() % 4u, epl, jobs});
            } else {
                specs.push_back(GroupSpec{n, nullptr, 0, 0, 0, jobs});
            }
            tiles += (uint64_t)tiles_per_job_of(n) * jobs;
        }
        if (tiles > 400000) continue;
        size_t batch = 0;
        for (const GroupSpec& s : specs) batch += s.jobs;
        std::vector<uint64_t> sizes(batch);
        {
            size_t j = 0;
            for (const GroupSpec& s : specs)
                for (uint32_t k = 0; k < s.jobs; ++k, ++j)
                    sizes[j] = header_bytes_of(s.n) +
                               4 * (rng() % (32 * ((s.n + kBlockElems - 1) / kBlockElems) + 1));
        }
        const std::vector<Chunk> chunks = split_chunks(specs);
        CHECK(chunks.size() == (specs.size() + kMaxGroups - 1) / kMaxGroups, "chunks");
        size_t first_job = 0;
        for (const Chunk& ch : chunks) {
            CHECK(ch.g1 - ch.g0 <= (size_t)kMaxGroups && ch.g1 > ch.g0, "chunk groups");
            check_launch(specs, ch, first_job, sizes, &tiles_checked);
            for (size_t gi = ch.g0; gi < ch.g1; ++gi) first_job += specs[gi].jobs;
            ++launches;
        }
        CHECK(first_job == batch, "jobs %zu of %zu", first_job, batch);
        if (chunks.size() == 1) {
            for (uint32_t G : {1u, 7u, 2048u}) {
                const uint32_t grid = G < chunks[0].tiles ? G : (uint32_t)chunks[0].tiles;
                check_runs(job_balanced_runs(specs, sizes.data(), batch, chunks[0].tiles, grid),
                           (uint32_t)chunks[0].tiles, "job-balanced runs");
            }
        }
    }

    // The kernels' division by a launch constant, against the hardware
    // division: every divisor class (1, powers of two and their neighbours,
    // the library's tile counts and layer sizes, random ones up to 2^32 - 1)
    // at the ends of the index range and at random indices below 2^29.
    {
        std::vector<uint32_t> ds{1u, 2u, 3u, 5u, 6u, 7u, 21u, 28u, 128u, 4096u, 28672u, 86016u,
                                 (1u << 29) - 1u, 1u << 29, (1u << 29) + 1u, 0xFFFFFFFFu,
                                 0xFFFFFFFEu, 0x80000000u, 0x80000001u};
        for (int k = 1; k < 32; ++k) {
            ds.push_back(1u << k);
            ds.push_back((1u << k) - 1u);
            ds.push_back((1u << k) + 1u);
        }
        for (int i = 0; i < 2000; ++i) ds.push_back(1u + (uint32_t)(rng() % 0xFFFFFFFFull));
        for (int i = 0; i < 2000; ++i) ds.push_back(1u + (uint32_t)(rng() % 100000u));
        long checked = 0;
        for (uint32_t d : ds) {
            const Divisor dv = divisor_of(d);
            std::vector<uint32_t> ns{0u, 1u, d - 1u, d, d + 1u, (1u << 29) - 1u, (1u << 29) - 2u};
            for (int i = 0; i < 200; ++i) ns.push_back((uint32_t)(rng() % (1u << 29)));
            for (uint32_t m = 1; m < 64 && (uint64_t)m * d < (1u << 29); ++m) {
                ns.push_back(m * d - 1u);
                ns.push_back(m * d);
            }
            for (uint32_t n : ns) {
                if (n >= (1u << 29)) continue;
                CHECK(divide(n, dv) == n / d, "%u / %u: %u", n, d, divide(n, dv));
                ++checked;
            }
        }
        // every index below 2^16 for small divisors
        for (uint32_t d = 1; d < 300; ++d) {
            const Divisor dv = divisor_of(d);
            for (uint32_t n = 0; n < (1u << 16); ++n) CHECK(divide(n, dv) == n / d, "%u / %u", n, d);
            checked += 1 << 16;
        }
        std::printf("divisions=%ld\n", checked);
    }

    // Plans that do not add up are rejected (planted on the host).
    {
        std::vector<GroupSpec> specs{GroupSpec{20000, nullptr, 0, 0, 0, 4},
                                     GroupSpec{8192, nullptr, 0, 0, 0, 5}};
        const Chunk ch = split_chunks(specs)[0];  // 4 x 3 + 5 x 1 = 17 tiles
        Group ok[kMaxGroups];
        const int ng = fill_groups(ok, specs, ch, 0);
        CHECK(tile_plan_ok(ok, ng, 17, 17, true, 9), "good plan rejected");
        Group g[kMaxGroups];
        auto reset = [&] { for (int i = 0; i < ng; ++i) g[i] = ok[i]; };
        reset(); CHECK(!tile_plan_ok(g, ng, 18, 17, false, 9), "tile count past the groups accepted");
        reset(); CHECK(!tile_plan_ok(g, ng, 17, 17, false, 8), "job past the table accepted");
        reset(); CHECK(!tile_plan_ok(g, ng, 17, 17, false, 0), "empty table accepted");
        reset(); g[1].first_job += 1; CHECK(!tile_plan_ok(g, ng, 17, 17, false, 9), "job gap accepted");
        reset(); g[1].first_tile -= 1; CHECK(!tile_plan_ok(g, ng, 17, 17, false, 9), "partial job accepted");
        reset(); g[0].first_tile = 1; CHECK(!tile_plan_ok(g, ng, 17, 17, false, 9), "plan not from tile 0 accepted");
        reset(); g[0].tiles_per_job = 2; CHECK(!tile_plan_ok(g, ng, 17, 17, false, 9), "tiles per job off accepted");
        reset(); CHECK(!tile_plan_ok(g, 0, 17, 17, false, 9), "no groups accepted");
        reset(); CHECK(!tile_plan_ok(g, ng, 17, 0, false, 9), "empty grid accepted");
        reset(); CHECK(!tile_plan_ok(g, kMaxGroups + 1, 17, 17, false, 9), "too many groups accepted");
        reset(); g[1].tiles_per_job_div.mul += 1; CHECK(!tile_plan_ok(g, ng, 17, 17, false, 9), "wrong divisor accepted");
        reset(); g[0].tiles_per_job_div = Divisor{0, 0}; CHECK(!tile_plan_ok(g, ng, 17, 17, false, 9), "missing divisor accepted");
    }

    // The persistent encoder's first tiles: a permutation of 0 .. G - 1 for
    // every grid of S workgroups on C units, so that the workgroups' walks
    // f, f + G, ... cover every tile of a launch exactly once; and the
    // launches that take the unit-major order.
    {
        long walked = 0;
        for (uint32_t C : {1u, 2u, 8u, 80u, 256u, 304u}) {
            for (uint32_t S = 1; S <= 8; ++S) {
                const uint32_t G = C * S;
                std::vector<int> seen(G, 0);
                for (uint32_t b = 0; b < G; ++b) {
                    const uint32_t f = persistent_first_tile(b, G, C);
                    CHECK(f < G, "C %u S %u: workgroup %u starts at %u", C, S, b, f);
                    if (f < G) seen[f] += 1;
                    if (S > 1 && b % C + 1 < C)  // unit r holds tiles r*S .. r*S + S - 1
                        CHECK(persistent_first_tile(b + 1, G, C) == f + S, "C %u S %u b %u", C, S, b);
                }
                for (uint32_t f = 0; f < G; ++f) CHECK(seen[f] == 1, "C %u S %u: tile %u", C, S, f);
                for (uint64_t T : {(uint64_t)G, (uint64_t)G + 1, (uint64_t)4 * G + G / 3 + 1, (uint64_t)17 * G - 1}) {
                    std::vector<int> cover(T, 0);
                    for (uint32_t b = 0; b < G; ++b)
                        for (uint64_t t = persistent_first_tile(b, G, C); t < T; t += G) cover[t] += 1;
                    for (uint64_t t = 0; t < T; ++t) CHECK(cover[t] == 1, "C %u S %u T %llu: tile %llu", C, S,
                                                           (unsigned long long)T, (unsigned long long)t);
                    walked += (long)T;
                }
            }
        }
        // Qwen2.5-1.5B 4K (7168 tiles) keeps workgroup order on 1536 = 6 x 256;
        // the 8192-page pool (229376 tiles) and longer take the unit-major order.
        CHECK(persistent_slot_cus(7168, 1536, 256, 1) == 0, "short launch mixed");
        CHECK(persistent_slot_cus(229376, 1536, 256, 1) == 256, "long launch not mixed");
        CHECK(persistent_slot_cus(7168, 1536, 256, 2) == 256, "mode 2");
        CHECK(persistent_slot_cus(229376, 1536, 256, 0) == 0, "mode 0");
        CHECK(persistent_slot_cus(229376, 1500, 256, 1) == 0, "grid not a multiple of the units");
        CHECK(persistent_slot_cus(229376, 256, 256, 1) == 0, "one workgroup per unit");
        std::printf("first-tile walks=%ld\n", walked);
    }

    std::printf("launches=%ld tiles=%ld mismatches=%ld\n", launches, tiles_checked, g_bad);
    return g_bad == 0 ? 0 : 1;
}
