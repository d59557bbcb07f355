// Host-side check of the persistent-grid work partition (rocmkernels_amd/csrc/attention_plan.hpp): every item of
// every sequence is dealt to exactly one (workgroup, round) slot, and for causal item costs (tile t streams t + 1 key
// tiles) the busiest workgroup carries no more than the average plus one item (any whole-item partition can do no
// better when the last round is partial) and, when every round is full, at most a few percent more than the average;
// the packed item table a launch reads holds every item once, and within a bin the four waves of each item (one per
// SIMD) end up with tile totals that differ by at most one.
// Prints "0 failure(s)" on success.
#include <attention_plan.hpp>

#include <cstdint>
#include <cstdio>
#include <vector>

static int failures = 0;

static void check(const long long seqs, const int tiles, const int cus, const bool causal, const double max_ratio) {
    const rk::Plan p = rk::make_plan(seqs, tiles, cus, causal);
    const int per_group = p.seqs * p.tiles;
    std::vector<int> hits(static_cast<size_t>(seqs) * tiles, 0);
    std::vector<long long> load(static_cast<size_t>(p.groups) * p.bins, 0);
    for (int g = 0; g < p.groups * p.bins; ++g) {
        const int x = g % p.groups, lb = g / p.groups;
        for (int j = 0; j < p.rounds; ++j) {
            const int pos = rk::plan_position(p, lb, j);
            if (pos >= per_group) continue;
            const rk::PlanItem it = rk::plan_item(p, x, pos);
            if (it.seq < 0 || it.seq >= seqs || it.tile < 0 || it.tile >= tiles || it.seq % p.groups != x) {
                std::printf("FAIL seqs=%lld tiles=%d: bad item (%d, %d)\n", seqs, tiles, it.seq, it.tile);
                ++failures;
                return;
            }
            ++hits[static_cast<size_t>(it.seq) * tiles + it.tile];
            load[g] += causal ? it.tile + 1 : 1;
        }
    }
    for (const int h : hits) {
        if (h != 1) {
            std::printf("FAIL seqs=%lld tiles=%d: an item is dealt %d times\n", seqs, tiles, h);
            ++failures;
            return;
        }
    }
    // The item table a launch reads (fill_item_table) holds the same items, and within each bin the SPLIT = 4 waves
    // of every item take its tiles from plan_lead: the per-sub totals (one SIMD each) differ by at most one tile.
    const auto cost = [&](const int tile) { return causal ? tile + 1 : 1; };
    const int heads = seqs % 3 == 0 ? 3 : 1;
    std::vector<uint32_t> table(rk::kMaxTableItems, 0u);
    const bool filled = rk::fill_item_table(table.data(), p, p.rounds, heads, cost);
    const bool fits = static_cast<long long>(p.groups) * p.bins * p.rounds <= rk::kMaxTableItems;
    if (filled != fits) {
        std::printf("FAIL seqs=%lld tiles=%d: table filled=%d, expected %d\n", seqs, tiles, filled ? 1 : 0, fits ? 1 : 0);
        ++failures;
        return;
    }
    if (filled) {
        std::vector<int> seen(static_cast<size_t>(seqs) * tiles, 0);
        for (int g = 0; g < p.groups * p.bins; ++g) {
            long long sub_tiles[4] = {0, 0, 0, 0};
            for (int j = 0; j < p.rounds; ++j) {
                const uint32_t e = table[static_cast<size_t>(g) * p.rounds + j];
                if (e == rk::kNoItem) continue;
                const int b = static_cast<int>(e & 1023u), head = static_cast<int>((e >> 10) & 1023u);
                const int rank = static_cast<int>((e >> 20) & 1023u), rotation = static_cast<int>(e >> 30);
                const int seq = b * heads + head;
                const int tile = causal ? tiles - 1 - rank : rank;
                if (head >= heads || seq >= seqs || rank >= tiles || seq % p.groups != g % p.groups) {
                    std::printf("FAIL seqs=%lld tiles=%d: bad table entry %08x\n", seqs, tiles, e);
                    ++failures;
                    return;
                }
                ++seen[static_cast<size_t>(seq) * tiles + tile];
                const int c = cost(tile);
                for (int sub = 0; sub < 4; ++sub) {
                    const int lead = rk::plan_lead(rotation, sub, 4);
                    sub_tiles[sub] += c > lead ? (c - lead + 3) / 4 : 0;
                }
            }
            long long lo = sub_tiles[0], hi = sub_tiles[0], sum = 0;
            for (const long long t : sub_tiles) {
                lo = t < lo ? t : lo;
                hi = t > hi ? t : hi;
                sum += t;
            }
            if (hi - lo > 1 || sum != load[g]) {
                std::printf("FAIL seqs=%lld tiles=%d: bin %d sub tiles %lld..%lld (sum %lld, bin load %lld)\n", seqs, tiles, g, lo,
                        hi, sum, load[g]);
                ++failures;
                return;
            }
        }
        for (const int h : seen) {
            if (h != 1) {
                std::printf("FAIL seqs=%lld tiles=%d: the table holds an item %d times\n", seqs, tiles, h);
                ++failures;
                return;
            }
        }
    }
    long long total = 0, most = 0;
    for (const long long l : load) {
        total += l;
        most = l > most ? l : most;
    }
    const double ratio = static_cast<double>(most) * load.size() / total;
    const double bound = static_cast<double>(total) / load.size() + (causal ? tiles : 1);
    if (most > bound) {
        std::printf("FAIL seqs=%lld tiles=%d: busiest bin %lld above average plus one item %.1f\n", seqs, tiles, most, bound);
        ++failures;
    }
    std::printf("seqs=%lld tiles=%d cus=%d causal=%d: groups=%d bins=%d rounds=%d max/avg=%.3f\n", seqs, tiles, cus, causal ? 1 : 0,
            p.groups, p.bins, p.rounds, ratio);
    if (ratio > max_ratio) {
        std::printf("FAIL seqs=%lld tiles=%d: max/avg %.3f > %.3f\n", seqs, tiles, ratio, max_ratio);
        ++failures;
    }
}

int main() {
    check(24, 32, 256, true, 1.02);   // the 24 x 1024 causal forward: three items per CU
    check(24, 16, 256, true, 1.30);   // 1.5 items per CU: a partial second round
    check(48, 32, 256, true, 1.02);   // six rounds: three snake pairs
    check(384, 32, 256, true, 1.01);
    check(32, 64, 256, true, 1.01);
    check(5, 7, 256, false, 1.0);     // fewer items than CUs, sequences not a multiple of 8
    check(3, 100, 256, true, 2.0);    // a partial last round: bounded by the largest single item
    check(7, 33, 96, true, 1.20);     // partial third round
    check(1, 1, 256, false, 1.0);
    std::printf("%d failure(s)\n", failures);
    return failures == 0 ? 0 : 1;
}
