// Host-side check of the fused backward's key-block partition (rocmkernels_amd/csrc/attention_block_plan.hpp):
//   * every query tile of every key block is covered by exactly one piece, and no piece reaches past its block;
//   * a piece is marked partial exactly when its block is split, and the blocks that are split are exactly those
//     seeing more than plan.chunk query tiles (the pre-pass zeroes dK/dV of those blocks only);
//   * with 8 | sequences and 8 | workgroups, workgroup g only takes sequences s with s mod 8 == g mod 8;
//   * the busiest workgroup carries no more than the average plus one piece (all the shapes here fill every bin);
//   * block_query_tiles agrees with a brute-force scan of the causal/radius windows.
// Prints "0 failure(s)" on success.
#include <attention_block_plan.hpp>

#include <cstdint>
#include <cstdio>
#include <vector>

static int failures = 0;

#define CHECK(cond, ...)                     \
    do {                                     \
        if (!(cond)) {                       \
            std::printf("FAIL: " __VA_ARGS__); \
            std::printf("\n");               \
            ++failures;                      \
            return;                          \
        }                                    \
    } while (0)

// Brute force: query tiles [first, first + count) of the queries that see some key of block kb.
static int brute_query_tiles(const int queries, const int keys, const int radius, const int causal, const int kb, int &first) {
    int lo = -1, hi = -1;
    for (int key = kb * rk::kBlockKeys; key < keys && key < (kb + 1) * rk::kBlockKeys; ++key) {
        for (int q = 0; q < queries; ++q) {
            const bool in = (!causal || key <= q) && (radius < 0 || (q - key <= radius && key - q <= radius));
            if (!in) continue;
            if (lo < 0 || q < lo) lo = q;
            if (q > hi) hi = q;
        }
    }
    if (lo < 0) {
        first = 0;
        return 0;
    }
    first = lo / 32;
    return hi / 32 + 1 - first;
}

static void check_ranges(const int queries, const int keys, const int radius, const int causal) {
    for (int kb = 0; kb * rk::kBlockKeys < keys; ++kb) {
        int f0 = 0, f1 = 0;
        const int c0 = rk::block_query_tiles(queries, keys, radius, causal, kb, f0);
        const int c1 = brute_query_tiles(queries, keys, radius, causal, kb, f1);
        // Both must cover the visible queries; the closed form may start a tile earlier only when the range is empty.
        CHECK(c0 == c1 && (c0 == 0 || f0 == f1), "block_query_tiles(q=%d k=%d r=%d c=%d kb=%d) = (%d, %d), brute (%d, %d)", queries,
                keys, radius, causal, kb, f0, c0, f1, c1);
    }
}

static void check_plan(const long long seqs, const int queries, const int keys, const int radius, const int causal, const int cus) {
    const int nblocks = (keys + rk::kBlockKeys - 1) / rk::kBlockKeys;
    std::vector<int> cost(static_cast<size_t>(nblocks));
    for (int kb = 0; kb < nblocks; ++kb) {
        int first;
        cost[static_cast<size_t>(kb)] = rk::block_query_tiles(queries, keys, radius, causal, kb, first);
    }
    std::vector<uint32_t> table(rk::kMaxPieces, 0u);
    rk::BlockPlan plan;
    const bool ok = rk::plan_blocks(seqs, nblocks, cus, 3, [&](const int kb) { return cost[static_cast<size_t>(kb)]; }, plan, table.data());
    if (!ok) return; // the launch takes the dispatch-order grid; nothing to check here
    for (int g = 0; g < plan.bins * plan.slots; ++g) {
        const uint32_t e = table[static_cast<size_t>(g)];
        if (e == rk::kNoPiece) continue;
        const rk::Piece p = rk::unpack_piece(e);
        CHECK(rk::pack_piece(p.block, p.start, p.count, p.partial) == e && p.start <= rk::kMaxPieceStart &&
                        p.count <= rk::kMaxPieceTiles, "piece fields overflow (seqs=%lld L=%d)", seqs, keys);
    }
    CHECK(plan.bins * plan.slots <= rk::kMaxPieces, "table overflow");
    std::vector<std::vector<int>> hits(static_cast<size_t>(seqs * nblocks));
    std::vector<int> pieces(static_cast<size_t>(seqs * nblocks), 0);
    long long total = 0, busiest = 0;
    int npieces = 0;
    for (int g = 0; g < plan.bins; ++g) {
        long long load = 0;
        for (int j = 0; j < plan.slots; ++j) {
            const uint32_t e = table[static_cast<size_t>(g * plan.slots + j)];
            if (e == rk::kNoPiece) continue;
            const rk::Piece p = rk::unpack_piece(e);
            const int seq = p.block / nblocks, kb = p.block % nblocks;
            CHECK(seq < seqs, "piece of sequence %d", seq);
            if (seqs % 8 == 0 && plan.bins % 8 == 0) CHECK(seq % 8 == g % 8, "sequence %d on workgroup %d", seq, g);
            const int c = cost[static_cast<size_t>(kb)];
            CHECK(p.start + p.count <= c, "piece past its block: %d + %d > %d", p.start, p.count, c);
            std::vector<int> &h = hits[static_cast<size_t>(p.block)];
            if (h.empty()) h.assign(static_cast<size_t>(c), 0);
            for (int t = p.start; t < p.start + p.count; ++t) ++h[static_cast<size_t>(t)];
            ++pieces[static_cast<size_t>(p.block)];
            load += p.count + rk::kPieceOverhead;
            ++npieces;
        }
        total += load;
        if (load > busiest) busiest = load;
    }
    for (long long blk = 0; blk < seqs * nblocks; ++blk) {
        const int c = cost[static_cast<size_t>(blk % nblocks)];
        CHECK(pieces[static_cast<size_t>(blk)] >= 1, "block %lld has no piece", blk);
        for (int t = 0; t < c; ++t) CHECK(hits[static_cast<size_t>(blk)][static_cast<size_t>(t)] == 1, "block %lld tile %d covered %d times", blk, t,
                hits[static_cast<size_t>(blk)][static_cast<size_t>(t)]);
        const bool split = pieces[static_cast<size_t>(blk)] > 1;
        CHECK(split == (c > plan.chunk), "block %lld (cost %d, chunk %d) split=%d", blk, c, plan.chunk, split ? 1 : 0);
    }
    for (int g = 0; g < plan.bins * plan.slots; ++g) {
        const uint32_t e = table[static_cast<size_t>(g)];
        if (e == rk::kNoPiece) continue;
        const rk::Piece p = rk::unpack_piece(e);
        CHECK(p.partial == (pieces[static_cast<size_t>(p.block)] > 1), "partial flag of block %d", p.block);
    }
    // Longest-first dealing keeps every workgroup within one piece of the average (the largest piece plus overhead).
    const double average = static_cast<double>(total) / plan.bins;
    CHECK(busiest <= average + plan.chunk + rk::kPieceOverhead + 1e-9, "seqs=%lld L=%d: busiest %lld, average %.2f, chunk %d", seqs, keys,
            busiest, average, plan.chunk);
    (void)npieces;
}

int main() {
    const int shapes[][4] = {{1024, 1024, -1, 1}, {2048, 2048, -1, 1}, {8192, 8192, 256, 1}, {700, 700, 40, 1}, {40, 200, 5, 0},
            {90, 50, 11, 1}, {1536, 1536, -1, 1}, {512, 512, 100, 0}, {1, 70, -1, 0}, {33, 33, 0, 0}, {130, 130, 17, 1},
            // Long rows: piece starts pass 255 query tiles, the width of the table's start field, so the plan must
            // either keep every start in range or be rejected (then the launch takes the dispatch-order grid).
            {10240, 10240, -1, 1}, {9000, 128, -1, 0}, {12288, 12288, -1, 1}};
    for (const auto &s : shapes) check_ranges(s[0], s[1], s[2], s[3]);
    const long long seqs[] = {1, 3, 8, 10, 16, 20, 24, 32, 48, 64};
    for (const auto &s : shapes) {
        for (const long long n : seqs) {
            check_plan(n, s[0], s[1], s[2], s[3], 256);
            check_plan(n, s[0], s[1], s[2], s[3], 80);
        }
    }
    std::printf("%d failure(s)\n", failures);
    return failures == 0 ? 0 : 1;
}
