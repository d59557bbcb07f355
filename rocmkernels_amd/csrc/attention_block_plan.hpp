// Work partition of the fused backward (attention_backward_fused.hip) over a persistent grid.
//
// The fused backward's work item is a key block: 128 consecutive keys (four 32-key tiles, one per wave of the
// workgroup) of one (batch, head) sequence, streamed over the query tiles that can see any of its keys. A block's
// cost is that number of query tiles (a function of the block index alone: causal and radius windows; the key mask is
// data and is ignored). Under a causal mask the costs fall linearly with the block index, and at the 24 x 1024 shape
// there are fewer blocks (192) than CUs (256), so whole blocks cannot balance the chip. The plan therefore cuts the
// blocks that cost more than the average workgroup load into pieces (contiguous query-tile ranges) of that load and
// deals all pieces to the workgroups longest first, each to the least-loaded workgroup that still has a free slot.
// A piece that covers only part of its block adds its dK/dV into memory zeroed beforehand; a whole block stores them.
//
// With both the sequences and the workgroups divisible by 8 the partition is done per XCD: workgroup g runs on XCD
// g mod 8 and only takes pieces of sequences s with s mod 8 == g mod 8, so each XCD streams its sequences from its own
// L2. Everything here is host code plus the block-range helper the kernel shares.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace rk {

constexpr int kBlockTiles = 4;  // 32-key tiles per key block: one per wave of a query stream
constexpr int kBlockKeys = 128; // keys per key block

// Query tiles [first_tile, first_tile + count) hold every query that sees some key of block kb through the causal and
// radius windows; returns count (0 when no query sees the block).
__host__ __device__ inline int block_query_tiles(const int queries, const int keys, const int radius, const int causal,
        const int kb, int &first_tile) {
    const int k0 = kb * kBlockKeys;
    const int k1 = (k0 + kBlockKeys < keys ? k0 + kBlockKeys : keys) - 1; // last key of the block
    int first = causal ? k0 : 0;
    int last = queries;
    if (radius >= 0) {
        first = k0 - radius > first ? k0 - radius : first;
        last = k1 + radius + 1 < last ? k1 + radius + 1 : last;
    }
    first = first > 0 ? first : 0;
    first_tile = first / 32;
    return last > first ? (last + 31) / 32 - first_tile : 0;
}

// ---- band walk (attention_backward_band.hip) ------------------------------------------------------------------
// Under a radius window each 32-key tile sees a band of query tiles, one tile later for each key tile. The band kernel
// walks a key block skewed: at step i the wave of key tile x works on query tile base + i + x, so each wave meets the
// tiles of its own band in order and no two waves share a tile within a step.

// Queries [first, last) that can see some key of 32-key tile kt through the causal and radius windows (the keys'
// padding mask aside); returns the number of 32-query tiles they span.
__host__ __device__ inline int key_tile_queries(const int queries, const int radius, const int causal, const int kt, int &first,
        int &last) {
    const int key0 = kt * 32;
    first = causal ? key0 : 0;
    last = queries;
    if (radius >= 0) {
        first = key0 - radius > first ? key0 - radius : first;
        last = key0 + 32 + radius < last ? key0 + 32 + radius : last;
    }
    first = first > 0 ? first : 0;
    return last > first ? (last - first + 31) / 32 : 0;
}

// Band of 32-key tile kt in whole query tiles [first, end): empty (first == end == 0) when the tile starts past the
// sequence's last key or no query sees it.
__host__ __device__ inline void key_tile_band(const int queries, const int keys, const int radius, const int causal, const int kt,
        int &first, int &end) {
    int q0 = 0, q1 = 0;
    if (kt * 32 < keys && key_tile_queries(queries, radius, causal, kt, q0, q1) > 0) {
        first = q0 / 32;
        end = (q1 + 31) / 32;
    } else {
        first = end = 0;
    }
}

struct BandWalk {
    int base = 0x7fffffff;      // query tile of the block's first key tile at step 0
    int nsteps = 0;             // steps of the walk (0: no query sees the block)
    int lo = 0x7fffffff;        // query tiles [lo, hi) of the union of the four bands
    int hi = -0x7fffffff;
};

// The walk of key block kb: base = min over the block's key tiles x of (band start - x), so that at step 0 no wave is
// past its band's start, and nsteps reaches the latest (band end - x).
__host__ __device__ inline BandWalk band_walk(const int queries, const int keys, const int radius, const int causal,
        const int kb) {
    BandWalk b;
    int stop = -0x7fffffff;
    for (int x = 0; x < kBlockTiles; ++x) {
        int f = 0, e = 0;
        key_tile_band(queries, keys, radius, causal, kb * kBlockTiles + x, f, e);
        if (e <= f) continue;
        b.base = b.base < f - x ? b.base : f - x;
        stop = stop > e - x ? stop : e - x;
        b.lo = b.lo < f ? b.lo : f;
        b.hi = b.hi > e ? b.hi : e;
    }
    b.nsteps = stop > b.base ? stop - b.base : 0;
    return b;
}

// ---- piece table ---------------------------------------------------------------------------------------------
// Entry g * slots + j of the table (passed by value in the kernel arguments) is the j-th piece of workgroup g:
// block index (sequence * blocks per sequence + kb) in bits 0-15, first query tile of the piece relative to the
// block's first query tile in bits 16-23, tile count in bits 24-30, and bit 31 set when the piece is part of a split
// block (its dK/dV are added, not stored). kNoPiece ends a workgroup's list.
constexpr int kMaxPieces = 768;
constexpr uint32_t kNoPiece = 0xffffffffu;
constexpr int kMaxPieceBlocks = 1 << 16;
constexpr int kMaxPieceStart = 255;
constexpr int kMaxPieceTiles = 127;

struct PieceTable {
    uint32_t entry[kMaxPieces];
};

struct Piece {
    int block, start, count;
    bool partial;
};

__host__ __device__ inline uint32_t pack_piece(const int block, const int start, const int count, const bool partial) {
    return static_cast<uint32_t>(block) | static_cast<uint32_t>(start) << 16 | static_cast<uint32_t>(count) << 24 |
            (partial ? 0x80000000u : 0u);
}

__host__ __device__ inline Piece unpack_piece(const uint32_t e) {
    return Piece{static_cast<int>(e & 0xffffu), static_cast<int>((e >> 16) & 0xffu), static_cast<int>((e >> 24) & 0x7fu),
            (e >> 31) != 0};
}

struct BlockPlan {
    int bins = 0;         // workgroups of the launch
    int slots = 0;        // table entries per workgroup
    int chunk = 0;        // piece length: exactly the blocks that see more query tiles are split
    bool partial = false; // some block is split (its dK/dV are accumulated with atomics)
    long long max_load = 0, total = 0; // busiest workgroup and all workgroups, in query-tile steps plus piece overheads
};

// Cost of a piece in the plan: its query tiles plus a fixed per-piece overhead (loading the block's K/V rows, the first
// tile's round trip, the dK/dV write), in tile steps.
constexpr int kPieceOverhead = 1;

// Partitions `seqs` sequences of `nblocks` key blocks (cost(kb) query tiles each) over at most `workgroups`
// workgroups, at most `max_slots` pieces per workgroup. Fills entry[0 .. bins * slots) and returns true; returns false
// (plan unusable: the launch then takes one workgroup per whole block) when the table or the entry fields are too
// small for the shape.
template<class Cost>
inline bool plan_blocks(const long long seqs, const int nblocks, const int workgroups, const int max_slots, const Cost &cost,
        BlockPlan &plan, uint32_t *entry) {
    plan = BlockPlan{};
    if (seqs <= 0 || nblocks <= 0 || workgroups <= 0 || seqs * nblocks > kMaxPieceBlocks) return false;
    std::vector<int> costs(static_cast<size_t>(nblocks));
    long long per_seq = 0;
    for (int kb = 0; kb < nblocks; ++kb) {
        costs[static_cast<size_t>(kb)] = cost(kb);
        per_seq += costs[static_cast<size_t>(kb)];
    }
    const int groups = (seqs % 8 == 0 && workgroups % 8 == 0) ? 8 : 1;
    const int bins = workgroups / groups; // per group
    const long long group_seqs = seqs / groups;
    const long long target = std::max<long long>(1, (group_seqs * per_seq + bins - 1) / bins);
    const int chunk = static_cast<int>(std::min<long long>(target, kMaxPieceTiles));
    plan.chunk = chunk;

    struct Item {
        int block, start, count;
        bool partial;
    };
    std::vector<Item> items;
    std::vector<std::vector<uint32_t>> lists(static_cast<size_t>(bins) * groups);
    std::vector<long long> load(static_cast<size_t>(bins));
    int slots = 1;
    for (int x = 0; x < groups; ++x) {
        items.clear();
        for (long long sl = 0; sl < group_seqs; ++sl) {
            const long long seq = x + groups * sl;
            for (int kb = 0; kb < nblocks; ++kb) {
                const int c = costs[static_cast<size_t>(kb)];
                const int block = static_cast<int>(seq * nblocks + kb);
                // A block that costs more than a workgroup's share is cut into pieces of exactly that share plus the
                // remainder; the remainders and the whole small blocks then fill the other workgroups. (Cutting it
                // into near-equal pieces instead leaves pieces that pair up badly: 74% of the ideal balance at the
                // 24 x 1024 causal shape against 93% here.)
                if (c <= chunk) {
                    items.push_back(Item{block, 0, c, false});
                    continue;
                }
                for (int a = 0; a < c; a += chunk) {
                    if (a > kMaxPieceStart) return false; // the start field holds 8 bits: take the dispatch-order grid
                    items.push_back(Item{block, a, std::min(chunk, c - a), true});
                }
            }
        }
        // Longest first; ties by block so the plan does not depend on the sort's stability.
        std::sort(items.begin(), items.end(), [](const Item &a, const Item &b) {
            return a.count != b.count ? a.count > b.count : (a.block != b.block ? a.block < b.block : a.start < b.start);
        });
        std::fill(load.begin(), load.end(), 0);
        for (const Item &it : items) {
            int best = -1;
            for (int lb = 0; lb < bins; ++lb) {
                const size_t g = static_cast<size_t>(lb) * groups + x;
                if (static_cast<int>(lists[g].size()) >= max_slots) continue;
                if (best < 0 || load[static_cast<size_t>(lb)] < load[static_cast<size_t>(best)]) best = lb;
            }
            if (best < 0) return false; // more pieces than slots
            const size_t g = static_cast<size_t>(best) * groups + x;
            lists[g].push_back(pack_piece(it.block, it.start, it.count, it.partial));
            load[static_cast<size_t>(best)] += it.count + kPieceOverhead;
            slots = std::max(slots, static_cast<int>(lists[g].size()));
            plan.partial = plan.partial || it.partial;
            plan.total += it.count + kPieceOverhead;
        }
        for (int lb = 0; lb < bins; ++lb) plan.max_load = std::max(plan.max_load, load[static_cast<size_t>(lb)]);
    }
    plan.bins = bins * groups;
    plan.slots = slots;
    if (static_cast<long long>(plan.bins) * slots > kMaxPieces) return false;
    for (int g = 0; g < plan.bins; ++g) {
        const std::vector<uint32_t> &l = lists[static_cast<size_t>(g)];
        for (int j = 0; j < slots; ++j) entry[g * slots + j] = j < static_cast<int>(l.size()) ? l[static_cast<size_t>(j)] : kNoPiece;
    }
    return true;
}

} // namespace rk
