// Static, cost-balanced partition of 32-row work items over a persistent grid (one workgroup per CU).
//
// A work item is one 32-row tile (of queries in the forward) of one (batch, head) sequence. Its cost is the number
// of 32-key tiles it streams, a function of the tile index alone (causal and radius windows; the key mask is data
// and is ignored here). Items are ranked heaviest first, rank-major and sequence-minor, and dealt to the
// workgroups in rounds of one item each, so that every workgroup's total is nearly the same:
//
//   * rounds are dealt in pairs, forward then backward ("snake"): for costs that fall linearly with the rank, the
//     two items of a pair always sum to the same cost;
//   * an odd number of rounds starts with three rounds whose positions sum to a constant (to within one) for
//     every workgroup: g, G + (g + G/2) mod G, and 2G + (G - 1 - 2g) or (2G - 2 - 2g) in the lower/upper half.
//
// When both the sequences and the workgroups divide by 8, the partition is done per XCD: workgroup g runs on XCD
// g mod 8 (round-robin dispatch) and only takes sequences s with s mod 8 == g mod 8, so the K/V rows each XCD streams
// stay in its own L2.
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

namespace rk {

struct Plan {
    int groups;  // 8 (one per XCD) or 1
    int bins;    // workgroups per group
    int seqs;    // sequences per group
    int tiles;   // 32-row tiles per sequence
    int rounds;  // items per workgroup, rounded up
    int reverse; // rank r is tile tiles-1-r (the last tiles are the heaviest, as under a causal mask)
};

struct PlanItem {
    int seq;  // (batch, head) sequence index, batch-major
    int tile; // 32-row tile within the sequence
};

// Position (in heaviest-first order, within the group) of the j-th item of bin lb; >= seqs * tiles when empty.
__host__ __device__ inline int plan_position(const Plan &p, const int lb, int j) {
    const int g = p.bins;
    int base = 0;
    if ((p.rounds & 1) && p.rounds >= 3 && (g & 1) == 0) {
        if (j == 0) return lb;
        if (j == 1) return g + (lb + g / 2) % g;
        if (j == 2) return 2 * g + (lb < g / 2 ? g - 1 - 2 * lb : 2 * g - 2 - 2 * lb);
        j -= 3;
        base = 3 * g;
    }
    return base + j * g + ((j & 1) ? g - 1 - lb : lb);
}

// Item at a position of group x; call only for positions < seqs * tiles.
__host__ __device__ inline PlanItem plan_item(const Plan &p, const int x, const int position) {
    const int rank = position / p.seqs;
    const int local = position - rank * p.seqs;
    return PlanItem{x + p.groups * local, p.reverse ? p.tiles - 1 - rank : rank};
}

// The SPLIT waves of an item take its tiles round-robin, and an item of c tiles leaves c mod split of them over.
// They are dealt round-robin over the subs across the bin: item i's tile j goes to sub (j + r) mod split, r = the
// rotation of slot i = the tiles of items 0 .. i-1. Wave `sub` of every slot runs on the same SIMD, so the SIMDs'
// tile counts then differ by at most one. cost(tile) = tiles streamed by the item of that 32-row tile.
template<class Cost>
inline int plan_rotation(const Plan &p, const int lb, const int slot, const Cost &cost) {
    int rotation = 0;
    for (int j = 0; j < slot; ++j) {
        const int position = plan_position(p, lb, j);
        if (position < p.seqs * p.tiles) rotation += cost(plan_item(p, 0, position).tile);
    }
    return rotation;
}

// Index (among its item's tiles) of the first tile taken by wave `sub` of an item whose slot has this rotation.
__host__ __device__ inline int plan_lead(const int rotation, const int sub, const int split) {
    return (sub + split - rotation % split) % split;
}

// ---- item table -------------------------------------------------------------------------------------------
// A persistent launch reads its items from a table passed by value in the kernel arguments: one scalar load per
// wave instead of the plan arithmetic above. The twelve waves of a CU share one scalar unit, and that arithmetic
// (integer divisions, the rotation loop) delayed the last waves' first loads by about 3 us at the 24 x 1024 causal
// shape. Entry g * ni + slot: batch in bits 0-9, head in 10-19, rank in 20-29, rotation mod 4 in 30-31.
constexpr int kMaxTableItems = 768; // 3 items on each of 256 CUs
constexpr int kItemFieldLimit = 1024;
constexpr uint32_t kNoItem = 0xffffffffu;

template<int NI>
struct ItemTable {
    uint32_t entry[NI > 0 ? kMaxTableItems : 1];
};

__host__ __device__ inline uint32_t pack_item(const int batch, const int head, const int rank, const int rotation) {
    return static_cast<uint32_t>(batch) | static_cast<uint32_t>(head) << 10 | static_cast<uint32_t>(rank) << 20 |
            static_cast<uint32_t>(rotation & 3) << 30;
}

// Fills entry[0 .. groups * bins * ni) for a plan of sequences with `heads` heads each; false (table untouched
// beyond what was written) when the launch does not fit the table.
template<class Cost>
inline bool fill_item_table(uint32_t *entry, const Plan &p, const int ni, const int heads, const Cost &cost) {
    const long long grid = static_cast<long long>(p.groups) * p.bins;
    const long long sequences = static_cast<long long>(p.groups) * p.seqs;
    if (grid * ni > kMaxTableItems || p.rounds > ni || p.tiles > kItemFieldLimit || heads > kItemFieldLimit ||
            sequences / heads > kItemFieldLimit)
        return false;
    for (int g = 0; g < grid; ++g) {
        const int x = g % p.groups, lb = g / p.groups;
        int rotation = 0;
        for (int slot = 0; slot < ni; ++slot) {
            const int position = plan_position(p, lb, slot);
            if (position >= p.seqs * p.tiles) {
                entry[g * ni + slot] = kNoItem;
                continue;
            }
            const PlanItem it = plan_item(p, x, position);
            const int rank = p.reverse ? p.tiles - 1 - it.tile : it.tile;
            entry[g * ni + slot] = pack_item(it.seq / heads, it.seq % heads, rank, rotation);
            rotation += cost(it.tile);
        }
    }
    return true;
}

// Plan for `seqs` sequences of `tiles` items each over at most `workgroups` workgroups (the CU count).
inline Plan make_plan(const long long seqs, const int tiles, const int workgroups, const bool reverse) {
    const long long items = seqs * tiles;
    const long long grid = items < workgroups ? items : workgroups;
    Plan p;
    p.groups = (seqs % 8 == 0 && grid % 8 == 0) ? 8 : 1;
    p.bins = static_cast<int>(grid / p.groups);
    p.seqs = static_cast<int>(seqs / p.groups);
    p.tiles = tiles;
    p.rounds = static_cast<int>((items / p.groups + p.bins - 1) / p.bins);
    p.reverse = reverse ? 1 : 0;
    return p;
}

} // namespace rk
