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
