// Device-side building blocks shared by the gfx950 FP32 attention kernels.
//
// Every contraction (Q·Kᵀ, P·V, dO·Vᵀ, Pᵀ·dO, dSᵀ·Q, dS·K) runs on v_mfma_f32_32x32x2f32. A wave owns one
// 32x32 tile of the score matrix at a time. The operand layouts are chosen so that the accumulator of one
// product is already the B operand of the next one, with no cross-lane transpose:
//
//   * A 32x32x2 MFMA takes A[m][k] from lane m + 32k and B[k][n] from lane n + 32k, and leaves D[i][n] in
//     lane n + 32h, accumulator register v, where i = 8*(v/4) + 4h + v%4 (tile_row below).
//   * For the reductions over features the k index is free: MFMA c pairs feature c (lanes 0..31) with
//     feature D/2 + c (lanes 32..63), so every lane holds D/2 contiguous features of one row and loads them
//     with 128-bit loads ("row layout").
//   * For the reductions over tile rows (keys in P·V, queries in Pᵀ·dO) MFMA j pairs tile row tile_row(j, 0)
//     with tile_row(j, 1); accumulator register j of the previous product then sits exactly where the B
//     operand of MFMA j is expected. The A operand of such a product is one 32-float row of the other tensor
//     per half-wave ("column layout": lane reads element [tile_row(j, h)][32t + lane%32]).
#pragma once

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "attention_block_plan.hpp"
#include "attention_plan.hpp"

namespace rk {

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;                 // CDNA wavefront width
constexpr int kTile = 32;                 // rows of one MFMA score tile (queries or keys)
constexpr int kWaves = 4;                 // waves per workgroup: one per SIMD, splitting the streamed dimension
constexpr int kThreads = kWave * kWaves;
constexpr float kLog2e = 1.4426950408889634f;

// Strided FP32 tensor [batch][head][token][D] with contiguous features (reference Attention.hip:14-20).
struct Tensor {
    const float *data;
    int sb, sh, st;
};

struct Shape {
    int batch, heads, queries, keys, radius, causal;
};

// Tile row held by accumulator register v of a lane in half h of the wave.
__device__ __forceinline__ constexpr int tile_row(const int v, const int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

__device__ __forceinline__ f32x16 mfma(const float a, const float b, const f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float exp2_fast(const float x) { return __builtin_amdgcn_exp2f(x); }

// Combine x with the value held by the lane 32 positions away (the other half of the wave) using
// v_permlane32_swap, a VALU op: no LDS round trip as with ds_bpermute.
__device__ __forceinline__ float halves_max(const float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float halves_sum(const float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// δ = Σ dO·O of a row is summed in one fixed order by every kernel that forms it, so all backward paths write the
// same bits: each 4-feature group is a product followed by an FMA chain (group_dot), and the groups are added as a
// pairwise tree (groups 2i and 2i + 1, then adjacent pairs, and so on up to the two half rows).
__device__ __forceinline__ float group_dot(const float *x, const float *y) {
    float p = x[0] * y[0];
    p = fmaf(x[1], y[1], p);
    p = fmaf(x[2], y[2], p);
    return fmaf(x[3], y[3], p);
}

// The tree over N consecutive groups held by one lane (N a power of two).
template<int N>
__device__ __forceinline__ float group_tree(float (&p)[N]) {
#pragma unroll
    for (int m = 1; m < N; m <<= 1) {
#pragma unroll
        for (int i = 0; i < N; i += 2 * m) p[i] += p[i + m];
    }
    return p[0];
}

// Bits lo..hi (inclusive, clamped to 0..31) set; 0 when the range is empty.
__device__ __forceinline__ uint32_t bit_range(const int lo, const int hi) {
    const int a = min(max(lo, 0), 32);
    const int b = min(max(hi + 1, 0), 32);
    return static_cast<uint32_t>(((1ull << b) - 1ull) & (~0ull << a));
}

__device__ __forceinline__ const float *sequence(const Tensor &t, const int b, const int head) {
    return t.data + (static_cast<int64_t>(b) * t.sb + static_cast<int64_t>(head) * t.sh);
}

// ---- buffer loads -----------------------------------------------------------------------------------------
// Streamed tensors are read through buffer resources (one per sequence, in SGPRs): offsets are 32-bit, a
// per-row SGPR offset replaces per-lane 64-bit address arithmetic, and the hardware range check returns 0 for
// any access at or beyond `bytes`, so rows past the end of a sequence need no clamping and cannot fault.
typedef __amdgpu_buffer_rsrc_t Buffer;
constexpr uint32_t kNoRow = 0x80000000u; // voffset beyond any sequence extent (host guarantees < 2 GiB): reads 0
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferWord3 = 0x00020000; // gfx9-family descriptor word 3: raw dword access

__device__ __forceinline__ Buffer make_buffer(const void *base, const uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), static_cast<short>(0), static_cast<int>(bytes), kBufferWord3);
}

// Byte extent of one sequence of a strided tensor: rows 0..rows-1 of `width` floats at `stride` floats.
__device__ __forceinline__ uint32_t sequence_bytes(const int rows, const int stride, const int width) {
    return static_cast<uint32_t>((static_cast<int64_t>(rows - 1) * stride + width) * 4);
}

__device__ __forceinline__ float buffer_load(const Buffer r, const uint32_t voffset, const uint32_t soffset) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(voffset), static_cast<int>(soffset), 0));
}

__device__ __forceinline__ f32x4 buffer_load4(const Buffer r, const uint32_t voffset, const uint32_t soffset) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voffset), static_cast<int>(soffset), 0));
}

__device__ __forceinline__ int buffer_load_byte(const Buffer r, const uint32_t voffset) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, static_cast<int>(voffset), 0, 0);
}

// The byte at voffset + soffset (soffset scalar).
__device__ __forceinline__ int buffer_load_byte_s(const Buffer r, const uint32_t voffset, const uint32_t soffset) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, static_cast<int>(voffset), static_cast<int>(soffset), 0);
}

// N contiguous floats at byte offset voffset (16-byte aligned when VEC).
template<bool VEC, int N>
__device__ __forceinline__ void buffer_load_span(float (&r)[N], const Buffer b, const uint32_t voffset) {
    static_assert(N % 4 == 0);
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const f32x4 x = buffer_load4(b, voffset + 16 * i, 0);
            r[4 * i + 0] = x[0];
            r[4 * i + 1] = x[1];
            r[4 * i + 2] = x[2];
            r[4 * i + 3] = x[3];
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) r[i] = buffer_load(b, voffset + 4 * i, 0);
    }
}

// N contiguous floats starting at p, or zeros when !ok. VEC uses 128-bit loads (p must be 16-byte aligned).
template<bool VEC, int N>
__device__ __forceinline__ void load_span(float (&r)[N], const float *p, const bool ok) {
    static_assert(N % 4 == 0);
    if (ok) {
        if constexpr (VEC) {
#pragma unroll
            for (int i = 0; i < N / 4; ++i) {
                const f32x4 x = *reinterpret_cast<const f32x4 *>(p + 4 * i);
                r[4 * i + 0] = x[0];
                r[4 * i + 1] = x[1];
                r[4 * i + 2] = x[2];
                r[4 * i + 3] = x[3];
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) r[i] = p[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) r[i] = 0.0f;
    }
}

// Stores accumulator tile acc (rows tile_row(v, h) of a 32-feature slice) as 4 groups of 4 contiguous floats; with
// ROWS = 16 (16-wide heads) only the groups holding features 0..15 (u = 0, 1).
template<bool VEC, int ROWS = 32>
__device__ __forceinline__ void store_tile_row(float *p, const f32x16 &acc, const float factor, const int h) {
    static_assert(ROWS == 16 || ROWS == 32);
#pragma unroll
    for (int u = 0; u < ROWS / 8; ++u) {
        float *dst = p + 8 * u + 4 * h;
        const f32x4 x = {acc[4 * u] * factor, acc[4 * u + 1] * factor, acc[4 * u + 2] * factor, acc[4 * u + 3] * factor};
        if constexpr (VEC) {
            *reinterpret_cast<f32x4 *>(dst) = x;
        } else {
            dst[0] = x[0];
            dst[1] = x[1];
            dst[2] = x[2];
            dst[3] = x[3];
        }
    }
}

// Orders this wave's LDS writes before its later LDS reads (and reads before later writes) without a
// workgroup barrier: the waves of a workgroup run different trip counts, so a __syncthreads inside the
// streaming loops would not be reached by all of them.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- coalesced row tiles -----------------------------------------------------------------------------------
// Row-layout operands (a lane holds D/2 contiguous features of one row) read straight from memory need 128-bit
// loads that each touch 32 different 128-byte lines. When every wave of the chip asks for its first tiles at once,
// those scattered requests queue up: the last waves of a CU received their first tile 3.4 us after launch against
// 1.6 us for loads that cover whole lines (12 waves per CU, 12 KiB each). So a 32-row tile is read with loads that
// cover whole lines (load i, lane L: 16-byte chunk i*64 + L of the tile in row-major order), written to the wave's
// LDS slot and read back in row layout (or, for products that reduce over the tile's rows, in column layout). Slot
// rows are D + 4 floats apart: the row-layout reads (lane%32 = row, 16 bytes each) and the column-layout reads (a
// half-wave reads 32 consecutive floats of one row) then meet no bank conflict over 32 banks, and every address is
// one per-lane base plus a constant.
template<int D>
constexpr int kSlotStride = D + 4;
template<int D>
constexpr int kSlotFloats = kTile * kSlotStride<D>;

template<int D>
struct RowTile {
    f32x4 x[D / 8]; // the tile's 32 * D floats, 16 bytes per lane per load
};

// Issues the loads of the 32 rows that start at byte offset row0 of b, rows `step` bytes apart (rows at or beyond
// the buffer's extent read 0: the range check covers voffset + soffset).
template<int D>
__device__ __forceinline__ void load_row_tile(RowTile<D> &t, const Buffer b, const uint32_t step, const uint32_t row0) {
    constexpr int CPR = D / 4;        // chunks per row
    constexpr int RPL = kWave / CPR;  // rows per load
    const int lane = threadIdx.x & (kWave - 1);
    const uint32_t voffset = static_cast<uint32_t>(lane / CPR) * step + 16u * static_cast<uint32_t>(lane % CPR);
#pragma unroll
    for (int i = 0; i < D / 8; ++i) t.x[i] = buffer_load4(b, voffset, row0 + static_cast<uint32_t>(i * RPL) * step);
}

// Writes a loaded tile to the wave's LDS slot (kSlotFloats<D> floats, 16-byte aligned), after the slot's previous
// reads.
template<int D>
__device__ __forceinline__ void write_row_tile(float *slot, const RowTile<D> &t) {
    constexpr int CPR = D / 4;
    constexpr int RPL = kWave / CPR;
    const int lane = threadIdx.x & (kWave - 1);
    float *base = slot + (lane / CPR) * kSlotStride<D> + 4 * (lane % CPR);
    wave_lds_sync(); // the previous tile's reads come first
#pragma unroll
    for (int i = 0; i < D / 8; ++i) *reinterpret_cast<f32x4 *>(base + i * RPL * kSlotStride<D>) = t.x[i];
}

// Row layout from a written slot: lane (col, h) receives features h*D/2 .. h*D/2 + D/2 - 1 of row col. Call
// wave_lds_sync() between the write and the first read.
template<int D>
__device__ __forceinline__ void read_row_layout(const float *slot, float (&r)[D / 2]) {
    const int lane = threadIdx.x & (kWave - 1);
    const float *base = slot + (lane & 31) * kSlotStride<D> + (lane >> 5) * (D / 2);
#pragma unroll
    for (int k = 0; k < D / 8; ++k) {
        const f32x4 x = *reinterpret_cast<const f32x4 *>(base + 4 * k);
        r[4 * k + 0] = x[0];
        r[4 * k + 1] = x[1];
        r[4 * k + 2] = x[2];
        r[4 * k + 3] = x[3];
    }
}

// Column layout from a written slot: element [tile_row(j, h)][32t + col] to c[t][j - J0] for j = J0 .. J0 + J - 1 (the
// A operands of MFMAs j of a product that reduces over the slot's rows).
template<int D, int J0 = 0, int J = 16>
__device__ __forceinline__ void read_column_layout(const float *slot, float (&c)[D / 32][J]) {
    const int lane = threadIdx.x & (kWave - 1);
    const float *base = slot + 4 * (lane >> 5) * kSlotStride<D> + (lane & 31);
#pragma unroll
    for (int j = J0; j < J0 + J; ++j) {
#pragma unroll
        for (int t = 0; t < D / 32; ++t) c[t][j - J0] = base[(8 * (j >> 2) + (j & 3)) * kSlotStride<D> + 32 * t];
    }
}

// Passes a loaded tile through the wave's LDS slot into row layout (write_row_tile, then read_row_layout).
template<int D>
__device__ __forceinline__ void stage_row_tile(float *slot, const RowTile<D> &t, float (&r)[D / 2]) {
    write_row_tile<D>(slot, t);
    wave_lds_sync();
    read_row_layout<D>(slot, r);
}

// Keys [first, last) cover every key the 32 queries of query tile qt can see through the causal and radius windows;
// returns the number of 32-key tiles they span (the work of one forward or dQ item).
__host__ __device__ inline int forward_key_range(const Shape &s, const int qt, int &first, int &last) {
    const int q0 = qt * kTile;
    first = 0;
    last = s.keys;
    if (s.radius >= 0) {
        first = q0 - s.radius > 0 ? q0 - s.radius : 0;
        last = q0 + kTile + s.radius < last ? q0 + kTile + s.radius : last;
    }
    if (s.causal && q0 + kTile < last) last = q0 + kTile;
    return last > first ? (last - first + kTile - 1) / kTile : 0;
}

// Queries [first, last) that can see some key of key tile kt through the causal and radius windows; returns the
// number of 32-query tiles they span (the work of one dK/dV item when any of its keys is unmasked).
__host__ __device__ inline int dkdv_query_range(const Shape &s, const int kt, int &first, int &last) {
    return key_tile_queries(s.queries, s.radius, s.causal, kt, first, last);
}

__host__ __device__ inline int forward_item_tiles(const Shape &s, const int qt) {
    int first, last;
    return forward_key_range(s, qt, first, last);
}

// Keys visible to `query` through the causal and radius windows form one interval [lo, hi].
__device__ __forceinline__ int window_lo(const Shape &s, const int query) { return s.radius >= 0 ? query - s.radius : -0x40000000; }
__device__ __forceinline__ int window_hi(const Shape &s, const int query) {
    int hi = s.causal ? query : 0x40000000;
    if (s.radius >= 0) hi = min(hi, query + s.radius);
    return hi;
}

// Queries that see `key` through the causal and radius windows form one interval [lo, hi].
__device__ __forceinline__ int window_query_lo(const Shape &s, const int key) {
    int lo = s.causal ? key : -0x40000000;
    if (s.radius >= 0) lo = max(lo, key - s.radius);
    return lo;
}
__device__ __forceinline__ int window_query_hi(const Shape &s, const int key) { return s.radius >= 0 ? key + s.radius : 0x40000000; }

// ---- work mapping ------------------------------------------------------------------------------------------
// A work item is one 32-row tile (of queries in the forward and dQ kernels, of keys in the dK/dV kernel) of one
// (batch, head) sequence. SPLIT waves of a workgroup share an item and split its streamed tiles round-robin;
// the workgroup's 4 waves therefore cover 4 / SPLIT items. Items are numbered rank-major (rank = position of the
// tile in the order the caller wants them dispatched, heaviest first), sequence-minor, so with B*H a multiple of
// 8 consecutive workgroups of one rank spread over the 8 XCDs while each XCD keeps a fixed subset of sequences.
struct WorkItem {
    int seq, b, head, rank, sub;
    int split; // waves sharing the item
    int lead;  // index of this wave's first tile among the item's tiles; it then takes every split-th tile
    bool valid;
};

//
// When the sequences and the grid split evenly over the 8 XCDs (workgroup g runs on XCD g mod 8), XCD x takes the
// sequences x, x + 8, ... only, still rank-major within them: every XCD then streams the K/V (or Q/dO) rows of a quarter
// or less of the sequences from its own L2, instead of every sequence at every other rank.
template<int SPLIT>
__device__ __forceinline__ WorkItem work_item(const Shape &s, const int tiles_per_seq) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform: keeps tile bookkeeping scalar
    const int seqs = s.batch * s.heads;
    constexpr int PER_GROUP = kWaves / SPLIT;
    const int items = seqs * tiles_per_seq;
    const bool by_xcd = seqs % 8 == 0 && gridDim.x % 8 == 0 && static_cast<int64_t>(gridDim.x) * PER_GROUP == items;
    WorkItem w;
    w.sub = wave % SPLIT;
    w.split = SPLIT;
    w.lead = w.sub;
    if (by_xcd) {
        const int xcd = static_cast<int>(blockIdx.x) & 7;
        const int local = (static_cast<int>(blockIdx.x) >> 3) * PER_GROUP + wave / SPLIT; // item index within the XCD
        const int own = seqs >> 3;                                                         // sequences of the XCD
        w.valid = true;
        w.rank = local / own;
        w.seq = xcd + 8 * (local - w.rank * own);
    } else {
        const int item = blockIdx.x * PER_GROUP + wave / SPLIT;
        w.valid = item < items;
        w.rank = item / seqs;
        w.seq = item - w.rank * seqs;
    }
    w.b = w.seq / s.heads;
    w.head = w.seq - w.b * s.heads;
    return w;
}

// Planned mapping (persistent grid, see attention_plan.hpp): the NI * SPLIT waves of workgroup blockIdx.x take the NI
// items of its bin from the launch's item table, item i on waves i*SPLIT .. i*SPLIT + SPLIT - 1. Waves are dealt to
// the 4 SIMDs round-robin (wave w and w + 4 share a SIMD), so with SPLIT = 4 every SIMD runs one quarter of every item
// of the bin, and the table's rotations deal the items' leftover tiles round-robin over the SIMDs. (Dealing them
// always from sub 0 put 9% more tiles than the average on one SIMD at 3 items per bin.)
template<int SPLIT, int NI>
__device__ __forceinline__ WorkItem planned_item(const Shape &s, const ItemTable<NI> &items) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform: keeps tile bookkeeping scalar
    const uint32_t e = items.entry[static_cast<int>(blockIdx.x) * NI + wave / SPLIT];
    WorkItem w;
    w.sub = wave % SPLIT;
    w.split = SPLIT;
    w.valid = e != kNoItem;
    // An empty slot reads sequence 0 (its loads stay in bounds) and visits no tile.
    w.b = w.valid ? static_cast<int>(e & 1023u) : 0;
    w.head = w.valid ? static_cast<int>((e >> 10) & 1023u) : 0;
    w.rank = w.valid ? static_cast<int>((e >> 20) & 1023u) : 0;
    w.lead = plan_lead(static_cast<int>(e >> 30), w.sub, SPLIT);
    w.seq = w.b * s.heads + w.head;
    return w;
}

// Host: the item table of a planned launch over shape s, or null when the launch does not fit one. Items are
// 32-query tiles (forward and dQ; KEY_ITEMS false) or 32-key tiles (dK/dV). Kept per host thread for the last
// shape, so repeated launches do not rebuild it.
template<int NI, bool KEY_ITEMS = false>
inline const ItemTable<NI> *item_table(const Shape &s, const Plan &p) {
    struct Cache {
        Shape s;
        Plan p;
        bool ok;
        ItemTable<NI> table;
    };
    thread_local Cache cache{Shape{}, Plan{}, false, {}};
    const bool same = cache.ok && cache.s.batch == s.batch && cache.s.heads == s.heads && cache.s.queries == s.queries &&
            cache.s.keys == s.keys && cache.s.radius == s.radius && cache.s.causal == s.causal && cache.p.groups == p.groups &&
            cache.p.bins == p.bins && cache.p.seqs == p.seqs && cache.p.tiles == p.tiles && cache.p.rounds == p.rounds &&
            cache.p.reverse == p.reverse;
    if (!same) {
        cache.ok = fill_item_table(cache.table.entry, p, NI, s.heads, [&](const int tile) {
            int first, last;
            return KEY_ITEMS ? dkdv_query_range(s, tile, first, last) : forward_item_tiles(s, tile);
        });
        cache.s = s;
        cache.p = p;
    }
    return cache.ok ? &cache.table : nullptr;
}

// Sums accumulator tiles over the SPLIT waves of an item through LDS; the wave with sub == 0 ends with the total.
// Every wave of the WG-wave workgroup must call it (it contains workgroup barriers when SPLIT > 1). `buffer` holds
// WG * 16 * N * 64 floats; the first barrier also orders it after the workgroup's earlier uses of that memory.
template<int SPLIT, int N, int WG>
__device__ __forceinline__ void split_sum_into(f32x16 (&acc)[N], const int sub, float *buffer) {
    if constexpr (SPLIT > 1) {
        const int lane = threadIdx.x & (kWave - 1);
        const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform: keeps tile bookkeeping scalar
        float *mine = buffer + wave * (16 * N * kWave) + lane;
        __syncthreads(); // a previous call, or the streaming loops, may still be reading this memory
        if (sub > 0) {
#pragma unroll
            for (int t = 0; t < N; ++t) {
#pragma unroll
                for (int j = 0; j < 16; ++j) mine[(16 * t + j) * kWave] = acc[t][j];
            }
        }
        __syncthreads();
        if (sub == 0) {
#pragma unroll
            for (int w = 1; w < SPLIT; ++w) {
#pragma unroll
                for (int t = 0; t < N; ++t) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) acc[t][j] += mine[w * (16 * N * kWave) + (16 * t + j) * kWave];
                }
            }
        }
    }
}

template<int SPLIT, int N, int WG = kWaves>
__device__ __forceinline__ void split_sum(f32x16 (&acc)[N], const int sub) {
    if constexpr (SPLIT > 1) {
        __shared__ float partial[WG * 16 * N * kWave];
        split_sum_into<SPLIT, N, WG>(acc, sub, partial);
    }
}

// True when every (query, key) pair of the 32x32 tile at (q0, key0) is inside the causal/radius window.
// Written as integer limits and two comparisons so that the test stays in scalar instructions (branchy boolean
// logic was lowered to lane masks and VALU selects, five VALU operations per tile).
__device__ __forceinline__ bool tile_in_window(const Shape &s, const int q0, const int key0) {
    const int reach = s.radius >= 0 ? s.radius : 0x40000000; // largest |query - key| allowed
    const int ahead = min(reach, s.causal ? 0 : 0x40000000);  // largest key - query allowed
    return key0 + kTile - 1 - q0 <= ahead && q0 + kTile - 1 - key0 <= reach;
}

} // namespace rk
