// Fused FP32 attention backward for radius windows on gfx950 (MI355X), head width 32 or 64, inputs with 128-bit
// access. The maths is the reference's backward (Attention.hip:32-169, Attention64.hip:34-191): P = exp(s - max)/sum from
// the forward's lse, δ = Σ dO·O, dS = P(dP - δ), dQ = Σ_k dS·k/√D, dK = Σ_q dS·q/√D, dV = Σ_q P·dO.
//
// Under a radius window every 32-key tile sees a band of query tiles that starts one tile later for each key tile: at
// radius 256 under the causal mask key tile kt sees query tiles kt .. kt + 8. A workgroup owns a key block (128 keys, four
// key tiles, one per wave, as in the key-block fused kernel) and walks the band skewed: at step i wave w works on query
// tile base + i + w, so every wave meets exactly the query tiles of its own band and a block takes 9 steps there instead
// of the 12 that a walk over the union of the four bands takes (a quarter of the wave-steps would see no key).
//
// Per step each wave stages nothing of its own: the four query tiles a step reads (and the one loaded for the next step,
// a quarter by each wave, whole 128-byte lines) sit in a ring of five LDS slots, row-major; the row layouts (S and dP A
// operands) and the column layouts (dVᵀ and dKᵀ A operands) are read from them. Each wave then computes, for its key tile
// and its query tile,
//   S = Q·Kᵀ and dP = dO·Vᵀ (v_mfma_f32_32x32x2f32, keys on lanes; the chains start from -(m·log2e + log2 l) and -δ,
//   so P = exp2(S chain) and dS = P·(dP chain)), dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS,
// and its own share of dQ for the query tile, dQᵀ = Kᵀ·dSᵀ over its 32 keys: dS goes through the wave's transpose buffer
// in LDS (queries onto lanes), K's column layout is held in registers (pre-scaled by 1/√D, zero for masked keys). The
// share is summed in the query tile's slot of a second ring of five LDS tiles, kept in the accumulator layout. Within a
// step the four waves work on four different query tiles, and query tile T meets wave 3, 2, 1 and 0 in four consecutive
// steps, so the sum needs no atomics (LDS float atomics cost several times the step's MFMAs): each wave that sees the
// tile loads the partial sum as the start of its dQ chain and stores the result. The last contribution comes from wave 0
// at step (tile - base); after that step's barrier the four waves add the slot to dQ with FP32 buffer atomics (one add
// per dQ element per key block, as in the key-block kernel) and zero it, so the ring is zero wherever a walk starts a
// tile (it is cleared once at the start).
// Blocks are never split: dK and dV are stored once.
//
// Work mapping: one persistent workgroup per CU walks the blocks g, g + G, ...; with the sequences and the grid divisible
// by 8, the workgroups of XCD x take only the sequences x, x + 8, ..., so the resident blocks of an XCD are neighbours that
// share most of their query tiles in the XCD's L2. A pre-pass (launch_backward_prepass) computes δ and zeroes dQ first.
#include "attention_block_plan.hpp"
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

namespace {

constexpr int kRing = 5;               // query tiles held at once: the four a step reads and the one loaded for the next
constexpr int kTrStride = kTile + 4;   // transpose buffer row stride: conflict-free row writes and 128-bit row reads
// dQ partial sums are kept in the accumulator layout every wave shares, lane-major: lane l's 16·D/32 registers at
// l·kDqStride, so a wave moves its partial sum with 128-bit accesses (four registers each) instead of one float per
// register; the 4 extra floats per lane keep 16 consecutive lanes of a 128-bit access on distinct banks.
template<int D>
constexpr int kDqStride = 16 * (D / 32) + 4;

template<int D>
struct BandShared {
    float q[kRing][kSlotFloats<D>];            // Q tiles, row-major, rows D + 4 floats apart
    float u[kRing][kSlotFloats<D>];            // dO tiles
    float seed_s[kRing][kTile];                // per query: -(m·log2e + log2 l), or -inf where P = 0
    float seed_d[kRing][kTile];                // per query: -δ
    float dq[kRing][kWave * kDqStride<D>];     // dQ partial sums of the query tiles in flight, [lane][register]
    float tr[kBlockTiles][kTile * kTrStride];  // per wave: dS transposed, [query][key]
};

// Quarter of a query tile (rows 8w .. 8w + 7) and the statistics of those rows, carried one step ahead.
template<int D>
struct BandQuarter {
    f32x4 q[D / 32], u[D / 32];
    float m, l, d;
};

// At D = 64 the Q and dO rows of the ring interleave the two 32-feature halves: feature f sits at position
// 2 (f mod 32) + f / 32. A lane's column-layout operands for both output slices (features col and 32 + col of a row)
// are then one 64-bit read instead of two 32-bit reads. The S and dP products reduce over the positions in order, so
// the K and V rows they pair with are loaded in the same order (load_row_positions).
template<int D>
constexpr bool kInterleaved = D == 64;

// Row of HALF = D/2 positions for half-wave h of a row in natural feature order at byte offset `row`: positions
// 32h .. 32h + 31 of the interleaved order, i.e. features 16h + m and 32 + 16h + m at r[2m] and r[2m + 1].
template<int D>
__device__ __forceinline__ void load_row_positions(float (&r)[D / 2], const Buffer b, const uint32_t row, const int h) {
    if constexpr (kInterleaved<D>) {
        float lo[16], hi[16];
        buffer_load_span<true>(lo, b, row + 64u * static_cast<uint32_t>(h));
        buffer_load_span<true>(hi, b, row + 128u + 64u * static_cast<uint32_t>(h));
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            r[2 * m] = lo[m];
            r[2 * m + 1] = hi[m];
        }
    } else {
        buffer_load_span<true>(r, b, row + 4u * static_cast<uint32_t>(h) * (D / 2));
    }
}

// Column layout of an interleaved slot: element [tile_row(j, h)][32t + col] to c[t][j - J0], both slices with one
// 64-bit read per row (the A operands of MFMAs j of a product that reduces over the slot's rows).
template<int D, int J0, int J>
__device__ __forceinline__ void read_column_pairs(const float *slot, float (&c)[D / 32][J]) {
    static_assert(D == 64, "two 32-feature slices");
    const int lane = threadIdx.x & (kWave - 1);
    const float *base = slot + 4 * (lane >> 5) * kSlotStride<D> + 2 * (lane & 31);
#pragma unroll
    for (int j = J0; j < J0 + J; ++j) {
        const f32x2 x = *reinterpret_cast<const f32x2 *>(base + (8 * (j >> 2) + (j & 3)) * kSlotStride<D>);
        c[0][j - J0] = x[0];
        c[1][j - J0] = x[1];
    }
}

template<int D, int J0, int J>
__device__ __forceinline__ void read_columns(const float *slot, float (&c)[D / 32][J]) {
    if constexpr (kInterleaved<D>) read_column_pairs<D, J0, J>(slot, c);
    else read_column_layout<D, J0, J>(slot, c);
}

template<int D>
__global__ __launch_bounds__(kWave * kBlockTiles) void attention_band_backward_kernel(const Tensor q, const Tensor k,
        const Tensor v, const uint8_t *__restrict__ mask, const float *__restrict__ lse, const Tensor du,
        const float *__restrict__ delta, float *__restrict__ dq, float *__restrict__ dk, float *__restrict__ dv, const Shape s,
        const int nblocks, const int groups, const float scale) {
    constexpr int HALF = D / 2;
    constexpr int DT = D / 32;
    constexpr int S = kSlotStride<D>;
    __shared__ __align__(16) BandShared<D> sh;

    const int lane = threadIdx.x & (kWave - 1);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // key tile of the block
    const int col = lane & 31;
    const int h = lane >> 5;
    const float c2 = scale * kLog2e;
    const int seqs = s.batch * s.heads;
    const int qtiles = (s.queries + kTile - 1) / kTile;
    const uint32_t kstep = 4u * k.st, vstep = 4u * v.st, qstep = 4u * q.st, ustep = 4u * du.st;

    // The dQ ring starts at zero; every flush zeroes the slot it empties (the first block's barrier orders these stores).
    for (int e = 4 * static_cast<int>(threadIdx.x); e < kRing * kWave * kDqStride<D>; e += 4 * kWave * kBlockTiles)
        *reinterpret_cast<f32x4 *>(&sh.dq[0][0] + e) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const int group = static_cast<int>(blockIdx.x) % groups;
    const int member = static_cast<int>(blockIdx.x) / groups;
    const int members = static_cast<int>(gridDim.x) / groups;
    const int group_blocks = seqs / groups * nblocks;
    // A block's coordinates and the buffer resources of its sequence.
    struct Block {
        int seq, kb;
        Buffer kbuf, vbuf, qbuf, ubuf, lbuf, dbuf, mbuf;
        BandWalk walk;
    };
    auto block_at = [&](const int index) __attribute__((always_inline)) {
        Block c;
        const int local_seq = index / nblocks;
        c.kb = index - local_seq * nblocks;
        c.seq = group + groups * local_seq;
        const int b = c.seq / s.heads;
        const int head = c.seq - b * s.heads;
        c.kbuf = make_buffer(sequence(k, b, head), sequence_bytes(s.keys, k.st, D));
        c.vbuf = make_buffer(sequence(v, b, head), sequence_bytes(s.keys, v.st, D));
        c.qbuf = make_buffer(sequence(q, b, head), sequence_bytes(s.queries, q.st, D));
        c.ubuf = make_buffer(sequence(du, b, head), sequence_bytes(s.queries, du.st, D));
        c.lbuf = make_buffer(lse + static_cast<int64_t>(c.seq) * s.queries * 2, static_cast<uint32_t>(s.queries) * 8u);
        c.dbuf = make_buffer(delta + static_cast<int64_t>(c.seq) * s.queries, static_cast<uint32_t>(s.queries) * 4u);
        c.mbuf = make_buffer(mask + static_cast<int64_t>(b) * s.keys, static_cast<uint32_t>(s.keys));
        // The skewed schedule (step i, wave w: query tile base + i + w) and the union of the bands.
        c.walk = band_walk(s.queries, s.keys, s.radius, s.causal, c.kb);
        return c;
    };
    // Query-tile quarters: rows 8w .. 8w + 7 of tile T, lane (row lane % 8, 16-byte chunk 8i + lane / 8), whole lines.
    // Rows outside the sequence (T < 0 or past the end) read 0 and get P = 0.
    auto load_quarter = [&](const Block &c, BandQuarter<D> &r, const int tile) __attribute__((always_inline)) {
        const int query = tile * kTile + 8 * w + (lane & 7);
        const bool ok = query >= 0 && query < s.queries; // kNoRow keeps the offset out of range for any stride
        const uint32_t row = static_cast<uint32_t>(query);
#pragma unroll
        for (int i = 0; i < D / 32; ++i) {
            const uint32_t chunk = static_cast<uint32_t>(8 * i + (lane >> 3));
            r.q[i] = buffer_load4(c.qbuf, (ok ? row * qstep : kNoRow) + 16u * chunk, 0);
            r.u[i] = buffer_load4(c.ubuf, (ok ? row * ustep : kNoRow) + 16u * chunk, 0);
        }
        r.m = buffer_load(c.lbuf, ok ? row * 8u : kNoRow, 0);
        r.l = buffer_load(c.lbuf, ok ? row * 8u + 4u : kNoRow, 0);
        r.d = buffer_load(c.dbuf, ok ? row * 4u : kNoRow, 0);
    };
    // The loads a block starts from: the key-mask byte (keys past the end read 0 through kNoRow rather than a branch),
    // this wave's K and V rows (row layout: B operands of S and dP) and the first four query tiles' quarters. The next
    // block's are issued as soon as a walk ends, before the walk's last dQ adds and the dK/dV stores: their round trip
    // overlaps the end of the block, and the in-order vector-memory counter does not make the next block wait for
    // those adds (all 256 workgroups end their blocks together, so the adds arrive at the L2 as one burst).
    struct BlockLoads {
        int mask_byte;
        float kr[HALF], vr[HALF]; // in the ring's position order (kInterleaved)
        BandQuarter<D> opening[kBlockTiles];
    };
    auto issue = [&](const Block &c, BlockLoads &ld) __attribute__((always_inline)) {
        const int key = (c.kb * kBlockTiles + w) * kTile + col;
        const bool in_range = key < s.keys;
        ld.mask_byte = buffer_load_byte(c.mbuf, in_range ? static_cast<uint32_t>(key) : kNoRow);
        load_row_positions<D>(ld.kr, c.kbuf, in_range ? static_cast<uint32_t>(key) * kstep : kNoRow, h);
        load_row_positions<D>(ld.vr, c.vbuf, in_range ? static_cast<uint32_t>(key) * vstep : kNoRow, h);
        // A block that no query sees reads nothing (its tiles would be outside every band).
        const int base = c.walk.nsteps > 0 ? c.walk.base : -0x10000;
#pragma unroll
        for (int x = 0; x < kBlockTiles; ++x) load_quarter(c, ld.opening[x], base + x);
    };

    // Adds this wave's quarter of a finished dQ tile into dQ: wave w holds registers RQ·w .. RQ·w + RQ - 1 of every
    // lane, and register (t, j) of lane (col, h) is query tile_row(j, h), feature 32t + col, so each atomic instruction
    // covers two whole 128-byte rows.
    constexpr int RQ = 4 * DT; // registers per wave: a quarter of the lane's 16·DT
    auto add_tile = [&](const Buffer gbuf, const int tile, const f32x4 (&x)[RQ / 4]) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < RQ; ++r) {
            const int reg = RQ * w + r, t = reg >> 4, j = reg & 15;
            const uint32_t voff = (static_cast<uint32_t>(tile * kTile + tile_row(j, h)) * D + static_cast<uint32_t>(32 * t + col)) * 4u;
            __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(x[r >> 2][r & 3], gbuf, static_cast<int>(voff), 0, 0);
        }
    };
    // The three query tiles still in flight when a walk ends are taken out of the ring at the block's end, but their
    // adds go out during the next block's first three steps, one tile per step: every workgroup ends its blocks at the
    // same time, and adding all three at once made each block end one burst of FP32 atomics on the L2.
    f32x4 tail[kBlockTiles - 1][RQ / 4];
    int tail_tile[kBlockTiles - 1] = {-1, -1, -1}; // -1: nothing pending
    Buffer tail_buf = make_buffer(dq, 0);           // dQ of the sequence the pending tiles belong to
    auto emit = [&](const int x) __attribute__((always_inline)) {
        if (tail_tile[x] >= 0) add_tile(tail_buf, tail_tile[x], tail[x]);
        tail_tile[x] = -1;
    };

    BlockLoads ld;
    if (member < group_blocks) issue(block_at(member), ld);
    for (int index = member; index < group_blocks; index += members) {
        const Block cur = block_at(index);
        const int seq = cur.seq, kb = cur.kb;
        const Buffer qgbuf = make_buffer(dq + static_cast<int64_t>(seq) * s.queries * D, static_cast<uint32_t>(s.queries) * (4u * D));
        const int base = cur.walk.base, nsteps = cur.walk.nsteps, union_lo = cur.walk.lo, union_hi = cur.walk.hi;
        int my_first, my_end; // this wave's band
        key_tile_band(s.queries, s.keys, s.radius, s.causal, kb * kBlockTiles + w, my_first, my_end);

        const int key0 = (kb * kBlockTiles + w) * kTile;
        const int key = key0 + col;
        float (&kr)[HALF] = ld.kr; // pre-scaled by scale·log2e below
        float (&vr)[HALF] = ld.vr;
        // K's column layout (A operand of dQᵀ: kc[t][j] = K[key0 + tile_row(j, h)][32t + col]) from the row layout,
        // one 32-feature slice at a time through this wave's transpose buffer (free until the walk): 4 128-bit writes
        // and 16 reads per slice instead of 16 single-float loads per slice from memory. Pre-scaled by 1/√D and zero
        // for masked keys below, whatever K holds there.
        float kc[DT][16];
        {
            float *const tb = sh.tr[w];
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                wave_lds_sync(); // the previous slice's reads (or the previous block's walk) are done
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    // Lane (key col, h) holds features 32t + 16h + 4u .. +3 (positions 2m + t at D = 64, m otherwise).
                    f32x4 x;
#pragma unroll
                    for (int e = 0; e < 4; ++e) x[e] = kInterleaved<D> ? kr[2 * (4 * u + e) + t] : kr[4 * u + e];
                    *reinterpret_cast<f32x4 *>(&tb[col * kTrStride + 16 * h + 4 * u]) = x;
                }
                wave_lds_sync();
#pragma unroll
                for (int j = 0; j < 16; ++j) kc[t][j] = tb[tile_row(j, h) * kTrStride + col];
            }
        }
        auto store_quarter = [&](const BandQuarter<D> &r, const int tile) __attribute__((always_inline)) {
            const int slot = (tile + kRing) % kRing;
            const int row = 8 * w + (lane & 7);
            if constexpr (kInterleaved<D>) {
                // The lane holds features 4c .. 4c + 3 and 32 + 4c .. 32 + 4c + 3 (c = lane / 8): positions 8c .. 8c + 7.
                const int at = row * S + 8 * (lane >> 3);
                auto put = [&](float *dst, const f32x4 (&x)[D / 32]) __attribute__((always_inline)) {
                    *reinterpret_cast<f32x4 *>(dst + at) = f32x4{x[0][0], x[1][0], x[0][1], x[1][1]};
                    *reinterpret_cast<f32x4 *>(dst + at + 4) = f32x4{x[0][2], x[1][2], x[0][3], x[1][3]};
                };
                put(sh.q[slot], r.q);
                put(sh.u[slot], r.u);
            } else {
#pragma unroll
                for (int i = 0; i < D / 32; ++i) {
                    const int at = row * S + 4 * (8 * i + (lane >> 3));
                    *reinterpret_cast<f32x4 *>(&sh.q[slot][at]) = r.q[i];
                    *reinterpret_cast<f32x4 *>(&sh.u[slot][at]) = r.u[i];
                }
            }
            const int query = tile * kTile + row;
            const bool ok = query >= 0 && query < s.queries && r.m != -INFINITY;
            // Straight-line arithmetic and a select: a branch here would let the compiler sink the statistic loads into
            // it and wait for each of them in turn. l >= 1 for every row that sees a key (v_log_f32 needs no denormal care).
            const float seed = -fmaf(r.m, kLog2e, __builtin_amdgcn_logf(r.l));
            sh.seed_s[slot][row] = ok ? seed : -INFINITY; // P = exp2(S·scale·log2e + this)
            sh.seed_d[slot][row] = -r.d;
        };
        // Takes query tile X's finished dQ slot (this wave's quarter) and zeroes it; false for tiles outside the
        // sequence or that no wave of the block touched (they hold zeros).
        auto take = [&](const int tile, f32x4 (&x)[RQ / 4]) __attribute__((always_inline)) {
            if (tile < 0 || tile >= qtiles || tile < union_lo || tile >= union_hi) return false;
            f32x4 *src = reinterpret_cast<f32x4 *>(&sh.dq[(tile + kRing) % kRing][lane * kDqStride<D> + RQ * w]);
#pragma unroll
            for (int c = 0; c < RQ / 4; ++c) {
                x[c] = src[c];
                src[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            return true;
        };
        auto flush = [&](const int tile) __attribute__((always_inline)) {
            f32x4 x[RQ / 4];
            if (take(tile, x)) add_tile(qgbuf, tile, x);
        };

        f32x16 acc_k[DT], acc_v[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            acc_k[t] = f32x16{};
            acc_v[t] = f32x16{};
        }
        const bool visible = ld.mask_byte != 0;
        const uint32_t bits = static_cast<uint32_t>(__ballot(visible));
        if (bits == 0) my_end = my_first; // no visible key: the wave only keeps the schedule
        const int qlo = window_query_lo(s, key);
        const int qhi = min(window_query_hi(s, key), s.queries - 1);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool kept = (bits >> tile_row(j, h)) & 1u;
#pragma unroll
            for (int t = 0; t < DT; ++t) kc[t][j] = kept ? kc[t][j] * scale : 0.0f;
        }
        if (nsteps > 0) { // a block that no query sees stores zero dK/dV below
    #pragma unroll
            for (int x = 0; x < kBlockTiles; ++x) store_quarter(ld.opening[x], base + x);
    #pragma unroll
            for (int c = 0; c < HALF; ++c) kr[c] *= c2;
            __syncthreads();

            float *const tr = sh.tr[w];
            for (int i = 0; i < nsteps; ++i) {
                const int tile = base + i + w;
                const int slot = (tile + kRing) % kRing;
                const bool has_next = i + 1 < nsteps;
                float *const dslot = sh.dq[slot];
                BandQuarter<D> next;
                if (has_next) load_quarter(cur, next, base + i + kBlockTiles);
                if (tile >= my_first && tile < my_end) {
                    const int q0 = tile * kTile;
                    // Each product's LDS reads are issued together, ahead of its MFMAs (sched_barrier keeps them there):
                    // with one wave per SIMD nothing else covers an LDS round trip, so the wave waits once per operand
                    // group instead of once per read. Accumulator register j holds query q0 + tile_row(j, h): the chains
                    // start from its seeds.
                    f32x16 sc, dp;
                    {
                        float qr[HALF];
    #pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const f32x4 a = *reinterpret_cast<const f32x4 *>(&sh.seed_s[slot][8 * u + 4 * h]);
                            const f32x4 d = *reinterpret_cast<const f32x4 *>(&sh.seed_d[slot][8 * u + 4 * h]);
    #pragma unroll
                            for (int x = 0; x < 4; ++x) {
                                sc[4 * u + x] = a[x];
                                dp[4 * u + x] = d[x];
                            }
                        }
                        read_row_layout<D>(sh.q[slot], qr);
                        __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
                        for (int c = 0; c < HALF; ++c) sc = mfma(qr[c], kr[c], sc);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    {
                        float ur[HALF];
                        read_row_layout<D>(sh.u[slot], ur);
                        __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
                        for (int c = 0; c < HALF; ++c) dp = mfma(ur[c], vr[c], dp);
                    }
                    __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float p = exp2_fast(sc[j]);
                        sc[j] = p;
                        dp[j] *= p;
                    }
                    if (bits != 0xffffffffu || q0 + kTile > s.queries || !tile_in_window(s, q0, key0)) {
                        const uint32_t keep = visible ? bit_range(qlo - q0, qhi - q0) >> (4 * h) : 0u;
    #pragma unroll
                        for (int j = 0; j < 16; ++j) {
                            const bool ok = (keep >> (8 * (j >> 2) + (j & 3))) & 1u;
                            sc[j] = ok ? sc[j] : 0.0f;
                            dp[j] = ok ? dp[j] : 0.0f;
                        }
                    }
                    // dS transposed through this wave's buffer: B operand of dQᵀ MFMA j is dS[query col][key tile_row(j, h)].
                    wave_lds_sync();
    #pragma unroll
                    for (int j = 0; j < 16; ++j) tr[tile_row(j, h) * kTrStride + col] = dp[j];
                    // dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS, column layouts read from the staged tiles eight rows at a time, each
                    // group read one group of MFMAs ahead of its use.
                    auto products = [&](const float (&c)[DT][8], const f32x16 &bop, const int j0, f32x16 (&acc)[DT]) __attribute__((always_inline)) {
    #pragma unroll
                        for (int j = 0; j < 8; ++j) {
    #pragma unroll
                            for (int t = 0; t < DT; ++t) acc[t] = mfma(c[t][j], bop[j0 + j], acc[t]);
                        }
                    };
                    {
                        float ca[DT][8], cb[DT][8];
                        read_columns<D, 0, 8>(sh.u[slot], ca);
                        __builtin_amdgcn_sched_barrier(0);
                        read_columns<D, 8, 8>(sh.u[slot], cb);
                        __builtin_amdgcn_sched_barrier(0);
                        products(ca, sc, 0, acc_v);
                        __builtin_amdgcn_sched_barrier(0);
                        read_columns<D, 0, 8>(sh.q[slot], ca);
                        __builtin_amdgcn_sched_barrier(0);
                        products(cb, sc, 8, acc_v);
                        __builtin_amdgcn_sched_barrier(0);
                        read_columns<D, 8, 8>(sh.q[slot], cb);
                        __builtin_amdgcn_sched_barrier(0);
                        products(ca, dp, 0, acc_k);
                        __builtin_amdgcn_sched_barrier(0);
                        products(cb, dp, 8, acc_k);
                    }
                    wave_lds_sync();
                    // dQ share of this key tile, dS·K over its 32 keys (A = dS rows, B = K's column layout), chained onto the
                    // query tile's partial sum: register j of slice t is query q0 + tile_row(j, h), feature 32t + col, and the
                    // partial sum is read and written in that register layout (four registers per 128-bit access).
                    float bq[16];
                    f32x16 acc_q[DT];
    #pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f32x4 x = *reinterpret_cast<const f32x4 *>(&tr[col * kTrStride + 8 * u + 4 * h]);
                        bq[4 * u + 0] = x[0];
                        bq[4 * u + 1] = x[1];
                        bq[4 * u + 2] = x[2];
                        bq[4 * u + 3] = x[3];
                    }
                    f32x4 *const mine = reinterpret_cast<f32x4 *>(dslot + lane * kDqStride<D>);
    #pragma unroll
                    for (int t = 0; t < DT; ++t) {
    #pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const f32x4 x = mine[4 * t + u];
    #pragma unroll
                            for (int e = 0; e < 4; ++e) acc_q[t][4 * u + e] = x[e];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
                    for (int t = 0; t < DT; ++t) {
    #pragma unroll
                        for (int j = 0; j < 16; ++j) acc_q[t] = mfma(bq[j], kc[t][j], acc_q[t]);
                    }
    #pragma unroll
                    for (int t = 0; t < DT; ++t) {
    #pragma unroll
                        for (int u = 0; u < 4; ++u)
                            mine[4 * t + u] = f32x4{acc_q[t][4 * u], acc_q[t][4 * u + 1], acc_q[t][4 * u + 2], acc_q[t][4 * u + 3]};
                    }
                }
                if (has_next) store_quarter(next, base + i + kBlockTiles);
                __syncthreads(); // this step's dQ shares and the next step's tile are in LDS
                flush(base + i); // wave 0 has just given query tile base + i its last share
                // The previous block's last tiles, one per step.
                if (i == 0) emit(0);
                else if (i == 1) emit(1);
                else if (i == 2) emit(2);
            }
        }
#pragma unroll
        for (int x = 0; x < kBlockTiles - 1; ++x) emit(x); // a walk shorter than three steps (or none) leaves some
        // This block's K/V rows and column layout are dead: the next block's loads go out now (see BlockLoads).
        const bool last_block = index + members >= group_blocks;
        if (!last_block) issue(block_at(index + members), ld);
        if (nsteps > 0) {
            // Query tiles still in flight after the walk (only waves 1..3 reached them): taken now, added during the
            // next block's first steps (or now, after the last block).
            tail_buf = qgbuf;
#pragma unroll
            for (int x = 0; x < kBlockTiles - 1; ++x) tail_tile[x] = take(base + nsteps + x, tail[x]) ? base + nsteps + x : -1;
            if (last_block) {
#pragma unroll
                for (int x = 0; x < kBlockTiles - 1; ++x) emit(x);
            }
        }

        // dK and dV of this wave's key tile (keys past the end fall outside the resources).
        const Buffer kg = make_buffer(dk + static_cast<int64_t>(seq) * s.keys * D, static_cast<uint32_t>(s.keys) * (4u * D));
        const Buffer vg = make_buffer(dv + static_cast<int64_t>(seq) * s.keys * D, static_cast<uint32_t>(s.keys) * (4u * D));
        const uint32_t row = static_cast<uint32_t>(key) * (4u * D) + 16u * h;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t off = row + 128u * t + 32u * u; // features 32t + 8u + 4h .. +3
                const f32x4 xk{acc_k[t][4 * u] * scale, acc_k[t][4 * u + 1] * scale, acc_k[t][4 * u + 2] * scale, acc_k[t][4 * u + 3] * scale};
                const f32x4 xv{acc_v[t][4 * u], acc_v[t][4 * u + 1], acc_v[t][4 * u + 2], acc_v[t][4 * u + 3]};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, xk), kg, static_cast<int>(off), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, xv), vg, static_cast<int>(off), 0, 0);
            }
        }
        __syncthreads(); // the next block overwrites both rings
    }
}

Tensor tensor(const float *p, const rocmkernels_strides &st) { return Tensor{p, st.batch, st.head, st.token}; }

template<int D>
hipError_t launch(const BackwardArgs &a, const int cus, hipStream_t stream) {
    const hipError_t error = launch_backward_prepass(D, a, stream);
    if (error != hipSuccess) return error;
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const int nblocks = (a.keys + kBlockKeys - 1) / kBlockKeys;
    const long long seqs = static_cast<long long>(a.batch) * a.heads;
    const long long blocks = seqs * nblocks;
    int grid = static_cast<int>(blocks < cus ? blocks : cus);
    const int groups = (seqs % 8 == 0 && grid % 8 == 0) ? 8 : 1;
    hipLaunchKernelGGL((attention_band_backward_kernel<D>), dim3(static_cast<unsigned>(grid)), dim3(kWave * kBlockTiles), 0, stream,
            tensor(a.q, a.qs), tensor(a.k, a.ks), tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), a.lse,
            tensor(a.upstream, a.us), a.delta, a.gradient_q, a.gradient_k, a.gradient_v, shape, nblocks, groups, scale);
    return hipGetLastError();
}

} // namespace

hipError_t launch_band_backward(const int D, const BackwardArgs &a, const int cus, hipStream_t stream) {
    return D == 32 ? launch<32>(a, cus, stream) : launch<64>(a, cus, stream);
}

} // namespace rk
