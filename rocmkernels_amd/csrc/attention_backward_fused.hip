// Fused FP32 attention backward for gfx950 (MI355X): one kernel computes dK, dV and dQ, head width 32 or 64, for
// inputs with 128-bit access (16-byte aligned, strides multiples of 4 floats). Selected by the fused flag of the _ex
// backward entry points (ROCMKERNELS_ATTENTION_FUSED_BACKWARD); the maths is the reference's backward
// (Attention.hip:32-169, Attention64.hip:34-191): P = exp(s - max)/sum from the forward's lse, δ = Σ dO·O,
// dS = P(dO·v - δ), dQ = Σ_k dS·k/√D, dK = Σ_q dS·q/√D, dV = Σ_q P·dO.
//
// Mapping. A workgroup owns a key block: 128 keys (four 32-key tiles) of one (batch, head) sequence, and streams the
// query tiles that see it. Wave w of each query stream owns key tile w of the block (its K and V rows stay in
// registers, its dKᵀ and dVᵀ accumulate in registers); at d = 32 two streams (8 waves, two per SIMD) take alternate
// query tiles and merge their dK/dV through LDS at the end, at d = 64 one stream (4 waves, up to 512 registers each).
// Per query tile, the four waves of a stream share the tile's Q, dO and softmax statistics, staged once in LDS
// (each wave loads a quarter, whole 128-byte lines, one tile ahead, double-buffered), and each computes
//   S = Q·Kᵀ and dP = dO·Vᵀ (v_mfma_f32_32x32x2f32, keys on lanes), P and dS = P(dP - δ),
//   dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS (the accumulators of S and dP are the B operands directly),
// and writes its 32 x 32 dS into the stream's dS tile [query][block key] in LDS. After one workgroup barrier every
// wave forms one 16-query x 16-feature quadrant of dQ = dS·K/√D over all 128 keys of the block
// (v_mfma_f32_16x16x4f32: A = dS from LDS, B = the block's K rows held in registers, pre-scaled and zero for masked
// keys) and adds it into dQ with FP32 buffer atomics: one add per dQ element per key block, a quarter of what adding
// each 32-key tile's product would take. Per tile and wave that is 5 GEMM tiles of MFMA work, the minimum for the
// backward (S is recomputed once).
//
// Work partition (attention_block_plan.hpp): with a plan, a persistent grid of one workgroup per CU takes
// cost-balanced pieces (blocks, or contiguous query-tile ranges of blocks too large for one workgroup's share); a piece
// of a split block adds its dK/dV into memory zeroed by the pre-pass, a whole block stores them. Without a plan (too
// many pieces for the kernel-argument table), one workgroup per whole block, heaviest first, in dispatch order.
//
// A pre-pass kernel computes δ (bit-identical to the deterministic backward's: 4-feature partial products added in
// the same pairwise tree, group_dot and group_tree) and zeroes dQ (and dK/dV when some block is split). dQ (and the dK/dV of split blocks) depend on the order in
// which the atomics land, so their low bits vary from run to run.
#include "attention_block_plan.hpp"
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

namespace {

__device__ __forceinline__ f32x4 mfma16(const float a, const float b, const f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

constexpr int kDsStride = kBlockKeys + 4; // floats between dS rows in LDS: conflict-free 128-bit reads of 16 rows

// Feature-major copies of the Q and dO tiles ([feature][query], rows kTStride floats apart) give the column layouts of
// the dKᵀ and dVᵀ products four tile rows per 128-bit read: accumulator rows tile_row(4u .. 4u + 3, h) are 8u + 4h + 0..3.
constexpr int kTStride = kTile + 4;

template<int D, int STREAMS>
struct FusedShared {
    float qs[STREAMS][2][kSlotFloats<D>]; // Q tile per stream and parity (rows D + 4 floats apart)
    float us[STREAMS][2][kSlotFloats<D>]; // dO tile
    float qt[STREAMS][2][D * kTStride];   // Q tile, feature-major
    float ut[STREAMS][2][D * kTStride];   // dO tile, feature-major
    float mc[STREAMS][2][kTile];          // per query: S chain seed -(m·log2e + log2 l) (-inf: P = 0)
    float dl[STREAMS][2][kTile];          // per query: dP chain seed -δ
    float ds[STREAMS][2][kTile * kDsStride]; // dS[query][block key]
    uint32_t kbits[kBlockTiles];          // key-mask ballots of the block's key tiles
};

template<int N>
struct PieceList {
    uint32_t entry[N];
};

// Quarter of a query tile (rows 8w .. 8w + 7) and the statistics of those rows, carried one tile ahead.
template<int D>
struct Quarter {
    f32x4 q[D / 32], u[D / 32];
    float m, l, d;
};

template<int D, int STREAMS, bool PLANNED>
__global__ __launch_bounds__(kWave * kBlockTiles * STREAMS) void attention_fused_backward_kernel(const Tensor q, const Tensor k,
        const Tensor v, const uint8_t *__restrict__ mask, const float *__restrict__ lse, const Tensor du,
        const float *__restrict__ delta, float *__restrict__ dq, float *__restrict__ dk, float *__restrict__ dv, const Shape s,
        const int nblocks, const int slots, const PieceList<PLANNED ? kMaxPieces : 1> table, const float scale) {
    constexpr int HALF = D / 2;
    constexpr int DT = D / 32;
    constexpr int CPR = D / 4; // 16-byte chunks per row
    __shared__ __align__(16) FusedShared<D, STREAMS> sh;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int stream = wave / kBlockTiles;
    const int w = wave - stream * kBlockTiles; // key tile of the block; waves w of both streams share a SIMD
    const int col = lane & 31;
    const int h = lane >> 5;
    const float c2 = scale * kLog2e;
    // dQ quadrants of this wave: features 16·fg .. +15 of rows 16·rh .. +15 (d = 32: one; d = 64: both row halves).
    const int fg = D == 32 ? (w & 1) : w;
    constexpr int RH = D == 32 ? 1 : 2;
    const int rh0 = D == 32 ? (w >> 1) : 0;

    const int seqs = s.batch * s.heads;
    const int npieces = PLANNED ? slots : 1;
    const uint32_t kstep = 4u * k.st, vstep = 4u * v.st, qstep = 4u * q.st, ustep = 4u * du.st;
    constexpr int WAVES = kBlockTiles * STREAMS;
    constexpr int KCH = kBlockKeys * CPR / (kWave * WAVES); // 16-byte chunks of the block's K rows per lane

    // A piece's coordinates, from its table entry (or, without a plan, from the workgroup index: rank-major,
    // sequence-minor, so under a causal mask block 0, the heaviest, of every sequence goes first).
    struct Ctx {
        bool valid, partial;
        int seq, kb, b, head, count, qt0;
    };
    auto decode = [&](const int slot) __attribute__((always_inline)) {
        Ctx c{};
        Piece pc{0, 0, 0, false};
        c.valid = slot < npieces;
        if constexpr (PLANNED) {
            const uint32_t e = c.valid ? table.entry[static_cast<int>(blockIdx.x) * slots + slot] : kNoPiece;
            c.valid = e != kNoPiece;
            if (c.valid) pc = unpack_piece(e);
        } else {
            const int rank = static_cast<int>(blockIdx.x) / seqs;
            pc = Piece{(static_cast<int>(blockIdx.x) - rank * seqs) * nblocks + rank, 0, 0, false};
        }
        c.partial = pc.partial;
        c.seq = pc.block / nblocks;
        c.kb = pc.block - c.seq * nblocks;
        c.b = c.seq / s.heads;
        c.head = c.seq - c.b * s.heads;
        int qt_first;
        const int full = block_query_tiles(s.queries, s.keys, s.radius, s.causal, c.kb, qt_first);
        c.count = PLANNED ? pc.count : full;
        c.qt0 = qt_first + pc.start;
        return c;
    };
    // Per-sequence buffer resources of a piece.
    struct Bufs {
        Buffer k, v, q, u, l, d, m;
    };
    auto buffers = [&](const Ctx &c) __attribute__((always_inline)) {
        return Bufs{make_buffer(sequence(k, c.b, c.head), sequence_bytes(s.keys, k.st, D)),
                make_buffer(sequence(v, c.b, c.head), sequence_bytes(s.keys, v.st, D)),
                make_buffer(sequence(q, c.b, c.head), sequence_bytes(s.queries, q.st, D)),
                make_buffer(sequence(du, c.b, c.head), sequence_bytes(s.queries, du.st, D)),
                make_buffer(lse + static_cast<int64_t>(c.seq) * s.queries * 2, static_cast<uint32_t>(s.queries) * 8u),
                make_buffer(delta + static_cast<int64_t>(c.seq) * s.queries, static_cast<uint32_t>(s.queries) * 4u),
                make_buffer(mask + static_cast<int64_t>(c.b) * s.keys, static_cast<uint32_t>(s.keys))};
    };

    // Quarter loads of a query tile: rows 8w .. 8w + 7, lane (row lane % 8, 16-byte chunk 8i + lane / 8) for load i, so
    // each load covers whole 128-byte lines and a half-wave's feature-major writes below spread over 8 rows (2-way bank
    // conflicts; with lanes along the row instead, 8-way at d = 64). The statistics are those of query
    // q0 + 8w + lane % 8. Rows past the sequence read 0.
    auto load_quarter = [&](Quarter<D> &r, const Bufs &bf, const int q0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < D / 32; ++i) {
            const uint32_t row = static_cast<uint32_t>(q0 + 8 * w + (lane & 7));
            const uint32_t chunk = static_cast<uint32_t>(8 * i + (lane >> 3));
            r.q[i] = buffer_load4(bf.q, row * qstep + 16u * chunk, 0);
            r.u[i] = buffer_load4(bf.u, row * ustep + 16u * chunk, 0);
        }
        const uint32_t qq = static_cast<uint32_t>(q0 + 8 * w + (lane & 7));
        r.m = buffer_load(bf.l, qq * 8u, 0);
        r.l = buffer_load(bf.l, qq * 8u + 4u, 0);
        r.d = buffer_load(bf.d, qq * 4u, 0);
    };
    auto store_quarter = [&](const Quarter<D> &r, const int q0, const int p) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < D / 32; ++i) {
            const int row = 8 * w + (lane & 7), chunk = 8 * i + (lane >> 3);
            const int at = row * kSlotStride<D> + 4 * chunk;
            *reinterpret_cast<f32x4 *>(&sh.qs[stream][p][at]) = r.q[i];
            *reinterpret_cast<f32x4 *>(&sh.us[stream][p][at]) = r.u[i];
            const int tat = 4 * chunk * kTStride + row;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sh.qt[stream][p][tat + e * kTStride] = r.q[i][e];
                sh.ut[stream][p][tat + e * kTStride] = r.u[i][e];
            }
        }
        // Every lane writes the statistics of row 8w + lane % 8 (eight lanes write each value, all equal): the loads then
        // stay with the tile's loads instead of sinking into a branch behind the wait for the tile.
        const int qq = q0 + 8 * w + (lane & 7);
        const bool ok = qq < s.queries && r.m != -INFINITY;
        sh.mc[stream][p][8 * w + (lane & 7)] = ok ? -fmaf(r.m, kLog2e, __log2f(r.l)) : -INFINITY; // P = exp2(s·c2 + this)
        sh.dl[stream][p][8 * w + (lane & 7)] = -r.d;
    };

    // The loads of a piece's prologue: this wave's K and V tile in row layout (B operands of S and dP), the block's K
    // rows (whole 128-byte lines, staged feature-major in LDS for the dQ B operands: lane (n, kk) holds
    // K[128 kb + 32 kk + i][16 fg + n], i = 0 .. 31; 32 single-float loads per lane instead took about 2 us per piece in
    // the texture addresser), the first query tile of this stream and the key mask byte (issued last: the piece then
    // waits for memory once). For every piece after the first they are issued during the previous piece's last
    // iteration, so their round trip overlaps its last dQ and its epilogue.
    struct Loads {
        f32x4 kraw[KCH];
        float kr[HALF], vr[HALF];
        Quarter<D> first;
        int mbyte;
    };
    auto issue = [&](const Ctx &c, Loads &ld) __attribute__((always_inline)) {
        const Bufs bf = buffers(c);
        const int key = (c.kb * kBlockTiles + w) * kTile + col;
        const bool in_range = key < s.keys;
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int ch = i * kWave * WAVES + static_cast<int>(threadIdx.x);
            ld.kraw[i] = buffer_load4(bf.k, static_cast<uint32_t>(c.kb * kBlockKeys + ch / CPR) * kstep + 16u * static_cast<uint32_t>(ch % CPR), 0);
        }
        buffer_load_span<true>(ld.kr, bf.k, in_range ? static_cast<uint32_t>(key) * kstep + 4u * h * HALF : kNoRow);
        buffer_load_span<true>(ld.vr, bf.v, in_range ? static_cast<uint32_t>(key) * vstep + 4u * h * HALF : kNoRow);
        if (stream < c.count) load_quarter(ld.first, bf, (c.qt0 + stream) * kTile);
        __builtin_amdgcn_sched_barrier(0);
        ld.mbyte = buffer_load_byte(bf.m, in_range ? static_cast<uint32_t>(key) : kNoRow);
    };

    Ctx cur = decode(0);
    Loads ld;
    if (cur.valid) issue(cur, ld);
    for (int slot = 0; slot < npieces && cur.valid; ++slot) {
        const Ctx nxt = decode(slot + 1);
        const int seq = cur.seq, kb = cur.kb, count = cur.count, qt0 = cur.qt0;
        const Bufs bf = buffers(cur);
        const Buffer qgbuf = make_buffer(dq + static_cast<int64_t>(seq) * s.queries * D, static_cast<uint32_t>(s.queries) * (4u * D));

        const int kt = kb * kBlockTiles + w;
        const int key0 = kt * kTile;
        const int key = key0 + col;
        const bool in_range = key < s.keys;
        int wfirst, wlast; // queries that see some key of this wave's tile
        dkdv_query_range(s, kt, wfirst, wlast);
        const int qlo = window_query_lo(s, key);
        const int qhi = min(window_query_hi(s, key), s.queries - 1);

        const bool visible = in_range && ld.mbyte != 0;
        const uint32_t bits = static_cast<uint32_t>(__ballot(visible));
        static_assert(D * kDsStride <= 2 * kTile * kDsStride, "K block staging region");
        float *const kblock = &sh.ds[0][0][0]; // K block, feature-major: kblock[f * kDsStride + key]
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int ch = i * kWave * WAVES + static_cast<int>(threadIdx.x);
#pragma unroll
            for (int e = 0; e < 4; ++e) kblock[(4 * (ch % CPR) + e) * kDsStride + ch / CPR] = ld.kraw[i][e];
        }
        if (stream < count) store_quarter(ld.first, (qt0 + stream) * kTile, 0);
        if (stream == 0 && lane == 0) sh.kbits[w] = bits;
        __syncthreads();
        float kq[32];
        {
            const uint32_t kk_bits = sh.kbits[lane >> 4];
            const float *src = kblock + (16 * fg + (lane & 15)) * kDsStride + 32 * (lane >> 4);
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const f32x4 x = *reinterpret_cast<const f32x4 *>(src + 4 * u);
#pragma unroll
                for (int e = 0; e < 4; ++e) kq[4 * u + e] = (kk_bits >> (4 * u + e)) & 1u ? x[e] * scale : 0.0f; // masked keys: 0
            }
        }
        const uint32_t any = __builtin_amdgcn_readfirstlane(sh.kbits[0] | sh.kbits[1] | sh.kbits[2] | sh.kbits[3]);
        // Every load of the prologue has landed: without this wait the compiler, merging the loop's entry state, keeps
        // waiting on the whole vector-memory queue (the next tile's prefetch included) inside every step's S and dP chain.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads(); // the staged K block is read: its memory holds dS from the first step on
        float (&kr)[HALF] = ld.kr;
        float (&vr)[HALF] = ld.vr;
        // S·scale·log2e comes straight out of the S MFMAs (K pre-scaled here), whose chain starts from the query's
        // -(m·log2e + log2 l), so P = exp2(chain); the dP chain starts from -δ, so dS = P·chain.
#pragma unroll
        for (int c = 0; c < HALF; ++c) kr[c] *= c2;

        f32x16 acc_k[DT], acc_v[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            acc_k[t] = f32x16{};
            acc_v[t] = f32x16{};
        }
        const int nsteps = any != 0 ? (count + STREAMS - 1) / STREAMS : 0;
        // dQ of a step's tile is formed in the next step, after the barrier that completes the block's dS (dS is
        // double-buffered): stream 0 does it before its own tile, stream 1 after, so the two waves that share a SIMD
        // are in different phases and cover each other's LDS waits.
        auto dq_quadrants = [&](const int i) __attribute__((always_inline)) {
            const int t = i * STREAMS + stream;
            if (i < 0 || t >= count) return;
            const int q0 = (qt0 + t) * kTile;
            const float *dsp = sh.ds[stream][i & 1];
#pragma unroll
            for (int r = 0; r < RH; ++r) {
                const int rh = rh0 + r;
                // Rows 16·rh + lane % 16, keys 32·(lane / 16) + 4u .. +3 of dS per 128-bit read.
                const float *arow = dsp + (16 * rh + (lane & 15)) * kDsStride + 32 * (lane >> 4);
                f32x4 a[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) a[u] = *reinterpret_cast<const f32x4 *>(arow + 4 * u);
                // Two accumulator chains (even and odd 4-key groups), added at the end.
                f32x4 acc{0.0f, 0.0f, 0.0f, 0.0f}, acc1{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int u = 0; u < 8; u += 2) {
#pragma unroll
                    for (int x = 0; x < 4; ++x) {
                        acc = mfma16(a[u][x], kq[4 * u + x], acc);
                        acc1 = mfma16(a[u + 1][x], kq[4 * u + 4 + x], acc1);
                    }
                }
                acc += acc1;
                // Register x of lane l: query q0 + 16 rh + 4 (l / 16) + x, feature 16 fg + l % 16. Rows past the last
                // query fall outside the resource and are dropped.
                const uint32_t voff = (static_cast<uint32_t>(q0 + 16 * rh + 4 * (lane >> 4)) * D + 16u * fg + (lane & 15)) * 4u;
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(acc[x], qgbuf, static_cast<int>(voff + 4u * D * x), 0, 0);
            }
        };
        for (int i = 0; i < nsteps; ++i) {
            const int p = i & 1;
            const int t = i * STREAMS + stream;
            const bool has = t < count;
            const bool has_next = t + STREAMS < count;
            const int q0 = (qt0 + t) * kTile;
            Quarter<D> next;
            if (has_next) load_quarter(next, bf, q0 + STREAMS * kTile);
            if (stream == 0) dq_quadrants(i - 1);
            float *const dsp = sh.ds[stream][p];
            if (has) {
                const bool active = bits != 0 && q0 < wlast && q0 + kTile > wfirst;
                if (active) {
                    const float *qslot = sh.qs[stream][p];
                    const float *uslot = sh.us[stream][p];
                    // Accumulator register j holds query q0 + tile_row(j, h): the chains start from its seeds.
                    f32x16 sc, dp;
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const f32x4 mcs = *reinterpret_cast<const f32x4 *>(&sh.mc[stream][p][8 * u + 4 * h]);
                        const f32x4 dls = *reinterpret_cast<const f32x4 *>(&sh.dl[stream][p][8 * u + 4 * h]);
#pragma unroll
                        for (int x = 0; x < 4; ++x) {
                            sc[4 * u + x] = mcs[x];
                            dp[4 * u + x] = dls[x];
                        }
                    }
                    {
                        // The S and dP chains are independent: interleaved, two accumulator chains are in flight.
                        float qr[HALF], ur[HALF];
                        read_row_layout<D>(qslot, qr);
                        read_row_layout<D>(uslot, ur);
#pragma unroll
                        for (int c = 0; c < HALF; ++c) {
                            sc = mfma(qr[c], kr[c], sc);
                            dp = mfma(ur[c], vr[c], dp);
                        }
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        const float pr = exp2_fast(sc[j]);
                        sc[j] = pr;
                        dp[j] *= pr;
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
#pragma unroll
                    for (int j = 0; j < 16; ++j) dsp[tile_row(j, h) * kDsStride + 32 * w + col] = dp[j];
                    // dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS: A operand of MFMA j is element [tile_row(j, h)][32t + col] of the
                    // tile, four consecutive j per 128-bit read of the feature-major copy.
                    // dVᵀ and dKᵀ interleaved (independent accumulator chains).
                    const float *ut_slot = sh.ut[stream][p];
                    const float *qt_slot = sh.qt[stream][p];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        f32x4 cv[DT], ck[DT];
#pragma unroll
                        for (int t2 = 0; t2 < DT; ++t2) {
                            cv[t2] = *reinterpret_cast<const f32x4 *>(ut_slot + (32 * t2 + col) * kTStride + 8 * u + 4 * h);
                            ck[t2] = *reinterpret_cast<const f32x4 *>(qt_slot + (32 * t2 + col) * kTStride + 8 * u + 4 * h);
                        }
#pragma unroll
                        for (int x = 0; x < 4; ++x) {
#pragma unroll
                            for (int t2 = 0; t2 < DT; ++t2) {
                                acc_v[t2] = mfma(cv[t2][x], sc[4 * u + x], acc_v[t2]);
                                acc_k[t2] = mfma(ck[t2][x], dp[4 * u + x], acc_k[t2]);
                            }
                        }
                    }
                } else {
#pragma unroll
                    for (int j = 0; j < 16; ++j) dsp[tile_row(j, h) * kDsStride + 32 * w + col] = 0.0f;
                }
            }
            if (stream != 0) dq_quadrants(i - 1);
            if (has_next) store_quarter(next, q0 + STREAMS * kTile, p ^ 1);
            __syncthreads(); // this step's dS and the next step's tiles are in LDS
        }
        // dQ of the last tile. This piece's K/V rows are dead: the next piece's loads go out first, and their round trip
        // overlaps this dQ and the epilogue below.
        if (nxt.valid) issue(nxt, ld);
        dq_quadrants(nsteps - 1);
        __syncthreads(); // every wave is done with the dS tiles: the merge below reuses their memory

        if constexpr (STREAMS == 2) {
            // Stream 1 hands its partial dKᵀ and dVᵀ to stream 0 through LDS (fixed order: deterministic).
            float *mine = &sh.ds[1][0][0] + w * (2 * 16 * DT * kWave) + lane;
            if (stream == 1) {
#pragma unroll
                for (int t = 0; t < DT; ++t) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        mine[(16 * t + j) * kWave] = acc_k[t][j];
                        mine[(16 * (DT + t) + j) * kWave] = acc_v[t][j];
                    }
                }
            }
            __syncthreads();
            if (stream == 0) {
#pragma unroll
                for (int t = 0; t < DT; ++t) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        acc_k[t][j] += mine[(16 * t + j) * kWave];
                        acc_v[t][j] += mine[(16 * (DT + t) + j) * kWave];
                    }
                }
            }
        }
        if (stream == 0) {
            if (!cur.partial) {
                // Buffer stores (sequence base in SGPRs, 32-bit offsets; keys past the end fall outside the resource):
                // 64-bit row pointers here were spilled to scratch, and the reload's wait then also waited for the next
                // piece's loads, which are in flight by now.
                const Buffer kg = make_buffer(dk + static_cast<int64_t>(seq) * s.keys * D, static_cast<uint32_t>(s.keys) * (4u * D));
                const Buffer vg = make_buffer(dv + static_cast<int64_t>(seq) * s.keys * D, static_cast<uint32_t>(s.keys) * (4u * D));
                const uint32_t row = static_cast<uint32_t>(key) * (4u * D) + 16u * h;
#pragma unroll
                for (int t = 0; t < DT; ++t) {
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const uint32_t off = row + 128u * t + 32u * u; // features 32t + 8u + 4h .. +3
                        const f32x4 xk{acc_k[t][4 * u] * scale, acc_k[t][4 * u + 1] * scale, acc_k[t][4 * u + 2] * scale,
                                acc_k[t][4 * u + 3] * scale};
                        const f32x4 xv{acc_v[t][4 * u], acc_v[t][4 * u + 1], acc_v[t][4 * u + 2], acc_v[t][4 * u + 3]};
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, xk), kg, static_cast<int>(off), 0, 0);
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, xv), vg, static_cast<int>(off), 0, 0);
                    }
                }
            } else {
                // Part of a split block: add into the zeroed dK/dV. The tile goes through this wave's LDS region
                // transposed (row = key, D + 1 floats apart) so each atomic instruction covers whole 128-byte lines.
                static_assert(kBlockTiles * kTile * (D + 1) <= 2 * kTile * kDsStride, "transpose region");
                float *tr = &sh.ds[0][0][0] + w * (kTile * (D + 1));
                auto add_tile = [&](const f32x16 (&acc)[DT], float *base, const float factor) __attribute__((always_inline)) {
                    const Buffer gbuf = make_buffer(base + static_cast<int64_t>(seq) * s.keys * D, static_cast<uint32_t>(s.keys) * (4u * D));
                    wave_lds_sync();
#pragma unroll
                    for (int t = 0; t < DT; ++t) {
#pragma unroll
                        for (int j = 0; j < 16; ++j) tr[col * (D + 1) + 32 * t + tile_row(j, h)] = acc[t][j] * factor;
                    }
                    wave_lds_sync();
#pragma unroll
                    for (int r = 0; r < kTile * D / kWave; ++r) {
                        const int e = r * kWave + lane;
                        const int row = e / D, f = e - row * D;
                        const uint32_t voff = (static_cast<uint32_t>(key0 + row) * D + static_cast<uint32_t>(f)) * 4u;
                        __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(tr[row * (D + 1) + f], gbuf, static_cast<int>(voff), 0, 0);
                    }
                };
                if (bits != 0) {
                    add_tile(acc_k, dk, scale);
                    add_tile(acc_v, dv, 1.0f);
                }
            }
        }
        __syncthreads(); // the next piece reuses the LDS tiles
        cur = nxt;
    }
}

// δ = Σ dO·O per query row, dQ = 0, and dK = dV = 0 on the key blocks that the plan splits (those that see more than
// `split_above` query tiles; their pieces add into dK/dV). Each thread takes one 16-byte group of a row: the D/4 lanes
// of a query row form δ with group_dot and the pairwise tree (shuffles at distance 1, 2, 4, ..., the same order as
// the deterministic backward's lane-local tree, so δ is bit-identical to that path's), and each thread clears its group
// of the dQ row and of the dK/dV row. Spreading δ over D/4 lanes per row keeps the loads of every workgroup in flight
// at once (two lanes per row left 576 of the 768 workgroups at 24 x 1024 with nothing to load).
template<int D>
__global__ __launch_bounds__(256) void attention_fused_prepass_kernel(const Tensor o, const Tensor du, float *__restrict__ delta,
        float *__restrict__ dq, float *__restrict__ dk, float *__restrict__ dv, const Shape s, const int64_t qrows,
        const int64_t krows, const int split_above) {
    constexpr int G = D / 4; // 16-byte groups per row: a power of two dividing the wave
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const f32x4 zero{0.0f, 0.0f, 0.0f, 0.0f};
    if (t < qrows * G) { // the G lanes of a row are all inside or all outside
        const int64_t r = t / G;
        const int g = static_cast<int>(t & (G - 1));
        // Sequence and query of the row; 32-bit arithmetic whenever the rows fit (always, short of 2^32 rows).
        int64_t seq;
        int query;
        if (qrows <= 0xffffffffLL) {
            const uint32_t r32 = static_cast<uint32_t>(r), nq = static_cast<uint32_t>(s.queries);
            seq = r32 / nq;
            query = static_cast<int>(r32 - static_cast<uint32_t>(seq) * nq);
        } else {
            seq = r / s.queries;
            query = static_cast<int>(r - seq * s.queries);
        }
        const int b = static_cast<int>(seq / s.heads), head = static_cast<int>(seq - static_cast<int64_t>(b) * s.heads);
        const float *orow = o.data + static_cast<int64_t>(b) * o.sb + static_cast<int64_t>(head) * o.sh + static_cast<int64_t>(query) * o.st + 4 * g;
        const float *urow = du.data + static_cast<int64_t>(b) * du.sb + static_cast<int64_t>(head) * du.sh + static_cast<int64_t>(query) * du.st + 4 * g;
        const f32x4 x = *reinterpret_cast<const f32x4 *>(urow);
        const f32x4 y = *reinterpret_cast<const f32x4 *>(orow);
        const float xs[4] = {x[0], x[1], x[2], x[3]}, ys[4] = {y[0], y[1], y[2], y[3]};
        float part = group_dot(xs, ys);
#pragma unroll
        for (int m = 1; m < G; m <<= 1) part += __shfl_xor(part, m);
        if (g == 0) delta[r] = part;
        reinterpret_cast<f32x4 *>(dq)[t] = zero;
    }
    if (t < krows * G) {
        const int64_t r = t / G;
        // Key index within its sequence; 32-bit arithmetic whenever the key rows fit (always, short of 2^32 rows).
        const int key = static_cast<int>(krows <= 0xffffffffLL ? static_cast<uint32_t>(r) % static_cast<uint32_t>(s.keys) : r % s.keys);
        int first;
        if (block_query_tiles(s.queries, s.keys, s.radius, s.causal, key / kBlockKeys, first) > split_above) {
            reinterpret_cast<f32x4 *>(dk)[t] = zero;
            reinterpret_cast<f32x4 *>(dv)[t] = zero;
        }
    }
}

Tensor tensor(const float *p, const rocmkernels_strides &s) { return Tensor{p, s.batch, s.head, s.token}; }

// The launch's piece table, kept per host thread for the last shape and CU count.
struct CachedPlan {
    Shape s{};
    int cus = -1;
    bool ok = false;
    BlockPlan plan;
    PieceList<kMaxPieces> table;
};

const CachedPlan &cached_plan(const Shape &s, const int cus) {
    thread_local CachedPlan cache;
    const bool same = cache.cus == cus && cache.s.batch == s.batch && cache.s.heads == s.heads && cache.s.queries == s.queries &&
            cache.s.keys == s.keys && cache.s.radius == s.radius && cache.s.causal == s.causal;
    if (!same) {
        const int nblocks = (s.keys + kBlockKeys - 1) / kBlockKeys;
        cache.ok = plan_blocks(static_cast<long long>(s.batch) * s.heads, nblocks, cus, 3, [&](const int kb) {
            int first;
            return block_query_tiles(s.queries, s.keys, s.radius, s.causal, kb, first);
        }, cache.plan, cache.table.entry);
        cache.s = s;
        cache.cus = cus;
    }
    return cache;
}

template<int D>
hipError_t launch(const BackwardArgs &a, const int cus, hipStream_t stream) {
    constexpr int STREAMS = D == 32 ? 2 : 1;
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const int nblocks = (a.keys + kBlockKeys - 1) / kBlockKeys;
    const long long seqs = static_cast<long long>(a.batch) * a.heads;
    const CachedPlan &cp = cached_plan(shape, cus);
    const bool planned = cp.ok;

    const int64_t qrows = seqs * a.queries, krows = seqs * a.keys;
    const int64_t rows = qrows > krows ? qrows : krows;
    // Blocks above the plan's piece length are split (no block is without a plan).
    const int split_above = planned && cp.plan.partial ? cp.plan.chunk : 0x7fffffff;
    const int64_t threads_pre = rows * (D / 4);
    hipLaunchKernelGGL((attention_fused_prepass_kernel<D>), dim3(static_cast<unsigned>((threads_pre + 255) / 256)), dim3(256), 0, stream,
            tensor(a.output, a.os), tensor(a.upstream, a.us), a.delta, a.gradient_q, a.gradient_k, a.gradient_v, shape, qrows, krows,
            split_above);
    hipError_t error = hipGetLastError();
    if (error != hipSuccess) return error;

    const unsigned threads = kWave * kBlockTiles * STREAMS;
    if (planned) {
        hipLaunchKernelGGL((attention_fused_backward_kernel<D, STREAMS, true>), dim3(static_cast<unsigned>(cp.plan.bins)), dim3(threads),
                0, stream, tensor(a.q, a.qs), tensor(a.k, a.ks), tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), a.lse,
                tensor(a.upstream, a.us), a.delta, a.gradient_q, a.gradient_k, a.gradient_v, shape, nblocks, cp.plan.slots, cp.table,
                scale);
    } else {
        const PieceList<1> none{};
        hipLaunchKernelGGL((attention_fused_backward_kernel<D, STREAMS, false>), dim3(static_cast<unsigned>(seqs * nblocks)), dim3(threads),
                0, stream, tensor(a.q, a.qs), tensor(a.k, a.ks), tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), a.lse,
                tensor(a.upstream, a.us), a.delta, a.gradient_q, a.gradient_k, a.gradient_v, shape, nblocks, 1, none, scale);
    }
    return hipGetLastError();
}

} // namespace

hipError_t launch_fused_backward(const int D, const BackwardArgs &a, const int cus, hipStream_t stream) {
    return D == 32 ? launch<32>(a, cus, stream) : launch<64>(a, cus, stream);
}

hipError_t launch_backward_prepass(const int D, const BackwardArgs &a, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const long long seqs = static_cast<long long>(a.batch) * a.heads;
    const int64_t qrows = seqs * a.queries;
    const int64_t threads = qrows * (D / 4); // dQ rows and delta; dK/dV are left alone
    const unsigned grid = static_cast<unsigned>((threads + 255) / 256);
    if (D == 32) {
        hipLaunchKernelGGL((attention_fused_prepass_kernel<32>), dim3(grid), dim3(256), 0, stream, tensor(a.output, a.os),
                tensor(a.upstream, a.us), a.delta, a.gradient_q, a.gradient_k, a.gradient_v, shape, qrows, int64_t{0}, 0x7fffffff);
    } else {
        hipLaunchKernelGGL((attention_fused_prepass_kernel<64>), dim3(grid), dim3(256), 0, stream, tensor(a.output, a.os),
                tensor(a.upstream, a.us), a.delta, a.gradient_q, a.gradient_k, a.gradient_v, shape, qrows, int64_t{0}, 0x7fffffff);
    }
    return hipGetLastError();
}

} // namespace rk
