// FP32 attention backward for gfx950 (MI355X), head width 32 or 64.
//
// Replaces the reference's backward kernels: attention_query<true> and attention_key_value
// (Attention.hip:32-169), attention_single_query_kv (Attention.hip:171-189), the tiled/tuned/profile instances
// (AttentionTile32.h:12-311) and attention64_query<true> / attention64_key_value (Attention64.hip:34-191).
// Gradients follow the reference's maths: P = exp(s - max)/sum from the forward's lse, δ = Σ dO·O,
// dS = P(dO·v - δ), dQ = Σ_k dS·k/√D, dK = Σ_q dS·q/√D, dV = Σ_q P·dO.
//
// Two deterministic kernels, no atomics and no workspace beyond the caller's delta buffer:
//   1. attention_dq_kernel (query-major): computes δ for its 32 queries and writes it, then streams the key
//      tiles: Sᵀ = K·Qᵀ, dPᵀ = V·dOᵀ, dSᵀ = Pᵀ(dPᵀ - δ), dQᵀ += Kᵀ·dSᵀ. The dSᵀ accumulator registers are the
//      B operand of the dQᵀ MFMAs directly.
//   2. attention_dkdv_kernel (key-major): for its 32 keys streams the query tiles: S = Q·Kᵀ, dP = dO·Vᵀ,
//      P and dS from lse/δ, dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS, again feeding accumulators straight into MFMAs.
// SPLIT waves share one 32-row item and split its streamed tiles; they sum their partial gradients through LDS.
// Kernel 2 reads the δ that kernel 1 wrote; they are ordered by the stream, as in the reference
// (Attention.hip:211-221). Streamed operands are read through buffer resources (see attention_device.hpp), and
// each tile's row-layout operands are loaded one tile ahead, after the current tile's MFMAs are issued.
//
// Per-key-tile fused variant (the fused flag's choice for inputs without 128-bit access; with it the key-block kernels
// of attention_backward_fused.hip and attention_backward_band.hip run): kernel 1 only computes δ and zeroes dQ;
// kernel 2 also forms dQ = dS·K/√D for each tile it visits and adds it into dQ with FP32 atomics. That is 5
// GEMMs per visited tile instead of 7 (kernel 1 no longer recomputes S and dP), at the price of a dQ whose
// low bits depend on the order in which the atomics land. run<D, VEC> at the end of this file picks the path.
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

enum DqMode { kDqAndDelta = 0, kDeltaOnly = 1, kDqFromDelta = 2, kDeltaZeroDq = 3 };

// NI = 0: items in dispatch order (work_item); NI > 0: persistent grid of NI * SPLIT-wave workgroups taking the NI
// items of their bin from the launch's item table (planned_item), as in the forward.
template<int D, int MODE, bool VEC, int SPLIT, int NI>
__global__ __launch_bounds__(kWave * (NI > 0 ? NI * SPLIT : kWaves)) void attention_dq_kernel(const Tensor q, const Tensor k,
        const Tensor v, const uint8_t *__restrict__ mask, const Tensor o, const float *__restrict__ lse, const Tensor du,
        float *__restrict__ dq, float *__restrict__ delta, const Shape s, const ItemTable<NI> items, const float scale) {
    constexpr int HALF = D / 2;
    constexpr int DT = D / 32;

    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 31;
    const int h = lane >> 5;

    const int qtiles = (s.queries + kTile - 1) / kTile;
    const WorkItem w = [&] {
        if constexpr (NI > 0) return planned_item<SPLIT, NI>(s, items);
        else return work_item<SPLIT>(s, qtiles);
    }();
    const int qt = s.causal ? qtiles - 1 - w.rank : w.rank;
    const int q0 = qt * kTile;
    const int query = q0 + col;
    const bool qvalid = w.valid && query < s.queries;
    const int64_t row = static_cast<int64_t>(w.seq) * s.queries + query;
    const float c2 = scale * kLog2e;

    int first, last;
    const int ntiles = w.valid ? forward_key_range(s, qt, first, last) : 0;
    const int mine = ntiles > w.lead ? (ntiles - w.lead + SPLIT - 1) / SPLIT : 0;
    const Buffer kbuf = make_buffer(sequence(k, w.b, w.head), sequence_bytes(s.keys, k.st, D));
    const Buffer vbuf = make_buffer(sequence(v, w.b, w.head), sequence_bytes(s.keys, v.st, D));
    const Buffer mbuf = make_buffer(mask + static_cast<int64_t>(w.b) * s.keys, static_cast<uint32_t>(s.keys));
    const uint32_t kstep = 4u * k.st;
    const uint32_t vstep = 4u * v.st;

    // With 128-bit access each K and V tile is loaded a whole line per request and staged through this wave's LDS slots,
    // which give the row layouts (Sᵀ, dPᵀ operands) and K's column layout (dQᵀ operand). The first tile's loads go out
    // before the query row's, so a wave waits for memory once before its first tile (issued after delta, they arrived
    // 3-9 us after launch at the 24 x 1024 causal shape). Reading K's columns straight from memory instead took 49
    // vector-memory loads per tile at d = 64, more than a wave can keep outstanding (63) with the next tile in flight:
    // staging made the d = 64 backward 9-15% faster (configs 4 and 5) and d = 32 up to 6% on large grids.
    constexpr bool STAGE = VEC && (MODE == kDqAndDelta || MODE == kDqFromDelta);
    struct Raw {
        RowTile<D> k, v;
        int mask;
    };
    auto load_raw = [&](Raw &r, const int key0) __attribute__((always_inline)) {
        r.mask = buffer_load_byte(mbuf, static_cast<uint32_t>(key0 + col)); // keys >= s.keys read 0: masked
        load_row_tile<D>(r.k, kbuf, kstep, static_cast<uint32_t>(key0) * kstep);
        load_row_tile<D>(r.v, vbuf, vstep, static_cast<uint32_t>(key0) * vstep);
    };
    Raw raw;
    if constexpr (STAGE) {
        if (mine > 0) load_raw(raw, first + w.lead * kTile);
    }

    const Buffer ubuf = make_buffer(sequence(du, w.b, w.head), sequence_bytes(s.queries, du.st, D));
    const uint32_t qoff = static_cast<uint32_t>(query) * (4u * du.st) + 4u * h * HALF;
    float dor[HALF];
    buffer_load_span<VEC>(dor, ubuf, qvalid ? qoff : kNoRow);
    // The query row and its statistics are requested before delta needs dO·O, so both round trips overlap.
    constexpr bool NEEDS_Q = MODE == kDqAndDelta || MODE == kDqFromDelta;
    const Buffer qbuf = make_buffer(sequence(q, w.b, w.head), sequence_bytes(s.queries, q.st, D));
    float qr[HALF];
    float m = -INFINITY, l = 0.0f;
    if constexpr (NEEDS_Q) {
        buffer_load_span<VEC>(qr, qbuf, qvalid ? static_cast<uint32_t>(query) * (4u * q.st) + 4u * h * HALF : kNoRow);
        if (qvalid) {
            m = lse[2 * row];
            l = lse[2 * row + 1];
        }
    }

    float dlt;
    if constexpr (MODE == kDqFromDelta) {
        dlt = qvalid ? delta[row] : 0.0f;
    } else {
        const Buffer obuf = make_buffer(sequence(o, w.b, w.head), sequence_bytes(s.queries, o.st, D));
        float orow[HALF];
        buffer_load_span<VEC>(orow, obuf, qvalid ? static_cast<uint32_t>(query) * (4u * o.st) + 4u * h * HALF : kNoRow);
        float part[HALF / 4];
#pragma unroll
        for (int i = 0; i < HALF / 4; ++i) part[i] = group_dot(dor + 4 * i, orow + 4 * i);
        dlt = halves_sum(group_tree(part));
        if (w.sub == 0 && h == 0 && qvalid) delta[row] = dlt;
        if constexpr (MODE == kDeltaZeroDq) {
            // The fused dK/dV/dQ kernel accumulates into dQ: start every row of this tile at zero.
            if (qvalid) {
                float *dst = dq + row * D + h * HALF;
#pragma unroll
                for (int c = 0; c < HALF; c += 4) {
                    if constexpr (VEC) {
                        *reinterpret_cast<f32x4 *>(dst + c) = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                    } else {
                        dst[c] = dst[c + 1] = dst[c + 2] = dst[c + 3] = 0.0f;
                    }
                }
            }
            return;
        }
        if constexpr (MODE == kDeltaOnly) return;
    }

    // P = exp(s - m) / l = exp2(s·c2 - (m·log2e + log2 l)): the normaliser folds into the exponent offset.
    // A row without visible keys gets offset +inf, so exp2(x - inf) = 0. At D = 32 the offset seeds every tile's
    // S chain and Q is pre-scaled by c2, so P = exp2(chain) (an FMA per element saved; 16 registers that the D = 64
    // kernel has no room for).
    const float mc = m != -INFINITY ? fmaf(m, kLog2e, __log2f(l)) : INFINITY;
    constexpr bool SEED = D == 32;
    f32x16 seed{};
    if constexpr (SEED) {
#pragma unroll
        for (int j = 0; j < 16; ++j) seed[j] = -mc;
#pragma unroll
        for (int c = 0; c < HALF; ++c) qr[c] *= c2;
    }

    const int wlo = window_lo(s, query);
    const int whi = window_hi(s, query);

    f32x16 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f32x16{};

    // K and V rows (Sᵀ and dPᵀ A operands) and the mask byte, one tile ahead.
    auto load_rows = [&](float (&kr)[HALF], float (&vr)[HALF], int &mb, const int key0) __attribute__((always_inline)) {
        const uint32_t key = static_cast<uint32_t>(key0 + col);
        mb = buffer_load_byte(mbuf, key);
        buffer_load_span<VEC>(kr, kbuf, key * kstep + 4u * h * HALF);
        buffer_load_span<VEC>(vr, vbuf, key * vstep + 4u * h * HALF);
    };

    // One key tile; the next tile's rows are loaded into the other register set after the MFMAs are issued.
    // key0 >= last marks the padding step of a wave with an odd number of tiles.
    auto step = [&](const float (&kr)[HALF], const float (&vr)[HALF], const int mb, const int key0, float (&kn)[HALF],
                        float (&vn)[HALF], int &mn, const int next_key0) __attribute__((always_inline)) {
        const uint32_t bits = key0 < last ? static_cast<uint32_t>(__ballot(mb != 0)) : 0u;
        if (bits == 0) {
            load_rows(kn, vn, mn, next_key0);
            return;
        }
        // K in column layout (dQᵀ A operand): row key0 + tile_row(j, h), feature 32t + col.
        float kc[DT][16];
        const uint32_t klane = static_cast<uint32_t>(key0 + 4 * h) * kstep + 4u * col;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
#pragma unroll
            for (int t = 0; t < DT; ++t) kc[t][j] = buffer_load(kbuf, klane + 128u * t, static_cast<uint32_t>(8 * (j >> 2) + (j & 3)) * kstep);
        }

        f32x16 sc = seed, dp{};
#pragma unroll
        for (int c = 0; c < HALF; ++c) {
            sc = mfma(kr[c], qr[c], sc);
            dp = mfma(vr[c], dor[c], dp);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_rows(kn, vn, mn, next_key0);
        __builtin_amdgcn_sched_barrier(0);

#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const float p = exp2_fast(SEED ? sc[j] : fmaf(sc[j], c2, -mc));
            sc[j] = p * (dp[j] - dlt);
        }
        if (bits != 0xffffffffu || !tile_in_window(s, q0, key0)) {
            const uint32_t visible = (bits & bit_range(wlo - key0, whi - key0)) >> (4 * h);
#pragma unroll
            for (int j = 0; j < 16; ++j) sc[j] = (visible >> (8 * (j >> 2) + (j & 3))) & 1u ? sc[j] : 0.0f;
            if (bits != 0xffffffffu) {
                const uint32_t kept = bits >> (4 * h); // masked keys contribute nothing, whatever K holds there
#pragma unroll
                for (int j = 0; j < 16; ++j) {
#pragma unroll
                    for (int t = 0; t < DT; ++t) kc[t][j] = (kept >> (8 * (j >> 2) + (j & 3))) & 1u ? kc[t][j] : 0.0f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
#pragma unroll
            for (int t = 0; t < DT; ++t) acc[t] = mfma(kc[t][j], sc[j], acc[t]);
        }
    };

    constexpr int WG = NI > 0 ? NI * SPLIT : kWaves;
    if constexpr (STAGE) {
        __shared__ __align__(16) float slots[WG * 2 * kSlotFloats<D>];
        float *const kslot = slots + 2 * static_cast<int>(threadIdx.x / kWave) * kSlotFloats<D>;
        float *const vslot = kslot + kSlotFloats<D>;
        // One key tile with some visible key (bits): stage r, then load the next tile into r while this one computes.
        auto stage_step = [&](Raw &r, const int key0, const int next_key0, const uint32_t bits) __attribute__((always_inline)) {
            write_row_tile<D>(kslot, r.k);
            write_row_tile<D>(vslot, r.v);
            wave_lds_sync();
            load_raw(r, next_key0);

            f32x16 sc = seed, dp{};
            {
                float kr[HALF];
                read_row_layout<D>(kslot, kr);
#pragma unroll
                for (int c = 0; c < HALF; ++c) sc = mfma(kr[c], qr[c], sc);
            }
            __builtin_amdgcn_sched_barrier(0);
            {
                float vr[HALF];
                read_row_layout<D>(vslot, vr);
#pragma unroll
                for (int c = 0; c < HALF; ++c) dp = mfma(vr[c], dor[c], dp);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float p = exp2_fast(SEED ? sc[j] : fmaf(sc[j], c2, -mc));
                sc[j] = p * (dp[j] - dlt);
            }
            const bool boundary = bits != 0xffffffffu || !tile_in_window(s, q0, key0);
            if (boundary) {
                const uint32_t visible = (bits & bit_range(wlo - key0, whi - key0)) >> (4 * h);
#pragma unroll
                for (int j = 0; j < 16; ++j) sc[j] = (visible >> (8 * (j >> 2) + (j & 3))) & 1u ? sc[j] : 0.0f;
            }
            // dQᵀ += Kᵀ·dSᵀ with K's column layout, eight rows at a time; masked keys contribute nothing,
            // whatever K holds there.
            const uint32_t kept = bits >> (4 * h);
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                __builtin_amdgcn_sched_barrier(0);
                float c[DT][8];
                if (half == 0) read_column_layout<D, 0, 8>(kslot, c);
                else read_column_layout<D, 8, 8>(kslot, c);
                if (bits != 0xffffffffu) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int jj = 8 * half + j;
#pragma unroll
                        for (int t = 0; t < DT; ++t) c[t][j] = (kept >> (8 * (jj >> 2) + (jj & 3))) & 1u ? c[t][j] : 0.0f;
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
#pragma unroll
                    for (int t = 0; t < DT; ++t) acc[t] = mfma(c[t][j], sc[8 * half + j], acc[t]);
                }
            }
        };
        // Fully masked tiles only advance the loads. At D = 64 they do so in a loop of their own: the dQ accumulators
        // are then updated on one path only and stay in place, where a skip branch joining the compute path cost a
        // copy of all 32 accumulator registers there and back per tile (configs 4 and 5: backward 1% faster). At
        // D = 32 the same form removed 16 copies per tile yet measured 1.5% slower (27.0 -> 27.4 us at 24 x 1024,
        // about four tiles per wave), so the skip stays a branch there.
        if constexpr (D == 64) {
            for (int i = 0; i < mine; ++i) {
                int key0 = first + (w.lead + i * SPLIT) * kTile;
                uint32_t bits = key0 < last ? static_cast<uint32_t>(__ballot(raw.mask != 0)) : 0u;
                while (bits == 0 && i < mine) {
                    load_raw(raw, key0 + SPLIT * kTile);
                    if (++i == mine) break;
                    key0 += SPLIT * kTile;
                    bits = key0 < last ? static_cast<uint32_t>(__ballot(raw.mask != 0)) : 0u;
                }
                if (bits == 0) break;
                stage_step(raw, key0, key0 + SPLIT * kTile, bits);
            }
        } else {
            for (int i = 0; i < mine; ++i) {
                const int key0 = first + (w.lead + i * SPLIT) * kTile;
                const uint32_t bits = key0 < last ? static_cast<uint32_t>(__ballot(raw.mask != 0)) : 0u;
                if (bits == 0) {
                    load_raw(raw, key0 + SPLIT * kTile);
                    continue;
                }
                stage_step(raw, key0, key0 + SPLIT * kTile, bits);
            }
        }
        // The slots are free once every wave has left its loop (split_sum_into's first barrier).
        static_assert(WG * 16 * DT * kWave <= WG * 2 * kSlotFloats<D>);
        split_sum_into<SPLIT, DT, WG>(acc, w.sub, slots);
    } else {
        // Tiles lead, lead + SPLIT, ...; the count is rounded up to even so the loop body is two straight-line steps.
        float ka[HALF], va[HALF], kb[HALF], vb[HALF];
        int ma = 0, mb = 0;
        if (mine > 0) load_rows(ka, va, ma, first + w.lead * kTile);
        for (int i = 0; i < mine; i += 2) {
            const int key0 = first + (w.lead + i * SPLIT) * kTile;
            step(ka, va, ma, key0, kb, vb, mb, key0 + SPLIT * kTile);
            step(kb, vb, mb, key0 + SPLIT * kTile, ka, va, ma, key0 + 2 * SPLIT * kTile);
        }
        split_sum<SPLIT, DT, WG>(acc, w.sub);
    }
    if (w.sub != 0 || !qvalid) return;
    float *dst = dq + row * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) store_tile_row<VEC>(dst + 32 * t, acc[t], scale, h);
}

// dK and dV contributions (and, FUSED, dQ, added with atomics) of key tile kt of sequence (b, head) over its query
// tiles start, start + stride, ... (at most `limit` of them), accumulated into acc_k (dKᵀ without the 1/√D factor)
// and acc_v (dVᵀ): accumulator register j of slice t is feature 32t + tile_row(j, h), lane%32 is key kt*32 + lane%32.
// A key tile at or past the last key contributes nothing. WAVES = the workgroup's waves (one LDS slice each).
// STAGE (128-bit access only): each Q and dO tile is loaded a whole line per request and staged through this wave's
// LDS slots, from which the wave reads both the row layout (S and dP operands) and the column layout (dK and dV
// operands); one register set of raw rows is carried a tile ahead. That needs about 70 fewer registers than the row
// spans plus column loads (two sets of rows in flight), enough for three waves per SIMD at D = 32, and 19 instead of 83
// vector-memory loads per tile at D = 64 (a wave keeps at most 63 outstanding).
// LDS slots of the staged dK/dV path: a Q tile and a dO tile per wave.
template<int D, int WAVES>
__device__ __forceinline__ float *dkdv_slots() {
    __shared__ __align__(16) float slots[WAVES * 2 * kSlotFloats<D>];
    return slots;
}

template<int D, bool VEC, bool FUSED, int WAVES, bool STAGE = false>
__device__ __forceinline__ void dkdv_tiles(const Tensor &q, const Tensor &k, const Tensor &v, const uint8_t *__restrict__ mask,
        const float *__restrict__ lse, const Tensor &du, const float *__restrict__ delta, float *__restrict__ dq, const Shape &s,
        const float scale, const int b, const int head, const int kt, const int start, const int stride, const int limit,
        f32x16 (&acc_k)[D / 32], f32x16 (&acc_v)[D / 32]) {
    constexpr int HALF = D / 2;
    constexpr int DT = D / 32;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform: keeps tile bookkeeping scalar
    const int col = lane & 31;
    const int h = lane >> 5;

    const int seq = b * s.heads + head;
    const int key0 = kt * kTile; // under a causal mask the first key tiles see the most queries
    const int key = key0 + col;
    const bool in_range = key < s.keys;
    const Buffer mbuf = make_buffer(mask + static_cast<int64_t>(b) * s.keys, static_cast<uint32_t>(s.keys));
    const bool visible = in_range && buffer_load_byte(mbuf, static_cast<uint32_t>(key)) != 0;
    const uint32_t bits = static_cast<uint32_t>(__ballot(visible));
    const float c2 = scale * kLog2e;

    const Buffer kbuf = make_buffer(sequence(k, b, head), sequence_bytes(s.keys, k.st, D));
    const Buffer vbuf = make_buffer(sequence(v, b, head), sequence_bytes(s.keys, v.st, D));
    float kr[HALF], vr[HALF];
    buffer_load_span<VEC>(kr, kbuf, in_range ? static_cast<uint32_t>(key) * (4u * k.st) + 4u * h * HALF : kNoRow);
    buffer_load_span<VEC>(vr, vbuf, in_range ? static_cast<uint32_t>(key) * (4u * v.st) + 4u * h * HALF : kNoRow);

    int first, last;
    const int range = dkdv_query_range(s, kt, first, last);
    const int ntiles = bits != 0 ? range : 0;
    // Queries that see this lane's key: [qlo, qhi] (also capped at the last query of the range).
    const int qlo = window_query_lo(s, key);
    const int qhi = min(window_query_hi(s, key), last - 1);

    const Buffer qbuf = make_buffer(sequence(q, b, head), sequence_bytes(s.queries, q.st, D));
    const Buffer ubuf = make_buffer(sequence(du, b, head), sequence_bytes(s.queries, du.st, D));
    const Buffer lbuf = make_buffer(lse + static_cast<int64_t>(seq) * s.queries * 2, static_cast<uint32_t>(s.queries) * 8u);
    const Buffer dbuf = make_buffer(delta + static_cast<int64_t>(seq) * s.queries, static_cast<uint32_t>(s.queries) * 4u);
    const uint32_t qstep = 4u * q.st;
    const uint32_t ustep = 4u * du.st;

    // Staged path: raw Q rows and softmax statistics of one query tile, one tile ahead. The first tile's loads go
    // out before the key tile's mask is known (a fully masked tile ignores them), so they overlap the K/V loads.
    struct Raw {
        RowTile<D> q;
        float m, l, d;
    };
    auto load_raw = [&](Raw &r, const int q0) __attribute__((always_inline)) {
        load_row_tile<D>(r.q, qbuf, qstep, static_cast<uint32_t>(q0) * qstep);
        const uint32_t qq = static_cast<uint32_t>(q0 + col);
        r.m = buffer_load(lbuf, qq * 8u, 0);
        r.l = buffer_load(lbuf, qq * 8u + 4u, 0);
        r.d = buffer_load(dbuf, qq * 4u, 0);
    };
    Raw raw;
    if constexpr (STAGE) {
        if (range > start && limit > 0) load_raw(raw, first + start * kTile);
    }
    // At D = 32, S·scale·log2e comes straight out of the S MFMAs: K is pre-scaled here, and every tile's S chain starts
    // from -(m·log2e + log2 l) of its queries (-inf for queries without keys), so P = exp2(chain); the dP chain starts
    // from -δ, so dS = P·chain. That saves an FMA and a subtraction per element and tile, and 9 registers. At D = 64
    // the kernels with two waves per item ran 4-9% slower seeded (the schedule at 256 registers waits on every LDS
    // read of the dO rows), so they subtract as before.
    constexpr bool SEED = D == 32;
    if constexpr (SEED) {
#pragma unroll
        for (int c = 0; c < HALF; ++c) kr[c] *= c2;
    }

    __shared__ __align__(16) float stats[WAVES][2][kTile]; // exp2 offset (seeded: its negation) and δ (seeded: -δ)
    // S and dP chain seeds of this wave's staged tile, in accumulator order (register j is query q0 + tile_row(j, h)).
    auto seeds = [&](f32x16 &sc, f32x16 &dp) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(&stats[wave][0][8 * u + 4 * h]);
            const f32x4 d = *reinterpret_cast<const f32x4 *>(&stats[wave][1][8 * u + 4 * h]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sc[4 * u + i] = a[i];
                dp[4 * u + i] = d[i];
            }
        }
    };
    // P and dS of a tile from the S and dP chains: four rows' constants at a time when not seeded (all sixteen at
    // once would hold 24 more registers).
    auto softmax = [&](f32x16 &sc, f32x16 &dp) __attribute__((always_inline)) {
        if constexpr (SEED) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float p = exp2_fast(sc[j]);
                sc[j] = p;
                dp[j] *= p;
            }
        } else {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                __builtin_amdgcn_sched_barrier(0);
                const f32x4 mcs = *reinterpret_cast<const f32x4 *>(&stats[wave][0][8 * u + 4 * h]);
                const f32x4 dls = *reinterpret_cast<const f32x4 *>(&stats[wave][1][8 * u + 4 * h]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int j = 4 * u + i;
                    const float p = exp2_fast(fmaf(sc[j], c2, -mcs[i]));
                    sc[j] = p;
                    dp[j] = p * (dp[j] - dls[i]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    // Fused dQ: K of this item in column layout (the B operand of dQ = dS·K, row key0 + tile_row(j, h), feature
    // 32t + col), pre-scaled by 1/√D and zero for masked keys, whatever K holds there. dS goes through the
    // wave's LDS slice (row stride kTile + 4 keeps both the row writes and the 128-bit column reads free of
    // bank conflicts), and dQ rows are added with buffer atomics: rows past the last query fall outside the
    // resource and are dropped by the hardware.
    constexpr int KC = FUSED ? DT : 0;
    float kq[KC > 0 ? KC : 1][16];
    __shared__ __align__(16) float dsl[FUSED ? WAVES : 1][kTile][kTile + 4];
    const Buffer qgbuf = make_buffer(dq + static_cast<int64_t>(seq) * s.queries * D, FUSED ? static_cast<uint32_t>(s.queries) * (4u * D) : 0u);
    if constexpr (FUSED) {
        const uint32_t klane = static_cast<uint32_t>(key0 + 4 * h) * (4u * k.st) + 4u * col;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const bool kept = (bits >> tile_row(j, h)) & 1u;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                const float x = buffer_load(kbuf, klane + 128u * t, static_cast<uint32_t>(8 * (j >> 2) + (j & 3)) * (4u * k.st));
                kq[t][j] = kept ? x * scale : 0.0f;
            }
        }
    }

#pragma unroll
    for (int t = 0; t < DT; ++t) {
        acc_k[t] = f32x16{};
        acc_v[t] = f32x16{};
    }

    // Q and dO rows (S and dP A operands) and the raw softmax statistics of query q0 + col, one tile ahead.
    struct Rows {
        float qr[HALF], ur[HALF];
        float m, l, d;
    };
    auto load_rows = [&](Rows &r, const int q0) __attribute__((always_inline)) {
        const uint32_t qq = static_cast<uint32_t>(q0 + col);
        buffer_load_span<VEC>(r.qr, qbuf, qq * qstep + 4u * h * HALF);
        buffer_load_span<VEC>(r.ur, ubuf, qq * ustep + 4u * h * HALF);
        r.m = buffer_load(lbuf, qq * 8u, 0);
        r.l = buffer_load(lbuf, qq * 8u + 4u, 0);
        r.d = buffer_load(dbuf, qq * 4u, 0);
    };

    // One query tile; the next tile's rows are loaded into the other set after the MFMAs are issued. An inactive
    // step (the padding step of a wave with an odd number of tiles) only issues the next loads.
    auto step = [&](const Rows &r, const int q0, const bool active, Rows &next, const int next_q0) __attribute__((always_inline)) {
        if (!active) {
            load_rows(next, next_q0);
            return;
        }
        // Per-query constants for the 32 queries of the tile, staged in this wave's LDS slice and read back in
        // accumulator order (lane needs queries q0 + tile_row(j, h)). Queries past the end get exp2(-inf) = 0.
        wave_lds_sync();
        if (h == 0) {
            const bool ok = q0 + col < last && r.m != -INFINITY;
            stats[wave][0][col] = SEED ? (ok ? -fmaf(r.m, kLog2e, __log2f(r.l)) : -INFINITY) : (ok ? fmaf(r.m, kLog2e, __log2f(r.l)) : INFINITY);
            stats[wave][1][col] = SEED ? -r.d : r.d;
        }
        wave_lds_sync();

        // Q and dO in column layout (dKᵀ and dVᵀ A operands): row q0 + tile_row(j, h), feature 32t + col.
        float qc[DT][16], uc[DT][16];
        const uint32_t qlane = static_cast<uint32_t>(q0 + 4 * h) * qstep + 4u * col;
        const uint32_t ulane = static_cast<uint32_t>(q0 + 4 * h) * ustep + 4u * col;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t r8 = static_cast<uint32_t>(8 * (j >> 2) + (j & 3));
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                uc[t][j] = buffer_load(ubuf, ulane + 128u * t, r8 * ustep);
                qc[t][j] = buffer_load(qbuf, qlane + 128u * t, r8 * qstep);
            }
        }

        f32x16 sc{}, dp{};
        if constexpr (SEED) seeds(sc, dp);
#pragma unroll
        for (int c = 0; c < HALF; ++c) {
            sc = mfma(r.qr[c], kr[c], sc);
            dp = mfma(r.ur[c], vr[c], dp);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_rows(next, next_q0);
        __builtin_amdgcn_sched_barrier(0);
        softmax(sc, dp);
        if (bits != 0xffffffffu || q0 + kTile > last || !tile_in_window(s, q0, key0)) {
            const uint32_t keep = visible ? bit_range(qlo - q0, qhi - q0) >> (4 * h) : 0u;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const bool ok = (keep >> (8 * (j >> 2) + (j & 3))) & 1u;
                sc[j] = ok ? sc[j] : 0.0f;
                dp[j] = ok ? dp[j] : 0.0f;
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                acc_v[t] = mfma(uc[t][j], sc[j], acc_v[t]);
                acc_k[t] = mfma(qc[t][j], dp[j], acc_k[t]);
            }
        }
        if constexpr (FUSED) {
            // dS (keys on lanes) → LDS [query][key] → queries on lanes: A operand of dQ MFMA j is
            // dS[q0 + col][key0 + tile_row(j, h)], four consecutive keys per 128-bit read.
#pragma unroll
            for (int j = 0; j < 16; ++j) dsl[wave][tile_row(j, h)][col] = dp[j];
            wave_lds_sync();
            float a[16];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const f32x4 x = *reinterpret_cast<const f32x4 *>(&dsl[wave][col][8 * u + 4 * h]);
                a[4 * u + 0] = x[0];
                a[4 * u + 1] = x[1];
                a[4 * u + 2] = x[2];
                a[4 * u + 3] = x[3];
            }
            wave_lds_sync(); // the next tile overwrites dsl only after these reads
            const uint32_t qrow = static_cast<uint32_t>(q0 + 4 * h) * (4u * D) + 4u * col;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                f32x16 acc_q{};
#pragma unroll
                for (int j = 0; j < 16; ++j) acc_q = mfma(a[j], kq[t][j], acc_q);
                // Accumulator register j is row q0 + tile_row(j, h), feature 32t + col.
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(acc_q[j], qgbuf, static_cast<int>(qrow + 128u * t),
                            static_cast<int>(static_cast<uint32_t>(8 * (j >> 2) + (j & 3)) * (4u * D)), 0);
            }
        }
    };

    const int mine = ntiles > start ? min(limit, (ntiles - start + stride - 1) / stride) : 0;
    if constexpr (STAGE) {
        static_assert(VEC, "staged tiles need 128-bit access");
        float *const qslot = dkdv_slots<D, WAVES>() + 2 * wave * kSlotFloats<D>;
        float *const uslot = qslot + kSlotFloats<D>;
        // One query tile: stage r, then load the next tile's rows into r while this one computes.
        auto stage_step = [&](Raw &r, const int q0, const int next_q0) __attribute__((always_inline)) {
            wave_lds_sync();
            if (h == 0) {
                const bool ok = q0 + col < last && r.m != -INFINITY;
                stats[wave][0][col] = SEED ? (ok ? -fmaf(r.m, kLog2e, __log2f(r.l)) : -INFINITY) : (ok ? fmaf(r.m, kLog2e, __log2f(r.l)) : INFINITY);
                stats[wave][1][col] = SEED ? -r.d : r.d;
            }
            {
                RowTile<D> u;
                load_row_tile<D>(u, ubuf, ustep, static_cast<uint32_t>(q0) * ustep);
                write_row_tile<D>(qslot, r.q);
                write_row_tile<D>(uslot, u);
            }
            wave_lds_sync();
            load_raw(r, next_q0);

            f32x16 sc{}, dp{};
            if constexpr (SEED) seeds(sc, dp);
            {
                float qr[HALF];
                read_row_layout<D>(qslot, qr);
#pragma unroll
                for (int c = 0; c < HALF; ++c) sc = mfma(qr[c], kr[c], sc);
            }
            __builtin_amdgcn_sched_barrier(0);
            {
                float ur[HALF];
                read_row_layout<D>(uslot, ur);
#pragma unroll
                for (int c = 0; c < HALF; ++c) dp = mfma(ur[c], vr[c], dp);
            }
            __builtin_amdgcn_sched_barrier(0);

            softmax(sc, dp);
            if (bits != 0xffffffffu || q0 + kTile > last || !tile_in_window(s, q0, key0)) {
                const uint32_t keep = visible ? bit_range(qlo - q0, qhi - q0) >> (4 * h) : 0u;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const bool ok = (keep >> (8 * (j >> 2) + (j & 3))) & 1u;
                    sc[j] = ok ? sc[j] : 0.0f;
                    dp[j] = ok ? dp[j] : 0.0f;
                }
            }
            // Column layouts eight rows at a time: all of both at once would hold 48 * D / 32 more registers.
            auto column_product = [&](const float *slot, const f32x16 &b, f32x16 (&acc)[DT]) __attribute__((always_inline)) {
                __builtin_amdgcn_sched_barrier(0);
                {
                    float c[DT][8];
                    read_column_layout<D, 0, 8>(slot, c);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
#pragma unroll
                        for (int t = 0; t < DT; ++t) acc[t] = mfma(c[t][j], b[j], acc[t]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
                {
                    float c[DT][8];
                    read_column_layout<D, 8, 8>(slot, c);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
#pragma unroll
                        for (int t = 0; t < DT; ++t) acc[t] = mfma(c[t][j], b[8 + j], acc[t]);
                    }
                }
            };
            column_product(uslot, sc, acc_v);
            column_product(qslot, dp, acc_k);
        };
        for (int i = 0; i < mine; ++i) {
            const int q0 = first + (start + i * stride) * kTile;
            stage_step(raw, q0, q0 + stride * kTile);
        }
    } else {
        // Tiles start, start + stride, ...; the count is rounded up to even so the loop body is two straight-line
        // steps.
        Rows ra, rb;
        if (mine > 0) load_rows(ra, first + start * kTile);
        for (int i = 0; i < mine; i += 2) {
            const int q0 = first + (start + i * stride) * kTile;
            step(ra, q0, true, rb, q0 + stride * kTile);
            step(rb, q0 + stride * kTile, i + 1 < mine, ra, q0 + 2 * stride * kTile);
        }
    }
}

// NI = 0: items (key tiles) in dispatch order, 4-wave workgroups; NI > 0: persistent grid of NI * SPLIT-wave workgroups
// taking the NI items of their bin from the launch's item table (staged Q/dO tiles, see dkdv_tiles), as in the forward.
template<int D, bool VEC, int SPLIT, bool FUSED, int NI = 0>
__global__ __launch_bounds__(kWave * (NI > 0 ? NI * SPLIT : kWaves)) void attention_dkdv_kernel(const Tensor q, const Tensor k,
        const Tensor v, const uint8_t *__restrict__ mask, const float *__restrict__ lse, const Tensor du,
        const float *__restrict__ delta, float *__restrict__ dk, float *__restrict__ dv, float *__restrict__ dq, const Shape s,
        const ItemTable<NI> items, const float scale) {
    constexpr int DT = D / 32;
    constexpr int WG = NI > 0 ? NI * SPLIT : kWaves;
    const int col = threadIdx.x & 31;
    const int h = (threadIdx.x >> 5) & 1;
    const int ktiles = (s.keys + kTile - 1) / kTile;
    const WorkItem w = [&] {
        if constexpr (NI > 0) return planned_item<SPLIT, NI>(s, items);
        else return work_item<SPLIT>(s, ktiles);
    }();
    const int kt = w.valid ? w.rank : ktiles; // past the last key tile: no work
    f32x16 acc_k[DT], acc_v[DT];
    constexpr bool STAGE = VEC && !FUSED;
    dkdv_tiles<D, VEC, FUSED, WG, STAGE>(q, k, v, mask, lse, du, delta, dq, s, scale, w.b, w.head, kt, w.lead, SPLIT,
            0x7fffffff, acc_k, acc_v);

    if constexpr (STAGE) { // the staged path's LDS slots are free once every wave has left its loop
        static_assert(WG * 16 * DT * kWave <= WG * 2 * kSlotFloats<D>);
        split_sum_into<SPLIT, DT, WG>(acc_k, w.sub, dkdv_slots<D, WG>());
        split_sum_into<SPLIT, DT, WG>(acc_v, w.sub, dkdv_slots<D, WG>());
    } else {
        split_sum<SPLIT, DT, WG>(acc_k, w.sub);
        split_sum<SPLIT, DT, WG>(acc_v, w.sub);
    }
    const int key = kt * kTile + col;
    if (w.sub != 0 || key >= s.keys) return;
    const int64_t krow = (static_cast<int64_t>(w.seq) * s.keys + key) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        store_tile_row<VEC>(dk + krow + 32 * t, acc_k[t], scale, h);
        store_tile_row<VEC>(dv + krow + 32 * t, acc_v[t], 1.0f, h);
    }
}

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool strides4(const rocmkernels_strides &s) { return ((s.batch | s.head | s.token) & 3) == 0; }

Tensor tensor(const float *p, const rocmkernels_strides &s) { return Tensor{p, s.batch, s.head, s.token}; }


template<int D, int MODE, bool VEC, int SPLIT, int NI = 0>
void launch_dq(const BackwardArgs &a, hipStream_t stream, const unsigned planned_grid = 0, const ItemTable<NI> &table = ItemTable<NI>{}) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const int64_t items = static_cast<int64_t>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    const unsigned grid = NI > 0 ? planned_grid : workgroups_for(items, SPLIT);
    const unsigned threads = kWave * (NI > 0 ? NI * SPLIT : kWaves);
    hipLaunchKernelGGL((attention_dq_kernel<D, MODE, VEC, SPLIT, NI>), dim3(grid), dim3(threads), 0, stream, tensor(a.q, a.qs),
            tensor(a.k, a.ks), tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), tensor(a.output, a.os), a.lse,
            tensor(a.upstream, a.us), a.gradient_q, a.delta, shape, table, scale);
}

// dQ pass (MODE kDqAndDelta or kDqFromDelta). At d=32 (about 155 VGPRs, 3 waves per SIMD) with more items than CUs but no
// more than 3 per CU, a persistent cost-balanced grid as in the forward; otherwise SPLIT waves per item in dispatch order.
template<int D, int MODE, bool VEC>
void launch_dq_mapped(const BackwardArgs &a, const int cus, hipStream_t stream) {
    const int qtiles = (a.queries + kTile - 1) / kTile;
    const int64_t items = static_cast<int64_t>(qtiles) * a.batch * a.heads;
    if constexpr (D == 32) {
        if (items > cus && items <= 3ll * cus) {
            const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
            const Plan plan = make_plan(static_cast<int64_t>(a.batch) * a.heads, qtiles, cus, a.causal != 0);
            const unsigned grid = static_cast<unsigned>(plan.groups * plan.bins);
            if (plan.rounds == 3) {
                if (const ItemTable<3> *table = item_table<3>(shape, plan)) {
                    launch_dq<D, MODE, VEC, 4, 3>(a, stream, grid, *table);
                    return;
                }
            } else if (const ItemTable<2> *table = item_table<2>(shape, plan)) {
                launch_dq<D, MODE, VEC, 4, 2>(a, stream, grid, *table);
                return;
            }
        }
    }
    const int split = backward_split_for(items);
    if (split == 1) launch_dq<D, MODE, VEC, 1>(a, stream);
    else if (split == 2) launch_dq<D, MODE, VEC, 2>(a, stream);
    else launch_dq<D, MODE, VEC, 4>(a, stream);
}

template<int D, bool VEC, int SPLIT, bool FUSED, int NI = 0>
void launch_dkdv(const BackwardArgs &a, hipStream_t stream, const unsigned planned_grid = 0, const ItemTable<NI> &table = ItemTable<NI>{}) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const int64_t items = static_cast<int64_t>((a.keys + kTile - 1) / kTile) * a.batch * a.heads;
    const unsigned grid = NI > 0 ? planned_grid : workgroups_for(items, SPLIT);
    const unsigned threads = kWave * (NI > 0 ? NI * SPLIT : kWaves);
    hipLaunchKernelGGL((attention_dkdv_kernel<D, VEC, SPLIT, FUSED, NI>), dim3(grid), dim3(threads), 0, stream, tensor(a.q, a.qs),
            tensor(a.k, a.ks), tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), a.lse, tensor(a.upstream, a.us), a.delta,
            a.gradient_k, a.gradient_v, a.gradient_q, shape, table, scale);
}

template<int D, bool VEC, bool FUSED>
void launch_dkdv_split(const BackwardArgs &a, const int split, hipStream_t stream) {
    if (split == 1) launch_dkdv<D, VEC, 1, FUSED>(a, stream);
    else if (split == 2) launch_dkdv<D, VEC, 2, FUSED>(a, stream);
    else launch_dkdv<D, VEC, 4, FUSED>(a, stream);
}

// Deterministic dK/dV pass. At d=32 with 128-bit access (staged Q/dO tiles: about 150 VGPRs, 3 waves per SIMD) and
// more key tiles than CUs but no more than 3 per CU, a persistent cost-balanced grid as in the forward; otherwise
// SPLIT waves per key tile in dispatch order.
template<int D, bool VEC>
void launch_dkdv_mapped(const BackwardArgs &a, const int cus, hipStream_t stream) {
    const int ktiles = (a.keys + kTile - 1) / kTile;
    const int64_t items = static_cast<int64_t>(ktiles) * a.batch * a.heads;
    if constexpr (D == 32 && VEC) {
        if (items > cus && items <= 3ll * cus) {
            const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
            const Plan plan = make_plan(static_cast<int64_t>(a.batch) * a.heads, ktiles, cus, false); // key tile 0 first
            const unsigned grid = static_cast<unsigned>(plan.groups * plan.bins);
            if (plan.rounds == 3) {
                if (const ItemTable<3> *table = item_table<3, true>(shape, plan)) {
                    launch_dkdv<D, VEC, 4, false, 3>(a, stream, grid, *table);
                    return;
                }
            } else if (const ItemTable<2> *table = item_table<2, true>(shape, plan)) {
                launch_dkdv<D, VEC, 4, false, 2>(a, stream, grid, *table);
                return;
            }
        }
    }
    launch_dkdv_split<D, VEC, false>(a, backward_split_for(items), stream);
}


// Smallest number of 128-key blocks per CU (num / den) at which Auto takes the band kernel under a radius window.
struct BlocksPerCu {
    int num, den;
};
constexpr BlocksPerCu kBandMinBlocksPerCu{5, 8};

template<int D, bool VEC>
hipError_t run(BackwardStage stage, const BackwardArgs &a, const int cus, hipStream_t stream) {
    const int64_t kitems = static_cast<int64_t>((a.keys + kTile - 1) / kTile) * a.batch * a.heads;
    const int64_t kblocks = static_cast<int64_t>((a.keys + kBlockKeys - 1) / kBlockKeys) * a.batch * a.heads;
    // The fused key-block kernels need 128-bit access; without it the deterministic kernels measured faster.
    // Auto takes the fused kernels wherever they exist (128-bit access): under a radius window the band kernel against
    // the deterministic pair, causal, measured 146.4 against 160.3 us at D = 32 (16 sequences x 8192 tokens, radius
    // 256), 124.9 against 147.8 us (32 x 2048, radius 512), 101.9 against 103.4 us (32 x 4096, radius 128), and 258
    // against 287 us at D = 64 (config 5). The band kernel runs one persistent workgroup per 128-key block and never
    // splits a block, so with fewer blocks than a grid that fills the CUs it leaves them idle while the deterministic
    // pair spreads 32-row tiles over every CU: measured, causal, 1 x 8192 at D = 64, radius 256 (64 blocks) 64.9
    // against 40.0 us, 2 x 8192 (128 blocks) 67.5 against 59.0 us, 4 x 8192 (256 blocks) 74.0 against 105.8 us; at
    // D = 32, 64 / 128 / 256 blocks 38.0 / 39.1 / 42.4 against 22.2 / 32.0 / 58.3 us. So under a radius window Auto
    // takes the band kernel only from kBandMinBlocksPerCu blocks per CU.
    if (stage == kBackwardAuto) {
        const bool band_fills = a.radius < 0 || kblocks * kBandMinBlocksPerCu.den >= static_cast<int64_t>(cus) * kBandMinBlocksPerCu.num;
        stage = VEC && band_fills ? kBackwardFused : kBackwardAll;
    }
    if (stage == kBackwardFused) {
        // Key-block kernels (one dQ add per element per 128 keys): without a radius window the piece-planned one; under a
        // radius window the band kernel, whose skewed walk visits each key tile's own band only (the key-block walk over
        // the union of the four bands idles a quarter of its wave-steps at radius 256).
        if constexpr (VEC) {
            if (a.radius < 0) return launch_fused_backward(D, a, cus, stream);
            return launch_band_backward(D, a, cus, stream);
        } else {
            // Without 128-bit access: delta and dQ = 0, then the per-key-tile dK/dV kernel adding dQ per 32 x 32 tile.
            launch_dq<D, kDeltaZeroDq, VEC, 1>(a, stream);
            const hipError_t error = hipGetLastError();
            if (error != hipSuccess) return error;
            launch_dkdv_split<D, VEC, true>(a, backward_split_for(kitems), stream);
            return hipGetLastError();
        }
    }
    if (stage == kBackwardAll || stage == kBackwardDelta || stage == kBackwardQuery) {
        if (stage == kBackwardDelta) launch_dq<D, kDeltaOnly, VEC, 1>(a, stream);
        else if (stage == kBackwardAll) launch_dq_mapped<D, kDqAndDelta, VEC>(a, cus, stream);
        else launch_dq_mapped<D, kDqFromDelta, VEC>(a, cus, stream);
        const hipError_t error = hipGetLastError();
        if (error != hipSuccess || stage != kBackwardAll) return error;
    }
    launch_dkdv_mapped<D, VEC>(a, cus, stream);
    return hipGetLastError();
}

} // namespace

hipError_t launch_backward(const int D, const BackwardStage stage, const BackwardArgs &a, hipStream_t stream) {
    const int64_t qblocks = static_cast<int64_t>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    const int64_t kblocks = static_cast<int64_t>((a.keys + kTile - 1) / kTile) * a.batch * a.heads;
    if (qblocks > 0x7fffffff || kblocks > 0x7fffffff || !sequence_fits(a.queries, a.qs, D) || !sequence_fits(a.keys, a.ks, D) ||
            !sequence_fits(a.keys, a.vs, D) || !sequence_fits(a.queries, a.os, D) || !sequence_fits(a.queries, a.us, D))
        return hipErrorInvalidValue;
    // The fused kernels address packed dQ (and dK/dV) through buffer resources: each sequence under 2 GiB.
    const bool packed_fits = sequence_fits(a.queries, rocmkernels_strides{0, 0, D}, D) && sequence_fits(a.keys, rocmkernels_strides{0, 0, D}, D);
    if (stage == kBackwardFused && !packed_fits) return hipErrorInvalidValue;
    const BackwardStage chosen = stage == kBackwardAuto && !packed_fits ? kBackwardAll : stage;
    const bool vec = aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.output) && aligned16(a.upstream) &&
            aligned16(a.gradient_q) && aligned16(a.gradient_k) && aligned16(a.gradient_v) && strides4(a.qs) && strides4(a.ks) &&
            strides4(a.vs) && strides4(a.os) && strides4(a.us);
    int cus = 0;
    const hipError_t error = compute_units(cus);
    if (error != hipSuccess) return error;
    if (D == 32) return vec ? run<32, true>(chosen, a, cus, stream) : run<32, false>(chosen, a, cus, stream);
    return vec ? run<64, true>(chosen, a, cus, stream) : run<64, false>(chosen, a, cus, stream);
}

} // namespace rk
