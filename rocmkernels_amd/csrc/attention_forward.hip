// FP32 online-softmax attention forward for gfx950 (MI355X), head width 16, 32 or 64.
//
// Replaces the reference's forward kernels: attention_query<false> (Attention.hip:32-115),
// attention_query_tiled_body (AttentionTile32.h:12-208), attention_query_flash_body (AttentionFlash32.h:23-170),
// the statistics-only instance (Attention.hip:252-261) and attention64_query<false> (Attention64.hip:34-129).
// The maths is the same (O = softmax(QKᵀ/√D + mask) V with lse = {max, Σexp(s - max)}); the mapping is not:
//
//   * A work item is one 32-query tile of one (batch, head). SPLIT waves (1, 2 or 4, one per SIMD) split the 32-key
//     tiles of its key range round-robin, each keeping its own online-softmax state (m, l, Oᵀ), and merge once
//     through LDS at the end. With few items (the causal 24x1024 shape has 768, under one per SIMD) the grid is
//     persistent: one workgroup per CU takes a bin of 2 or 3 items chosen so that every bin costs the same number
//     of key tiles (attention_plan.hpp), 4 waves per item; otherwise items go to 4-wave workgroups in dispatch
//     order and the hardware balances them.
//   * Sᵀ = K·Qᵀ and Oᵀ += Vᵀ·Pᵀ run on v_mfma_f32_32x32x2f32; the Sᵀ accumulator register j is the B operand
//     of Oᵀ MFMA j, so P never leaves registers. Each lane owns one query, so the row maximum is 15 VALU max
//     plus one exchange with the other half-wave, and the rescale of Oᵀ is lane-local.
//   * exp(s - m) is evaluated as exp2(s·(log2e/√D) - m·(log2e/√D)) with one FMA feeding v_exp_f32.
//   * FP32 MFMAs and VALU instructions share the SIMD's ALU on gfx950 (they never co-execute, in one wave or across
//     waves), so every VALU instruction of the inner loop adds to the MFMA time: the loop keeps them few.
//   * Q and K tiles are read with loads that cover whole 128-byte lines and staged into row layout through each
//     wave's LDS slot (attention_device.hpp); the persistent grid reads each wave's item from a host-built table.
//   * blockIdx → work: in dispatch order the heaviest query tiles (the last ones under a causal mask) go first, and
//     consecutive workgroups take consecutive (batch, head) pairs of the same tile; in both mappings, with B·H a
//     multiple of 8, each XCD (workgroup index mod 8) keeps a fixed subset of sequences in its own L2.
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

// NI = 0: one work item per SPLIT waves of 4-wave workgroups, in dispatch order (work_item). NI > 0: persistent grid
// of NI * SPLIT-wave workgroups, each taking the NI items of its bin from the launch's item table (planned_item).
template<int D, bool STATS, bool VEC, int SPLIT, int NI>
__global__ __launch_bounds__(kWave * (NI > 0 ? NI * SPLIT : kWaves)) void attention_forward_kernel(const Tensor q, const Tensor k,
        const Tensor v, const uint8_t *__restrict__ mask, float *__restrict__ out, const int osb, const int osh, const int ost,
        float *__restrict__ lse, const Shape s, const ItemTable<NI> items, const float scale) {
    constexpr int HALF = D / 2; // features per lane in row layout
    constexpr int DT = (D + 31) / 32; // 32-feature slices of the output (a 16-wide head uses half of one)
    constexpr int ROWS = D < 32 ? D : 32; // valid features per slice
    constexpr int NREG = STATS ? 0 : 16 * DT;
    constexpr int WG = NI > 0 ? NI * SPLIT : kWaves; // waves per workgroup

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform: keeps tile bookkeeping scalar
    const int col = lane & 31;
    const int h = lane >> 5;

    const int qtiles = (s.queries + kTile - 1) / kTile;
    const WorkItem w = [&] {
        if constexpr (NI > 0) return planned_item<SPLIT, NI>(s, items);
        else return work_item<SPLIT>(s, qtiles);
    }();
    const int seq = w.seq, b = w.b, head = w.head, sub = w.sub;
    constexpr int split = SPLIT; // waves sharing this item
    const int qt = s.causal ? qtiles - 1 - w.rank : w.rank;
    const int q0 = qt * kTile;
    const int query = q0 + col;
    const float c2 = scale * kLog2e;

    int first, last;
    const int ntiles = w.valid ? forward_key_range(s, qt, first, last) : 0;
    // This lane's query sees keys [wlo, whi] through the causal/radius window.
    const int wlo = window_lo(s, query);
    const int whi = window_hi(s, query);

    const Buffer qbuf = make_buffer(sequence(q, b, head), sequence_bytes(s.queries, q.st, D));
    const Buffer kbuf = make_buffer(sequence(k, b, head), sequence_bytes(s.keys, k.st, D));
    const Buffer vbuf = make_buffer(sequence(v, b, head), sequence_bytes(s.keys, v.st, D));
    const Buffer mbuf = make_buffer(mask + static_cast<int64_t>(b) * s.keys, static_cast<uint32_t>(s.keys));
    const uint32_t kstep = 4u * k.st; // bytes between consecutive keys
    const uint32_t vstep = 4u * v.st;

    // With 128-bit access (VEC) the row-layout operands (Q once; K per tile at D <= 32) are loaded a whole line per
    // request and staged through this wave's LDS slot; otherwise each lane reads its own row span. (At D = 64 the
    // staged K tile pushes the kernel past the 256 registers that two waves per SIMD allow.)
    constexpr bool STAGE_K = VEC && D <= 32;
    __shared__ __align__(16) float row_slots[VEC ? WG : 1][VEC ? kSlotFloats<D> : 1];
    float *const slot = row_slots[VEC ? wave : 0];
    float qr[HALF];
    RowTile<D> qraw;
    if constexpr (VEC) load_row_tile<D>(qraw, qbuf, 4u * q.st, static_cast<uint32_t>(q0) * (4u * q.st)); // rows >= queries read 0
    else buffer_load_span<VEC>(qr, qbuf, static_cast<uint32_t>(query) * (4u * q.st) + 4u * h * HALF);

    // Online-softmax state of this lane's query over the tiles this wave visits. m_half is the raw maximum of q·k
    // over the keys this half-wave holds (16 of each tile); the row maximum is the larger of the two halves', formed
    // only when it is needed (a re-base, and once at the end), so a tile costs no cross-half exchange.
    // The exponentials are taken against a reference offset mc (in log2 units, c2-scaled): p = exp2(s·c2 - mc).
    // mc moves only when the running maximum exceeds it by more than kLazy (so p <= 2^kLazy, far from overflow);
    // o and l are then rescaled by exp2(mc_old - mc_new). The test compares raw maxima with m_lazy, the raw
    // score at which p would reach 2^kLazy: a row's maximum exceeds it exactly when one of its halves' does.
    // The lse sum is brought to the true maximum once at the end. Skipping most rescales removes 16·D/32 VALU
    // multiplies per tile, which matters because FP32 MFMA and VALU share the SIMD on gfx950: every VALU cycle
    // adds to the MFMA time.
    constexpr float kLazy = 8.0f;
    const float lazy_raw = kLazy / c2; // kLazy in raw score units
    float m_half = -INFINITY;
    float m_lazy = -INFINITY; // re-base when a maximum exceeds this (-inf: any visible key)
    float mc = -INFINITY;     // offset of the state; -inf until the row has a visible key
    float mcx = 0.0f;         // finite stand-in used in the exponent (masked scores are -inf there, giving 0)
    float l_run = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x16{};

    // K rows (Sᵀ A operand, row layout), V columns (PV A operand) and the mask byte of the tile after next are
    // loaded while the current tile computes. The loads are unconditional: past the last tile they read rows
    // that are never used (or, beyond the sequence, zeros), which keeps the two register sets free of copies.
    struct Tile {
        float k[STAGE_K ? 1 : HALF]; // row layout
        RowTile<D> kraw;             // whole-line loads, staged into row layout when the tile is used (STAGE_K)
        float v[STATS ? 1 : DT][16];
        int mask;
    };
    auto load_tile = [&](Tile &t, const int key0) __attribute__((always_inline)) {
        const uint32_t key = static_cast<uint32_t>(key0 + col);
        t.mask = buffer_load_byte(mbuf, key); // keys >= s.keys read 0: masked
        if constexpr (STAGE_K) load_row_tile<D>(t.kraw, kbuf, kstep, static_cast<uint32_t>(key0) * kstep);
        else buffer_load_span<VEC>(t.k, kbuf, key * kstep + 4u * h * HALF);
        if constexpr (!STATS) {
            // Lanes past a 16-wide head's last feature read 0 (offset beyond the sequence).
            const uint32_t vlane = col < ROWS ? static_cast<uint32_t>(key0 + 4 * h) * vstep + 4u * col : kNoRow;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
#pragma unroll
                for (int t2 = 0; t2 < DT; ++t2)
                    t.v[t2][j] = buffer_load(vbuf, vlane + 128u * t2, static_cast<uint32_t>(8 * (j >> 2) + (j & 3)) * vstep);
            }
        }
    };

    auto step = [&](Tile &t, const int key0, Tile &next, const int next_key0) __attribute__((always_inline)) {
        // key0 >= last marks the padding step of a wave with an odd number of tiles.
        const uint32_t bits = key0 < last ? static_cast<uint32_t>(__ballot(t.mask != 0)) : 0u;
        if (bits == 0) { // every key of the tile is masked: contributes nothing
            load_tile(next, next_key0);
            return;
        }
        f32x16 sc{};
        if constexpr (STAGE_K) {
            float kr[HALF];
            stage_row_tile<D>(slot, t.kraw, kr);
#pragma unroll
            for (int c = 0; c < HALF; ++c) sc = mfma(kr[c], qr[c], sc);
        } else {
#pragma unroll
            for (int c = 0; c < HALF; ++c) sc = mfma(t.k[c], qr[c], sc);
        }
        __builtin_amdgcn_sched_barrier(0);
        load_tile(next, next_key0);
        __builtin_amdgcn_sched_barrier(0);

        if (bits != 0xffffffffu || !tile_in_window(s, q0, key0)) {
            // Boundary tile: keep (query, key) pairs whose key is unmasked and inside this query's window.
            const uint32_t visible = (bits & bit_range(wlo - key0, whi - key0)) >> (4 * h);
#pragma unroll
            for (int j = 0; j < 16; ++j) sc[j] = (visible >> (8 * (j >> 2) + (j & 3))) & 1u ? sc[j] : -INFINITY;
            if constexpr (!STATS) {
                if (bits != 0xffffffffu) {
                    // Masked keys contribute exactly nothing, whatever their stored values hold.
                    const uint32_t kept = bits >> (4 * h);
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
#pragma unroll
                        for (int t2 = 0; t2 < DT; ++t2) t.v[t2][j] = (kept >> (8 * (j >> 2) + (j & 3))) & 1u ? t.v[t2][j] : 0.0f;
                    }
                }
            }
        }

        float mx = m_half; // starting from the running maximum folds its update into the three-input maxima
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sc[j]);
        m_half = mx;

        // exp, row sum and PV; instantiated on both sides of the re-base branch so that each side ends in the
        // MFMA chain that writes o (a join after a conditional o *= alpha would cost a copy of o on every tile).
        auto finish = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 16; ++j) sc[j] = exp2_fast(fmaf(sc[j], c2, -mcx));
            float psum = sc[0]; // not 0 + sc[0]: the compiler keeps that add (0 + -0 is +0)
#pragma unroll
            for (int j = 1; j < 16; ++j) psum += sc[j];
            l_run += psum;
            if constexpr (!STATS) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
#pragma unroll
                    for (int t2 = 0; t2 < DT; ++t2) o[t2] = mfma(t.v[t2][j], sc[j], o[t2]);
                }
            }
        };
        // The common case (no re-base) is the fall-through path, so the exponentials follow the maxima without a
        // branch (a jump there also made the compiler wait out the full MFMA result latency again).
        if (__builtin_expect(__ballot(m_half > m_lazy) == 0, 1)) {
            finish();
        } else {
            // Re-base every lane on its row's current maximum. A row without a visible key yet keeps offset -inf (its
            // l and o are 0); the first finite offset multiplies them by exp2(-inf) = 0.
            const float m_row = halves_max(m_half);
            const float mc_new = m_row == -INFINITY ? -INFINITY : m_row * c2;
            m_lazy = m_row + lazy_raw;
            const float alpha = mc_new == -INFINITY ? 1.0f : exp2_fast(mc - mc_new);
            l_run *= alpha;
            if constexpr (!STATS) {
#pragma unroll
                for (int t2 = 0; t2 < DT; ++t2) o[t2] *= alpha;
            }
            mc = mc_new;
            mcx = mc_new == -INFINITY ? 0.0f : mc_new;
            finish();
        }
    };

    // The wave visits tiles lead, lead + split, ...; their count is rounded up to even so the loop body is two
    // straight-line steps (the padding step sees no key).
    const int lead = w.lead;
    const int mine = ntiles > lead ? (ntiles - lead + split - 1) / split : 0;
    Tile ta, tb;
    if (mine > 0) load_tile(ta, first + lead * kTile);
    if constexpr (VEC) stage_row_tile<D>(slot, qraw, qr); // after the first tile's loads are issued
    for (int i = 0; i < mine; i += 2) {
        const int key0 = first + (lead + i * split) * kTile;
        step(ta, key0, tb, key0 + split * kTile);
        step(tb, key0 + split * kTile, ta, key0 + 2 * split * kTile);
    }
    const float mc_run = mc; // offset the wave's (l_run, o) are expressed against
    const float m_run = halves_max(m_half); // raw maximum of the row over the wave's tiles

    // Merge the states of the `split` waves of the item. Every state satisfies l_w = Σ exp2(s·c2 - mc_w); they are
    // combined against the largest offset, and lse's sum is then expressed against the true maximum. The sum runs in
    // the same order whichever wave computes it (state 0 scaled, then states 1 .. SPLIT - 1 added).
    //   * Dispatch order (NI = 0): waves with sub > 0 publish (m, l, mc, Oᵀ) in LDS and the wave with sub == 0
    //     combines and stores everything; other workgroups keep the CU busy meanwhile.
    //   * Persistent bins (NI > 0): the item's end is on the CU's critical path, so every wave publishes its state and
    //     after the barrier each merges and stores its own share of the output registers (NREG / SPLIT of them, whole
    //     16-byte row chunks): config 2 forward 19.04 -> 18.9 us (the last item's merge and store end sooner). In
    //     dispatch order the extra LDS traffic made configs 4 and 5 2-2.5% slower.
    constexpr int SHARERS = NI > 0 ? SPLIT : 1; // waves that finalise the item's output
    constexpr int NR = NREG / SHARERS;          // output registers each of them finalises
    float m_all = m_run;
    float mc_all = mc_run;
    float base = 0.0f, l_all = l_run;
    float share[SHARERS > 1 && NR > 0 ? NR : 1];
    const int r0 = sub * NR; // first of them (register j of slice t is 16t + j)
    if constexpr (SPLIT > 1) {
        __shared__ float partial[WG][NREG + 3][kWave];
        if (SHARERS > 1 || sub > 0) {
            partial[wave][0][lane] = m_run;
            partial[wave][1][lane] = l_run;
            partial[wave][2 + NREG][lane] = mc_run;
            if constexpr (!STATS) {
#pragma unroll
                for (int t = 0; t < DT; ++t) {
#pragma unroll
                    for (int j = 0; j < 16; ++j) partial[wave][2 + 16 * t + j][lane] = o[t][j];
                }
            }
        }
        __syncthreads();
        if (sub >= SHARERS) return;
        if constexpr (SHARERS > 1) {
            const int w0 = wave - sub; // the item's first wave
            m_all = partial[w0][0][lane];
            mc_all = partial[w0][2 + NREG][lane];
#pragma unroll
            for (int x = 1; x < split; ++x) {
                m_all = fmaxf(m_all, partial[w0 + x][0][lane]);
                mc_all = fmaxf(mc_all, partial[w0 + x][2 + NREG][lane]);
            }
            base = mc_all == -INFINITY ? 0.0f : mc_all;
            float a[SPLIT];
#pragma unroll
            for (int x = 0; x < split; ++x) a[x] = exp2_fast(partial[w0 + x][2 + NREG][lane] - base);
            l_all = partial[w0][1][lane] * a[0];
#pragma unroll
            for (int x = 1; x < split; ++x) l_all = fmaf(partial[w0 + x][1][lane], a[x], l_all);
            if constexpr (!STATS) {
#pragma unroll
                for (int k = 0; k < NR; ++k) {
                    float acc = partial[w0][2 + r0 + k][lane] * a[0];
#pragma unroll
                    for (int x = 1; x < split; ++x) acc = fmaf(partial[w0 + x][2 + r0 + k][lane], a[x], acc);
                    share[k] = acc;
                }
            }
        } else {
#pragma unroll
            for (int x = 1; x < split; ++x) {
                m_all = fmaxf(m_all, partial[wave + x][0][lane]);
                mc_all = fmaxf(mc_all, partial[wave + x][2 + NREG][lane]);
            }
            base = mc_all == -INFINITY ? 0.0f : mc_all;
            const float a0 = exp2_fast(mc_run - base);
            l_all = l_run * a0;
            if constexpr (!STATS) {
#pragma unroll
                for (int t = 0; t < DT; ++t) o[t] *= a0;
            }
#pragma unroll
            for (int x = 1; x < split; ++x) {
                const float aw = exp2_fast(partial[wave + x][2 + NREG][lane] - base);
                l_all = fmaf(partial[wave + x][1][lane], aw, l_all);
                if constexpr (!STATS) {
#pragma unroll
                    for (int t = 0; t < DT; ++t) {
#pragma unroll
                        for (int j = 0; j < 16; ++j) o[t][j] = fmaf(partial[wave + x][2 + 16 * t + j][lane], aw, o[t][j]);
                    }
                }
            }
        }
    } else {
        base = mc_run == -INFINITY ? 0.0f : mc_run;
    }
    l_all = halves_sum(l_all); // each half-wave summed the exponentials of its own 16 keys per tile
    // O is o / l in any offset; lse's sum is Σ exp(s - max) = l · exp2(offset - max·c2).
    const float sum_at_max = m_all == -INFINITY ? l_all : l_all * exp2_fast(base - m_all * c2);

    if (!w.valid || query >= s.queries) return;
    const bool nan_row = isnan(l_all);
    const bool has_keys = l_all > 0.0f;
    if constexpr (!STATS) {
        const float factor = has_keys ? 1.0f / l_all : (nan_row ? NAN : 0.0f);
        float *orow = out + static_cast<int64_t>(b) * osb + static_cast<int64_t>(head) * osh + static_cast<int64_t>(query) * ost;
        if constexpr (SHARERS == 1) {
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                if (has_keys) {
                    store_tile_row<VEC, ROWS>(orow + 32 * t, o[t], factor, h);
                } else {
                    const f32x16 fill{};
                    store_tile_row<VEC, ROWS>(orow + 32 * t, fill + factor, 1.0f, h);
                }
            }
        } else {
            // Registers 16t + 4u .. +3 are features 32t + 8u + 4h .. +3 of this lane's query; a 16-wide head stores only
            // its first two chunks (u < 2).
#pragma unroll
            for (int q4 = 0; q4 < NR / 4; ++q4) {
                const int r = r0 + 4 * q4, t = r >> 4, u = (r & 15) >> 2;
                if (u >= ROWS / 8) continue;
                const f32x4 x = has_keys ? f32x4{share[4 * q4] * factor, share[4 * q4 + 1] * factor, share[4 * q4 + 2] * factor,
                                                 share[4 * q4 + 3] * factor}
                                         : f32x4{factor, factor, factor, factor};
                float *dst = orow + 32 * t + 8 * u + 4 * h;
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
    }
    if (h == 0 && sub == 0) {
        const int64_t row = static_cast<int64_t>(seq) * s.queries + query;
        lse[2 * row] = has_keys ? m_all * scale : (nan_row ? NAN : -INFINITY);
        lse[2 * row + 1] = has_keys ? sum_at_max : (nan_row ? NAN : 0.0f);
    }
}

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool strides4(const rocmkernels_strides &s) { return ((s.batch | s.head | s.token) & 3) == 0; }

template<int D, bool STATS, bool VEC, int SPLIT, int NI>
void launch(const ForwardArgs &a, const unsigned grid, const ItemTable<NI> &table, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const unsigned threads = kWave * (NI > 0 ? NI * SPLIT : kWaves);
    hipLaunchKernelGGL((attention_forward_kernel<D, STATS, VEC, SPLIT, NI>), dim3(grid), dim3(threads), 0, stream,
            Tensor{a.q, a.qs.batch, a.qs.head, a.qs.token}, Tensor{a.k, a.ks.batch, a.ks.head, a.ks.token},
            Tensor{a.v, a.vs.batch, a.vs.head, a.vs.token}, reinterpret_cast<const uint8_t *>(a.mask), a.output, a.os.batch,
            a.os.head, a.os.token, a.lse, shape, table, scale);
}

// Items (32-query tiles) of 4 waves each that one CU runs at once: 3 at d<=32 (about 155 VGPRs per wave), 2 at d=64
// (about 250).
template<int D>
constexpr int resident_items_per_cu() { return D <= 32 ? 3 : 2; }

template<int D, bool STATS, bool VEC, int NI>
bool launch_planned(const ForwardArgs &a, const Plan &plan, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const ItemTable<NI> *table = item_table<NI>(shape, plan);
    if (table == nullptr) return false;
    launch<D, STATS, VEC, 4, NI>(a, static_cast<unsigned>(plan.groups * plan.bins), *table, stream);
    return true;
}

// Waves per item in dispatch order. Under a causal mask without a radius window item costs run from one tile to the
// whole sequence, and more waves per item (forward_split_for) even out the SIMDs' loads: config 4 forward 145.5 µs with
// four waves per item against 153.4 with two and 197.1 with one. Otherwise (no mask, or a radius window of at most a
// quarter of the sequence) items cost about the same, and the fewest waves that still fill every SIMD's resident slots
// (two waves per SIMD at d = 64, three at d <= 32) win, since a wave's start and the merge of an item's waves cost more
// than they balance: config 5 forward 90.2 µs with one wave per item against 96.5 with two and 114.4 with four; without
// a mask, 32 x 2048 at d = 64 256.8 against 266.6 µs (four waves) and 16 x 8192 at d = 64, radius 256, 149.9 against
// 158.3 µs (two).
template<int D>
int dispatch_split(const ForwardArgs &a, const int64_t items, const int cus) {
    // A radius window over more than a quarter of the sequence ramps item costs up over most of it.
    const bool varied = (a.causal && a.radius < 0) || (a.radius >= 0 && 4LL * a.radius > a.queries);
    if (varied) return forward_split_for(items);
    const int64_t slots = static_cast<int64_t>(cus) * kWaves * (D == 64 ? 2 : 3);
    return items >= slots ? 1 : 2 * items >= slots ? 2 : 4;
}

template<int D, bool STATS, bool VEC>
void launch_mapped(const ForwardArgs &a, const int64_t items, const int cus, hipStream_t stream) {
    if (items > cus && items <= static_cast<int64_t>(resident_items_per_cu<D>()) * cus) {
        // Every CU holds its whole bin at once: one persistent workgroup per CU takes a cost-balanced bin of items (the
        // causal mask makes item costs range from 1 to L/32 tiles), each item on 4 waves, one per SIMD, so that every
        // SIMD carries a quarter of the bin.
        const int qtiles = (a.queries + kTile - 1) / kTile;
        const Plan plan = make_plan(static_cast<int64_t>(a.batch) * a.heads, qtiles, cus, a.causal != 0);
        if constexpr (resident_items_per_cu<D>() >= 3) {
            if (plan.rounds == 3 && launch_planned<D, STATS, VEC, 3>(a, plan, stream)) return;
        }
        if (plan.rounds <= 2 && launch_planned<D, STATS, VEC, 2>(a, plan, stream)) return;
    }
    // Otherwise one item per 1, 2 or 4 waves of 4-wave workgroups, heaviest first, left to the hardware dispatcher.
    const ItemTable<0> none{};
    switch (dispatch_split<D>(a, items, cus)) {
        case 1: launch<D, STATS, VEC, 1, 0>(a, workgroups_for(items, 1), none, stream); break;
        case 2: launch<D, STATS, VEC, 2, 0>(a, workgroups_for(items, 2), none, stream); break;
        default: launch<D, STATS, VEC, 4, 0>(a, workgroups_for(items, 4), none, stream); break;
    }
}

template<int D>
void dispatch(const bool statistics_only, const ForwardArgs &a, const int64_t items, const int cus, hipStream_t stream) {
    bool vec = aligned16(a.q) && aligned16(a.k) && strides4(a.qs) && strides4(a.ks);
    if (!statistics_only) vec = vec && aligned16(a.v) && aligned16(a.output) && strides4(a.vs) && strides4(a.os);
    if (statistics_only) {
        if (vec) launch_mapped<D, true, true>(a, items, cus, stream);
        else launch_mapped<D, true, false>(a, items, cus, stream);
    } else {
        if (vec) launch_mapped<D, false, true>(a, items, cus, stream);
        else launch_mapped<D, false, false>(a, items, cus, stream);
    }
}

} // namespace

hipError_t launch_forward(const int D, const bool statistics_only, const ForwardArgs &a, hipStream_t stream) {
    const int64_t tiles = static_cast<int64_t>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    if (tiles > 0x7fffffff || !sequence_fits(a.queries, a.qs, D) || !sequence_fits(a.keys, a.ks, D) ||
            (!statistics_only && !sequence_fits(a.keys, a.vs, D)))
        return hipErrorInvalidValue;
    int cus = 0;
    const hipError_t error = compute_units(cus);
    if (error != hipSuccess) return error;
    if (D == 16) dispatch<16>(statistics_only, a, tiles, cus, stream);
    else if (D == 32) dispatch<32>(statistics_only, a, tiles, cus, stream);
    else dispatch<64>(statistics_only, a, tiles, cus, stream);
    return hipGetLastError();
}

} // namespace rk
