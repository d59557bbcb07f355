// FP16-storage online-softmax attention forward for gfx950 (MI355X), head width 16, 32 or 64: the fp16 instance of
// the reference's attention_generic_forward (Generic/Attention/AttentionGeneric.hip:141-236).
//
// The reference reads fp16 Q/K/V, forms scores and the softmax in fp32, rounds each probability to fp16 before the
// P·V product (accumulated in fp32), and rounds the normalised output to fp16; lse stays fp32. The arithmetic here is
// the same, on the FP16 matrix cores:
//
//   * Sᵀ = K·Qᵀ and Oᵀ += Vᵀ·Pᵀ run on v_mfma_f32_32x32x16_f16 (fp16 operands, fp32 accumulation). A lane of
//     half-wave h supplies features 16i + 8h .. 16i + 8h + 7 of its key (A) or query (B) row to MFMA i of Sᵀ.
//   * For Oᵀ the MFMA's 16-long reduction index is mapped onto the Sᵀ accumulator layout: MFMA u takes from lane
//     (query, h) the probabilities held in accumulator registers 8u .. 8u + 7, i.e. keys tile_row(8u + j, h), so
//     P is converted to fp16 in place (4 v_cvt_pk_f16_f32) and never leaves the lane; the Vᵀ operand of the same
//     lane (feature, h) holds V[tile_row(8u + j, h)][feature]. With 16-byte aligned V rows (d = 32, 64) a tile's V
//     rows arrive as 128-bit loads, pass through the wave's LDS slot and come back in that operand layout through
//     ds_read_b64_tr_b16 (a transposing 16-bit LDS read, two per MFMA); otherwise each element is a 16-bit load.
//   * The online softmax (lazy re-basing, exp2 with the scale folded into one FMA), the masks, the work mapping and
//     the merge of the waves sharing a query tile follow attention_forward.hip.
//   * Two kernels: attention_forward_f16_kernel gives each wave its own K/V tiles (1, 2 or 4 waves per query tile);
//     at d = 64 on grids that fill the chip, attention_forward_f16_shared_kernel has the waves of a workgroup (four query
//     tiles of one sequence) share each K/V tile through LDS, a quarter of the per-wave kernel's L2 traffic; its tiles
//     are loaded straight into LDS (buffer loads with the LDS bit).
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Strided fp16 tensor [batch][head][token][D] with contiguous features.
struct TensorH {
    const _Float16 *data;
    int sb, sh, st;
};

__device__ __forceinline__ f32x16 mfma16(const f16x8 a, const f16x8 b, const f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Byte extent of one sequence of a strided fp16 tensor: rows 0..rows-1 of `width` halves at `stride` halves.
__device__ __forceinline__ uint32_t sequence_bytes_h(const int rows, const int stride, const int width) {
    return static_cast<uint32_t>((static_cast<int64_t>(rows - 1) * stride + width) * 2);
}

// 8 contiguous halves at byte offset voffset (16-byte aligned when VEC).
template<bool VEC>
__device__ __forceinline__ f16x8 load8h(const Buffer b, const uint32_t voffset) {
    if constexpr (VEC) {
        return __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(b, static_cast<int>(voffset), 0, 0));
    } else {
        f16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[i] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(b, static_cast<int>(voffset + 2 * i), 0, 0));
        return r;
    }
}

// Row stride (halves) of a wave's staged V tile: rows are unpadded (padded strides that put the four rows of one
// transposing read on distinct banks measured no faster).
template<int D>
constexpr int kVStride = D;

// Operand of Oᵀ MFMA (t2, u) from the staged tile: lane (col, h) gets V[tile_row(8u + j, h)][32 t2 + col], j = 0..7,
// as two transposing reads of 4 rows each. In each 16-lane group, lane L points at row r0 + L / 4, features
// f0 + 4 (L mod 4) .. +3, and receives feature f0 + L of rows r0 .. r0 + 3 (r0 = 16u + 8p + 4h, f0 = 32 t2 + 16 (col / 16)).
template<int D, int T2, int U, int STRIDE = kVStride<D>>
__device__ __forceinline__ f16x8 read_v_operand(const _Float16 *slot, const int lane_off) {
    typedef __fp16 v4h __attribute__((ext_vector_type(4))); // the builtin's element type
    const _Float16 *p = slot + lane_off + 16 * U * STRIDE + 32 * T2;
    const f16x4 lo = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) v4h *)(p)));
    const f16x4 hi = __builtin_bit_cast(f16x4,
            __builtin_amdgcn_ds_read_tr16_b64_v4f16((__attribute__((address_space(3))) v4h *)(p + 8 * STRIDE)));
    return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// STAGE_V (d = 32 or 64, 16-byte aligned V rows): a tile's V rows arrive with 128-bit loads and pass through the wave's
// LDS slot, read back by transposing LDS reads into the Vᵀ operand layout (2 per MFMA) instead of one 16-bit load per
// operand element (16·D/32 per lane and tile).
template<int D, bool VEC, int SPLIT, bool STAGE_V>
__global__ __launch_bounds__(kThreads) void attention_forward_f16_kernel(const TensorH q, const TensorH k, const TensorH v,
        const uint8_t *__restrict__ mask, _Float16 *__restrict__ out, const int osb, const int osh, const int ost,
        float *__restrict__ lse, const Shape s, const float scale) {
    constexpr int KC = D / 16;            // 16-feature chunks of a row: MFMAs per Sᵀ tile
    constexpr int DT = (D + 31) / 32;     // 32-feature slices of the output
    constexpr int ROWS = D < 32 ? D : 32; // valid features per slice
    static_assert(!STAGE_V || (VEC && D >= 32), "staged V needs 128-bit rows of at least 32 features");
    constexpr int VLOADS = STAGE_V ? D / 16 : 1; // 128-bit loads per lane for a 32-row V tile
    constexpr int VCPR = D / 8;                  // 16-byte chunks per V row
    constexpr int VRPL = kWave / VCPR;           // V rows per 128-bit load

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); // wave-uniform: keeps tile bookkeeping scalar
    const int col = lane & 31;
    const int h = lane >> 5;

    const int qtiles = (s.queries + kTile - 1) / kTile;
    const WorkItem w = work_item<SPLIT>(s, qtiles);
    const int b = w.b, head = w.head, sub = w.sub;
    const int qt = s.causal ? qtiles - 1 - w.rank : w.rank;
    const int q0 = qt * kTile;
    const int query = q0 + col;
    const float c2 = scale * kLog2e;

    int first = 0, last = s.keys;
    if (s.radius >= 0) {
        first = max(0, q0 - s.radius);
        last = min(last, q0 + kTile + s.radius);
    }
    if (s.causal) last = min(last, q0 + kTile);
    const int ntiles = (w.valid && last > first) ? (last - first + kTile - 1) / kTile : 0;
    const int wlo = window_lo(s, query);
    const int whi = window_hi(s, query);

    auto seq_base = [&](const TensorH &t) {
        return t.data + (static_cast<int64_t>(b) * t.sb + static_cast<int64_t>(head) * t.sh);
    };
    const Buffer qbuf = make_buffer(seq_base(q), sequence_bytes_h(s.queries, q.st, D));
    const Buffer kbuf = make_buffer(seq_base(k), sequence_bytes_h(s.keys, k.st, D));
    const Buffer vbuf = make_buffer(seq_base(v), sequence_bytes_h(s.keys, v.st, D));
    const Buffer mbuf = make_buffer(mask + static_cast<int64_t>(b) * s.keys, static_cast<uint32_t>(s.keys));
    const uint32_t kstep = 2u * k.st; // bytes between consecutive keys
    const uint32_t vstep = 2u * v.st;

    f16x8 qr[KC];
#pragma unroll
    for (int i = 0; i < KC; ++i) qr[i] = load8h<VEC>(qbuf, static_cast<uint32_t>(query) * (2u * q.st) + 2u * (16 * i + 8 * h));

    // Lazy re-basing as in the FP32 forward: m_half is the maximum over this half-wave's keys, the row maximum is
    // formed only on a re-base and at the end, and m_lazy is the raw score at which p would reach 2^kLazy.
    constexpr float kLazy = 8.0f; // p = exp2(s·c2 - mc) <= 2^8: also within fp16 range
    const float lazy_raw = kLazy / c2;
    float m_half = -INFINITY;
    float m_lazy = -INFINITY;
    float mc = -INFINITY;
    float mcx = 0.0f;
    float l_run = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x16{};

    struct Tile {
        f16x8 k[KC];
        f16x8 v[STAGE_V ? 1 : DT][2];
        u32x4 vraw[VLOADS]; // STAGE_V: rows VRPL·i + lane / VCPR, 16-byte chunk lane mod VCPR
        int mask;
    };
    // STAGE_V: this wave's V slot, and the lane's offsets into it for the 128-bit row writes and the transposing reads.
    __shared__ __align__(16) _Float16 vslots[STAGE_V ? kWaves : 1][STAGE_V ? kTile * kVStride<D> : 1];
    _Float16 *const vslot = vslots[STAGE_V ? wave : 0];
    const int vrow = lane / VCPR; // row of the lane's chunk within each group of VRPL rows
    const int vwrite = vrow * kVStride<D> + 8 * (lane % VCPR);
    const int vread = (4 * h + ((lane & 15) >> 2)) * kVStride<D> + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    // With 128-bit rows the lane's offset within a tile is fixed (voffset) and the tile's row offset is scalar
    // (soffset): no per-tile address arithmetic in the VALU.
    const uint32_t kk_lane = static_cast<uint32_t>(col) * kstep + 16u * static_cast<uint32_t>(h);
    const uint32_t vv_lane = static_cast<uint32_t>(vrow) * vstep + 16u * static_cast<uint32_t>(lane % VCPR);
    auto load_tile = [&](Tile &t, const int key0) __attribute__((always_inline)) {
        const uint32_t key = static_cast<uint32_t>(key0 + col);
        if constexpr (VEC) {
            const uint32_t k0 = static_cast<uint32_t>(key0);
            t.mask = buffer_load_byte_s(mbuf, static_cast<uint32_t>(col), k0);
#pragma unroll
            for (int i = 0; i < KC; ++i)
                t.k[i] = __builtin_bit_cast(f16x8, __builtin_amdgcn_raw_buffer_load_b128(kbuf, static_cast<int>(kk_lane + 32u * i),
                        static_cast<int>(k0 * kstep), 0));
        } else {
            t.mask = buffer_load_byte(mbuf, key);
#pragma unroll
            for (int i = 0; i < KC; ++i) t.k[i] = load8h<VEC>(kbuf, key * kstep + 2u * (16 * i + 8 * h));
        }
        if constexpr (STAGE_V) {
            // Rows past the sequence read 0 through the range check (which covers voffset + soffset).
#pragma unroll
            for (int i = 0; i < VLOADS; ++i) {
                t.vraw[i] = __builtin_amdgcn_raw_buffer_load_b128(vbuf, static_cast<int>(vv_lane + static_cast<uint32_t>(VRPL * i) * vstep),
                        static_cast<int>(static_cast<uint32_t>(key0) * vstep), 0);
            }
        } else {
            // V[key0 + tile_row(8u + j, h)][32 t2 + col]; lanes past a 16-wide head's last feature read 0.
            const uint32_t vlane = col < ROWS ? static_cast<uint32_t>(key0 + 4 * h) * vstep + 2u * col : kNoRow;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const uint32_t row = static_cast<uint32_t>(16 * u + 8 * (j >> 2) + (j & 3));
#pragma unroll
                    for (int t2 = 0; t2 < DT; ++t2)
                        t.v[t2][u][j] = __builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(vbuf,
                                static_cast<int>(vlane + 64u * t2), static_cast<int>(row * vstep), 0));
                }
            }
        }
    };
    // STAGE_V: the tile's V rows into the slot, rows of masked keys as zeros (they contribute exactly nothing, whatever
    // their stored values hold). The previous tile's reads of the slot are complete first.
    auto stage_v = [&](const Tile &t, const uint32_t bits) __attribute__((always_inline)) {
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < VLOADS; ++i) {
            if (__builtin_expect(bits == 0xffffffffu, 1)) {
                *reinterpret_cast<u32x4 *>(vslot + vwrite + VRPL * i * kVStride<D>) = t.vraw[i];
            } else {
                const bool kept = (bits >> (VRPL * i + vrow)) & 1u;
                __asm__ volatile("" ::: "memory"); // keeps the two stores apart (no select on the common path)
                *reinterpret_cast<u32x4 *>(vslot + vwrite + VRPL * i * kVStride<D>) = kept ? t.vraw[i] : u32x4{0u, 0u, 0u, 0u};
            }
        }
    };

    auto step = [&](Tile &t, const int key0, Tile &next, const int next_key0) __attribute__((always_inline)) {
        const uint32_t bits = key0 < last ? static_cast<uint32_t>(__ballot(t.mask != 0)) : 0u;
        if (bits == 0) {
            load_tile(next, next_key0);
            return;
        }
        f32x16 sc{};
#pragma unroll
        for (int i = 0; i < KC; ++i) sc = mfma16(t.k[i], qr[i], sc);
        __builtin_amdgcn_sched_barrier(0);
        load_tile(next, next_key0);
        // STAGE_V: the tile's V rows go through the slot now, and the operand reads are issued before the softmax,
        // whose VALU work covers their LDS round trip.
        f16x8 vop[DT][2];
        if constexpr (STAGE_V) {
            stage_v(t, bits);
            wave_lds_sync(); // the slot's rows are written
            vop[0][0] = read_v_operand<D, 0, 0>(vslot, vread);
            vop[0][1] = read_v_operand<D, 0, 1>(vslot, vread);
            if constexpr (DT > 1) {
                vop[DT - 1][0] = read_v_operand<D, DT - 1, 0>(vslot, vread);
                vop[DT - 1][1] = read_v_operand<D, DT - 1, 1>(vslot, vread);
            }
        }
        __builtin_amdgcn_sched_barrier(0);

        if (bits != 0xffffffffu || !tile_in_window(s, q0, key0)) {
            const uint32_t visible = (bits & bit_range(wlo - key0, whi - key0)) >> (4 * h);
#pragma unroll
            for (int j = 0; j < 16; ++j) sc[j] = (visible >> (8 * (j >> 2) + (j & 3))) & 1u ? sc[j] : -INFINITY;
            if constexpr (!STAGE_V) { // (staged rows were zeroed by stage_v)
                if (bits != 0xffffffffu) {
                    // Masked keys contribute exactly nothing, whatever their stored values hold.
                    const uint32_t kept = bits >> (4 * h);
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const bool ok = (kept >> (16 * u + 8 * (j >> 2) + (j & 3))) & 1u;
#pragma unroll
                            for (int t2 = 0; t2 < DT; ++t2) t.v[t2][u][j] = ok ? t.v[t2][u][j] : static_cast<_Float16>(0.0f);
                        }
                    }
                }
            }
        }

        float mx = m_half;
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sc[j]);
        m_half = mx;

        auto finish = [&]() __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 16; ++j) sc[j] = exp2_fast(fmaf(sc[j], c2, -mcx));
            float psum = sc[0];
#pragma unroll
            for (int j = 1; j < 16; ++j) psum += sc[j];
            l_run += psum;
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                f16x8 p;
#pragma unroll
                for (int j = 0; j < 8; j += 2) {
                    const f16x2 pair = {static_cast<_Float16>(sc[8 * u + j]), static_cast<_Float16>(sc[8 * u + j + 1])};
                    p[j] = pair[0];
                    p[j + 1] = pair[1];
                }
#pragma unroll
                for (int t2 = 0; t2 < DT; ++t2) {
                    if constexpr (STAGE_V) o[t2] = mfma16(vop[t2][u], p, o[t2]);
                    else o[t2] = mfma16(t.v[t2][u], p, o[t2]);
                }
            }
        };
        if (__builtin_expect(__ballot(m_half > m_lazy) == 0, 1)) {
            finish();
        } else {
            const float m_row = halves_max(m_half);
            const float mc_new = m_row == -INFINITY ? -INFINITY : m_row * c2;
            m_lazy = m_row + lazy_raw;
            const float alpha = mc_new == -INFINITY ? 1.0f : exp2_fast(mc - mc_new);
            l_run *= alpha;
#pragma unroll
            for (int t2 = 0; t2 < DT; ++t2) o[t2] *= alpha;
            mc = mc_new;
            mcx = mc_new == -INFINITY ? 0.0f : mc_new;
            finish();
        }
    };

    const int mine = ntiles > sub ? (ntiles - sub + SPLIT - 1) / SPLIT : 0;
    Tile ta, tb;
    if (mine > 0) load_tile(ta, first + sub * kTile);
    for (int i = 0; i < mine; i += 2) {
        const int key0 = first + (sub + i * SPLIT) * kTile;
        step(ta, key0, tb, key0 + SPLIT * kTile);
        step(tb, key0 + SPLIT * kTile, ta, key0 + 2 * SPLIT * kTile);
    }
    const float mc_run = mc;
    const float m_run = halves_max(m_half);

    float m_all = m_run;
    float base = 0.0f, l_all = l_run;
    if constexpr (SPLIT > 1) {
        constexpr int NREG = 16 * DT;
        __shared__ float partial[kWaves][NREG + 3][kWave];
        if (sub > 0) {
            partial[wave][0][lane] = m_run;
            partial[wave][1][lane] = l_run;
            partial[wave][2 + NREG][lane] = mc_run;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
#pragma unroll
                for (int j = 0; j < 16; ++j) partial[wave][2 + 16 * t + j][lane] = o[t][j];
            }
        }
        __syncthreads();
        if (sub != 0) return;
        float mc_all = mc_run;
#pragma unroll
        for (int x = 1; x < SPLIT; ++x) {
            m_all = fmaxf(m_all, partial[wave + x][0][lane]);
            mc_all = fmaxf(mc_all, partial[wave + x][2 + NREG][lane]);
        }
        base = mc_all == -INFINITY ? 0.0f : mc_all;
        const float a0 = exp2_fast(mc_run - base);
        l_all = l_run * a0;
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= a0;
#pragma unroll
        for (int x = 1; x < SPLIT; ++x) {
            const float aw = exp2_fast(partial[wave + x][2 + NREG][lane] - base);
            l_all = fmaf(partial[wave + x][1][lane], aw, l_all);
#pragma unroll
            for (int t = 0; t < DT; ++t) {
#pragma unroll
                for (int j = 0; j < 16; ++j) o[t][j] = fmaf(partial[wave + x][2 + 16 * t + j][lane], aw, o[t][j]);
            }
        }
    } else {
        base = mc_run == -INFINITY ? 0.0f : mc_run;
    }
    l_all = halves_sum(l_all);
    const float sum_at_max = m_all == -INFINITY ? l_all : l_all * exp2_fast(base - m_all * c2);

    if (!w.valid || query >= s.queries) return;
    const bool nan_row = isnan(l_all);
    const bool has_keys = l_all > 0.0f;
    const float factor = has_keys ? 1.0f / l_all : (nan_row ? NAN : 0.0f);
    _Float16 *orow = out + static_cast<int64_t>(b) * osb + static_cast<int64_t>(head) * osh + static_cast<int64_t>(query) * ost;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int u = 0; u < ROWS / 8; ++u) {
            // Features 32t + 8u + 4h .. +3 of this lane's query: accumulator registers 4u .. 4u + 3.
            f16x4 x;
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = static_cast<_Float16>(has_keys ? o[t][4 * u + i] * factor : factor);
            _Float16 *dst = orow + 32 * t + 8 * u + 4 * h;
            if constexpr (VEC) {
                *reinterpret_cast<f16x4 *>(dst) = x;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) dst[i] = x[i];
            }
        }
    }
    if (h == 0) {
        const int64_t row = static_cast<int64_t>(w.seq) * s.queries + query;
        lse[2 * row] = has_keys ? m_all * scale : (nan_row ? NAN : -INFINITY);
        lse[2 * row + 1] = has_keys ? sum_at_max : (nan_row ? NAN : 0.0f);
    }
}

// Shared K/V tiles: QB = 4 query tiles of one sequence per workgroup (d = 64, 16-byte aligned rows, every stride a
// multiple of 8). Wave w of the workgroup owns query tile 4·block + w mod 4 and key stream w / 4: the KS streams take
// alternate key tiles of the union of the workgroup's windows. The four waves of a stream stream its tiles together:
// each loads a quarter of a tile's K and V rows (one 16-byte chunk per lane of each, whole 128-byte lines) straight into
// the stream's double-buffered LDS stage (buffer loads with the LDS bit: no registers, no LDS store instructions), which
// all of them read, so every K/V byte crosses from L2 once per four waves instead of once per wave. Per step: one
// workgroup barrier (its fence waits for this wave's loads, so after it every wave's share of the tile is in place and
// every wave is done reading the other stage); then the loads of the next tile into the other stage; then each wave
// whose window meets the tile computes it as attention_forward_f16_kernel does (K's row layout read with 128-bit LDS
// reads, V's operand with transposing reads; V elements of masked keys are zeroed in registers, only on tiles with a
// masked key). Loads write 64 consecutive 16-byte chunks per instruction, so the stage rows are unpadded and the
// chunks of each row are permuted (an XOR of the chunk index with a function of the row) to keep the reads free of
// bank conflicts. Every wave runs every step (the barriers are uniform); a wave past the last query tile or outside the
// tile's window only loads its share. With KS = 2 the second stream's softmax state is merged into the first through
// LDS at the end (a fixed order: deterministic). The kernel is held to 128 VGPRs, so four waves fit on every SIMD.
template<int D, int QB, int KS>
__global__ __launch_bounds__(kWave * QB * KS) __attribute__((amdgpu_waves_per_eu(4))) void attention_forward_f16_shared_kernel(
        const TensorH q, const TensorH k, const TensorH v, const uint8_t *__restrict__ mask, _Float16 *__restrict__ out,
        const int osb, const int osh, const int ost, float *__restrict__ lse, const Shape s, const float scale) {
    static_assert(D == 64, "shared K/V tiles are for 64-wide heads (at d = 32 the per-wave kernel is faster)");
    static_assert(QB == 4 && (KS == 1 || KS == 2));
    constexpr int KC = D / 16;                  // MFMAs per Sᵀ tile
    constexpr int DT = D / 32;                  // 32-feature output slices
    constexpr int CPR = D / 8;                  // 16-byte chunks per row
    static_assert(kTile * CPR == QB * kWave, "each wave of a stream loads one chunk per lane of a K tile and of a V tile");
    constexpr int TILE = kTile * D;             // halves of one staged K or V tile (rows D halves apart)
    constexpr int STAGE_BYTES = 2 * KS * 2 * TILE * 2;
    constexpr int NREG = 16 * DT + 3;           // merged per lane: m, l, mc and the output accumulators
    constexpr int MERGE_BYTES = KS > 1 ? QB * NREG * kWave * 4 : 0;
    __shared__ __align__(16) unsigned char smem[STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES];
    // Stage (stream x, parity p): the K tile, then the V tile.
    auto kstage = [&](const int x, const int p) { return reinterpret_cast<_Float16 *>(smem) + (2 * x + p) * (2 * TILE); };
    auto vstage = [&](const int x, const int p) { return kstage(x, p) + TILE; };
    // Chunk c of row r is stored at position c ^ kswz(r) (K) or c ^ vswz(r) (V) of the row. K's row-layout reads (16
    // lanes: 16 rows, one chunk each) then meet 16 distinct 16-byte bank groups, and V's transposing reads (16 lanes: 4
    // rows of 32 bytes) 8; the V permutation leaves rows 4 apart alike, so a read 8 or 16 rows further is an offset.
    auto kswz = [](const int r) { return (r & 7) ^ ((r >> 3) & 1); };
    auto vswz = [](const int r) { return 2 * (r & 3); };

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int qi = wave % QB;     // query tile of the workgroup
    const int stream = wave / QB; // key stream
    const int col = lane & 31;
    const int h = lane >> 5;
    const float c2 = scale * kLog2e;

    // Workgroup g takes query block g / seqs of sequence g % seqs: with B·H a multiple of 8 (workgroup g runs on XCD
    // g mod 8), each XCD streams the K/V rows of its own eighth of the sequences from its L2.
    const int seqs = s.batch * s.heads;
    const int seq = static_cast<int>(blockIdx.x) % seqs;
    const int qb = static_cast<int>(blockIdx.x) / seqs;
    const int b = seq / s.heads, head = seq - b * s.heads;
    const int q0 = (qb * QB + qi) * kTile;
    const int query = q0 + col;
    const bool tile_valid = q0 < s.queries;

    // Keys [first, last) seen by query tile t0's queries.
    auto key_window = [&](const int t0, int &first, int &last) __attribute__((always_inline)) {
        first = 0;
        last = s.keys;
        if (s.radius >= 0) {
            first = max(0, t0 - s.radius);
            last = min(last, t0 + kTile + s.radius);
        }
    };
    // This wave's window, and the workgroup's union (from its first query tile's start to its last valid one's end).
    int first, last, ufirst, ulast, unused;
    key_window(q0, first, last);
    key_window(qb * QB * kTile, ufirst, unused);
    key_window(min(qb * QB + QB - 1, (s.queries - 1) / kTile) * kTile, unused, ulast);
    const int ntiles = ulast > ufirst ? (ulast - ufirst + kTile - 1) / kTile : 0;
    const int nsteps = (ntiles + KS - 1) / KS; // steps of every stream; tile of stream x at step i: i·KS + x
    const int wlo = window_lo(s, query);
    const int whi = window_hi(s, query);

    auto seq_base = [&](const TensorH &t) {
        return t.data + (static_cast<int64_t>(b) * t.sb + static_cast<int64_t>(head) * t.sh);
    };
    const Buffer qbuf = make_buffer(seq_base(q), sequence_bytes_h(s.queries, q.st, D));
    const Buffer kbuf = make_buffer(seq_base(k), sequence_bytes_h(s.keys, k.st, D));
    const Buffer vbuf = make_buffer(seq_base(v), sequence_bytes_h(s.keys, v.st, D));
    const Buffer mbuf = make_buffer(mask + static_cast<int64_t>(b) * s.keys, static_cast<uint32_t>(s.keys));
    const uint32_t kstep = 2u * k.st;
    const uint32_t vstep = 2u * v.st;

    f16x8 qr[KC];
#pragma unroll
    for (int i = 0; i < KC; ++i)
        qr[i] = load8h<true>(qbuf, tile_valid ? static_cast<uint32_t>(query) * (2u * q.st) + 2u * (16 * i + 8 * h) : kNoRow);

    // This lane's load of a stream tile fills stage chunk 64·qi + lane: row lrow, position lane mod 8, i.e. the
    // row's chunk (lane mod 8) ^ swz(lrow). Its offset within a tile is fixed (voffset); the tile's row offset is
    // scalar (soffset), and a tile past the last one gets soffset kNoRow, read as 0 by the range check (which covers
    // voffset + soffset), as are rows past the sequence's end.
    const int lrow = (kWave * qi + lane) / CPR;
    const uint32_t kv_lane = static_cast<uint32_t>(lrow) * kstep + 16u * static_cast<uint32_t>((lane & 7) ^ kswz(lrow));
    const uint32_t vv_lane = static_cast<uint32_t>(lrow) * vstep + 16u * static_cast<uint32_t>((lane & 7) ^ vswz(lrow));
    // Issues step i's loads into stage p: K and V rows into LDS, the tile's mask bytes (one per key, lane col) into the
    // returned register.
    auto issue = [&](const int i, const int p) __attribute__((always_inline)) {
        const int t = i * KS + stream;
        const bool live = t < ntiles;
        const uint32_t key0 = static_cast<uint32_t>(ufirst + t * kTile);
        const int mbyte = buffer_load_byte_s(mbuf, static_cast<uint32_t>(col), live ? key0 : kNoRow); // keys past the end read 0
        __builtin_amdgcn_raw_ptr_buffer_load_lds(kbuf, (__attribute__((address_space(3))) void *)(kstage(stream, p) + kWave * 8 * qi), 16,
                static_cast<int>(kv_lane), static_cast<int>(live ? key0 * kstep : kNoRow), 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(vbuf, (__attribute__((address_space(3))) void *)(vstage(stream, p) + kWave * 8 * qi), 16,
                static_cast<int>(vv_lane), static_cast<int>(live ? key0 * vstep : kNoRow), 0, 0);
        return mbyte;
    };

    constexpr float kLazy = 8.0f; // p = exp2(s·c2 - mc) <= 2^8: also within fp16 range
    const float lazy_raw = kLazy / c2;
    float m_half = -INFINITY, m_lazy = -INFINITY, mc = -INFINITY, mcx = 0.0f, l_run = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x16{};
    // Lane offsets (halves) of this lane's reads within a stage: K rows col, chunks 2i + h (row layout); V as the
    // transposing reads of read_v_operand address them (16-lane group: rows 4h + (lane mod 16) / 4, features
    // 32 t2 + 16 ((lane / 16) mod 2) + 4 (lane mod 4)), permuted as the loads stored them.
    int kread[KC];
#pragma unroll
    for (int i = 0; i < KC; ++i) kread[i] = col * D + 8 * ((2 * i + h) ^ kswz(col));
    int vread[DT];
#pragma unroll
    for (int t2 = 0; t2 < DT; ++t2) {
        const int vrow = 4 * h + ((lane & 15) >> 2);
        const int chunk = 4 * t2 + 2 * ((lane >> 4) & 1) + ((lane & 3) >> 1);
        vread[t2] = vrow * D + 8 * (chunk ^ vswz(vrow)) + 4 * (lane & 1);
    }

    // The MFMA operands of the tile in this stream's stage p: K's row layout (Sᵀ A operands) and V's transposed layout
    // (Oᵀ A operands).
    struct Operands {
        f16x8 k[KC];
        f16x8 v[DT][2];
    };
    auto read_operands = [&](Operands &op, const int p) __attribute__((always_inline)) {
        const _Float16 *ks = kstage(stream, p);
        const _Float16 *vs = vstage(stream, p);
#pragma unroll
        for (int i = 0; i < KC; ++i) op.k[i] = *reinterpret_cast<const f16x8 *>(ks + kread[i]);
#pragma unroll
        for (int t2 = 0; t2 < DT; ++t2) {
            op.v[t2][0] = read_v_operand<D, 0, 0, D>(vs, vread[t2]);
            op.v[t2][1] = read_v_operand<D, 0, 1, D>(vs, vread[t2]);
        }
    };
    // The product of the tile at key0 for this wave's query tile.
    auto compute = [&](Operands &op, const int key0, const uint32_t bits) __attribute__((always_inline)) {
        auto &vop = op.v;
        f32x16 sc{};
#pragma unroll
        for (int i = 0; i < KC; ++i) sc = mfma16(op.k[i], qr[i], sc);
        if (bits != 0xffffffffu || !tile_in_window(s, q0, key0)) {
            const uint32_t visible = (bits & bit_range(wlo - key0, whi - key0)) >> (4 * h);
#pragma unroll
            for (int j = 0; j < 16; ++j) sc[j] = (visible >> (8 * (j >> 2) + (j & 3))) & 1u ? sc[j] : -INFINITY;
            if (bits != 0xffffffffu) {
                // Masked keys contribute exactly nothing, whatever their stored V rows hold: element j of operand u
                // is key 16u + 8 (j / 4) + 4h + j mod 4.
                const uint32_t kept = bits >> (4 * h);
#pragma unroll
                for (int t2 = 0; t2 < DT; ++t2) {
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            vop[t2][u][j] = (kept >> (16 * u + 8 * (j >> 2) + (j & 3))) & 1u ? vop[t2][u][j] : static_cast<_Float16>(0.0f);
                    }
                }
            }
        }
        float mx = m_half;
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, sc[j]);
        m_half = mx;
        if (__builtin_expect(__ballot(m_half > m_lazy) != 0, 0)) {
            const float m_row = halves_max(m_half);
            const float mc_new = m_row == -INFINITY ? -INFINITY : m_row * c2;
            m_lazy = m_row + lazy_raw;
            const float alpha = mc_new == -INFINITY ? 1.0f : exp2_fast(mc - mc_new);
            l_run *= alpha;
#pragma unroll
            for (int t2 = 0; t2 < DT; ++t2) o[t2] *= alpha;
            mc = mc_new;
            mcx = mc_new == -INFINITY ? 0.0f : mc_new;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) sc[j] = exp2_fast(fmaf(sc[j], c2, -mcx));
        float psum = sc[0];
#pragma unroll
        for (int j = 1; j < 16; ++j) psum += sc[j];
        l_run += psum;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            f16x8 pv;
#pragma unroll
            for (int j = 0; j < 8; ++j) pv[j] = static_cast<_Float16>(sc[8 * u + j]);
#pragma unroll
            for (int t2 = 0; t2 < DT; ++t2) o[t2] = mfma16(vop[t2][u], pv, o[t2]);
        }
    };

    // Step i of stream x: tile i·KS + x, loaded into stage i mod 2 during step i - 1. A step: barrier (its fence waits
    // for this wave's outstanding loads: stage i mod 2 is complete, and every wave is done reading the other stage);
    // the operands of step i's tile from the stage; step i + 1's loads into the other stage; then step i's product: the
    // loads have the product and the barrier to land. The operand reads come before the loads are issued: the compiler
    // makes an LDS read that follows an LDS-bound load wait for that load, whatever the addresses. The loop runs the
    // steps in pairs (stages 0 and 1 at fixed offsets; an odd count gets one empty step).
    if (nsteps > 0) {
        int mnext = issue(0, 0);
        auto step = [&](const int i, const int p) __attribute__((always_inline)) {
            __syncthreads();
            const uint32_t bits = static_cast<uint32_t>(__ballot(mnext != 0));
            const int t = i * KS + stream;
            const int key0 = ufirst + t * kTile;
            const bool work = t < ntiles && tile_valid && bits != 0 && key0 < last && key0 + kTile > first;
            Operands op;
            if (work) read_operands(op, p);
            __builtin_amdgcn_sched_barrier(0);
            mnext = issue(i + 1, p ^ 1);
            __builtin_amdgcn_sched_barrier(0);
            if (work) compute(op, key0, bits);
        };
        for (int i = 0; i < nsteps; i += 2) {
            step(i, 0);
            step(i + 1, 1);
        }
        // The last step's loads (past the last tile: zeros) write LDS: they land before the stages are reused or the
        // workgroup ends.
        __syncthreads();
    }

    const float m_run = halves_max(m_half);
    float m_all = m_run, base = mc == -INFINITY ? 0.0f : mc, l_all = l_run;
    if constexpr (KS > 1) {
        // Stream 1 hands (row maximum, sum, base, accumulators) to stream 0 through LDS; stream 0 rescales both to the
        // larger base and adds.
        float *const slot = reinterpret_cast<float *>(smem) + qi * (NREG * kWave) + lane;
        __syncthreads(); // every wave is done with the stages
        if (stream == 1) {
            slot[0] = m_run;
            slot[kWave] = l_run;
            slot[2 * kWave] = mc;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
#pragma unroll
                for (int j = 0; j < 16; ++j) slot[(3 + 16 * t + j) * kWave] = o[t][j];
            }
        }
        __syncthreads();
        if (stream == 1) return;
        const float m1 = slot[0], l1 = slot[kWave], mc1 = slot[2 * kWave];
        m_all = fmaxf(m_run, m1);
        const float mc_all = fmaxf(mc, mc1);
        base = mc_all == -INFINITY ? 0.0f : mc_all;
        const float a0 = exp2_fast(mc - base), a1 = exp2_fast(mc1 - base);
        l_all = fmaf(l1, a1, l_run * a0);
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int j = 0; j < 16; ++j) o[t][j] = fmaf(slot[(3 + 16 * t + j) * kWave], a1, o[t][j] * a0);
        }
    }

    if (!tile_valid || query >= s.queries) return;
    l_all = halves_sum(l_all);
    const float sum_at_max = m_all == -INFINITY ? l_all : l_all * exp2_fast(base - m_all * c2);
    const bool nan_row = isnan(l_all);
    const bool has_keys = l_all > 0.0f;
    const float factor = has_keys ? 1.0f / l_all : (nan_row ? NAN : 0.0f);
    _Float16 *orow = out + static_cast<int64_t>(b) * osb + static_cast<int64_t>(head) * osh + static_cast<int64_t>(query) * ost;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            f16x4 x;
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = static_cast<_Float16>(has_keys ? o[t][4 * u + i] * factor : factor);
            *reinterpret_cast<f16x4 *>(orow + 32 * t + 8 * u + 4 * h) = x;
        }
    }
    if (h == 0) {
        const int64_t row = static_cast<int64_t>(seq) * s.queries + query;
        lse[2 * row] = has_keys ? m_all * scale : (nan_row ? NAN : -INFINITY);
        lse[2 * row + 1] = has_keys ? sum_at_max : (nan_row ? NAN : 0.0f);
    }
}

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }
bool strides8(const rocmkernels_strides &s) { return ((s.batch | s.head | s.token) & 7) == 0; }
bool strides4(const rocmkernels_strides &s) { return ((s.batch | s.head | s.token) & 3) == 0; }

// Buffer resources use 32-bit byte offsets: every sequence, padded by one 32-row tile, must span less than 2 GiB.
bool fits_h(const int rows, const rocmkernels_strides &s, const int width) {
    const long long extent = (static_cast<long long>(rows) + 32) * s.token + width;
    return s.token >= 0 && extent * 2 < (1ll << 31);
}

TensorH tensor_h(const void *p, const rocmkernels_strides &s) {
    return TensorH{static_cast<const _Float16 *>(p), s.batch, s.head, s.token};
}

template<int D, int QB, int KS>
void launch_shared(const HalfForwardArgs &a, const int64_t groups, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, 0};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    hipLaunchKernelGGL((attention_forward_f16_shared_kernel<D, QB, KS>), dim3(static_cast<unsigned>(groups)), dim3(kWave * QB * KS), 0,
            stream,
            tensor_h(a.q, a.qs), tensor_h(a.k, a.ks), tensor_h(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask),
            static_cast<_Float16 *>(a.output), a.os.batch, a.os.head, a.os.token, a.lse, shape, scale);
}

template<int D, bool VEC, int SPLIT, bool STAGE_V>
void launch(const HalfForwardArgs &a, const int64_t items, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, 0};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    hipLaunchKernelGGL((attention_forward_f16_kernel<D, VEC, SPLIT, STAGE_V>), dim3(workgroups_for(items, SPLIT)), dim3(kThreads), 0, stream,
            tensor_h(a.q, a.qs), tensor_h(a.k, a.ks), tensor_h(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask),
            static_cast<_Float16 *>(a.output), a.os.batch, a.os.head, a.os.token, a.lse, shape, scale);
}

// Waves per item: the fewest of 1, 2 and 4 that still give every SIMD its resident waves (two at d = 64, three at
// d = 32, four at d = 16). An fp16 tile costs a fraction of an FP32 one, so a wave's start and the merge of an item's
// waves weigh more here than in the FP32 kernel, whose own rule (forward_split_for) keeps more waves per item. Measured
// on the generic fp16 forward: 32 x 2048 x 64 82.1 -> 76.7 µs and 16 x 8192 x 64 (radius 256) 65.5 -> 54.6 µs with one
// wave per item; 24 x 2048 x 64 62.7 µs with two against 64.8 with four; 24 x 1024 x 32 keeps four (14.0 µs against
// 14.7 with two and 17.6 with one).
int f16_split_for(const int64_t items, const int D, const int cus) {
    const int64_t slots = static_cast<int64_t>(cus) * kWaves * (D == 64 ? 2 : D == 32 ? 3 : 4);
    if (items >= slots) return 1;
    if (2 * items >= slots) return 2;
    return 4;
}

template<int D, bool VEC, bool STAGE_V>
void launch_split(const HalfForwardArgs &a, const int64_t items, const int split, hipStream_t stream) {
    if (split == 1) launch<D, VEC, 1, STAGE_V>(a, items, stream);
    else if (split == 2) launch<D, VEC, 2, STAGE_V>(a, items, stream);
    else launch<D, VEC, 4, STAGE_V>(a, items, stream);
}

template<int D>
void dispatch(const HalfForwardArgs &a, const int64_t items, const int cus, hipStream_t stream) {
    // 128-bit row loads need 16-byte aligned rows; the output's 4-half stores 8-byte alignment.
    const bool vec = aligned16(a.q) && aligned16(a.k) && strides8(a.qs) && strides8(a.ks) && aligned8(a.output) && strides4(a.os);
    const int split = f16_split_for(items, D, cus);
    // V rows staged through LDS need 16-byte aligned rows too (d = 32 and 64).
    bool stage = false;
    if constexpr (D >= 32) stage = vec && aligned16(a.v) && strides8(a.vs);
    if (stage) {
        if constexpr (D >= 32) {
            // d = 64: shared K/V tiles (four query tiles per workgroup) when those workgroups give every CU one; two key
            // streams per workgroup (eight waves) until there are four workgroups per CU, so that each SIMD holds four
            // waves. Measured on the generic fp16 forward (the per-wave kernel against the shared one): 32 x 2048
            // 76.7 -> 48.3 µs (two streams; one: 51.8), 16 x 8192 radius 256 51.9 -> 34.7 µs (one stream), 8 x 16 x
            // 1024 80.9 -> 49.9 µs. At d = 32 the per-wave kernel stays: its tiles carry half the bytes, and the
            // shared kernel's barrier per tile cost more than the loads it saves (24 x 1024 9.6 against 13.5 µs,
            // 2 x 16 x 2048 radius 300 14.3 against 17.1 µs, 4 x 8 x 2048 37.1 against 36.0 µs).
            if constexpr (D == 64) {
                const int64_t seqs = static_cast<int64_t>(a.batch) * a.heads;
                const int64_t groups = seqs * ((a.queries + 4 * kTile - 1) / (4 * kTile));
                if (groups >= cus) {
                    if (groups >= 4 * cus) launch_shared<64, 4, 1>(a, groups, stream);
                    else launch_shared<64, 4, 2>(a, groups, stream);
                    return;
                }
            }
            launch_split<D, true, true>(a, items, split, stream);
        }
    } else if (vec) {
        launch_split<D, true, false>(a, items, split, stream);
    } else {
        launch_split<D, false, false>(a, items, split, stream);
    }
}

} // namespace

hipError_t launch_forward_f16(const int D, const HalfForwardArgs &a, hipStream_t stream) {
    const int64_t items = static_cast<int64_t>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    if (items > 0x7fffffff || !fits_h(a.queries, a.qs, D) || !fits_h(a.keys, a.ks, D) || !fits_h(a.keys, a.vs, D)) return hipErrorInvalidValue;
    int cus = 0;
    const hipError_t error = compute_units(cus);
    if (error != hipSuccess) return error;
    if (D == 16) dispatch<16>(a, items, cus, stream);
    else if (D == 32) dispatch<32>(a, items, cus, stream);
    else dispatch<64>(a, items, cus, stream);
    return hipGetLastError();
}

} // namespace rk
