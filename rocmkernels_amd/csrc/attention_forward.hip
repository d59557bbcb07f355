// FP32 online-softmax attention forward for gfx950 (MI355X), head width 32 or 64.
//
// Replaces the reference's forward kernels: attention_query<false> (Attention.hip:32-115),
// attention_query_tiled_body (AttentionTile32.h:12-208), attention_query_flash_body (AttentionFlash32.h:23-170),
// the statistics-only instance (Attention.hip:252-261) and attention64_query<false> (Attention64.hip:34-129).
// The maths is the same (O = softmax(QKᵀ/√D + mask) V with lse = {max, Σexp(s - max)}); the mapping is not:
//
//   * A workgroup owns one 32-query tile of one (batch, head) and runs 4 waves, one per SIMD. The waves split
//     the 32-key tiles of the query tile's key range round-robin, each keeping its own online-softmax state
//     (m, l, Oᵀ), and merge once through LDS at the end. That bounds the longest workgroup to a quarter of a
//     row, which matters at the causal 24x1024 shape where rows are short and the grid is small.
//   * Sᵀ = K·Qᵀ and Oᵀ += Vᵀ·Pᵀ run on v_mfma_f32_32x32x2f32; the Sᵀ accumulator register j is the B operand
//     of Oᵀ MFMA j, so P never leaves registers. Each lane owns one query, so the row maximum is 15 VALU max
//     plus one exchange with the other half-wave, and the rescale of Oᵀ is lane-local.
//   * exp(s - m) is evaluated as exp2(s·(log2e/√D) - m·(log2e/√D)) with one FMA feeding v_exp_f32.
//   * blockIdx → work: the heaviest query tiles (the last ones under a causal mask) are dispatched first, and
//     consecutive workgroups take consecutive (batch, head) pairs of the same tile, so with B·H a multiple of 8
//     each XCD keeps a fixed subset of sequences in its own L2.
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

template<int D, bool STATS, bool VEC>
__global__ __launch_bounds__(kThreads) void attention_forward_kernel(const Tensor q, const Tensor k, const Tensor v,
        const uint8_t *__restrict__ mask, float *__restrict__ out, const int osb, const int osh, const int ost,
        float *__restrict__ lse, const Shape s, const float scale) {
    constexpr int HALF = D / 2; // features per lane in row layout
    constexpr int DT = D / 32;  // 32-feature slices of the output
    constexpr int NREG = STATS ? 0 : 16 * DT;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 31;
    const int h = lane >> 5;

    const int seqs = s.batch * s.heads;
    const int qtiles = (s.queries + kTile - 1) / kTile;
    const int rank = blockIdx.x / seqs;
    const int seq = blockIdx.x - rank * seqs;
    const int qt = s.causal ? qtiles - 1 - rank : rank;
    const int b = seq / s.heads;
    const int head = seq - b * s.heads;
    const int q0 = qt * kTile;
    const int query = q0 + col;
    const float c2 = scale * kLog2e;

    int first = 0, last = s.keys;
    if (s.radius >= 0) {
        first = max(0, q0 - s.radius);
        last = min(last, q0 + kTile + s.radius);
    }
    if (s.causal) last = min(last, q0 + kTile);
    const int ntiles = last > first ? (last - first + kTile - 1) / kTile : 0;

    float qr[HALF];
    load_span<VEC>(qr, sequence(q, b, head) + static_cast<int64_t>(query) * q.st + h * HALF, query < s.queries);

    const float *kbase = sequence(k, b, head);
    const float *vbase = sequence(v, b, head);
    const uint8_t *mrow = mask + static_cast<int64_t>(b) * s.keys;

    float m_run = -INFINITY;
    float l_run = 0.0f;
    f32x16 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x16{};

    for (int tile = wave; tile < ntiles; tile += kWaves) {
        const int key0 = first + tile * kTile;
        const int key = key0 + col;
        const bool in_range = key < s.keys;
        const bool visible = in_range && mrow[key] != 0;
        const uint32_t bits = static_cast<uint32_t>(__ballot(visible));
        if (bits == 0) continue; // every key of the tile is masked: contributes nothing

        float kr[HALF];
        load_span<VEC>(kr, kbase + static_cast<int64_t>(key) * k.st + h * HALF, in_range);
        float vc[DT][16];
        if constexpr (!STATS) {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int r = tile_row(j, h);
                const bool ok = (bits >> r) & 1u;
                const float *vrow = vbase + static_cast<int64_t>(key0 + r) * v.st + col;
#pragma unroll
                for (int t = 0; t < DT; ++t) vc[t][j] = ok ? vrow[32 * t] : 0.0f;
            }
        }

        f32x16 sc{};
#pragma unroll
        for (int c = 0; c < HALF; ++c) sc = mfma(kr[c], qr[c], sc);

        const bool full = bits == 0xffffffffu && tile_in_window(s, q0, key0);
        if (!full) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = tile_row(v, h);
                const bool ok = ((bits >> r) & 1u) && in_window(s, query, key0 + r);
                sc[v] = ok ? sc[v] : -INFINITY;
            }
        }

        float mx = sc[0];
#pragma unroll
        for (int v = 1; v < 16; ++v) mx = fmaxf(mx, sc[v]);
        mx = fmaxf(mx, other_half(mx));
        const float m_new = fmaxf(m_run, mx);
        const float mc = m_new == -INFINITY ? 0.0f : m_new * c2;
        const float alpha = exp2_fast(fmaf(m_run, c2, -mc));
        float psum = 0.0f;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            sc[v] = exp2_fast(fmaf(sc[v], c2, -mc));
            psum += sc[v];
        }
        l_run = fmaf(l_run, alpha, psum);
        m_run = m_new;

        if constexpr (!STATS) {
#pragma unroll
            for (int t = 0; t < DT; ++t) o[t] *= alpha;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
#pragma unroll
                for (int t = 0; t < DT; ++t) o[t] = mfma(vc[t][j], sc[j], o[t]);
            }
        }
    }

    // Merge the per-wave states of the workgroup: waves 1..3 publish (m, l, Oᵀ) in LDS, wave 0 combines.
    __shared__ float partial[kWaves - 1][NREG + 2][kWave];
    if (wave > 0) {
        partial[wave - 1][0][lane] = m_run;
        partial[wave - 1][1][lane] = l_run;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                if constexpr (!STATS) partial[wave - 1][2 + 16 * t + v][lane] = o[t][v];
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;

    float m_all = m_run;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w) m_all = fmaxf(m_all, partial[w][0][lane]);
    const float mc = m_all == -INFINITY ? 0.0f : m_all * c2;
    const float a0 = exp2_fast(fmaf(m_run, c2, -mc));
    float l_all = l_run * a0;
    if constexpr (!STATS) {
#pragma unroll
        for (int t = 0; t < DT; ++t) o[t] *= a0;
    }
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w) {
        const float aw = exp2_fast(fmaf(partial[w][0][lane], c2, -mc));
        l_all = fmaf(partial[w][1][lane], aw, l_all);
        if constexpr (!STATS) {
#pragma unroll
            for (int t = 0; t < DT; ++t) {
#pragma unroll
                for (int v = 0; v < 16; ++v) o[t][v] = fmaf(partial[w][2 + 16 * t + v][lane], aw, o[t][v]);
            }
        }
    }
    l_all += other_half(l_all); // each half-wave summed the exponentials of its own 16 keys per tile

    if (query >= s.queries) return;
    const bool nan_row = isnan(l_all);
    const bool has_keys = l_all > 0.0f;
    if constexpr (!STATS) {
        const float factor = has_keys ? 1.0f / l_all : (nan_row ? NAN : 0.0f);
        float *orow = out + static_cast<int64_t>(b) * osb + static_cast<int64_t>(head) * osh + static_cast<int64_t>(query) * ost;
#pragma unroll
        for (int t = 0; t < DT; ++t) {
            if (has_keys) {
                store_tile_row<VEC>(orow + 32 * t, o[t], factor, h);
            } else {
                const f32x16 fill{};
                store_tile_row<VEC>(orow + 32 * t, fill + factor, 1.0f, h);
            }
        }
    }
    if (h == 0) {
        const int64_t row = static_cast<int64_t>(seq) * s.queries + query;
        lse[2 * row] = has_keys ? m_all * scale : (nan_row ? NAN : -INFINITY);
        lse[2 * row + 1] = has_keys ? l_all : (nan_row ? NAN : 0.0f);
    }
}

namespace {

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool strides4(const rocmkernels_strides &s) { return ((s.batch | s.head | s.token) & 3) == 0; }

template<int D, bool STATS, bool VEC>
void launch(const ForwardArgs &a, const dim3 grid, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    hipLaunchKernelGGL((attention_forward_kernel<D, STATS, VEC>), grid, dim3(kThreads), 0, stream, Tensor{a.q, a.qs.batch, a.qs.head, a.qs.token},
            Tensor{a.k, a.ks.batch, a.ks.head, a.ks.token}, Tensor{a.v, a.vs.batch, a.vs.head, a.vs.token},
            reinterpret_cast<const uint8_t *>(a.mask), a.output, a.os.batch, a.os.head, a.os.token, a.lse, shape, scale);
}

template<int D>
void dispatch(const bool statistics_only, const ForwardArgs &a, const dim3 grid, hipStream_t stream) {
    bool vec = aligned16(a.q) && aligned16(a.k) && strides4(a.qs) && strides4(a.ks);
    if (!statistics_only) vec = vec && aligned16(a.v) && aligned16(a.output) && strides4(a.vs) && strides4(a.os);
    if (statistics_only) {
        if (vec) launch<D, true, true>(a, grid, stream);
        else launch<D, true, false>(a, grid, stream);
    } else {
        if (vec) launch<D, false, true>(a, grid, stream);
        else launch<D, false, false>(a, grid, stream);
    }
}

} // namespace

hipError_t launch_forward(const int D, const bool statistics_only, const ForwardArgs &a, hipStream_t stream) {
    const int64_t tiles = static_cast<int64_t>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    if (tiles > 0x7fffffff) return hipErrorInvalidValue;
    const dim3 grid(static_cast<unsigned>(tiles));
    if (D == 32) dispatch<32>(statistics_only, a, grid, stream);
    else dispatch<64>(statistics_only, a, grid, stream);
    return hipGetLastError();
}

} // namespace rk
