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
// In both, the 4 waves of a workgroup split the streamed tiles and sum their partial gradients through LDS.
// Kernel 2 reads the δ that kernel 1 wrote; they are ordered by the stream, as in the reference
// (Attention.hip:211-221).
#include "attention_device.hpp"
#include "attention_launch.hpp"

namespace rk {

enum DqMode { kDqAndDelta = 0, kDeltaOnly = 1, kDqFromDelta = 2 };

template<int D, int MODE, bool VEC>
__global__ __launch_bounds__(kThreads) void attention_dq_kernel(const Tensor q, const Tensor k, const Tensor v,
        const uint8_t *__restrict__ mask, const Tensor o, const float *__restrict__ lse, const Tensor du,
        float *__restrict__ dq, float *__restrict__ delta, const Shape s, const float scale) {
    constexpr int HALF = D / 2;
    constexpr int DT = D / 32;

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
    const bool qvalid = query < s.queries;
    const int64_t row = static_cast<int64_t>(seq) * s.queries + query;
    const float c2 = scale * kLog2e;

    float dor[HALF];
    load_span<VEC>(dor, sequence(du, b, head) + static_cast<int64_t>(query) * du.st + h * HALF, qvalid);

    float dlt;
    if constexpr (MODE == kDqFromDelta) {
        dlt = qvalid ? delta[row] : 0.0f;
    } else {
        float orow[HALF];
        load_span<VEC>(orow, sequence(o, b, head) + static_cast<int64_t>(query) * o.st + h * HALF, qvalid);
        dlt = 0.0f;
#pragma unroll
        for (int c = 0; c < HALF; ++c) dlt = fmaf(dor[c], orow[c], dlt);
        dlt = halves_sum(dlt);
        if (wave == 0 && h == 0 && qvalid) delta[row] = dlt;
        if constexpr (MODE == kDeltaOnly) return;
    }

    float qr[HALF];
    load_span<VEC>(qr, sequence(q, b, head) + static_cast<int64_t>(query) * q.st + h * HALF, qvalid);
    const float m = qvalid ? lse[2 * row] : -INFINITY;
    const float l = qvalid ? lse[2 * row + 1] : 0.0f;
    const bool row_ok = m != -INFINITY;
    const float mc = row_ok ? m * kLog2e : INFINITY; // exp2(x - inf) = 0 for a row without visible keys
    const float il = row_ok ? 1.0f / l : 0.0f;

    int first = 0, last = s.keys;
    if (s.radius >= 0) {
        first = max(0, q0 - s.radius);
        last = min(last, q0 + kTile + s.radius);
    }
    if (s.causal) last = min(last, q0 + kTile);
    const int ntiles = last > first ? (last - first + kTile - 1) / kTile : 0;

    const float *kbase = sequence(k, b, head);
    const float *vbase = sequence(v, b, head);
    const uint8_t *mrow = mask + static_cast<int64_t>(b) * s.keys;

    f32x16 acc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) acc[t] = f32x16{};

    for (int tile = wave; tile < ntiles; tile += kWaves) {
        const int key0 = first + tile * kTile;
        const int key = key0 + col;
        const bool in_range = key < s.keys;
        const bool visible = in_range && mrow[key] != 0;
        const uint32_t bits = static_cast<uint32_t>(__ballot(visible));
        if (bits == 0) continue;

        float kr[HALF], vr[HALF];
        load_span<VEC>(kr, kbase + static_cast<int64_t>(key) * k.st + h * HALF, in_range);
        load_span<VEC>(vr, vbase + static_cast<int64_t>(key) * v.st + h * HALF, in_range);
        float kc[DT][16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = tile_row(j, h);
            const bool ok = (bits >> r) & 1u;
            const float *krow = kbase + static_cast<int64_t>(key0 + r) * k.st + col;
#pragma unroll
            for (int t = 0; t < DT; ++t) kc[t][j] = ok ? krow[32 * t] : 0.0f;
        }

        f32x16 sc{}, dp{};
#pragma unroll
        for (int c = 0; c < HALF; ++c) {
            sc = mfma(kr[c], qr[c], sc);
            dp = mfma(vr[c], dor[c], dp);
        }

        const bool full = bits == 0xffffffffu && tile_in_window(s, q0, key0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const float p = exp2_fast(fmaf(sc[v], c2, -mc)) * il;
            float ds = p * (dp[v] - dlt);
            if (!full) {
                const int r = tile_row(v, h);
                const bool ok = ((bits >> r) & 1u) && key0 + r >= window_lo(s, query) && key0 + r <= window_hi(s, query);
                ds = ok ? ds : 0.0f;
            }
            sc[v] = ds;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
#pragma unroll
            for (int t = 0; t < DT; ++t) acc[t] = mfma(kc[t][j], sc[j], acc[t]);
        }
    }

    __shared__ float partial[kWaves - 1][16 * DT][kWave];
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) partial[wave - 1][16 * t + v][lane] = acc[t][v];
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[t][v] += partial[w][16 * t + v][lane];
        }
    }
    if (!qvalid) return;
    float *dst = dq + row * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) store_tile_row<VEC>(dst + 32 * t, acc[t], scale, h);
}

template<int D, bool VEC>
__global__ __launch_bounds__(kThreads) void attention_dkdv_kernel(const Tensor q, const Tensor k, const Tensor v,
        const uint8_t *__restrict__ mask, const float *__restrict__ lse, const Tensor du, const float *__restrict__ delta,
        float *__restrict__ dk, float *__restrict__ dv, const Shape s, const float scale) {
    constexpr int HALF = D / 2;
    constexpr int DT = D / 32;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int col = lane & 31;
    const int h = lane >> 5;

    const int seqs = s.batch * s.heads;
    const int rank = blockIdx.x / seqs;
    const int seq = blockIdx.x - rank * seqs;
    const int b = seq / s.heads;
    const int head = seq - b * s.heads;
    const int key0 = rank * kTile; // under a causal mask the first key tiles see the most queries
    const int key = key0 + col;
    const bool in_range = key < s.keys;
    const bool visible = in_range && mask[static_cast<int64_t>(b) * s.keys + key] != 0;
    const uint32_t bits = static_cast<uint32_t>(__ballot(visible));
    const float c2 = scale * kLog2e;

    float kr[HALF], vr[HALF];
    load_span<VEC>(kr, sequence(k, b, head) + static_cast<int64_t>(key) * k.st + h * HALF, visible);
    load_span<VEC>(vr, sequence(v, b, head) + static_cast<int64_t>(key) * v.st + h * HALF, visible);

    int first = s.causal ? key0 : 0;
    int last = s.queries;
    if (s.radius >= 0) {
        first = max(first, key0 - s.radius);
        last = min(last, key0 + kTile + s.radius);
    }
    first = max(first, 0);
    const int ntiles = (bits != 0 && last > first) ? (last - first + kTile - 1) / kTile : 0;

    const float *qbase = sequence(q, b, head);
    const float *ubase = sequence(du, b, head);
    const int64_t rows = static_cast<int64_t>(seq) * s.queries;

    __shared__ __align__(16) float stats[kWaves][3][kTile];

    f32x16 acc_k[DT], acc_v[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) {
        acc_k[t] = f32x16{};
        acc_v[t] = f32x16{};
    }

    for (int tile = wave; tile < ntiles; tile += kWaves) {
        const int q0 = first + tile * kTile;

        // Per-query softmax constants for the 32 queries of the tile, staged once in this wave's LDS slice and
        // read back in accumulator order (lane needs queries tile_row(v, h), v = 0..15).
        wave_lds_sync();
        if (h == 0) {
            const int qq = q0 + col;
            float mcv = INFINITY, ilv = 0.0f, dl = 0.0f;
            if (qq < s.queries) {
                const float m = lse[2 * (rows + qq)];
                if (m != -INFINITY) {
                    mcv = m * kLog2e;
                    ilv = 1.0f / lse[2 * (rows + qq) + 1];
                }
                dl = delta[rows + qq];
            }
            stats[wave][0][col] = mcv;
            stats[wave][1][col] = ilv;
            stats[wave][2][col] = dl;
        }
        wave_lds_sync();
        float mcs[16], ils[16], dls[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f32x4 a = *reinterpret_cast<const f32x4 *>(&stats[wave][0][8 * u + 4 * h]);
            const f32x4 bb = *reinterpret_cast<const f32x4 *>(&stats[wave][1][8 * u + 4 * h]);
            const f32x4 c = *reinterpret_cast<const f32x4 *>(&stats[wave][2][8 * u + 4 * h]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                mcs[4 * u + i] = a[i];
                ils[4 * u + i] = bb[i];
                dls[4 * u + i] = c[i];
            }
        }

        const int qrow = q0 + col;
        float qr[HALF], dor[HALF];
        load_span<VEC>(qr, qbase + static_cast<int64_t>(qrow) * q.st + h * HALF, qrow < s.queries);
        load_span<VEC>(dor, ubase + static_cast<int64_t>(qrow) * du.st + h * HALF, qrow < s.queries);
        float qc[DT][16], uc[DT][16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = q0 + tile_row(j, h);
            const bool ok = r < s.queries;
            const float *qp = qbase + static_cast<int64_t>(r) * q.st + col;
            const float *up = ubase + static_cast<int64_t>(r) * du.st + col;
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                qc[t][j] = ok ? qp[32 * t] : 0.0f;
                uc[t][j] = ok ? up[32 * t] : 0.0f;
            }
        }

        f32x16 sc{}, dp{};
#pragma unroll
        for (int c = 0; c < HALF; ++c) {
            sc = mfma(qr[c], kr[c], sc);
            dp = mfma(dor[c], vr[c], dp);
        }

        const bool full = bits == 0xffffffffu && q0 + kTile <= s.queries && tile_in_window(s, q0, key0);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            float p = exp2_fast(fmaf(sc[v], c2, -mcs[v])) * ils[v];
            float ds = p * (dp[v] - dls[v]);
            if (!full) {
                const int qq = q0 + tile_row(v, h);
                const bool ok = visible && qq < s.queries && qq >= window_query_lo(s, key) && qq <= window_query_hi(s, key);
                p = ok ? p : 0.0f;
                ds = ok ? ds : 0.0f;
            }
            sc[v] = p;
            dp[v] = ds;
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
#pragma unroll
            for (int t = 0; t < DT; ++t) {
                acc_v[t] = mfma(uc[t][j], sc[j], acc_v[t]);
                acc_k[t] = mfma(qc[t][j], dp[j], acc_k[t]);
            }
        }
    }

    __shared__ float partial[kWaves - 1][32 * DT][kWave];
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                partial[wave - 1][16 * t + v][lane] = acc_k[t][v];
                partial[wave - 1][16 * DT + 16 * t + v][lane] = acc_v[t][v];
            }
        }
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int w = 0; w < kWaves - 1; ++w) {
#pragma unroll
        for (int t = 0; t < DT; ++t) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                acc_k[t][v] += partial[w][16 * t + v][lane];
                acc_v[t][v] += partial[w][16 * DT + 16 * t + v][lane];
            }
        }
    }
    if (!in_range) return;
    const int64_t krow = (static_cast<int64_t>(seq) * s.keys + key) * D;
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

template<int D, int MODE, bool VEC>
void launch_dq(const BackwardArgs &a, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const unsigned blocks = static_cast<unsigned>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    hipLaunchKernelGGL((attention_dq_kernel<D, MODE, VEC>), dim3(blocks), dim3(kThreads), 0, stream, tensor(a.q, a.qs),
            tensor(a.k, a.ks), tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), tensor(a.output, a.os), a.lse,
            tensor(a.upstream, a.us), a.gradient_q, a.delta, shape, scale);
}

template<int D, bool VEC>
void launch_dkdv(const BackwardArgs &a, hipStream_t stream) {
    const Shape shape{a.batch, a.heads, a.queries, a.keys, a.radius, a.causal};
    const float scale = 1.0f / sqrtf(static_cast<float>(D));
    const unsigned blocks = static_cast<unsigned>((a.keys + kTile - 1) / kTile) * a.batch * a.heads;
    hipLaunchKernelGGL((attention_dkdv_kernel<D, VEC>), dim3(blocks), dim3(kThreads), 0, stream, tensor(a.q, a.qs), tensor(a.k, a.ks),
            tensor(a.v, a.vs), reinterpret_cast<const uint8_t *>(a.mask), a.lse, tensor(a.upstream, a.us), a.delta, a.gradient_k,
            a.gradient_v, shape, scale);
}

template<int D, bool VEC>
hipError_t run(const BackwardStage stage, const BackwardArgs &a, hipStream_t stream) {
    if (stage == kBackwardAll || stage == kBackwardDelta || stage == kBackwardQuery) {
        if (stage == kBackwardAll) launch_dq<D, kDqAndDelta, VEC>(a, stream);
        else if (stage == kBackwardDelta) launch_dq<D, kDeltaOnly, VEC>(a, stream);
        else launch_dq<D, kDqFromDelta, VEC>(a, stream);
        const hipError_t error = hipGetLastError();
        if (error != hipSuccess || stage != kBackwardAll) return error;
    }
    launch_dkdv<D, VEC>(a, stream);
    return hipGetLastError();
}

} // namespace

hipError_t launch_backward(const int D, const BackwardStage stage, const BackwardArgs &a, hipStream_t stream) {
    const int64_t qblocks = static_cast<int64_t>((a.queries + kTile - 1) / kTile) * a.batch * a.heads;
    const int64_t kblocks = static_cast<int64_t>((a.keys + kTile - 1) / kTile) * a.batch * a.heads;
    if (qblocks > 0x7fffffff || kblocks > 0x7fffffff || !sequence_fits(a.queries, a.qs, D) || !sequence_fits(a.keys, a.ks, D) ||
            !sequence_fits(a.keys, a.vs, D) || !sequence_fits(a.queries, a.os, D) || !sequence_fits(a.queries, a.us, D))
        return hipErrorInvalidValue;
    const bool vec = aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.output) && aligned16(a.upstream) &&
            aligned16(a.gradient_q) && aligned16(a.gradient_k) && aligned16(a.gradient_v) && strides4(a.qs) && strides4(a.ks) &&
            strides4(a.vs) && strides4(a.os) && strides4(a.us);
    if (D == 32) return vec ? run<32, true>(stage, a, stream) : run<32, false>(stage, a, stream);
    return vec ? run<64, true>(stage, a, stream) : run<64, false>(stage, a, stream);
}

} // namespace rk
