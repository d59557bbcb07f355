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

namespace rk {

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

// Value of x held by the lane 32 positions away (the other half of the wave).
__device__ __forceinline__ float other_half(const float x) { return __shfl_xor(x, 32); }

__device__ __forceinline__ const float *sequence(const Tensor &t, const int b, const int head) {
    return t.data + (static_cast<int64_t>(b) * t.sb + static_cast<int64_t>(head) * t.sh);
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

// Stores accumulator tile acc (rows tile_row(v, h) of a 32-feature slice) as 4 groups of 4 contiguous floats.
template<bool VEC>
__device__ __forceinline__ void store_tile_row(float *p, const f32x16 &acc, const float factor, const int h) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
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

// Visibility of (query, key) beyond the key mask: causal (key <= query) and local radius (|query - key| <= radius).
__device__ __forceinline__ bool in_window(const Shape &s, const int query, const int key) {
    bool ok = true;
    if (s.causal) ok = ok && key <= query;
    if (s.radius >= 0) ok = ok && abs(query - key) <= s.radius;
    return ok;
}

// True when every (query, key) pair of the 32x32 tile at (q0, key0) is inside the causal/radius window.
__device__ __forceinline__ bool tile_in_window(const Shape &s, const int q0, const int key0) {
    bool ok = true;
    if (s.causal) ok = ok && key0 + kTile - 1 <= q0;
    if (s.radius >= 0) ok = ok && q0 + kTile - 1 - key0 <= s.radius && key0 + kTile - 1 - q0 <= s.radius;
    return ok;
}

} // namespace rk
