// 32-wide rotary position embedding for gfx950 (MI355X): the reference's rotary_fp32 (Positional/Rotary.hip:10-56),
// the step that prepares Q and K for attention.
//
// For each (sample, token, head) row of Q and of K, column c < 16 pairs with c + 16:
//   forward:  out[c] = x[c]·cos[c] − x[c+16]·sin[c],   out[c+16] = x[c+16]·cos[c+16] + x[c]·sin[c+16]
//   backward: out[c] = x[c]·cos[c] + x[c+16]·sin[c+16], out[c+16] = x[c+16]·cos[c+16] − x[c]·sin[c]
// (the backward is the transpose of the forward rotation). cos/sin hold 32 values per (sample, token), shared by the
// heads. Each product is rounded before the sum (no contraction: the library is built with -ffp-contract=off), which
// is how the reference's CPU reference evaluates it (PositionalTests.cpp:18-51), so results match it bit for bit.
//
// The work is HBM-bound (per row 128 B read and 128 B written for each of Q and K; the tables are shared by the heads
// and stay in cache). Mapping: 4 lanes per row; lane r owns columns 4r..4r+3 and 16+4r..16+4r+3 and moves each half
// with one 128-bit load/store when aligned. Rows are numbered in output order [batch][token][head] (the reference's
// token-major output), so consecutive lanes write consecutive 16-byte chunks.
#include <rocmkernels_attention.h>

#include <hip/hip_runtime.h>

#include <stdint.h>

#include "attention_launch.hpp"

namespace rk {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template<bool VEC>
__device__ __forceinline__ f32x4 load4(const float *p) {
    if constexpr (VEC) return *reinterpret_cast<const f32x4 *>(p);
    else return f32x4{p[0], p[1], p[2], p[3]};
}

template<bool VEC>
__device__ __forceinline__ void store4(float *p, const f32x4 x) {
    if constexpr (VEC) {
        *reinterpret_cast<f32x4 *>(p) = x;
    } else {
        p[0] = x[0];
        p[1] = x[1];
        p[2] = x[2];
        p[3] = x[3];
    }
}

template<bool BACKWARD, bool VEC>
__global__ __launch_bounds__(256) void rotary_kernel(const float *__restrict__ q, const float *__restrict__ k, const float *__restrict__ cos,
        const float *__restrict__ sin, float *__restrict__ oq, float *__restrict__ ok, const int heads, const int length, const int64_t rows,
        const rocmkernels_strides qs, const rocmkernels_strides ks, const rocmkernels_strides cs, const rocmkernels_strides ss) {
    const int64_t thread = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = thread >> 2;
    if (row >= rows) return;
    const int part = 4 * static_cast<int>(thread & 3);
    // Head, token and sample of the row; 32-bit divisions whenever the rows fit (64-bit ones are long VALU sequences).
    int head, token;
    int64_t sample;
    if (rows <= 0xffffffffLL) {
        const uint32_t r32 = static_cast<uint32_t>(row), nh = static_cast<uint32_t>(heads), nl = static_cast<uint32_t>(length);
        const uint32_t sample_token = r32 / nh;
        head = static_cast<int>(r32 - sample_token * nh);
        const uint32_t s32 = sample_token / nl;
        token = static_cast<int>(sample_token - s32 * nl);
        sample = s32;
    } else {
        head = static_cast<int>(row % heads);
        const int64_t sample_token = row / heads;
        token = static_cast<int>(sample_token % length);
        sample = sample_token / length;
    }

    const float *qrow = q + sample * qs.batch + static_cast<int64_t>(head) * qs.head + static_cast<int64_t>(token) * qs.token + part;
    const float *krow = k + sample * ks.batch + static_cast<int64_t>(head) * ks.head + static_cast<int64_t>(token) * ks.token + part;
    const float *crow = cos + sample * cs.batch + static_cast<int64_t>(token) * cs.token + part;
    const float *srow = sin + sample * ss.batch + static_cast<int64_t>(token) * ss.token + part;
    const f32x4 c_lo = load4<VEC>(crow), c_hi = load4<VEC>(crow + 16);
    const f32x4 s_lo = load4<VEC>(srow), s_hi = load4<VEC>(srow + 16);

    auto rotate = [&](const float *x, float *out) __attribute__((always_inline)) {
        const f32x4 lo = load4<VEC>(x), hi = load4<VEC>(x + 16);
        f32x4 out_lo, out_hi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (BACKWARD) {
                out_lo[i] = lo[i] * c_lo[i] + hi[i] * s_hi[i];
                out_hi[i] = hi[i] * c_hi[i] - lo[i] * s_lo[i];
            } else {
                out_lo[i] = lo[i] * c_lo[i] - hi[i] * s_lo[i];
                out_hi[i] = hi[i] * c_hi[i] + lo[i] * s_hi[i];
            }
        }
        store4<VEC>(out, out_lo);
        store4<VEC>(out + 16, out_hi);
    };
    rotate(qrow, oq + row * 32 + part);
    rotate(krow, ok + row * 32 + part);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool strides4(const rocmkernels_strides &s, const bool with_head) {
    return ((s.batch | s.token | (with_head ? s.head : 0)) & 3) == 0;
}

template<bool BACKWARD, bool VEC>
void launch(const RotaryArgs &a, const int64_t rows, hipStream_t stream) {
    const unsigned blocks = static_cast<unsigned>((rows * 4 + 255) / 256);
    hipLaunchKernelGGL((rotary_kernel<BACKWARD, VEC>), dim3(blocks), dim3(256), 0, stream, a.q, a.k, a.cos, a.sin, a.oq, a.ok, a.heads,
            a.length, rows, a.qs, a.ks, a.cs, a.ss);
}

} // namespace

hipError_t launch_rotary(const RotaryArgs &a, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(a.batch) * a.length * a.heads;
    if ((rows * 4 + 255) / 256 > 0x7fffffff) return hipErrorInvalidValue;
    const bool vec = aligned16(a.q) && aligned16(a.k) && aligned16(a.cos) && aligned16(a.sin) && aligned16(a.oq) && aligned16(a.ok) &&
            strides4(a.qs, true) && strides4(a.ks, true) && strides4(a.cs, false) && strides4(a.ss, false);
    if (a.backward) {
        if (vec) launch<true, true>(a, rows, stream);
        else launch<true, false>(a, rows, stream);
    } else {
        if (vec) launch<false, true>(a, rows, stream);
        else launch<false, false>(a, rows, stream);
    }
    return hipGetLastError();
}

} // namespace rk
