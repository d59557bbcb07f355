#pragma once

// Throwing C++ wrappers over the 64-wide FP32 attention C entry points. Names and arguments follow the
// reference's ROCmKernels.Kernels/include/ROCmKernels/Kernels/Attention/Attention64.hpp:17-32; layouts match the
// 32-wide family with D = 64.

#include <ROCmKernels/Common/Error.hpp>
#include <ROCmKernels/Kernels/Strides.hpp>

#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    inline void Attention64Forward(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks,
            const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(
                attention64_fp32_forward(q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream));
    }

    inline void Attention64Backward(const float *q, const float *k, const float *v, const bool *mask, const float *output,
            const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, const int batch,
            const int heads, const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks, const Strides &vs,
            const Strides &os, const Strides &us, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention64_fp32_backward(q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch,
                heads, queries, keys, radius, qs, ks, vs, os, us, stream));
    }

    /// Causal-capable 64-wide forward (no reference counterpart): flags bit 0 restricts each query to keys <= query.
    inline void Attention64ForwardEx(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const int flags, const Strides &qs,
            const Strides &ks, const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention64_fp32_forward_ex(
                q, k, v, mask, output, lse, batch, heads, queries, keys, radius, flags, qs, ks, vs, os, stream));
    }

    /// Causal-capable 64-wide backward (no reference counterpart).
    inline void Attention64BackwardEx(const float *q, const float *k, const float *v, const bool *mask, const float *output,
            const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, const int batch,
            const int heads, const int queries, const int keys, const int radius, const int flags, const Strides &qs, const Strides &ks,
            const Strides &vs, const Strides &os, const Strides &us, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention64_fp32_backward_ex(q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta,
                batch, heads, queries, keys, radius, flags, qs, ks, vs, os, us, stream));
    }
} // namespace ROCmKernels::Kernels
