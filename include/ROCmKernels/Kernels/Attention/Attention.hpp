#pragma once

// Throwing C++ wrappers over the 32-wide FP32 attention C entry points. Names, argument order and the
// defaulted stream follow the reference's ROCmKernels.Kernels/include/ROCmKernels/Kernels/Attention/Attention.hpp:39-109,
// so C++ callers of the reference compile against this header unchanged. Each wrapper throws
// ROCmKernels::HipError when the entry point returns a non-zero hipError_t.
//
// mask is [batch][keys]; radius < 0 attends globally; lse receives {row maximum, exponent sum} per (batch, head, query).
// output honours os; lse, delta and the gradients are packed [batch][head][query|key][32].

#include <ROCmKernels/Common/Error.hpp>
#include <ROCmKernels/Kernels/Strides.hpp>

#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    inline void AttentionForward(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse, const int batch,
            const int heads, const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks, const Strides &vs,
            const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_forward(q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream));
    }

    inline void AttentionForwardTiled(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks,
            const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(
                attention_fp32_forward_tiled(q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream));
    }

    inline void AttentionBackward(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
            const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, const int batch, const int heads,
            const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks, const Strides &vs, const Strides &os,
            const Strides &us, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_backward(q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta, batch,
                heads, queries, keys, radius, qs, ks, vs, os, us, stream));
    }

    inline void AttentionBackwardTiled(const float *q, const float *k, const float *v, const bool *mask, const float *output,
            const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, const int batch,
            const int heads, const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks, const Strides &vs,
            const Strides &os, const Strides &us, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_backward_tiled(q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta,
                batch, heads, queries, keys, radius, qs, ks, vs, os, us, stream));
    }

    /// Softmax statistics only: no value reads, no output write.
    inline void AttentionStatistics(const float *q, const float *k, const bool *mask, float *lse, const int batch, const int heads,
            const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_statistics(q, k, mask, lse, batch, heads, queries, keys, radius, qs, ks, stream));
    }

    inline void AttentionForwardTuned(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const int group, const Strides &qs,
            const Strides &ks, const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(
                attention_fp32_forward_tuned(q, k, v, mask, output, lse, batch, heads, queries, keys, radius, group, qs, ks, vs, os, stream));
    }

    /// Flash attention forward: online softmax over 32-key MFMA tiles.
    inline void AttentionForwardFlash(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const Strides &qs, const Strides &ks,
            const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_forward_flash(q, k, v, mask, output, lse, batch, heads, queries, keys, radius, qs, ks, vs, os, stream));
    }

    /// Variant selector kept from the reference's tuning sweep: 0 through 18 are accepted.
    inline void AttentionForwardFlashTuned(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const int variant, const Strides &qs,
            const Strides &ks, const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_forward_flash_tuned(
                q, k, v, mask, output, lse, batch, heads, queries, keys, radius, variant, qs, ks, vs, os, stream));
    }

    inline void AttentionBackwardTuned(const float *q, const float *k, const float *v, const bool *mask, const float *output,
            const float *lse, const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, const int batch,
            const int heads, const int queries, const int keys, const int radius, const int group, const Strides &qs, const Strides &ks,
            const Strides &vs, const Strides &os, const Strides &us, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_backward_tuned(q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta,
                batch, heads, queries, keys, radius, group, qs, ks, vs, os, us, stream));
    }

    /// Causal-capable flash forward (no reference counterpart): flags bit 0 restricts each query to keys <= query.
    inline void AttentionForwardFlashEx(const float *q, const float *k, const float *v, const bool *mask, float *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int radius, const int flags, const Strides &qs,
            const Strides &ks, const Strides &vs, const Strides &os, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_forward_flash_ex(
                q, k, v, mask, output, lse, batch, heads, queries, keys, radius, flags, qs, ks, vs, os, stream));
    }

    /// Causal-capable backward (no reference counterpart): flags as in AttentionForwardFlashEx.
    inline void AttentionBackwardEx(const float *q, const float *k, const float *v, const bool *mask, const float *output, const float *lse,
            const float *upstream, float *gradient_q, float *gradient_k, float *gradient_v, float *delta, const int batch, const int heads,
            const int queries, const int keys, const int radius, const int flags, const Strides &qs, const Strides &ks, const Strides &vs,
            const Strides &os, const Strides &us, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_fp32_backward_ex(q, k, v, mask, output, lse, upstream, gradient_q, gradient_k, gradient_v, delta,
                batch, heads, queries, keys, radius, flags, qs, ks, vs, os, us, stream));
    }
} // namespace ROCmKernels::Kernels
