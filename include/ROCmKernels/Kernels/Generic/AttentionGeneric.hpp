#pragma once

// Throwing C++ wrapper over attention_generic_forward. Name, arguments and the defaulted stream follow the
// reference's ROCmKernels.Kernels/include/ROCmKernels/Kernels/Generic/AttentionGeneric.hpp:15-25.
//
// Windowed attention forward for 16-, 32- or 64-wide heads with fp32 or fp16 q, k, v and output (fp32 lse).
// mask is [batch][keys]; radius < 0 attends globally; lse receives {row maximum, exponent sum} per (batch, head, query).

#include <ROCmKernels/Common/Error.hpp>
#include <ROCmKernels/Kernels/DType.hpp>
#include <ROCmKernels/Kernels/Strides.hpp>

#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    inline void AttentionGenericForward(const void *q, const void *k, const void *v, const bool *mask, void *output, float *lse,
            const int batch, const int heads, const int queries, const int keys, const int headWidth, const int radius, const Strides &qs,
            const Strides &ks, const Strides &vs, const Strides &os, const DType dtype, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(attention_generic_forward(q, k, v, mask, output, lse, batch, heads, queries, keys, headWidth, radius, qs, ks,
                vs, os, static_cast<rocmkernels_dtype>(dtype), stream));
    }
} // namespace ROCmKernels::Kernels
