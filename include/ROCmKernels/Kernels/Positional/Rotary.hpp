#pragma once

// Throwing C++ wrapper over rotary_fp32. Name, arguments and the defaulted stream follow the reference's
// ROCmKernels.Kernels/include/ROCmKernels/Kernels/Positional/Rotary.hpp:13-22.
//
// Rotary embedding for 32-wide heads. Outputs are token-major [batch][token][head][32]. Input strides are honoured for
// q, k, cos and sin; cos/sin hold 32 values per token.

#include <ROCmKernels/Common/Error.hpp>
#include <ROCmKernels/Kernels/Strides.hpp>

#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    inline void Rotary(const float *q, const float *k, const float *cos, const float *sin, float *oq, float *ok, const int batch,
            const int heads, const int length, const bool backward, const Strides &qs, const Strides &ks, const Strides &cs,
            const Strides &ss, hipStream_t stream = nullptr) {
        ROCMKERNELS_HIP_CHECK(rotary_fp32(q, k, cos, sin, oq, ok, batch, heads, length, backward ? 1 : 0, qs, ks, cs, ss, stream));
    }
} // namespace ROCmKernels::Kernels
