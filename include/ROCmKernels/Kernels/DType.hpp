#pragma once

// Storage type of attention_generic_forward's tensors; accumulation is always fp32. Same enumerators, underlying
// type and values as the reference's ROCmKernels.Kernels/include/ROCmKernels/Kernels/DType.hpp:7-8, so that a
// C++ caller of the reference passes it unchanged; converts to the C ABI's rocmkernels_dtype.
#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    enum class DType : unsigned char { Float32 = ROCMKERNELS_DTYPE_FLOAT32, Float16 = ROCMKERNELS_DTYPE_FLOAT16 };
} // namespace ROCmKernels::Kernels
