#pragma once

// ROCmKernels::Kernels::Strides is the C struct of the library's ABI, so C and C++ callers pass the same
// three ints by value (reference layout: ROCmKernels.Kernels/include/ROCmKernels/Kernels/Strides.hpp:5-9).
#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    using Strides = ::rocmkernels_strides;
} // namespace ROCmKernels::Kernels
