#pragma once

// Host-side error type of the C++ wrapper layer: every wrapper turns a non-zero hipError_t returned by a
// C entry point into a ROCmKernels::HipError carrying the status, the failing expression and its location.
// Interface follows the reference's ROCmKernels.Common/include/ROCmKernels/Common/Error.hpp:14-45.

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace ROCmKernels {
    class HipError final : public std::runtime_error {
      public:
        HipError(const hipError_t status, const std::string &message) : std::runtime_error(message), status_(status) {}

        [[nodiscard]] hipError_t Status() const noexcept { return status_; }

      private:
        hipError_t status_;
    };

    [[noreturn]] inline void ThrowHipError(const hipError_t status, const char *expression, const char *file, const int line) {
        throw HipError(status, std::string("HIP call failed: ") + expression + " -> " + hipGetErrorString(status) + " (" + file + ":" +
                std::to_string(line) + ")");
    }
} // namespace ROCmKernels

#define ROCMKERNELS_HIP_CHECK(expression)                                                                                    \
    do {                                                                                                                     \
        const hipError_t rocmkernels_status_ = static_cast<hipError_t>(expression);                                          \
        if (rocmkernels_status_ != hipSuccess) ::ROCmKernels::ThrowHipError(rocmkernels_status_, #expression, __FILE__, __LINE__); \
    } while (false)
