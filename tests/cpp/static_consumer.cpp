// A C++ consumer of the static target ROCmKernels.Kernels (libROCmKernels.Kernels.a), linked the way a C++ program
// links the reference's static library: the wrapper's invalid-argument path must throw ROCmKernels::HipError with
// hipErrorInvalidValue (no GPU needed: validation happens before any HIP call). Exit code 0 on success.
#include <ROCmKernels/Kernels/Attention/Attention.hpp>
#include <ROCmKernels/Kernels/Attention/Attention64.hpp>

#include <cstdio>

int main() {
    using namespace ROCmKernels::Kernels;
    const Strides s{0, 0, 0};
    float dummy[4] = {};
    const bool mask[1] = {true};
    int ok = 0;
    try {
        AttentionForwardFlash(nullptr, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -1, s, s, s, s);
    } catch (const ROCmKernels::HipError &error) {
        ok += error.Status() == hipErrorInvalidValue;
        std::printf("%s\n", error.what());
    }
    try {
        Attention64BackwardEx(dummy, dummy, dummy, mask, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1, 1, 1, 1, -1, 6, s, s, s, s, s);
    } catch (const ROCmKernels::HipError &error) {
        ok += error.Status() == hipErrorInvalidValue;
        std::printf("%s\n", error.what());
    }
    return ok == 2 ? 0 : 1;
}
