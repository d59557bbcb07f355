// Host-only check of the C++ wrapper layer (no GPU needed): every wrapper must turn an invalid-argument return
// into ROCmKernels::HipError carrying hipErrorInvalidValue, exactly as the reference's wrappers do
// (ROCmKernels.Common/include/ROCmKernels/Common/Error.hpp:24-45). Prints one line per case; exit code = failures.
#include <ROCmKernels/Kernels/Attention/Attention.hpp>
#include <ROCmKernels/Kernels/Attention/Attention64.hpp>
#include <ROCmKernels/Kernels/Generic/AttentionGeneric.hpp>
#include <ROCmKernels/Kernels/Positional/Rotary.hpp>

#include <cstdio>
#include <functional>
#include <string>

namespace {
int failures = 0;

void expect_invalid(const char *name, const std::function<void()> &call) {
    try {
        call();
        std::printf("FAIL %s: no exception\n", name);
        ++failures;
    } catch (const ROCmKernels::HipError &error) {
        const bool ok = error.Status() == hipErrorInvalidValue && std::string(error.what()).find("HIP call failed") == 0;
        std::printf("%s %s: %s\n", ok ? "ok" : "FAIL", name, error.what());
        failures += ok ? 0 : 1;
    }
}
} // namespace

int main() {
    using namespace ROCmKernels::Kernels;
    const Strides s{0, 0, 0};
    float dummy[4] = {};
    const bool mask[1] = {true};
    expect_invalid("AttentionForward null q", [&] { AttentionForward(nullptr, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -1, s, s, s, s); });
    expect_invalid("AttentionForwardTiled zero batch",
            [&] { AttentionForwardTiled(dummy, dummy, dummy, mask, dummy, dummy, 0, 1, 1, 1, -1, s, s, s, s); });
    expect_invalid("AttentionForwardFlash radius -2",
            [&] { AttentionForwardFlash(dummy, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -2, s, s, s, s); });
    expect_invalid("AttentionForwardFlashTuned variant 19",
            [&] { AttentionForwardFlashTuned(dummy, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -1, 19, s, s, s, s); });
    expect_invalid("AttentionForwardTuned group 3",
            [&] { AttentionForwardTuned(dummy, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -1, 3, s, s, s, s); });
    expect_invalid("AttentionStatistics null lse", [&] { AttentionStatistics(dummy, dummy, mask, nullptr, 1, 1, 1, 1, -1, s, s); });
    expect_invalid("AttentionBackward null delta", [&] {
        AttentionBackward(dummy, dummy, dummy, mask, dummy, dummy, dummy, dummy, dummy, dummy, nullptr, 1, 1, 1, 1, -1, s, s, s, s, s);
    });
    expect_invalid("AttentionBackwardTiled zero keys", [&] {
        AttentionBackwardTiled(dummy, dummy, dummy, mask, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1, 1, 1, 0, -1, s, s, s, s, s);
    });
    expect_invalid("AttentionBackwardTuned group 5", [&] {
        AttentionBackwardTuned(dummy, dummy, dummy, mask, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1, 1, 1, 1, -1, 5, s, s, s, s, s);
    });
    expect_invalid("Attention64Forward null mask", [&] { Attention64Forward(dummy, dummy, dummy, nullptr, dummy, dummy, 1, 1, 1, 1, -1, s, s, s, s); });
    expect_invalid("Attention64Backward zero heads", [&] {
        Attention64Backward(dummy, dummy, dummy, mask, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1, 0, 1, 1, -1, s, s, s, s, s);
    });
    expect_invalid("AttentionForwardFlashEx flags 2",
            [&] { AttentionForwardFlashEx(dummy, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -1, 2, s, s, s, s); });
    expect_invalid("AttentionBackwardEx null upstream", [&] {
        AttentionBackwardEx(dummy, dummy, dummy, mask, dummy, dummy, nullptr, dummy, dummy, dummy, dummy, 1, 1, 1, 1, -1, 1, s, s, s, s, s);
    });
    expect_invalid("Attention64ForwardEx radius -3",
            [&] { Attention64ForwardEx(dummy, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, -3, 1, s, s, s, s); });
    expect_invalid("Attention64BackwardEx flags -1", [&] {
        Attention64BackwardEx(dummy, dummy, dummy, mask, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1, 1, 1, 1, -1, -1, s, s, s, s, s);
    });
    expect_invalid("AttentionGenericForward head width 48", [&] {
        AttentionGenericForward(dummy, dummy, dummy, mask, dummy, dummy, 1, 1, 1, 1, 48, -1, s, s, s, s, DType::Float32);
    });
    expect_invalid("AttentionGenericForward fp16 null output", [&] {
        AttentionGenericForward(dummy, dummy, dummy, mask, nullptr, dummy, 1, 1, 1, 1, 16, -1, s, s, s, s, DType::Float16);
    });
    expect_invalid("Rotary zero heads", [&] { Rotary(dummy, dummy, dummy, dummy, dummy, dummy, 1, 0, 1, false, s, s, s, s); });
    std::printf("%d failure(s)\n", failures);
    return failures;
}
