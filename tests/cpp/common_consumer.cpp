// A C++ caller written in the pattern of the reference's generic tests (ROCmKernels.Tests/Generic/
// AttentionGenericTests.cpp:106-139): ROCmKernels::DeviceBuffer<T> storage, AttentionGenericForward(...,
// DTypeOf<T>::value), ROCMKERNELS_HIP_CHECK and the device queries of ROCmKernels/Common/Device.hpp. It compiles
// against the public headers only and links the ROCmKernels.Common target with a kernel target.
//
// Two uses:
//   - CPU (tests/test_abi.py): built with COMMON_CONSUMER_MAIN against the static archives; main() checks what needs no
//     GPU (DTypeOf, an empty DeviceBuffer, the wrapper's invalid-argument throw, the device queries reporting a missing
//     device as HipError) and prints "<n> failure(s)".
//   - GPU (tests/test_common_gpu.py): built by the CMake project as librocmkernels_common_consumer.so and called in the
//     test's own process through ctypes; common_consumer_gpu_check() queries device 0 and runs fp32 and fp16 windowed
//     cases on DeviceBuffer storage, checked against their closed form: with constant Q and K every visible key gets
//     the same score, so the output is the mean of the visible V rows and lse = {score, number of visible keys}.
#include <ROCmKernels/Common/Device.hpp>
#include <ROCmKernels/Common/DeviceBuffer.hpp>
#include <ROCmKernels/Common/Error.hpp>
#include <ROCmKernels/Kernels/DType.hpp>
#include <ROCmKernels/Kernels/Generic/AttentionGeneric.hpp>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <type_traits>
#include <vector>

namespace {

static_assert(ROCmKernels::Kernels::DTypeOf<float>::value == ROCmKernels::Kernels::DType::Float32);
static_assert(ROCmKernels::Kernels::DTypeOf<__half>::value == ROCmKernels::Kernels::DType::Float16);
static_assert(static_cast<rocmkernels_dtype>(ROCmKernels::Kernels::DTypeOf<__half>::value) == ROCMKERNELS_DTYPE_FLOAT16);
static_assert(std::is_same_v<std::underlying_type_t<ROCmKernels::Kernels::DType>, unsigned char>);

struct Report {
    std::string text;
    int failures = 0;
    void expect(const bool ok, const std::string &what) {
        if (!ok) {
            ++failures;
            text += "FAIL " + what + "\n";
        }
    }
};

template<typename T> T narrow(const float x) {
    if constexpr (std::is_same_v<T, __half>) return __float2half(x);
    else return x;
}

template<typename T> float widen(const T x) {
    if constexpr (std::is_same_v<T, __half>) return __half2float(x);
    else return x;
}

// One windowed forward on [batch][head][token][W] packed storage of type T. V values are multiples of 1/16 in
// [-0.5, 0.5], exact in fp16, and every probability is exp(0) = 1, so the fp32 sums are exact and only the final
// division (and, for fp16, the output's rounding) rounds.
template<typename T, int W> void run_case(Report &report, const int batch, const int heads, const int queries, const int keys, const int radius) {
    const std::size_t qn = static_cast<std::size_t>(batch) * heads * queries * W;
    const std::size_t kn = static_cast<std::size_t>(batch) * heads * keys * W;
    std::vector<T> q(qn, narrow<T>(0.5f)), k(kn, narrow<T>(0.5f)), v(kn);
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < heads; ++h)
            for (int key = 0; key < keys; ++key)
                for (int f = 0; f < W; ++f)
                    v[((static_cast<std::size_t>(b) * heads + h) * keys + key) * W + f] =
                            narrow<T>(static_cast<float>((key * 7 + f * 3 + b + 2 * h) % 17 - 8) / 16.0f);
    std::vector<std::uint8_t> mask(static_cast<std::size_t>(batch) * keys, 1);
    mask[3] = 0;

    ROCmKernels::DeviceBuffer<T> deviceQ(qn), deviceK(kn), deviceV(kn), deviceOutput(qn);
    ROCmKernels::DeviceBuffer<std::uint8_t> deviceMask(mask.size());
    ROCmKernels::DeviceBuffer<float> deviceLse(static_cast<std::size_t>(batch) * heads * queries * 2);
    deviceQ.CopyFromHost(q.data(), q.size());
    deviceK.CopyFromHost(k.data(), k.size());
    deviceV.CopyFromHost(v.data(), v.size());
    deviceMask.CopyFromHost(mask.data(), mask.size());

    const ROCmKernels::Kernels::Strides qs{heads * queries * W, queries * W, W};
    const ROCmKernels::Kernels::Strides ks{heads * keys * W, keys * W, W};
    ROCmKernels::Kernels::AttentionGenericForward(deviceQ.Data(), deviceK.Data(), deviceV.Data(),
            reinterpret_cast<const bool *>(deviceMask.Data()), deviceOutput.Data(), deviceLse.Data(), batch, heads, queries, keys, W,
            radius, qs, ks, ks, qs, ROCmKernels::Kernels::DTypeOf<T>::value);
    ROCMKERNELS_HIP_CHECK(hipDeviceSynchronize());

    std::vector<T> output(qn);
    std::vector<float> lse(deviceLse.Count());
    deviceOutput.CopyToHost(output.data(), output.size());
    deviceLse.CopyToHost(lse.data(), lse.size());

    const double score = 0.25 * W / std::sqrt(static_cast<double>(W)); // 0.5 * 0.5 * W, scaled by 1/sqrt(W)
    const double tolerance = std::is_same_v<T, __half> ? 2e-3 : 1e-6;
    double worst_o = 0.0, worst_max = 0.0;
    int bad_sum = 0;
    for (int b = 0; b < batch; ++b) {
        for (int h = 0; h < heads; ++h) {
            for (int query = 0; query < queries; ++query) {
                const std::size_t row = (static_cast<std::size_t>(b) * heads + h) * queries + query;
                int visible = 0;
                std::vector<double> sum(W, 0.0);
                for (int key = 0; key < keys; ++key) {
                    if (!mask[static_cast<std::size_t>(b) * keys + key] || (radius >= 0 && std::abs(query - key) > radius)) continue;
                    ++visible;
                    for (int f = 0; f < W; ++f) sum[f] += widen(v[((static_cast<std::size_t>(b) * heads + h) * keys + key) * W + f]);
                }
                for (int f = 0; f < W; ++f) {
                    const double want = visible ? sum[f] / visible : 0.0;
                    worst_o = std::fmax(worst_o, std::fabs(widen(output[row * W + f]) - want));
                }
                if (visible) {
                    worst_max = std::fmax(worst_max, std::fabs(lse[2 * row] - score) / score);
                    bad_sum += lse[2 * row + 1] != static_cast<float>(visible);
                } else {
                    bad_sum += !(std::isinf(lse[2 * row]) && lse[2 * row] < 0 && lse[2 * row + 1] == 0.0f);
                }
            }
        }
    }
    char line[256];
    std::snprintf(line, sizeof line, "%s W=%d B%d H%d %dx%d radius %d: O max-abs %.3g, lse max rel %.3g, %d bad sums\n",
            std::is_same_v<T, __half> ? "fp16" : "fp32", W, batch, heads, queries, keys, radius, worst_o, worst_max, bad_sum);
    report.text += line;
    report.expect(worst_o <= tolerance, std::string("output within tolerance: ") + line);
    report.expect(worst_max <= 1e-6 && bad_sum == 0, std::string("lse closed form: ") + line);
}

} // namespace

// GPU check (device 0 must be an MI355X): returns the number of failures, or -1 when a HIP call or a wrapper threw;
// the report (one line per case, then any failure or the exception's message) is written to `text` (size bytes).
extern "C" __attribute__((visibility("default"))) int common_consumer_gpu_check(char *text, const int size) {
    Report report;
    int result = 0;
    try {
        const int devices = ROCmKernels::GetDeviceCount();
        report.expect(devices >= 1, "at least one device");
        const ROCmKernels::DeviceInfo info = ROCmKernels::QueryDevice(0);
        report.text += "device 0: " + info.name + " (" + info.gcnArchName + "), " + std::to_string(info.computeUnitCount) + " CUs, wave" +
                std::to_string(info.warpSize) + "\n";
        report.expect(info.gcnArchName.rfind("gfx950", 0) == 0, "device 0 is a gfx950");
        report.expect(info.computeUnitCount > 0 && info.warpSize == 64 && info.totalGlobalMemory > 0, "device properties");
        run_case<float, 32>(report, 2, 2, 40, 48, -1);
        run_case<float, 64>(report, 2, 1, 33, 37, 3);
        run_case<__half, 16>(report, 2, 2, 40, 48, -1);
        run_case<__half, 32>(report, 2, 1, 33, 37, 3);
        run_case<__half, 64>(report, 1, 2, 70, 70, 5);
        ROCmKernels::SynchronizeDevice(0);
        result = report.failures;
    } catch (const std::exception &error) {
        report.text += std::string("exception: ") + error.what() + "\n";
        result = -1;
    }
    if (text && size > 0) {
        std::strncpy(text, report.text.c_str(), static_cast<std::size_t>(size) - 1);
        text[size - 1] = '\0';
    }
    return result;
}

#ifdef COMMON_CONSUMER_MAIN
// CPU checks: nothing here needs a GPU.
int main() {
    Report report;
    {
        ROCmKernels::DeviceBuffer<__half> empty;
        report.expect(empty.Data() == nullptr && empty.Count() == 0 && empty.ByteSize() == 0, "empty DeviceBuffer");
        bool threw = false;
        const __half one = __float2half(1.0f);
        try {
            empty.CopyFromHost(&one, 1);
        } catch (const std::out_of_range &) {
            threw = true;
        }
        report.expect(threw, "copy past the allocation throws std::out_of_range");
        empty.Resize(0);
        ROCmKernels::DeviceBuffer<__half> moved(std::move(empty));
        report.expect(moved.Data() == nullptr && moved.Count() == 0, "moved empty DeviceBuffer");
        report.expect(sizeof(__half) == 2 && ROCmKernels::DeviceBuffer<float>().ByteSize() == 0, "element sizes");
    }
    try {
        const ROCmKernels::Kernels::Strides s{0, 0, 0};
        float lse[2] = {};
        ROCmKernels::Kernels::AttentionGenericForward(nullptr, nullptr, nullptr, nullptr, nullptr, lse, 1, 1, 1, 1, 16, -1, s, s, s, s,
                ROCmKernels::Kernels::DTypeOf<__half>::value);
        report.expect(false, "invalid arguments throw");
    } catch (const ROCmKernels::HipError &error) {
        report.expect(error.Status() == hipErrorInvalidValue, "invalid arguments throw HipError(hipErrorInvalidValue)");
        std::printf("%s\n", error.what());
    }
    // Without a GPU the runtime reports no device: GetDeviceCount either throws HipError or returns 0, and QueryDevice(0)
    // throws HipError.
    try {
        const int devices = ROCmKernels::GetDeviceCount();
        std::printf("devices: %d\n", devices);
        if (devices == 0) {
            bool threw = false;
            try {
                static_cast<void>(ROCmKernels::QueryDevice(0));
            } catch (const ROCmKernels::HipError &error) {
                threw = true;
                std::printf("%s\n", error.what());
            }
            report.expect(threw, "QueryDevice(0) without a device throws HipError");
        }
    } catch (const ROCmKernels::HipError &error) {
        std::printf("devices: none (%s)\n", error.what());
    }
    std::printf("%s%d failure(s)\n", report.text.c_str(), report.failures);
    return report.failures == 0 ? 0 : 1;
}
#endif
