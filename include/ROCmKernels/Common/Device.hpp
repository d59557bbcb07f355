#pragma once

// Device queries for host code that drives the kernels. Interface of the reference's
// ROCmKernels.Common/include/ROCmKernels/Common/Device.hpp:12-33 (DeviceInfo and the four functions, same names,
// arguments and defaults); defined in rocmkernels_amd/csrc/device.cpp, part of the ROCmKernels.Common static target.
// Every function throws ROCmKernels::HipError when a HIP call fails (for example hipErrorNoDevice on a host without a
// GPU).
#include <cstdint>
#include <string>

namespace ROCmKernels {
    // What HIP reports for one device.
    struct DeviceInfo {
        std::string name;        // marketing name
        std::string gcnArchName; // e.g. "gfx950:sramecc+:xnack-"
        std::uint64_t totalGlobalMemory = 0; // bytes
        std::uint32_t computeUnitCount = 0;
        std::uint32_t clockRateKHz = 0;
        std::uint32_t warpSize = 0;
        int runtimeVersion = 0;
        int driverVersion = 0;
    };

    // Devices visible to the HIP runtime.
    [[nodiscard]] int GetDeviceCount();

    // Properties of device deviceIndex.
    [[nodiscard]] DeviceInfo QueryDevice(int deviceIndex = 0);

    // Makes deviceIndex current and waits until all work queued on it has finished.
    void SynchronizeDevice(int deviceIndex = 0);

    // Makes deviceIndex current and resets it: its allocations and streams are destroyed.
    void ResetDevice(int deviceIndex = 0);
} // namespace ROCmKernels
