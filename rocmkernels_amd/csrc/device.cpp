// Host-side device queries of the ROCmKernels.Common target (declared in include/ROCmKernels/Common/Device.hpp;
// interface of the reference's ROCmKernels.Common/src/Device.cpp). Plain C++ against the HIP runtime API: no kernels.
#include <ROCmKernels/Common/Device.hpp>

#include <ROCmKernels/Common/Error.hpp>

#include <hip/hip_runtime_api.h>

namespace ROCmKernels {
    int GetDeviceCount() {
        int count = 0;
        ROCMKERNELS_HIP_CHECK(hipGetDeviceCount(&count));
        return count;
    }

    DeviceInfo QueryDevice(const int deviceIndex) {
        hipDeviceProp_t props{};
        ROCMKERNELS_HIP_CHECK(hipGetDeviceProperties(&props, deviceIndex));
        DeviceInfo info;
        info.name = props.name;
        info.gcnArchName = props.gcnArchName;
        info.totalGlobalMemory = static_cast<std::uint64_t>(props.totalGlobalMem);
        info.computeUnitCount = static_cast<std::uint32_t>(props.multiProcessorCount);
        info.clockRateKHz = static_cast<std::uint32_t>(props.clockRate);
        info.warpSize = static_cast<std::uint32_t>(props.warpSize);
        ROCMKERNELS_HIP_CHECK(hipRuntimeGetVersion(&info.runtimeVersion));
        ROCMKERNELS_HIP_CHECK(hipDriverGetVersion(&info.driverVersion));
        return info;
    }

    void SynchronizeDevice(const int deviceIndex) {
        ROCMKERNELS_HIP_CHECK(hipSetDevice(deviceIndex));
        ROCMKERNELS_HIP_CHECK(hipDeviceSynchronize());
    }

    void ResetDevice(const int deviceIndex) {
        ROCMKERNELS_HIP_CHECK(hipSetDevice(deviceIndex));
        ROCMKERNELS_HIP_CHECK(hipDeviceReset());
    }
} // namespace ROCmKernels
