#pragma once

// Storage types of the generic kernels' tensors; accumulation is always fp32. Interface of the reference's
// ROCmKernels.Kernels/include/ROCmKernels/Kernels/DType.hpp:1-44: the DType enumerators (same underlying type and
// values, convertible to the C ABI's rocmkernels_dtype), the DTypeOf<T> trait a templated caller passes as
// `DTypeOf<T>::value` (float and __half), and the scalar/pair load-store helpers for device code, which widen __half
// to float on load and round to nearest even on store.
//
// Host compilers see this header too (g++ with __HIP_PLATFORM_AMD__ defined, as for every header of this library):
// <hip/hip_fp16.h> declares __half for host code, and the device helpers are only instantiated in HIP device code.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>

#include <rocmkernels_attention.h>

namespace ROCmKernels::Kernels {
    enum class DType : unsigned char { Float32 = ROCMKERNELS_DTYPE_FLOAT32, Float16 = ROCMKERNELS_DTYPE_FLOAT16 };

    // DTypeOf<T>::value names the storage type T; only float and __half are defined.
    template<typename T> struct DTypeOf;
    template<> struct DTypeOf<float> {
        static constexpr DType value = DType::Float32;
    };
    template<> struct DTypeOf<__half> {
        static constexpr DType value = DType::Float16;
    };

    namespace Detail {
        template<typename T> inline constexpr bool kIsHalf = std::is_same_v<T, __half>;
    } // namespace Detail

    // One element of storage type T, as float.
    template<typename T> __device__ __forceinline__ float LoadScalar(const T *pointer) {
        static_assert(std::is_same_v<T, float> || Detail::kIsHalf<T>, "storage type must be float or __half");
        if constexpr (Detail::kIsHalf<T>) {
            return __half2float(pointer[0]);
        } else {
            return pointer[0];
        }
    }

    // Stores value as storage type T (__half: rounded to nearest even).
    template<typename T> __device__ __forceinline__ void StoreScalar(T *pointer, const float value) {
        static_assert(std::is_same_v<T, float> || Detail::kIsHalf<T>, "storage type must be float or __half");
        if constexpr (Detail::kIsHalf<T>) {
            pointer[0] = __float2half_rn(value);
        } else {
            pointer[0] = value;
        }
    }

    // Two consecutive elements (pointer aligned to two elements), as float2.
    template<typename T> __device__ __forceinline__ float2 LoadPair(const T *pointer) {
        static_assert(std::is_same_v<T, float> || Detail::kIsHalf<T>, "storage type must be float or __half");
        if constexpr (Detail::kIsHalf<T>) {
            return __half22float2(*reinterpret_cast<const __half2 *>(pointer));
        } else {
            return *reinterpret_cast<const float2 *>(pointer);
        }
    }

    // Stores two consecutive elements (pointer aligned to two elements); __half rounds each to nearest even.
    template<typename T> __device__ __forceinline__ void StorePair(T *pointer, const float2 value) {
        static_assert(std::is_same_v<T, float> || Detail::kIsHalf<T>, "storage type must be float or __half");
        if constexpr (Detail::kIsHalf<T>) {
            *reinterpret_cast<__half2 *>(pointer) = __floats2half2_rn(value.x, value.y);
        } else {
            *reinterpret_cast<float2 *>(pointer) = value;
        }
    }
} // namespace ROCmKernels::Kernels
