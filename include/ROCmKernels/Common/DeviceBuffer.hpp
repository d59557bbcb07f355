#pragma once

// Owning handle to one HIP device allocation of `Count()` elements of T, for host code that calls the kernels (tests,
// benchmarks, training harnesses). Interface of the reference's
// ROCmKernels.Common/include/ROCmKernels/Common/DeviceBuffer.hpp:15-101: constructed empty or with an element count,
// move-only, Resize/Release, host copies bounded by the allocation (std::out_of_range beyond it), Data/Count/ByteSize.
// A failing HIP call throws ROCmKernels::HipError. The library's kernels themselves never allocate: this type is for
// their callers.
//
// Copies with a null stream are synchronous (hipMemcpy); with a stream they are queued on it (hipMemcpyAsync), and the
// host memory must stay valid until the stream reaches them.
#include <ROCmKernels/Common/Error.hpp>

#include <cstddef>
#include <stdexcept>
#include <utility>

namespace ROCmKernels {
    template<typename T> class DeviceBuffer {
      public:
        DeviceBuffer() = default;

        explicit DeviceBuffer(const std::size_t elementCount) { Resize(elementCount); }

        // Frees the allocation. A destructor cannot report an error, so a failing hipFree here is ignored (call
        // Release() first to have it thrown).
        ~DeviceBuffer() {
            if (data_ != nullptr) static_cast<void>(hipFree(data_));
        }

        DeviceBuffer(const DeviceBuffer &) = delete;
        DeviceBuffer &operator=(const DeviceBuffer &) = delete;

        DeviceBuffer(DeviceBuffer &&other) noexcept : data_(other.data_), count_(other.count_) {
            other.data_ = nullptr;
            other.count_ = 0;
        }

        DeviceBuffer &operator=(DeviceBuffer &&other) noexcept {
            if (this != &other) {
                DeviceBuffer old(std::move(*this)); // freed when `old` goes out of scope
                std::swap(data_, other.data_);
                std::swap(count_, other.count_);
            }
            return *this;
        }

        // Replaces the allocation with one of elementCount elements (none for 0); the contents are not kept.
        void Resize(const std::size_t elementCount) {
            Release();
            if (elementCount == 0) return;
            if (elementCount > static_cast<std::size_t>(-1) / sizeof(T)) throw std::length_error("DeviceBuffer: element count too large");
            void *allocation = nullptr;
            ROCMKERNELS_HIP_CHECK(hipMalloc(&allocation, elementCount * sizeof(T)));
            data_ = static_cast<T *>(allocation);
            count_ = elementCount;
        }

        // Frees the allocation (if any); the buffer is empty afterwards even when hipFree fails (which throws).
        void Release() {
            T *const allocation = data_;
            data_ = nullptr;
            count_ = 0;
            if (allocation != nullptr) ROCMKERNELS_HIP_CHECK(hipFree(allocation));
        }

        // Copies elementCount elements from host memory to the start of the buffer.
        void CopyFromHost(const T *source, const std::size_t elementCount, hipStream_t stream = nullptr) {
            Copy(data_, source, elementCount, hipMemcpyHostToDevice, stream);
        }

        // Copies the buffer's first elementCount elements to host memory.
        void CopyToHost(T *destination, const std::size_t elementCount, hipStream_t stream = nullptr) const {
            Copy(destination, data_, elementCount, hipMemcpyDeviceToHost, stream);
        }

        [[nodiscard]] T *Data() const noexcept { return data_; }
        [[nodiscard]] std::size_t Count() const noexcept { return count_; }
        [[nodiscard]] std::size_t ByteSize() const noexcept { return count_ * sizeof(T); }

      private:
        void Copy(void *to, const void *from, const std::size_t elementCount, const hipMemcpyKind kind, hipStream_t stream) const {
            if (elementCount > count_) throw std::out_of_range("DeviceBuffer: copy of more elements than the buffer holds");
            if (elementCount == 0) return;
            const std::size_t bytes = elementCount * sizeof(T);
            if (stream == nullptr) {
                ROCMKERNELS_HIP_CHECK(hipMemcpy(to, from, bytes, kind));
            } else {
                ROCMKERNELS_HIP_CHECK(hipMemcpyAsync(to, from, bytes, kind, stream));
            }
        }

        T *data_ = nullptr;
        std::size_t count_ = 0;
    };
} // namespace ROCmKernels
