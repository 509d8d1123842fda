#pragma once

// Owner of one device allocation, the counterpart of the reference's
// DeviceBuffer<T> (include/cuvit/device_buffer.hpp:22-244): move-only, records
// the device it lives on, synchronous and stream-ordered copies with bounds
// checks, rejects cross-device and overlapping self copies, zero fills.

#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <limits>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>

namespace cuvit {

template <typename T> class DeviceBuffer final {
    static_assert(!std::is_const<T>::value, "DeviceBuffer cannot own const elements");
    static_assert(!std::is_reference<T>::value, "DeviceBuffer cannot own references");
    static_assert(std::is_trivially_copyable<T>::value,
                  "DeviceBuffer elements must be trivially copyable");

  public:
    DeviceBuffer() noexcept = default;
    explicit DeviceBuffer(std::size_t count) { allocate(count); }
    ~DeviceBuffer() { release(); }

    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;

    DeviceBuffer(DeviceBuffer&& other) noexcept { swap(other); }
    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
        if (this != &other) {
            release();
            swap(other);
        }
        return *this;
    }

    /// Owns exactly @p count elements on the current device. Asking for the
    /// size already held keeps the allocation, its contents and its device.
    void allocate(std::size_t count) {
        if (count == size_) {
            return;
        }
        DeviceBuffer fresh;
        if (count != 0) {
            CUVIT_HIP_CHECK(hipGetDevice(&fresh.device_));
            void* memory = nullptr;
            CUVIT_HIP_CHECK(hipMalloc(&memory, byte_count(count)));
            fresh.data_ = static_cast<T*>(memory);
            fresh.size_ = count;
        }
        swap(fresh);
    }

    void reset() noexcept { release(); }

    void copy_from_host(const T* source, std::size_t count, std::size_t offset = 0) {
        if (prepare(count, offset, source, "source")) {
            CUVIT_HIP_CHECK(hipMemcpy(data_ + offset, source, byte_count(count), hipMemcpyHostToDevice));
        }
    }

    void copy_from_host_async(const T* source, std::size_t count, hipStream_t stream,
                              std::size_t offset = 0) {
        if (prepare(count, offset, source, "source")) {
            CUVIT_HIP_CHECK(hipMemcpyAsync(data_ + offset, source, byte_count(count),
                                           hipMemcpyHostToDevice, stream));
        }
    }

    void copy_to_host(T* destination, std::size_t count, std::size_t offset = 0) const {
        if (prepare(count, offset, destination, "destination")) {
            CUVIT_HIP_CHECK(hipMemcpy(destination, data_ + offset, byte_count(count), hipMemcpyDeviceToHost));
        }
    }

    void copy_to_host_async(T* destination, std::size_t count, hipStream_t stream,
                            std::size_t offset = 0) const {
        if (prepare(count, offset, destination, "destination")) {
            CUVIT_HIP_CHECK(hipMemcpyAsync(destination, data_ + offset, byte_count(count),
                                           hipMemcpyDeviceToHost, stream));
        }
    }

    void copy_from_device(const DeviceBuffer& source, std::size_t count,
                          std::size_t source_offset = 0, std::size_t destination_offset = 0) {
        if (prepare_device(source, count, source_offset, destination_offset)) {
            CUVIT_HIP_CHECK(hipMemcpy(data_ + destination_offset, source.data_ + source_offset,
                                      byte_count(count), hipMemcpyDeviceToDevice));
        }
    }

    void copy_from_device_async(const DeviceBuffer& source, std::size_t count, hipStream_t stream,
                                std::size_t source_offset = 0, std::size_t destination_offset = 0) {
        if (prepare_device(source, count, source_offset, destination_offset)) {
            CUVIT_HIP_CHECK(hipMemcpyAsync(data_ + destination_offset, source.data_ + source_offset,
                                           byte_count(count), hipMemcpyDeviceToDevice, stream));
        }
    }

    void fill_zero() {
        if (!empty()) {
            CUVIT_HIP_CHECK(hipMemset(data_, 0, bytes()));
        }
    }

    void fill_zero_async(hipStream_t stream) {
        if (!empty()) {
            CUVIT_HIP_CHECK(hipMemsetAsync(data_, 0, bytes(), stream));
        }
    }

    void swap(DeviceBuffer& other) noexcept {
        std::swap(data_, other.data_);
        std::swap(size_, other.size_);
        std::swap(device_, other.device_);
    }

    [[nodiscard]] T* data() noexcept { return data_; }
    [[nodiscard]] const T* data() const noexcept { return data_; }
    [[nodiscard]] std::size_t size() const noexcept { return size_; }
    [[nodiscard]] std::size_t bytes() const noexcept { return size_ * sizeof(T); }
    [[nodiscard]] bool empty() const noexcept { return size_ == 0; }
    /// Device holding the allocation, or -1 when empty.
    [[nodiscard]] int device() const noexcept { return device_; }

  private:
    static std::size_t byte_count(std::size_t count) {
        if (count > std::numeric_limits<std::size_t>::max() / sizeof(T)) {
            throw std::overflow_error("DeviceBuffer byte size overflow");
        }
        return count * sizeof(T);
    }

    void check_range(std::size_t count, std::size_t offset) const {
        if (offset > size_ || count > size_ - offset) {
            throw std::out_of_range("DeviceBuffer copy exceeds allocation bounds");
        }
    }

    /// Validates a host copy; false when there is nothing to copy.
    bool prepare(std::size_t count, std::size_t offset, const void* host, const char* role) const {
        check_range(count, offset);
        if (count == 0) {
            return false;
        }
        if (host == nullptr) {
            throw std::invalid_argument(std::string("Host ") + role + " pointer cannot be null");
        }
        return true;
    }

    bool prepare_device(const DeviceBuffer& source, std::size_t count, std::size_t source_offset,
                        std::size_t destination_offset) const {
        source.check_range(count, source_offset);
        check_range(count, destination_offset);
        if (count == 0) {
            return false;
        }
        if (source.device_ != device_) {
            throw std::invalid_argument("DeviceBuffer copies between different devices are not supported");
        }
        if (this == &source) {
            const std::size_t gap = source_offset > destination_offset ? source_offset - destination_offset
                                                                       : destination_offset - source_offset;
            if (gap < count) {
                throw std::invalid_argument("DeviceBuffer device-to-device copy ranges must not overlap");
            }
        }
        return true;
    }

    void release() noexcept {
        if (data_ != nullptr) {
            // hipFree wants the owning device current.
            int current = -1;
            const bool switched = hipGetDevice(&current) == hipSuccess && current != device_ &&
                                  hipSetDevice(device_) == hipSuccess;
            static_cast<void>(hipFree(data_));
            if (switched) {
                static_cast<void>(hipSetDevice(current));
            }
        }
        data_ = nullptr;
        size_ = 0;
        device_ = -1;
    }

    T* data_ = nullptr;
    std::size_t size_ = 0;
    int device_ = -1;
};

template <typename T> void swap(DeviceBuffer<T>& left, DeviceBuffer<T>& right) noexcept {
    left.swap(right);
}

} // namespace cuvit
