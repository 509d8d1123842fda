#pragma once

// One device allocation owned by one object. Interface of the reference's
// DeviceBuffer<T> (include/cuvit/device_buffer.hpp:22-244): an element count,
// allocate / reset, blocking and stream-ordered copies to and from the host
// and between buffers of one device, zero fills, moves, and the device the
// memory lives on.
//
// The allocation sits in a unique_ptr whose deleter remembers the owning
// device and makes it current for hipFree. Every copy goes through one routine
// that checks the element range first, then skips empty copies, then checks
// the other side (a host pointer, or a device buffer: same device, and for a
// copy within one buffer, ranges that do not overlap).

#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <memory>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>

namespace cuvit {

template <typename T> class DeviceBuffer final {
    static_assert(std::is_trivially_copyable<T>::value && !std::is_const<T>::value &&
                      !std::is_reference<T>::value,
                  "DeviceBuffer holds mutable, trivially copyable elements");

  public:
    DeviceBuffer() noexcept = default;
    explicit DeviceBuffer(std::size_t count) { allocate(count); }

    DeviceBuffer(DeviceBuffer&& other) noexcept
        : memory_(std::move(other.memory_)), count_(std::exchange(other.count_, 0)) {}

    DeviceBuffer& operator=(DeviceBuffer&& other) noexcept {
        DeviceBuffer(std::move(other)).swap(*this);
        return *this;
    }

    /// Holds exactly @p count elements on the current device afterwards. The
    /// count already held changes nothing (memory, contents and device stay);
    /// any other count replaces the allocation, zero releases it.
    void allocate(std::size_t count) {
        if (count != count_) {
            DeviceBuffer(Sized{}, count).swap(*this);
        }
    }

    void reset() noexcept { DeviceBuffer().swap(*this); }

    void copy_from_host(const T* source, std::size_t count, std::size_t offset = 0) {
        from_host(source, count, offset, nullptr);
    }
    void copy_from_host_async(const T* source, std::size_t count, hipStream_t stream,
                              std::size_t offset = 0) {
        from_host(source, count, offset, &stream);
    }
    void copy_to_host(T* destination, std::size_t count, std::size_t offset = 0) const {
        to_host(destination, count, offset, nullptr);
    }
    void copy_to_host_async(T* destination, std::size_t count, hipStream_t stream,
                            std::size_t offset = 0) const {
        to_host(destination, count, offset, &stream);
    }
    void copy_from_device(const DeviceBuffer& source, std::size_t count,
                          std::size_t source_offset = 0, std::size_t destination_offset = 0) {
        from_device(source, count, source_offset, destination_offset, nullptr);
    }
    void copy_from_device_async(const DeviceBuffer& source, std::size_t count, hipStream_t stream,
                                std::size_t source_offset = 0, std::size_t destination_offset = 0) {
        from_device(source, count, source_offset, destination_offset, &stream);
    }

    void fill_zero() {
        if (count_ != 0) {
            CUVIT_HIP_CHECK(hipMemset(data(), 0, bytes()));
        }
    }
    void fill_zero_async(hipStream_t stream) {
        if (count_ != 0) {
            CUVIT_HIP_CHECK(hipMemsetAsync(data(), 0, bytes(), stream));
        }
    }

    void swap(DeviceBuffer& other) noexcept {
        memory_.swap(other.memory_);
        std::swap(count_, other.count_);
    }

    [[nodiscard]] T* data() noexcept { return memory_.get(); }
    [[nodiscard]] const T* data() const noexcept { return memory_.get(); }
    [[nodiscard]] std::size_t size() const noexcept { return count_; }
    [[nodiscard]] std::size_t bytes() const noexcept { return count_ * sizeof(T); }
    [[nodiscard]] bool empty() const noexcept { return count_ == 0; }
    /// The device holding the memory; -1 when there is none.
    [[nodiscard]] int device() const noexcept {
        return memory_ ? memory_.get_deleter().device : -1;
    }

  private:
    struct FreeOnDevice {
        int device = -1;
        void operator()(T* memory) const noexcept {
            int current = -1;
            const bool away = hipGetDevice(&current) == hipSuccess && current != device;
            if (away) {
                static_cast<void>(hipSetDevice(device));
            }
            static_cast<void>(hipFree(memory));
            if (away) {
                static_cast<void>(hipSetDevice(current));
            }
        }
    };
    struct Sized {};

    DeviceBuffer(Sized, std::size_t count) : count_(count) {
        if (count == 0) {
            return;
        }
        int device = -1;
        CUVIT_HIP_CHECK(hipGetDevice(&device));
        void* memory = nullptr;
        CUVIT_HIP_CHECK(hipMalloc(&memory, byte_count(count)));
        memory_ = Memory(static_cast<T*>(memory), FreeOnDevice{device});
    }

    static std::size_t byte_count(std::size_t count) {
        std::size_t total = 0;
        if (__builtin_mul_overflow(count, sizeof(T), &total)) {
            throw std::overflow_error("DeviceBuffer byte size overflow");
        }
        return total;
    }

    /// Whether [offset, offset + count) lies inside the buffer; throws if not.
    void require_range(std::size_t count, std::size_t offset) const {
        if (offset <= count_ && count <= count_ - offset) {
            return;
        }
        throw std::out_of_range("DeviceBuffer copy of " + std::to_string(count) +
                                " elements at offset " + std::to_string(offset) +
                                " leaves the allocation of " + std::to_string(count_));
    }

    static void move_bytes(void* to, const void* from, std::size_t bytes, hipMemcpyKind kind,
                           const hipStream_t* stream) {
        if (stream != nullptr) {
            CUVIT_HIP_CHECK(hipMemcpyAsync(to, from, bytes, kind, *stream));
        } else {
            CUVIT_HIP_CHECK(hipMemcpy(to, from, bytes, kind));
        }
    }

    void from_host(const T* source, std::size_t count, std::size_t offset, const hipStream_t* stream) {
        require_range(count, offset);
        if (count == 0) {
            return;
        }
        if (source == nullptr) {
            throw std::invalid_argument("DeviceBuffer copy: the host source is null");
        }
        move_bytes(data() + offset, source, count * sizeof(T), hipMemcpyHostToDevice, stream);
    }

    void to_host(T* destination, std::size_t count, std::size_t offset, const hipStream_t* stream) const {
        require_range(count, offset);
        if (count == 0) {
            return;
        }
        if (destination == nullptr) {
            throw std::invalid_argument("DeviceBuffer copy: the host destination is null");
        }
        move_bytes(destination, data() + offset, count * sizeof(T), hipMemcpyDeviceToHost, stream);
    }

    void from_device(const DeviceBuffer& source, std::size_t count, std::size_t source_offset,
                     std::size_t destination_offset, const hipStream_t* stream) {
        source.require_range(count, source_offset);
        require_range(count, destination_offset);
        if (count == 0) {
            return;
        }
        if (source.device() != device()) {
            throw std::invalid_argument("DeviceBuffer copy: the buffers live on different devices");
        }
        const bool overlapping = &source == this && (source_offset < destination_offset + count &&
                                                     destination_offset < source_offset + count);
        if (overlapping) {
            throw std::invalid_argument("DeviceBuffer copy: source and destination ranges overlap");
        }
        move_bytes(data() + destination_offset, source.data() + source_offset, count * sizeof(T),
                   hipMemcpyDeviceToDevice, stream);
    }

    using Memory = std::unique_ptr<T, FreeOnDevice>;
    Memory memory_;
    std::size_t count_ = 0;
};

template <typename T> void swap(DeviceBuffer<T>& left, DeviceBuffer<T>& right) noexcept {
    left.swap(right);
}

} // namespace cuvit
