#pragma once

// Bump allocator over one device allocation, the counterpart of the reference's
// DeviceArena (include/cuvit/device_arena.hpp:26-113). Every carve is padded
// to 256 bytes, so every tensor in an arena starts 16-byte aligned, which is
// what lets the kernels use dwordx4 traffic on interior buffers. reset()
// rewinds everything at once; nothing is freed individually.

#include "cuvit/device_buffer.hpp"
#include "cuvit/tensor.hpp"

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <stdexcept>
#include <string>

namespace cuvit {

class DeviceArena final {
  public:
    static constexpr std::size_t kAlignment = 256;

    DeviceArena() noexcept = default;
    explicit DeviceArena(std::size_t capacity_bytes) { reserve(capacity_bytes); }

    /// Replaces the backing allocation and forgets everything carved from it.
    void reserve(std::size_t capacity_bytes) {
        storage_.allocate(capacity_bytes);
        used_ = 0;
    }

    void reset() noexcept { used_ = 0; }

    /// Arena bytes a tensor of @p count elements takes, padding included.
    template <typename T> [[nodiscard]] static std::size_t reserved_bytes(std::size_t count) {
        return round_up(element_bytes<T>(count));
    }

    template <typename T> [[nodiscard]] TensorView<T> allocate(std::initializer_list<Extent> extents) {
        Extent count = 1;
        for (const Extent e : extents) {
            if (e < 0) {
                throw std::invalid_argument("DeviceArena extents cannot be negative");
            }
            count *= e;
        }
        return TensorView<T>(static_cast<T*>(carve(element_bytes<T>(static_cast<std::size_t>(count)),
                                                   alignof(T))),
                             extents);
    }

    template <typename T> [[nodiscard]] T* allocate_raw(std::size_t count) {
        return static_cast<T*>(carve(element_bytes<T>(count), alignof(T)));
    }

    void fill_zero() { storage_.fill_zero(); }
    void fill_zero_async(hipStream_t stream) { storage_.fill_zero_async(stream); }

    [[nodiscard]] std::size_t capacity() const noexcept { return storage_.size(); }
    [[nodiscard]] std::size_t used() const noexcept { return used_; }
    [[nodiscard]] std::size_t remaining() const noexcept { return capacity() - used_; }
    [[nodiscard]] const std::byte* data() const noexcept { return storage_.data(); }

  private:
    static constexpr std::size_t round_up(std::size_t bytes) noexcept {
        return (bytes + kAlignment - 1) / kAlignment * kAlignment;
    }

    template <typename T> static std::size_t element_bytes(std::size_t count) {
        if (count > SIZE_MAX / sizeof(T)) {
            throw std::overflow_error("DeviceArena allocation size overflow");
        }
        return count * sizeof(T);
    }

    void* carve(std::size_t bytes, std::size_t alignment) {
        if (alignment > kAlignment) {
            throw std::invalid_argument("DeviceArena cannot satisfy an over-aligned type");
        }
        const std::size_t padded = round_up(bytes);
        if (padded > remaining()) {
            throw std::runtime_error("DeviceArena is out of capacity: " + std::to_string(padded) +
                                     " bytes requested, " + std::to_string(remaining()) + " of " +
                                     std::to_string(capacity()) + " remaining");
        }
        std::byte* const pointer = storage_.data() + used_;
        used_ += padded;
        return pointer;
    }

    DeviceBuffer<std::byte> storage_;
    std::size_t used_ = 0;
};

} // namespace cuvit
