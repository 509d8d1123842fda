#pragma once

// A bump allocator over one device allocation. Interface of the reference's
// DeviceArena (include/cuvit/device_arena.hpp:26-113): reserve a capacity,
// carve tensors (as TensorViews) or raw arrays from it, rewind everything at
// once with reset(); nothing is freed on its own.
//
// Every carve starts on a 256-byte boundary and takes a whole number of
// 256-byte granules, so every tensor in an arena is 16-byte aligned and the
// kernels' 16-byte vector paths apply to all of them. A carve that does not
// fit throws and leaves the arena as it was.

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

    /// A fresh backing allocation of @p capacity_bytes; earlier carves are void.
    void reserve(std::size_t capacity_bytes) {
        granules_.allocate(capacity_bytes);
        cursor_ = 0;
    }

    void reset() noexcept { cursor_ = 0; }

    /// The arena bytes @p count elements of T occupy, padding included.
    template <typename T> [[nodiscard]] static std::size_t reserved_bytes(std::size_t count) {
        return granule_bytes(bytes_of<T>(count));
    }

    template <typename T> [[nodiscard]] TensorView<T> allocate(std::initializer_list<Extent> extents) {
        std::size_t count = 1;
        for (const Extent extent : extents) {
            if (extent < 0) {
                throw std::invalid_argument("DeviceArena extents cannot be negative");
            }
            if (__builtin_mul_overflow(count, static_cast<std::size_t>(extent), &count)) {
                throw std::overflow_error("DeviceArena allocation size overflow");
            }
        }
        return TensorView<T>(allocate_raw<T>(count), extents);
    }

    template <typename T> [[nodiscard]] T* allocate_raw(std::size_t count) {
        static_assert(alignof(T) <= kAlignment, "DeviceArena cannot align this type");
        return reinterpret_cast<T*>(take(granule_bytes(bytes_of<T>(count))));
    }

    void fill_zero() { granules_.fill_zero(); }
    void fill_zero_async(hipStream_t stream) { granules_.fill_zero_async(stream); }

    [[nodiscard]] std::size_t capacity() const noexcept { return granules_.size(); }
    [[nodiscard]] std::size_t used() const noexcept { return cursor_; }
    [[nodiscard]] std::size_t remaining() const noexcept { return granules_.size() - cursor_; }
    [[nodiscard]] const std::byte* data() const noexcept { return granules_.data(); }

  private:
    template <typename T> static std::size_t bytes_of(std::size_t count) {
        std::size_t bytes = 0;
        if (__builtin_mul_overflow(count, sizeof(T), &bytes)) {
            throw std::overflow_error("DeviceArena allocation size overflow");
        }
        return bytes;
    }

    /// @p bytes rounded up to whole granules.
    static std::size_t granule_bytes(std::size_t bytes) {
        constexpr std::size_t mask = kAlignment - 1;
        static_assert((kAlignment & mask) == 0, "granules are a power of two");
        std::size_t padded = 0;
        if (__builtin_add_overflow(bytes, mask, &padded)) {
            throw std::overflow_error("DeviceArena allocation size overflow");
        }
        return padded & ~mask;
    }

    std::byte* take(std::size_t padded) {
        if (padded > remaining()) {
            throw std::runtime_error("DeviceArena is out of capacity: " + std::to_string(padded) +
                                     " bytes asked for, " + std::to_string(remaining()) +
                                     " of " + std::to_string(capacity()) + " left");
        }
        std::byte* const start = granules_.data() + cursor_;
        cursor_ += padded;
        return start;
    }

    DeviceBuffer<std::byte> granules_;
    std::size_t cursor_ = 0;
};

} // namespace cuvit
