#pragma once

// Owner of pinned host memory, the counterpart of the reference's HostBuffer<T>
// (include/cuvit/host_buffer.hpp:25-134). Memory comes from hipHostMalloc, so
// stream-ordered copies from it are truly asynchronous. Allocate once and reuse:
// pinning is expensive.

#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace cuvit {

template <typename T> class HostBuffer final {
    static_assert(!std::is_const<T>::value, "HostBuffer cannot own const elements");
    static_assert(!std::is_reference<T>::value, "HostBuffer cannot own references");
    static_assert(std::is_trivially_copyable<T>::value,
                  "HostBuffer elements must be trivially copyable");

  public:
    HostBuffer() noexcept = default;
    explicit HostBuffer(std::size_t count) { allocate(count); }
    ~HostBuffer() { release(); }

    HostBuffer(const HostBuffer&) = delete;
    HostBuffer& operator=(const HostBuffer&) = delete;

    HostBuffer(HostBuffer&& other) noexcept { swap(other); }
    HostBuffer& operator=(HostBuffer&& other) noexcept {
        if (this != &other) {
            release();
            swap(other);
        }
        return *this;
    }

    /// Owns exactly @p count pinned elements; the current size is a no-op.
    void allocate(std::size_t count) {
        if (count == size_) {
            return;
        }
        HostBuffer fresh;
        if (count != 0) {
            if (count > std::numeric_limits<std::size_t>::max() / sizeof(T)) {
                throw std::overflow_error("HostBuffer byte size overflow");
            }
            void* memory = nullptr;
            CUVIT_HIP_CHECK(hipHostMalloc(&memory, count * sizeof(T), hipHostMallocDefault));
            fresh.data_ = static_cast<T*>(memory);
            fresh.size_ = count;
        }
        swap(fresh);
    }

    void reset() noexcept { release(); }

    void fill_zero() noexcept {
        if (data_ != nullptr) {
            std::memset(static_cast<void*>(data_), 0, bytes());
        }
    }

    void swap(HostBuffer& other) noexcept {
        std::swap(data_, other.data_);
        std::swap(size_, other.size_);
    }

    [[nodiscard]] T& operator[](std::size_t index) noexcept { return data_[index]; }
    [[nodiscard]] const T& operator[](std::size_t index) const noexcept { return data_[index]; }

    [[nodiscard]] T& at(std::size_t index) {
        if (index >= size_) {
            throw std::out_of_range("HostBuffer index is out of range");
        }
        return data_[index];
    }
    [[nodiscard]] const T& at(std::size_t index) const {
        if (index >= size_) {
            throw std::out_of_range("HostBuffer index is out of range");
        }
        return data_[index];
    }

    [[nodiscard]] T* data() noexcept { return data_; }
    [[nodiscard]] const T* data() const noexcept { return data_; }
    [[nodiscard]] T* begin() noexcept { return data_; }
    [[nodiscard]] const T* begin() const noexcept { return data_; }
    [[nodiscard]] T* end() noexcept { return data_ + size_; }
    [[nodiscard]] const T* end() const noexcept { return data_ + size_; }
    [[nodiscard]] std::size_t size() const noexcept { return size_; }
    [[nodiscard]] std::size_t bytes() const noexcept { return size_ * sizeof(T); }
    [[nodiscard]] bool empty() const noexcept { return size_ == 0; }

  private:
    void release() noexcept {
        if (data_ != nullptr) {
            static_cast<void>(hipHostFree(data_));
        }
        data_ = nullptr;
        size_ = 0;
    }

    T* data_ = nullptr;
    std::size_t size_ = 0;
};

template <typename T> void swap(HostBuffer<T>& left, HostBuffer<T>& right) noexcept {
    left.swap(right);
}

} // namespace cuvit
