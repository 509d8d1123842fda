#pragma once

// Page-locked host memory owned by one object. Interface of the reference's
// HostBuffer<T> (include/cuvit/host_buffer.hpp:25-134): an element count,
// allocate / reset, indexed and checked access, iteration, zero fill, moves.
// Pinned pages make stream-ordered copies from and to them asynchronous, and
// pinning is slow, so a buffer is meant to be sized once and reused.
//
// The pages sit in a unique_ptr whose deleter returns them with hipHostFree;
// the element count travels beside it.

#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace cuvit {

template <typename T> class HostBuffer final {
    static_assert(std::is_trivially_copyable<T>::value && !std::is_const<T>::value &&
                      !std::is_reference<T>::value,
                  "HostBuffer holds mutable, trivially copyable elements");

  public:
    HostBuffer() noexcept = default;
    explicit HostBuffer(std::size_t count) { allocate(count); }

    HostBuffer(HostBuffer&& other) noexcept
        : pages_(std::move(other.pages_)), count_(std::exchange(other.count_, 0)) {}

    HostBuffer& operator=(HostBuffer&& other) noexcept {
        HostBuffer(std::move(other)).swap(*this);
        return *this;
    }

    /// Holds exactly @p count elements afterwards. The count already held
    /// changes nothing, so the contents survive; any other count replaces
    /// the pages (contents not kept), zero releases them.
    void allocate(std::size_t count) {
        if (count != count_) {
            HostBuffer(Sized{}, count).swap(*this);
        }
    }

    void reset() noexcept { HostBuffer().swap(*this); }

    void fill_zero() noexcept {
        if (count_ != 0) {
            std::memset(static_cast<void*>(pages_.get()), 0, bytes());
        }
    }

    void swap(HostBuffer& other) noexcept {
        pages_.swap(other.pages_);
        std::swap(count_, other.count_);
    }

    [[nodiscard]] T& operator[](std::size_t i) noexcept { return pages_.get()[i]; }
    [[nodiscard]] const T& operator[](std::size_t i) const noexcept { return pages_.get()[i]; }

    [[nodiscard]] T& at(std::size_t i) { return pages_.get()[checked(i)]; }
    [[nodiscard]] const T& at(std::size_t i) const { return pages_.get()[checked(i)]; }

    [[nodiscard]] T* data() noexcept { return pages_.get(); }
    [[nodiscard]] const T* data() const noexcept { return pages_.get(); }
    [[nodiscard]] T* begin() noexcept { return data(); }
    [[nodiscard]] const T* begin() const noexcept { return data(); }
    [[nodiscard]] T* end() noexcept { return data() + count_; }
    [[nodiscard]] const T* end() const noexcept { return data() + count_; }
    [[nodiscard]] std::size_t size() const noexcept { return count_; }
    [[nodiscard]] std::size_t bytes() const noexcept { return count_ * sizeof(T); }
    [[nodiscard]] bool empty() const noexcept { return count_ == 0; }

  private:
    struct Unpin {
        void operator()(T* pages) const noexcept { static_cast<void>(hipHostFree(pages)); }
    };
    struct Sized {};

    HostBuffer(Sized, std::size_t count) : count_(count) {
        if (count == 0) {
            return;
        }
        std::size_t total = 0;
        if (__builtin_mul_overflow(count, sizeof(T), &total)) {
            throw std::overflow_error("HostBuffer byte size overflow");
        }
        void* pages = nullptr;
        CUVIT_HIP_CHECK(hipHostMalloc(&pages, total, hipHostMallocDefault));
        pages_.reset(static_cast<T*>(pages));
    }

    std::size_t checked(std::size_t i) const {
        if (i < count_) {
            return i;
        }
        throw std::out_of_range("HostBuffer index is out of range");
    }

    std::unique_ptr<T, Unpin> pages_;
    std::size_t count_ = 0;
};

template <typename T> void swap(HostBuffer<T>& left, HostBuffer<T>& right) noexcept {
    left.swap(right);
}

} // namespace cuvit
