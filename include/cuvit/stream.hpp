#pragma once

// Owning wrapper of a HIP stream, the counterpart of the reference's Stream
// (include/cuvit/stream.hpp:19-75). Default construction makes a non-blocking
// stream at the default priority; a moved-from Stream is empty and get()
// returns nullptr, the default stream.

#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime_api.h>

#include <utility>

namespace cuvit {

class Stream final {
  public:
    Stream() : Stream(hipStreamNonBlocking) {}

    explicit Stream(unsigned int flags) { CUVIT_HIP_CHECK(hipStreamCreateWithFlags(&stream_, flags)); }

    ~Stream() { release(); }

    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;

    Stream(Stream&& other) noexcept : stream_(std::exchange(other.stream_, nullptr)) {}

    Stream& operator=(Stream&& other) noexcept {
        if (this != &other) {
            release();
            stream_ = std::exchange(other.stream_, nullptr);
        }
        return *this;
    }

    /// Blocks until everything queued on the stream has finished.
    void synchronize() const { CUVIT_HIP_CHECK(hipStreamSynchronize(stream_)); }

    /// True when all queued work has finished; never blocks.
    [[nodiscard]] bool query() const {
        const hipError_t status = hipStreamQuery(stream_);
        if (status == hipErrorNotReady) {
            return false;
        }
        CUVIT_HIP_CHECK(status);
        return true;
    }

    void swap(Stream& other) noexcept { std::swap(stream_, other.stream_); }

    [[nodiscard]] hipStream_t get() const noexcept { return stream_; }
    [[nodiscard]] bool empty() const noexcept { return stream_ == nullptr; }

  private:
    void release() noexcept {
        if (stream_ != nullptr) {
            static_cast<void>(hipStreamDestroy(stream_));
            stream_ = nullptr;
        }
    }

    hipStream_t stream_ = nullptr;
};

inline void swap(Stream& left, Stream& right) noexcept { left.swap(right); }

} // namespace cuvit
