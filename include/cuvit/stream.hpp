#pragma once

// An owned HIP stream. Interface of the reference's Stream
// (include/cuvit/stream.hpp:19-75): created non-blocking unless flags are
// given, destroyed with its owner, movable but not copyable; an empty Stream
// (default-moved-from) hands out nullptr, the null stream.
//
// Ownership sits in a unique_ptr whose deleter destroys the stream, so moves,
// swaps and destruction need no code of their own. Streams keep the default
// priority.

#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime_api.h>

#include <memory>
#include <type_traits>

namespace cuvit {

class Stream final {
  public:
    Stream() : Stream(hipStreamNonBlocking) {}

    explicit Stream(unsigned int flags) : handle_(create(flags)) {}

    /// Waits for all work queued on the stream.
    void synchronize() const { CUVIT_HIP_CHECK(hipStreamSynchronize(get())); }

    /// Whether all queued work has finished, without waiting.
    [[nodiscard]] bool query() const {
        const hipError_t state = hipStreamQuery(get());
        if (state != hipErrorNotReady) {
            CUVIT_HIP_CHECK(state);
        }
        return state == hipSuccess;
    }

    void swap(Stream& other) noexcept { handle_.swap(other.handle_); }

    [[nodiscard]] hipStream_t get() const noexcept { return handle_.get(); }
    [[nodiscard]] bool empty() const noexcept { return !handle_; }

  private:
    struct Destroy {
        void operator()(hipStream_t stream) const noexcept {
            static_cast<void>(hipStreamDestroy(stream));
        }
    };
    using Handle = std::unique_ptr<std::remove_pointer_t<hipStream_t>, Destroy>;

    static Handle create(unsigned int flags) {
        hipStream_t stream = nullptr;
        CUVIT_HIP_CHECK(hipStreamCreateWithFlags(&stream, flags));
        return Handle(stream);
    }

    Handle handle_;
};

inline void swap(Stream& left, Stream& right) noexcept { left.swap(right); }

} // namespace cuvit
