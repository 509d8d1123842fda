#pragma once

// HIP error handling for the host side: the counterpart of the reference's
// CudaError / CUVIT_CUDA_CHECK (include/cuvit/cuda_check.hpp:11-36). A failed
// HIP call becomes a HipError, a std::runtime_error that keeps the hipError_t
// and whose message names the expression, the location and the error.

#include <hip/hip_runtime_api.h>

#include <sstream>
#include <stdexcept>
#include <string>

namespace cuvit {

class HipError final : public std::runtime_error {
  public:
    HipError(hipError_t code, const std::string& message)
        : std::runtime_error(message), code_(code) {}

    [[nodiscard]] hipError_t code() const noexcept { return code_; }

  private:
    hipError_t code_;
};

inline void check_hip(hipError_t result, const char* expression, const char* file, int line) {
    if (result == hipSuccess) {
        return;
    }
    std::ostringstream message;
    message << "HIP call failed: " << expression << " at " << file << ':' << line << " ("
            << hipGetErrorName(result) << ": " << hipGetErrorString(result) << ')';
    throw HipError(result, message.str());
}

} // namespace cuvit

#define CUVIT_HIP_CHECK(expression) ::cuvit::check_hip((expression), #expression, __FILE__, __LINE__)
