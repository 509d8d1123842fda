#pragma once

// Host-side HIP error reporting. Interface of the reference's CudaError and
// CUVIT_CUDA_CHECK (include/cuvit/cuda_check.hpp:11-36): a failed runtime call
// becomes an exception derived from std::runtime_error that keeps the error
// code and whose text names the error, the call and where it was made.

#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace cuvit {

/// The source position of one checked HIP call.
struct HipCallSite {
    const char* expression;
    const char* file;
    int line;
};

class HipError final : public std::runtime_error {
  public:
    /// An error whose text the caller composed (the C ABI's last-error text).
    HipError(hipError_t code, const std::string& what) : std::runtime_error(what), code_(code) {}

    /// An error from a checked call: "<name> (<description>) from <call> at
    /// <file>:<line>".
    HipError(hipError_t code, const HipCallSite& site)
        : std::runtime_error(compose(code, site)), code_(code) {}

    [[nodiscard]] hipError_t code() const noexcept { return code_; }

  private:
    static std::string compose(hipError_t code, const HipCallSite& site) {
        std::string text = hipGetErrorName(code);
        text.append(" (").append(hipGetErrorString(code)).append(") from ");
        text.append(site.expression).append(" at ").append(site.file);
        text.push_back(':');
        text.append(std::to_string(site.line));
        return text;
    }

    hipError_t code_;
};

/// Throws HipError unless @p result is hipSuccess.
inline void check_hip(hipError_t result, const char* expression, const char* file, int line) {
    if (result != hipSuccess) {
        throw HipError(result, HipCallSite{expression, file, line});
    }
}

} // namespace cuvit

#define CUVIT_HIP_CHECK(call) ::cuvit::check_hip((call), #call, __FILE__, __LINE__)
