// Status plumbing for the C ABI: the thread-local last error, and the mapping
// from C++ exceptions (thrown by the host-side classes) to status codes.
#pragma once

#include "cuvit/capi.h"
#include "cuvit/hip_check.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>
#include <new>
#include <stdexcept>
#include <string>

namespace cuvit::capi {

/// Records @p message as this thread's last error and returns @p status.
int fail(cuvit_status status, const std::string& message);

/// Records success and returns CUVIT_OK.
int ok();

/// Turns a launch result into a status, naming the failed call.
int from_hip(hipError_t result, const char* what);

/// Stores the hipError_t reported by cuvit_last_hip_error().
void set_hip_error(int code);

/// cuvit_gemm_f32 plus an [m, n] addend (row stride ld_addend, the same for
/// every batch entry) added after the bias. Not part of the C ABI, whose
/// problem struct is the reference's GemmProblem: the model uses it to fold
/// the positional add into the patch-embedding GEMM.
int gemm_f32_with_addend(const float* a, const float* b, const float* bias, const float* addend,
                         int ld_addend, float* c, const cuvit_gemm_problem* problem,
                         hipStream_t stream);

/// gemm_f32_with_addend's bf16 twin: bf16 A, B and C, fp32 bias and addend,
/// one rounding at the store.
int gemm_bf16_with_addend(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                          const float* addend, int ld_addend, std::uint16_t* c,
                          const cuvit_gemm_problem* problem, hipStream_t stream);

/// cuvit_layer_norm_f32 / _bf16 with plain (cached) output stores, for a
/// caller whose next launch reads the output: the model's blocks, where the
/// normalised rows feed a GEMM at once. Same validation and values as the C
/// ABI's entry points, which store non-temporally.
/// Input rows sit @p input_stride elements apart (0: packed); output rows are
/// packed.
int layer_norm_cached(const float* input, const float* gamma, const float* beta, float* output,
                      int rows, int columns, float epsilon, hipStream_t stream,
                      std::int64_t input_stride = 0);
int layer_norm_cached(const std::uint16_t* input, const float* gamma, const float* beta,
                      std::uint16_t* output, int rows, int columns, float epsilon,
                      hipStream_t stream, std::int64_t input_stride = 0);

/// fp32 images into the bf16 model's patch rows in one pass (bitwise the
/// conversion to bf16 followed by the bf16 gather) when the layout allows it:
/// 16-byte aligned pointers, patch size and image width multiples of 8.
/// @p fused tells whether it ran; when it did not, nothing was launched and
/// the caller converts and gathers.
int extract_patches_f32_to_bf16(const float* images, std::uint16_t* patches, int batch,
                                int channels, int height, int width, int patch,
                                hipStream_t stream, bool* fused);

/// The checks of preprocess (image.cpp:96-104, 126-128), in its order: an
/// empty image, a non-positive size, a crop fraction outside (0, 1], a zero
/// standard deviation.
int check_preprocess_settings(int width, int height, const cuvit_preprocessing& settings);

/// Runs @p body, mapping any exception it throws to the matching status.
template <typename Body> int guarded(Body&& body) {
    try {
        return body();
    } catch (const HipError& error) {
        const int status = fail(CUVIT_ERROR_HIP, error.what());
        set_hip_error(static_cast<int>(error.code()));
        return status;
    } catch (const std::invalid_argument& error) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, error.what());
    } catch (const std::length_error& error) {
        return fail(CUVIT_ERROR_LENGTH, error.what());
    } catch (const std::out_of_range& error) {
        return fail(CUVIT_ERROR_OUT_OF_RANGE, error.what());
    } catch (const std::bad_alloc&) {
        return fail(CUVIT_ERROR_RUNTIME, "host allocation failed");
    } catch (const std::exception& error) {
        return fail(CUVIT_ERROR_RUNTIME, error.what());
    } catch (...) {
        return fail(CUVIT_ERROR_RUNTIME, "unknown exception");
    }
}

} // namespace cuvit::capi
