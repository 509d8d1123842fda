// The C++ launchers of cuvit/kernels.hpp: each forwards to the C ABI and turns
// a failure back into the exception the reference's launcher throws
// (src/kernels/normalization.cu:224-350, src/kernels/gemm.cu:199-242).
#include "cuvit/kernels.hpp"

#include "cuvit/capi.h"
#include "cuvit/hip_check.hpp"

#include <cstddef>
#include <stdexcept>
#include <string>

namespace cuvit {
namespace {

// GemmProblem and cuvit_gemm_problem must be the same bytes, so a C++ problem
// can be handed to the C ABI as is.
static_assert(sizeof(GemmProblem) == sizeof(cuvit_gemm_problem), "GemmProblem layout drifted");
static_assert(offsetof(GemmProblem, layout) == offsetof(cuvit_gemm_problem, layout), "layout");
static_assert(offsetof(GemmProblem, alpha) == offsetof(cuvit_gemm_problem, alpha), "alpha");
static_assert(offsetof(GemmProblem, ldc) == offsetof(cuvit_gemm_problem, ldc), "ldc");
static_assert(offsetof(GemmProblem, batch) == offsetof(cuvit_gemm_problem, batch), "batch");
static_assert(offsetof(GemmBatch, inner) == offsetof(cuvit_gemm_batch, inner), "inner");
static_assert(offsetof(GemmBatch, outer_stride_c) == offsetof(cuvit_gemm_batch, outer_stride_c),
              "outer_stride_c");
static_assert(offsetof(GemmProblem, epilogue) == offsetof(cuvit_gemm_problem, epilogue),
              "epilogue");
static_assert(offsetof(GemmEpilogue, gelu) == offsetof(cuvit_gemm_epilogue, gelu), "gelu");
static_assert(sizeof(GemmLayout) == sizeof(std::int32_t), "GemmLayout is an int");
static_assert(static_cast<int>(GemmLayout::kTransposed) == CUVIT_GEMM_TRANSPOSED, "layout value");

cuvit_stream_t as_c(hipStream_t stream) { return reinterpret_cast<cuvit_stream_t>(stream); }

const cuvit_gemm_problem* as_c(const GemmProblem& problem) {
    return reinterpret_cast<const cuvit_gemm_problem*>(&problem);
}

} // namespace

void throw_on_error(int status) {
    switch (status) {
    case CUVIT_OK:
        return;
    case CUVIT_ERROR_INVALID_ARGUMENT:
        throw std::invalid_argument(cuvit_last_error());
    case CUVIT_ERROR_LENGTH:
        throw std::length_error(cuvit_last_error());
    case CUVIT_ERROR_OUT_OF_RANGE:
        throw std::out_of_range(cuvit_last_error());
    case CUVIT_ERROR_HIP:
        throw HipError(static_cast<hipError_t>(cuvit_last_hip_error()), cuvit_last_error());
    default:
        throw std::runtime_error(cuvit_last_error());
    }
}

void launch_gemm(const float* a, const float* b, const float* bias, float* c,
                 const GemmProblem& problem, hipStream_t stream) {
    throw_on_error(cuvit_gemm_f32(a, b, bias, c, as_c(problem), as_c(stream)));
}

void launch_layer_norm(const float* input, const float* gamma, const float* beta, float* output,
                       int rows, int columns, float epsilon, hipStream_t stream) {
    throw_on_error(
        cuvit_layer_norm_f32(input, gamma, beta, output, rows, columns, epsilon, as_c(stream)));
}

void launch_gelu(const float* input, float* output, std::int64_t count, hipStream_t stream) {
    throw_on_error(cuvit_gelu_f32(input, output, count, as_c(stream)));
}

void launch_softmax(const float* input, float* output, int rows, int columns, hipStream_t stream) {
    throw_on_error(cuvit_softmax_f32(input, output, rows, columns, as_c(stream)));
}

void launch_extract_patches(const float* images, float* patches, int batch, int channels,
                            int height, int width, int patch, hipStream_t stream) {
    throw_on_error(cuvit_extract_patches_f32(images, patches, batch, channels, height, width, patch,
                                             as_c(stream)));
}

void launch_add(float* accumulator, const float* addend, std::int64_t count, hipStream_t stream) {
    throw_on_error(cuvit_add_f32(accumulator, addend, count, as_c(stream)));
}

void launch_add_broadcast(float* accumulator, const float* addend, std::int64_t count, int batch,
                          hipStream_t stream) {
    throw_on_error(cuvit_add_broadcast_f32(accumulator, addend, count, batch, as_c(stream)));
}

void launch_broadcast(float* destination, const float* source, std::int64_t count,
                      std::int64_t destination_stride, int batch, hipStream_t stream) {
    throw_on_error(
        cuvit_broadcast_f32(destination, source, count, destination_stride, batch, as_c(stream)));
}

void launch_gemm(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                 std::uint16_t* c, const GemmProblem& problem, hipStream_t stream) {
    throw_on_error(cuvit_gemm_bf16(a, b, bias, c, as_c(problem), as_c(stream)));
}

void launch_layer_norm(const std::uint16_t* input, const float* gamma, const float* beta,
                       std::uint16_t* output, int rows, int columns, float epsilon,
                       hipStream_t stream) {
    throw_on_error(
        cuvit_layer_norm_bf16(input, gamma, beta, output, rows, columns, epsilon, as_c(stream)));
}

void launch_gelu(const std::uint16_t* input, std::uint16_t* output, std::int64_t count,
                 hipStream_t stream) {
    throw_on_error(cuvit_gelu_bf16(input, output, count, as_c(stream)));
}

void launch_softmax(const std::uint16_t* input, std::uint16_t* output, int rows, int columns,
                    hipStream_t stream) {
    throw_on_error(cuvit_softmax_bf16(input, output, rows, columns, as_c(stream)));
}

void launch_extract_patches(const std::uint16_t* images, std::uint16_t* patches, int batch,
                            int channels, int height, int width, int patch, hipStream_t stream) {
    throw_on_error(cuvit_extract_patches_bf16(images, patches, batch, channels, height, width,
                                              patch, as_c(stream)));
}

void launch_broadcast(std::uint16_t* destination, const std::uint16_t* source, std::int64_t count,
                      std::int64_t destination_stride, int batch, hipStream_t stream) {
    throw_on_error(
        cuvit_broadcast_bf16(destination, source, count, destination_stride, batch, as_c(stream)));
}

} // namespace cuvit
