#pragma once

// The kernel launcher API: the reference's include/cuvit/kernels.hpp:9-154 with
// the same names, argument order, defaults and exceptions, taking a
// hipStream_t. Each launcher forwards to the C ABI in cuvit/capi.h and turns a
// failure status back into the exception the reference throws:
//   CUVIT_ERROR_INVALID_ARGUMENT -> std::invalid_argument
//   CUVIT_ERROR_LENGTH           -> std::length_error
//   CUVIT_ERROR_HIP              -> cuvit::HipError (a std::runtime_error)
// Launchers only enqueue work: they never synchronize and never allocate.

#include "cuvit/capi.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>

namespace cuvit {

/// How the right-hand operand is stored (kernels.hpp:16-21).
enum class GemmLayout {
    /// B is [K, N]: C[m][n] = sum_k A[m][k] * B[k][n].
    kNoTranspose,
    /// B is [N, K]: C[m][n] = sum_k A[m][k] * B[n][k], a Linear layer's weight.
    kTransposed,
};

/// What happens to each result before it is stored (kernels.hpp:30-36).
struct GemmEpilogue {
    /// C += value instead of C = value (a residual connection).
    bool accumulate = false;
    /// erf GELU after the bias.
    bool gelu = false;
};

/// Batch addressing (kernels.hpp:46-59). With @p inner positive, entry i is
/// (i / inner, i % inner) and the first part advances by the outer strides.
struct GemmBatch {
    int count = 1;
    std::int64_t stride_a = 0;
    std::int64_t stride_b = 0;
    std::int64_t stride_c = 0;
    int inner = 0;
    std::int64_t outer_stride_a = 0;
    std::int64_t outer_stride_b = 0;
    std::int64_t outer_stride_c = 0;
};

/// C[i][m][n] = epilogue(alpha * sum_k A[i][m][k] * B_layout[i][k][n] + bias[n])
/// (kernels.hpp:74-85). A zero leading dimension selects the packed one.
struct GemmProblem {
    int m = 0;
    int n = 0;
    int k = 0;
    GemmLayout layout = GemmLayout::kNoTranspose;
    float alpha = 1.0F;
    int lda = 0;
    int ldb = 0;
    int ldc = 0;
    GemmBatch batch;
    GemmEpilogue epilogue;
};

/// One un-batched problem with packed operands and no epilogue (kernels.hpp:89-96).
[[nodiscard]] inline GemmProblem gemm_problem(int m, int n, int k, GemmLayout layout) {
    GemmProblem problem;
    problem.m = m;
    problem.n = n;
    problem.k = k;
    problem.layout = layout;
    return problem;
}

void launch_gemm(const float* a, const float* b, const float* bias, float* c,
                 const GemmProblem& problem, hipStream_t stream = nullptr);

/// out[r][c] = (in[r][c] - mean) / sqrt(var + eps) * gamma[c] + beta[c], biased var.
void launch_layer_norm(const float* input, const float* gamma, const float* beta, float* output,
                       int rows, int columns, float epsilon = 1.0e-6F,
                       hipStream_t stream = nullptr);

/// Exact GELU, x * 0.5 * (1 + erf(x / sqrt(2))), not the tanh form.
void launch_gelu(const float* input, float* output, std::int64_t count,
                 hipStream_t stream = nullptr);

/// Row softmax in the max-subtracted form; input may equal output.
void launch_softmax(const float* input, float* output, int rows, int columns,
                    hipStream_t stream = nullptr);

/// [B, C, H, W] images -> [B * (H/P) * (W/P), C * P * P] patch rows, channel-major.
void launch_extract_patches(const float* images, float* patches, int batch, int channels,
                            int height, int width, int patch, hipStream_t stream = nullptr);

/// accumulator[i] += addend[i].
void launch_add(float* accumulator, const float* addend, std::int64_t count,
                hipStream_t stream = nullptr);

/// accumulator[s * count + i] += addend[i] for each of @p batch blocks.
void launch_add_broadcast(float* accumulator, const float* addend, std::int64_t count, int batch,
                          hipStream_t stream = nullptr);

/// destination[s * destination_stride + i] = source[i] for each of @p batch slots.
void launch_broadcast(float* destination, const float* source, std::int64_t count,
                      std::int64_t destination_stride, int batch, hipStream_t stream = nullptr);

// bfloat16-storage overloads (an extension; the reference is fp32 only). The
// data type is hip_bfloat16's bit pattern carried as std::uint16_t; statistics,
// accumulation, gamma, beta and bias are fp32.
void launch_gemm(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                 std::uint16_t* c, const GemmProblem& problem, hipStream_t stream = nullptr);
void launch_layer_norm(const std::uint16_t* input, const float* gamma, const float* beta,
                       std::uint16_t* output, int rows, int columns, float epsilon = 1.0e-6F,
                       hipStream_t stream = nullptr);
void launch_gelu(const std::uint16_t* input, std::uint16_t* output, std::int64_t count,
                 hipStream_t stream = nullptr);
void launch_softmax(const std::uint16_t* input, std::uint16_t* output, int rows, int columns,
                    hipStream_t stream = nullptr);
void launch_extract_patches(const std::uint16_t* images, std::uint16_t* patches, int batch,
                            int channels, int height, int width, int patch,
                            hipStream_t stream = nullptr);
void launch_broadcast(std::uint16_t* destination, const std::uint16_t* source, std::int64_t count,
                      std::int64_t destination_stride, int batch, hipStream_t stream = nullptr);

/// Throws the exception matching a C-ABI status (no-op on CUVIT_OK).
void throw_on_error(int status);

} // namespace cuvit
