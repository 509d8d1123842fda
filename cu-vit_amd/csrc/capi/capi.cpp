// The C ABI's kernel entry points: validation in the reference's order and
// wording (src/kernels/normalization.cu:214-350, src/kernels/gemm.cu:199-231),
// then the launch, then the launch status. Nothing here throws.
#include "cuvit/capi.h"
#include "status.hpp"

#include "../kernels/launch.hpp"

#include <cmath>
#include <cstdint>
#include <string>

namespace cuvit::capi {
namespace {

thread_local std::string last_message;
thread_local int last_hip = 0;

/// The reference's elementwise_blocks limit (normalization.cu:214-220): a
/// launch of ceil(total / 256) blocks above 2^31 - 1 is a length error. The
/// kernels here loop over any size, but the contract is kept.
constexpr std::int64_t kElementwiseThreads = 256;
constexpr std::int64_t kMaxBlocks = 0x7FFFFFFF;

bool exceeds_grid(std::int64_t total) {
    return (total + kElementwiseThreads - 1) / kElementwiseThreads > kMaxBlocks;
}

int grid_error() {
    return fail(CUVIT_ERROR_LENGTH, "Elementwise launch exceeds the grid limit");
}

/// a * b for non-negative values, saturating at INT64_MAX.
std::int64_t saturating_product(std::int64_t a, std::int64_t b) {
    if (a != 0 && b > INT64_MAX / a) {
        return INT64_MAX;
    }
    return a * b;
}

hipStream_t as_hip(cuvit_stream_t stream) { return reinterpret_cast<hipStream_t>(stream); }

int check_layer_norm(const void* input, const void* gamma, const void* beta, const void* output,
                     int rows, int columns, bool* empty) {
    *empty = rows == 0 || columns == 0;
    if (*empty) {
        return ok();
    }
    if (rows < 0 || columns < 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Layer norm dimensions cannot be negative");
    }
    if (input == nullptr || gamma == nullptr || beta == nullptr || output == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Layer norm operands cannot be null");
    }
    return ok();
}

int check_softmax(const void* input, const void* output, int rows, int columns, bool* empty) {
    *empty = rows == 0 || columns == 0;
    if (*empty) {
        return ok();
    }
    if (rows < 0 || columns < 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Softmax dimensions cannot be negative");
    }
    if (input == nullptr || output == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Softmax operands cannot be null");
    }
    return ok();
}

int check_gelu(const void* input, const void* output, std::int64_t count, bool* empty) {
    *empty = count == 0;
    if (*empty) {
        return ok();
    }
    if (count < 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GELU element count cannot be negative");
    }
    if (input == nullptr || output == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GELU operands cannot be null");
    }
    if (exceeds_grid(count)) {
        return grid_error();
    }
    return ok();
}

/// Validation shared by the fp32 and bf16 fused attention (@p element_size
/// bytes an element); @p empty is set for a launch with nothing to do.
int check_attention(const void* qkv, const void* context, int images, int heads, int tokens,
                    int head_dim, int element_size, bool* empty) {
    *empty = images == 0 || heads == 0 || tokens == 0 || head_dim == 0;
    if (*empty) {
        return ok();
    }
    if (images < 0 || heads < 0 || tokens < 0 || head_dim < 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Attention extents cannot be negative");
    }
    if (qkv == nullptr || context == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Attention operands cannot be null");
    }
    if (!detail::attention_supported(tokens, head_dim)) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT,
                          "Fused attention supports head_dim 64 and at most 256 tokens");
    }
    if (((reinterpret_cast<std::uintptr_t>(qkv) | reinterpret_cast<std::uintptr_t>(context)) & 15U) != 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Fused attention needs 16-byte aligned operands");
    }
    if (saturating_product(images, heads) > 65535) {
        return fail(CUVIT_ERROR_LENGTH, "Fused attention takes at most 65535 (image, head) pairs");
    }
    // The kernels address an image's rows of the packed projection with
    // 32-bit byte offsets from the image's first row, inside a buffer range of
    // 0x7FFFFFF0 bytes.
    if (static_cast<std::int64_t>(tokens) * 3 * heads * head_dim * element_size > 0x7FFFFFF0) {
        return fail(CUVIT_ERROR_LENGTH, "Fused attention takes at most 2^31 - 16 bytes of an image's QKV rows");
    }
    return ok();
}

int check_broadcast(const void* destination, const void* source, std::int64_t count,
                    std::int64_t destination_stride, int batch, bool* empty) {
    *empty = count == 0 || batch == 0;
    if (*empty) {
        return ok();
    }
    if (count < 0 || batch < 0 || destination_stride < count) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Broadcast extents are inconsistent");
    }
    if (destination == nullptr || source == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Broadcast operands cannot be null");
    }
    if (exceeds_grid(saturating_product(count, batch))) {
        return grid_error();
    }
    return ok();
}

int check_patches(const void* images, const void* patches, int batch, int channels, int height,
                  int width, int patch, bool* empty) {
    *empty = batch == 0;
    if (*empty) {
        return ok();
    }
    if (batch < 0 || channels <= 0 || height <= 0 || width <= 0 || patch <= 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Patch extraction dimensions must be positive");
    }
    if (height % patch != 0 || width % patch != 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT,
                    "Patch extraction needs the image to divide into whole patches");
    }
    if (images == nullptr || patches == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Patch extraction operands cannot be null");
    }
    const std::int64_t total = saturating_product(
        saturating_product(saturating_product(batch, channels), height), width);
    if (exceeds_grid(total)) {
        return grid_error();
    }
    return ok();
}

struct ResolvedGemm {
    detail::GemmArgs args;
    bool empty;
};

int check_gemm(const void* a, const void* b, const void* c, const cuvit_gemm_problem* problem,
               ResolvedGemm* out) {
    if (problem == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GEMM problem cannot be null");
    }
    const cuvit_gemm_problem& p = *problem;
    out->empty = p.m == 0 || p.n == 0 || p.batch.count == 0;
    if (out->empty) {
        return ok();
    }
    if (p.m < 0 || p.n < 0 || p.k < 0 || p.batch.count < 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GEMM dimensions cannot be negative");
    }
    if (p.batch.inner > 0 && p.batch.count % p.batch.inner != 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT,
                    "A split GEMM batch must divide into whole inner groups");
    }
    if (a == nullptr || b == nullptr || c == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GEMM operands cannot be null");
    }
    if (p.layout != CUVIT_GEMM_NO_TRANSPOSE && p.layout != CUVIT_GEMM_TRANSPOSED) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GEMM layout is not a GemmLayout value");
    }
    const bool transposed = p.layout == CUVIT_GEMM_TRANSPOSED;
    const int lda = p.lda != 0 ? p.lda : p.k;
    const int ldb = p.ldb != 0 ? p.ldb : (transposed ? p.k : p.n);
    const int ldc = p.ldc != 0 ? p.ldc : p.n;
    if (lda < p.k || ldc < p.n || ldb < (transposed ? p.k : p.n)) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "A GEMM leading dimension is smaller than its row");
    }

    detail::GemmArgs& args = out->args;
    args.m = p.m;
    args.n = p.n;
    args.k = p.k;
    args.transposed = transposed;
    args.alpha = p.alpha;
    args.lda = lda;
    args.ldb = ldb;
    args.ldc = ldc;
    args.count = p.batch.count;
    args.stride_a = p.batch.stride_a;
    args.stride_b = p.batch.stride_b;
    args.stride_c = p.batch.stride_c;
    // One outer group reaches nothing a flat index would not (gemm.cu:218-223).
    args.inner = p.batch.inner > 0 && p.batch.inner < p.batch.count ? p.batch.inner : 0;
    args.outer_stride_a = p.batch.outer_stride_a;
    args.outer_stride_b = p.batch.outer_stride_b;
    args.outer_stride_c = p.batch.outer_stride_c;
    args.accumulate = p.epilogue.accumulate != 0;
    args.gelu = p.epilogue.gelu != 0;
    return ok();
}

/// Largest output side: size * size stays within a 32-bit pixel index.
constexpr int kMaxPreprocessSize = 32768;

/// check_preprocess_settings with the batch, the settings pointer and the
/// operands around it.
int check_preprocess(const void* pixels, int batch, int width, int height,
                     const cuvit_preprocessing* settings, const void* tensor, bool* empty) {
    *empty = batch == 0;
    if (*empty) {
        return ok();
    }
    if (batch < 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "The preprocessing batch cannot be negative");
    }
    if (settings == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Preprocessing settings cannot be null");
    }
    if (const int s = check_preprocess_settings(width, height, *settings); s != CUVIT_OK) {
        return s;
    }
    if (pixels == nullptr || tensor == nullptr) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Preprocessing operands cannot be null");
    }
    if (settings->size > kMaxPreprocessSize) {
        return fail(CUVIT_ERROR_LENGTH, "The preprocessing size exceeds the grid limit");
    }
    if (saturating_product(saturating_product(saturating_product(batch, width), height), 3) ==
        INT64_MAX) {
        return fail(CUVIT_ERROR_LENGTH, "The preprocessing images exceed the addressable size");
    }
    return ok();
}

/// Resize-and-crop geometry (image.cpp:113-121), each step rounded to float
/// on its own: the shorter side goes to round(size / crop_fraction), the crop
/// of size * scale source pixels is centred, and output pixels are step apart.
detail::PreprocessGeometry preprocess_geometry(int width, int height,
                                               const cuvit_preprocessing& settings) {
#pragma clang fp contract(off)
    const float size = static_cast<float>(settings.size);
    const float resized = std::round(size / settings.crop_fraction);
    const int shorter = width < height ? width : height;
    const float scale = static_cast<float>(shorter) / resized;
    const float crop = size * scale;
    detail::PreprocessGeometry geometry{};
    geometry.origin_x = (static_cast<float>(width) - crop) * 0.5F;
    geometry.origin_y = (static_cast<float>(height) - crop) * 0.5F;
    geometry.step = crop / size;
    for (int channel = 0; channel < 3; ++channel) {
        geometry.mean[channel] = settings.mean[channel];
        geometry.stddev[channel] = settings.stddev[channel];
    }
    return geometry;
}

} // namespace

int fail(cuvit_status status, const std::string& message) {
    last_message = message;
    if (status != CUVIT_ERROR_HIP) {
        last_hip = 0;
    }
    return status;
}

int ok() { return CUVIT_OK; }

void set_hip_error(int code) { last_hip = code; }

int from_hip(hipError_t result, const char* what) {
    if (result == hipSuccess) {
        return CUVIT_OK;
    }
    const int status = fail(CUVIT_ERROR_HIP, std::string("HIP call failed: ") + what + " (" +
                                                 hipGetErrorName(result) + ": " +
                                                 hipGetErrorString(result) + ')');
    last_hip = static_cast<int>(result);
    return status;
}

int check_preprocess_settings(int width, int height, const cuvit_preprocessing& settings) {
    if (width <= 0 || height <= 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "Cannot preprocess an empty image");
    }
    if (settings.size <= 0) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "The preprocessing size must be positive");
    }
    if (!(settings.crop_fraction > 0.0F) || settings.crop_fraction > 1.0F) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "The crop fraction must lie in (0, 1]");
    }
    for (const float deviation : settings.stddev) {
        if (deviation == 0.0F) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT,
                        "A preprocessing standard deviation cannot be zero");
        }
    }
    return ok();
}

int gemm_f32_with_addend(const float* a, const float* b, const float* bias, const float* addend,
                         int ld_addend, float* c, const cuvit_gemm_problem* problem,
                         hipStream_t stream) {
    ResolvedGemm resolved{};
    if (const int s = check_gemm(a, b, c, problem, &resolved); s != CUVIT_OK || resolved.empty) {
        return s;
    }
    if (addend == nullptr || ld_addend < problem->n) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GEMM addend needs a row of at least n values");
    }
    resolved.args.addend = addend;
    resolved.args.ld_addend = ld_addend;
    return from_hip(detail::gemm_f32(a, b, bias, c, resolved.args, stream), "gemm launch");
}

int gemm_bf16_with_addend(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                          const float* addend, int ld_addend, std::uint16_t* c,
                          const cuvit_gemm_problem* problem, hipStream_t stream) {
    ResolvedGemm resolved{};
    if (const int s = check_gemm(a, b, c, problem, &resolved); s != CUVIT_OK || resolved.empty) {
        return s;
    }
    if (addend == nullptr || ld_addend < problem->n) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "GEMM addend needs a row of at least n values");
    }
    resolved.args.addend = addend;
    resolved.args.ld_addend = ld_addend;
    return from_hip(detail::gemm_bf16(a, b, bias, c, resolved.args, stream), "gemm launch");
}

int extract_patches_f32_to_bf16(const float* images, std::uint16_t* patches, int batch,
                                int channels, int height, int width, int patch,
                                hipStream_t stream, bool* fused) {
    const hipError_t result = detail::extract_patches_f32_to_bf16(images, patches, batch, channels,
                                                                  height, width, patch, stream);
    *fused = result != hipErrorNotSupported;
    if (!*fused) {
        return ok();
    }
    return from_hip(result, "extract_patches launch");
}

int layer_norm_cached(const float* input, const float* gamma, const float* beta, float* output,
                      int rows, int columns, float epsilon, hipStream_t stream,
                      std::int64_t input_stride) {
    bool empty = false;
    if (const int s = check_layer_norm(input, gamma, beta, output, rows, columns, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    if (input_stride != 0 && input_stride < columns) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "layer_norm rows overlap");
    }
    return from_hip(detail::layer_norm_f32(input, gamma, beta, output, rows, columns, epsilon,
                                           stream, false, input_stride),
                    "layer_norm launch");
}

int layer_norm_cached(const std::uint16_t* input, const float* gamma, const float* beta,
                      std::uint16_t* output, int rows, int columns, float epsilon,
                      hipStream_t stream, std::int64_t input_stride) {
    bool empty = false;
    if (const int s = check_layer_norm(input, gamma, beta, output, rows, columns, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    if (input_stride != 0 && input_stride < columns) {
        return fail(CUVIT_ERROR_INVALID_ARGUMENT, "layer_norm rows overlap");
    }
    return from_hip(detail::layer_norm_bf16(input, gamma, beta, output, rows, columns, epsilon,
                                            stream, false, input_stride),
                    "layer_norm launch");
}

} // namespace cuvit::capi

using namespace cuvit;
using capi::from_hip;

extern "C" {

const char* cuvit_last_error(void) { return capi::last_message.c_str(); }

int cuvit_last_hip_error(void) { return capi::last_hip; }

int cuvit_version(void) { return 100; }

void cuvit_gemm_problem_init(cuvit_gemm_problem* problem, int m, int n, int k, int layout) {
    if (problem == nullptr) {
        return;
    }
    *problem = cuvit_gemm_problem{};
    problem->m = m;
    problem->n = n;
    problem->k = k;
    problem->layout = layout;
    problem->alpha = 1.0F;
    problem->batch.count = 1;
}

int cuvit_layer_norm_f32(const float* input, const float* gamma, const float* beta, float* output,
                         int rows, int columns, float epsilon, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_layer_norm(input, gamma, beta, output, rows, columns, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::layer_norm_f32(input, gamma, beta, output, rows, columns, epsilon,
                                           capi::as_hip(stream)),
                    "layer_norm launch");
}

int cuvit_layer_norm_bf16(const cuvit_bf16* input, const float* gamma, const float* beta,
                          cuvit_bf16* output, int rows, int columns, float epsilon,
                          cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_layer_norm(input, gamma, beta, output, rows, columns, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::layer_norm_bf16(input, gamma, beta, output, rows, columns, epsilon,
                                            capi::as_hip(stream)),
                    "layer_norm launch");
}

int cuvit_softmax_f32(const float* input, float* output, int rows, int columns,
                      cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_softmax(input, output, rows, columns, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::softmax_f32(input, output, rows, columns, capi::as_hip(stream)),
                    "softmax launch");
}

int cuvit_softmax_bf16(const cuvit_bf16* input, cuvit_bf16* output, int rows, int columns,
                       cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_softmax(input, output, rows, columns, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::softmax_bf16(input, output, rows, columns, capi::as_hip(stream)),
                    "softmax launch");
}

int cuvit_gelu_f32(const float* input, float* output, int64_t count, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_gelu(input, output, count, &empty); s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::gelu_f32(input, output, count, capi::as_hip(stream)), "gelu launch");
}

int cuvit_gelu_bf16(const cuvit_bf16* input, cuvit_bf16* output, int64_t count,
                    cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_gelu(input, output, count, &empty); s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::gelu_bf16(input, output, count, capi::as_hip(stream)), "gelu launch");
}

int cuvit_extract_patches_f32(const float* images, float* patches, int batch, int channels,
                              int height, int width, int patch, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_patches(images, patches, batch, channels, height, width, patch,
                                          &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::extract_patches(images, patches, 4, batch, channels, height, width,
                                            patch, capi::as_hip(stream)),
                    "extract_patches launch");
}

int cuvit_extract_patches_bf16(const cuvit_bf16* images, cuvit_bf16* patches, int batch,
                               int channels, int height, int width, int patch,
                               cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_patches(images, patches, batch, channels, height, width, patch,
                                          &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::extract_patches(images, patches, 2, batch, channels, height, width,
                                            patch, capi::as_hip(stream)),
                    "extract_patches launch");
}

int cuvit_extract_patches_f32_to_bf16(const float* images, cuvit_bf16* patches, int batch,
                                      int channels, int height, int width, int patch,
                                      cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_patches(images, patches, batch, channels, height, width, patch,
                                          &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::extract_patches_f32_to_bf16_any(images, patches, batch, channels,
                                                            height, width, patch,
                                                            capi::as_hip(stream)),
                    "extract_patches launch");
}

void cuvit_preprocessing_default(cuvit_preprocessing* settings) {
    if (settings == nullptr) {
        return;
    }
    settings->size = 224;
    settings->crop_fraction = 0.9F;
    for (int channel = 0; channel < 3; ++channel) {
        settings->mean[channel] = 0.5F;
        settings->stddev[channel] = 0.5F;
    }
}

int cuvit_preprocess_u8(const uint8_t* pixels, int batch, int width, int height,
                        const cuvit_preprocessing* settings, float* tensor,
                        cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_preprocess(pixels, batch, width, height, settings, tensor, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    const detail::PreprocessGeometry geometry = capi::preprocess_geometry(width, height, *settings);
    return from_hip(detail::preprocess_u8(pixels, batch, width, height, tensor, settings->size,
                                          geometry, capi::as_hip(stream)),
                    "preprocess launch");
}

int cuvit_add_f32(float* accumulator, const float* addend, int64_t count, cuvit_stream_t stream) {
    if (count == 0) {
        return capi::ok();
    }
    if (count < 0) {
        return capi::fail(CUVIT_ERROR_INVALID_ARGUMENT,
                          "Residual add element count cannot be negative");
    }
    if (accumulator == nullptr || addend == nullptr) {
        return capi::fail(CUVIT_ERROR_INVALID_ARGUMENT, "Residual add operands cannot be null");
    }
    if (capi::exceeds_grid(count)) {
        return capi::grid_error();
    }
    return from_hip(detail::add_f32(accumulator, addend, count, capi::as_hip(stream)), "add launch");
}

int cuvit_add_broadcast_f32(float* accumulator, const float* addend, int64_t count, int batch,
                            cuvit_stream_t stream) {
    if (count == 0 || batch == 0) {
        return capi::ok();
    }
    if (count < 0 || batch < 0) {
        return capi::fail(CUVIT_ERROR_INVALID_ARGUMENT, "Broadcast add extents cannot be negative");
    }
    if (accumulator == nullptr || addend == nullptr) {
        return capi::fail(CUVIT_ERROR_INVALID_ARGUMENT, "Broadcast add operands cannot be null");
    }
    if (capi::exceeds_grid(capi::saturating_product(count, batch))) {
        return capi::grid_error();
    }
    return from_hip(detail::add_broadcast_f32(accumulator, addend, count, batch, capi::as_hip(stream)),
                    "add_broadcast launch");
}

int cuvit_attention_supported(int tokens, int head_dim) {
    return detail::attention_supported(tokens, head_dim) ? 1 : 0;
}

int cuvit_attention_f32(const float* qkv, float* context, int images, int heads, int tokens,
                        int head_dim, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_attention(qkv, context, images, heads, tokens, head_dim, 4, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::attention_f32(qkv, context, images, heads, tokens, head_dim,
                                          capi::as_hip(stream)),
                    "attention launch");
}

int cuvit_attention_bf16(const cuvit_bf16* qkv, cuvit_bf16* context, int images, int heads,
                         int tokens, int head_dim, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_attention(qkv, context, images, heads, tokens, head_dim, 2, &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::attention_bf16(qkv, context, images, heads, tokens, head_dim,
                                           capi::as_hip(stream)),
                    "attention launch");
}

int cuvit_broadcast_f32(float* destination, const float* source, int64_t count,
                        int64_t destination_stride, int batch, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_broadcast(destination, source, count, destination_stride, batch,
                                            &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::broadcast_f32(destination, source, count, destination_stride, batch,
                                          capi::as_hip(stream)),
                    "broadcast launch");
}

int cuvit_broadcast_bf16(cuvit_bf16* destination, const cuvit_bf16* source, int64_t count,
                         int64_t destination_stride, int batch, cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_broadcast(destination, source, count, destination_stride, batch,
                                            &empty);
        s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::broadcast_bf16(destination, source, count, destination_stride, batch,
                                           capi::as_hip(stream)),
                    "broadcast launch");
}

int cuvit_convert_f32_to_bf16(const float* input, cuvit_bf16* output, int64_t count,
                              cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_gelu(input, output, count, &empty); s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::convert_f32_to_bf16(input, output, count, capi::as_hip(stream)),
                    "convert launch");
}

int cuvit_convert_bf16_to_f32(const cuvit_bf16* input, float* output, int64_t count,
                              cuvit_stream_t stream) {
    bool empty = false;
    if (const int s = capi::check_gelu(input, output, count, &empty); s != CUVIT_OK || empty) {
        return s;
    }
    return from_hip(detail::convert_bf16_to_f32(input, output, count, capi::as_hip(stream)),
                    "convert launch");
}

int cuvit_gemm_f32(const float* a, const float* b, const float* bias, float* c,
                   const cuvit_gemm_problem* problem, cuvit_stream_t stream) {
    capi::ResolvedGemm resolved{};
    if (const int s = capi::check_gemm(a, b, c, problem, &resolved); s != CUVIT_OK || resolved.empty) {
        return s;
    }
    return from_hip(detail::gemm_f32(a, b, bias, c, resolved.args, capi::as_hip(stream)),
                    "gemm launch");
}

int cuvit_gemm_bf16(const cuvit_bf16* a, const cuvit_bf16* b, const float* bias, cuvit_bf16* c,
                    const cuvit_gemm_problem* problem, cuvit_stream_t stream) {
    capi::ResolvedGemm resolved{};
    if (const int s = capi::check_gemm(a, b, c, problem, &resolved); s != CUVIT_OK || resolved.empty) {
        return s;
    }
    return from_hip(detail::gemm_bf16(a, b, bias, c, resolved.args, capi::as_hip(stream)),
                    "gemm launch");
}

} // extern "C"
