// Internal interface between the C ABI (validation, status codes) and the
// kernel files (grid shaping, launch). Every function here assumes its
// arguments were already validated and returns the launch's hipError_t.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

namespace cuvit::detail {

// preprocess.hip. The crop geometry of image.cpp:113-121, worked out on the
// host, and the per-channel normalisation.
struct PreprocessGeometry {
    float origin_x;
    float origin_y;
    float step;
    float mean[3];
    float stddev[3];
};
hipError_t preprocess_u8(const std::uint8_t* pixels, int batch, int width, int height,
                         float* tensor, int size, const PreprocessGeometry& geometry,
                         hipStream_t stream);

// layer_norm.hip. With @p streaming the output is stored non-temporally
// (best when it is read back from HBM later); without, it stays in the
// caches for a kernel that reads it next. The values are the same. Input
// rows sit @p input_stride elements apart (0: packed, @p columns); output
// rows are packed.
hipError_t layer_norm_f32(const float* input, const float* gamma, const float* beta, float* output,
                          int rows, int columns, float epsilon, hipStream_t stream,
                          bool streaming = true, std::int64_t input_stride = 0);
hipError_t layer_norm_bf16(const std::uint16_t* input, const float* gamma, const float* beta,
                           std::uint16_t* output, int rows, int columns, float epsilon,
                           hipStream_t stream, bool streaming = true,
                           std::int64_t input_stride = 0);

// softmax.hip
hipError_t softmax_f32(const float* input, float* output, int rows, int columns,
                       hipStream_t stream);
hipError_t softmax_bf16(const std::uint16_t* input, std::uint16_t* output, int rows, int columns,
                        hipStream_t stream);

// patches.hip. The gather is a pure permutation, so it is typed only by the
// element size (4 for fp32, 2 for bf16).
hipError_t extract_patches(const void* images, void* patches, int element_size, int batch,
                           int channels, int height, int width, int patch, hipStream_t stream);
/// fp32 images into bf16 patch rows in one pass (bitwise the conversion then
/// the bf16 gather); hipErrorNotSupported unless both pointers are 16-byte
/// aligned and the patch and image widths are multiples of 8.
hipError_t extract_patches_f32_to_bf16(const float* images, std::uint16_t* patches, int batch,
                                      int channels, int height, int width, int patch,
                                      hipStream_t stream);
/// The same for any alignment and geometry: the strip kernel where it
/// applies, else one element per thread.
hipError_t extract_patches_f32_to_bf16_any(const float* images, std::uint16_t* patches, int batch,
                                          int channels, int height, int width, int patch,
                                          hipStream_t stream);
hipError_t broadcast_f32(float* destination, const float* source, std::int64_t count,
                         std::int64_t destination_stride, int batch, hipStream_t stream);
hipError_t broadcast_bf16(std::uint16_t* destination, const std::uint16_t* source,
                          std::int64_t count, std::int64_t destination_stride, int batch,
                          hipStream_t stream);
hipError_t add_broadcast_f32(float* accumulator, const float* addend, std::int64_t count, int batch,
                             hipStream_t stream);

// elementwise.hip
hipError_t add_f32(float* accumulator, const float* addend, std::int64_t count,
                   hipStream_t stream);
hipError_t gelu_f32(const float* input, float* output, std::int64_t count, hipStream_t stream);
hipError_t gelu_bf16(const std::uint16_t* input, std::uint16_t* output, std::int64_t count,
                     hipStream_t stream);
hipError_t convert_f32_to_bf16(const float* input, std::uint16_t* output, std::int64_t count,
                               hipStream_t stream);
hipError_t convert_bf16_to_f32(const std::uint16_t* input, float* output, std::int64_t count,
                               hipStream_t stream);

// gemm.hip. Leading dimensions are already resolved (never zero) and the
// batch is already flattened when it has a single outer group.
struct GemmArgs {
    int m;
    int n;
    int k;
    bool transposed;
    float alpha;
    int lda;
    int ldb;
    int ldc;
    int count;
    std::int64_t stride_a;
    std::int64_t stride_b;
    std::int64_t stride_c;
    int inner;
    std::int64_t outer_stride_a;
    std::int64_t outer_stride_b;
    std::int64_t outer_stride_c;
    bool accumulate;
    bool gelu;
    /// Optional [m, n] term added after the bias (row stride ld_addend), the
    /// same for every batch entry; no counterpart in the reference's
    /// GemmProblem, used by the model to fold the positional add into the
    /// patch-embedding GEMM.
    const float* addend = nullptr;
    int ld_addend = 0;
    /// When > 0, the m rows are consecutive batch entries of rows_per_entry
    /// rows each, run as one problem (A rows contiguous across the entries,
    /// count 1): output row p is row p % rows_per_entry of entry
    /// p / rows_per_entry, stored at entry * stride_c, and its addend row is
    /// p % rows_per_entry. Set by the dispatch only, for the tile that takes it.
    int rows_per_entry = 0;
};

hipError_t gemm_f32(const float* a, const float* b, const float* bias, float* c,
                    const GemmArgs& args, hipStream_t stream);
hipError_t gemm_bf16(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                     std::uint16_t* c, const GemmArgs& args, hipStream_t stream);

/// Fused softmax(Q.K^T / sqrt(head_dim)).V per (image, head) from the packed
/// [images, tokens, 3, heads, head_dim] projection into [images, tokens,
/// heads, head_dim]; bitwise equal to the GEMM -> softmax -> GEMM sequence.
bool attention_supported(int tokens, int head_dim);
hipError_t attention_f32(const float* qkv, float* context, int images, int heads, int tokens,
                         int head_dim, hipStream_t stream);
/// attention_f32's bf16 twin: bitwise equal to the bf16 GEMM -> softmax ->
/// GEMM sequence (logits and probabilities rounded to bf16 as stored there).
bool attention_bf16_supported(int tokens, int head_dim);
hipError_t attention_bf16(const std::uint16_t* qkv, std::uint16_t* context, int images, int heads,
                          int tokens, int head_dim, hipStream_t stream);

// Device facts used to shape grids, cached per device.
int compute_units();

/// Lets @p kernel use @p bytes of dynamic LDS (an opt-in above 64 KiB) on the
/// current device, once per device; @p devices is the kernel's own bit set of
/// the devices already done.
hipError_t allow_lds(const void* kernel, std::size_t bytes, std::atomic<std::uint64_t>& devices);

/// Grid size for a grid-stride kernel: enough blocks to cover @p units of work,
/// capped so the work-item count stays far inside the 32-bit dispatch limit.
unsigned int stride_grid(std::int64_t units, int units_per_block, int cap_per_cu);

} // namespace cuvit::detail
