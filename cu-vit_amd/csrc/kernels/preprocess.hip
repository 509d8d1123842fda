// Image preprocessing for gfx950: interleaved 8-bit RGB images to the planar
// float tensor the model reads (reference: include/cuvit/image.hpp:30-52,
// src/runtime/image.cpp:37-55 and 95-135, there a host loop per image).
//
// Per output pixel (row, column) of an S x S tensor, with the crop geometry
// (origin_x, origin_y, step) worked out once on the host:
//   x = origin_x + (column + 0.5) * step - 0.5,  y likewise with row
//   left = floor(x), top = floor(y), dx = x - left, dy = y - top
//   p(c, r) = pixel at clamp(c, 0, W-1), clamp(r, 0, H-1)
//   sample = (p(l,t)(1-dx) + p(l+1,t)dx)(1-dy) + (p(l,t+1)(1-dx) + p(l+1,t+1)dx)dy
//   out[channel][row][column] = (sample / 255 - mean[channel]) / stddev[channel]
// Every operation is rounded on its own, in the order written (no FMA
// contraction, divisions rounded as IEEE division rounds them), which is how
// the reference's host code evaluates it, so the tensor is bit-identical to
// it. The two divisions are multiply-and-correct sequences of fused
// multiply-adds that round exactly as the division operator does (see
// divide_by_255 and divide), about a third of the division operator's
// instructions; settings outside their guarded range use the operator.
//
// Vector path (size a multiple of 2, 16-byte aligned tensor, images at least
// two pixels wide): one thread computes two consecutive output pixels of a
// row for all three channels. The row's y, top and dy are worked out once.
// The two horizontal neighbours of a sample are adjacent pixels, 6 contiguous
// bytes starting at pixel clamp(left, 0, W-2), so each (row, column) is one
// unaligned 4-byte and one 2-byte load (the edge clamps pick which of the two
// pixels each neighbour is) instead of six byte loads; neighbouring threads
// read neighbouring bytes, served from cache. Away from the left and right
// edges each byte's place in the pair is fixed, one conversion a sample. The
// results go out as one 8-byte store per channel plane. Measured at 32 images
// of 320 x 240 to 224, against the same kernel with the division operator at
// four pixels a thread (12.4 us): corrected divisions and fixed byte places
// 11.2 us at four pixels, 11.0 at two, 12.4 at one, 13.7 at eight. Other
// shapes run one pixel per thread with byte loads. The grid covers (pixels,
// image); images beyond gridDim.y loop.
#include "device_common.hpp"
#include "launch.hpp"

#include <cmath>
#include <type_traits>

namespace cuvit::detail {
namespace {

using cuvit::device::aligned16;

constexpr int kBlock = 256;
constexpr std::int64_t kMaxGridY = 65535;

/// Output pixels per thread on the vector path.
constexpr int kColumns = 2;

/// Bilinear sample of one channel: the reference's order of operations,
/// x weights first, each product and sum rounded on its own.
__device__ __forceinline__ float blend(float p00, float p01, float p10, float p11, float dx,
                                       float dy) {
#pragma clang fp contract(off)
    const float upper = p00 * (1.0F - dx) + p01 * dx;
    const float lower = p10 * (1.0F - dx) + p11 * dx;
    return upper * (1.0F - dy) + lower * dy;
}

/// sample / 255 rounded as IEEE division rounds it, in three operations: the
/// product with 1/255 (rounded), the residual sample - 255 q (exact, one
/// fused multiply-add) and q + residual / 255 (one more). Equal to the IEEE
/// quotient for every float in [0, 255], the blend's range (an exhaustive
/// host comparison over all 1.13e9 of them, denormals included).
__device__ __forceinline__ float divide_by_255(float sample) {
#pragma clang fp contract(off)
    constexpr float kInverse = 1.0F / 255.0F;
    const float q = sample * kInverse;
    return fmaf(fmaf(-255.0F, q, sample), kInverse, q);
}

/// a / b rounded as IEEE division rounds it, from @p inverse = 1/b rounded:
/// the product a * inverse is within two units in the last place, one
/// residual correction makes it faithful, and a second gives the correctly
/// rounded quotient (Markstein's theorem: with the residual a - b q exact and
/// 1/b correctly rounded, q + residual / b rounded once is a / b rounded).
/// The residuals are exact while they stay normal, which the host guarantees
/// by the range it takes this path for (preprocess_u8).
__device__ __forceinline__ float divide(float a, float b, float inverse) {
#pragma clang fp contract(off)
    const float q0 = a * inverse;
    const float q1 = fmaf(fmaf(-b, q0, a), inverse, q0);
    return fmaf(fmaf(-b, q1, a), inverse, q1);
}

/// (sample / 255 - mean) / stddev, two divisions rounded as IEEE division
/// rounds them: with @p kCorrected by the multiply-and-correct forms above
/// (@p inverse = 1/stddev rounded), otherwise by the division operator.
template <bool kCorrected>
__device__ __forceinline__ float normalise(float sample, float mean, float stddev, float inverse) {
#pragma clang fp contract(off)
    if constexpr (kCorrected) {
        return divide(divide_by_255(sample) - mean, stddev, inverse);
    } else {
        return (sample / 255.0F - mean) / stddev;
    }
}

/// 1/stddev per channel, rounded (host IEEE division), for the corrected forms.
struct Inverse {
    float stddev[3];
};

/// Source coordinate of output index @p i along one axis.
__device__ __forceinline__ float source_coordinate(float origin, float step, int i) {
#pragma clang fp contract(off)
    return origin + (static_cast<float>(i) + 0.5F) * step - 0.5F;
}

/// Two adjacent RGB pixels (6 bytes from @p p, any alignment): bytes 0-3 in
/// @p low, 4-5 in the low half of @p high.
struct PixelPair {
    std::uint32_t low;
    std::uint32_t high;
};

__device__ __forceinline__ PixelPair load_pair(const std::uint8_t* p) {
    std::uint32_t low = 0;
    std::uint16_t high = 0;
    __builtin_memcpy(&low, p, sizeof(low));
    __builtin_memcpy(&high, p + 4, sizeof(high));
    return {low, high};
}

/// Channel @p channel of pixel @p pixel (0 or 1) of a pair, as a float.
__device__ __forceinline__ float pair_byte(const PixelPair& pair, int pixel, int channel) {
    const std::uint64_t bits = static_cast<std::uint64_t>(pair.low) | (static_cast<std::uint64_t>(pair.high) << 32);
    return static_cast<float>(static_cast<std::uint8_t>(bits >> (8 * (pixel * 3 + channel))));
}

/// Byte @p k (0-5, a constant) of a pair, as a float: one byte conversion of
/// the 32-bit word that holds it (v_cvt_f32_ubyte0-3).
__device__ __forceinline__ float pair_byte_at(const PixelPair& pair, int k) {
    return static_cast<float>(((k < 4 ? pair.low : pair.high) >> (8 * (k & 3))) & 0xFFU);
}

template <bool kCorrected>
__global__ __launch_bounds__(kBlock) void preprocess_vector_kernel(
    const std::uint8_t* __restrict__ pixels, int width, int height, float* __restrict__ tensor,
    int size, PreprocessGeometry geometry, Inverse inverse, int batch) {
#pragma clang fp contract(off)
    const int quads_per_row = size / kColumns;
    const int quad = blockIdx.x * kBlock + threadIdx.x;
    if (quad >= quads_per_row * size) {
        return;
    }
    const int row = quad / quads_per_row;
    const int first = (quad - row * quads_per_row) * kColumns;
    const int plane = size * size;

    const float y = source_coordinate(geometry.origin_y, geometry.step, row);
    const int top = static_cast<int>(floorf(y));
    const float dy = y - static_cast<float>(top);
    const std::int64_t row0 = static_cast<std::int64_t>(min(max(top, 0), height - 1)) * width;
    const std::int64_t row1 = static_cast<std::int64_t>(min(max(top + 1, 0), height - 1)) * width;

    float dx[kColumns];
    int pair[kColumns];  // byte offset in a row of the 6-byte pixel pair
    int left[kColumns];  // which pixel of the pair (0 or 1) the left neighbour is
    int right[kColumns]; // ... and the right one
#pragma unroll
    for (int j = 0; j < kColumns; ++j) {
        const float x = source_coordinate(geometry.origin_x, geometry.step, first + j);
        const int x0 = static_cast<int>(floorf(x));
        dx[j] = x - static_cast<float>(x0);
        const int start = min(max(x0, 0), width - 2);
        pair[j] = start * 3;
        left[j] = min(max(x0, 0), width - 1) - start;
        right[j] = min(max(x0 + 1, 0), width - 1) - start;
    }

    // Away from the left and right edges each column's neighbours are the
    // two pixels of its pair, in order.
    bool interior = true;
#pragma unroll
    for (int j = 0; j < kColumns; ++j) {
        interior = interior && left[j] == 0 && right[j] == 1;
    }

    const std::int64_t image_bytes = static_cast<std::int64_t>(width) * height * 3;
    for (std::int64_t image = blockIdx.y; image < batch; image += gridDim.y) {
        const std::uint8_t* const top_row = pixels + image * image_bytes + row0 * 3;
        const std::uint8_t* const bottom_row = pixels + image * image_bytes + row1 * 3;
        PixelPair upper[kColumns];
        PixelPair lower[kColumns];
#pragma unroll
        for (int j = 0; j < kColumns; ++j) {
            upper[j] = load_pair(top_row + pair[j]);
            lower[j] = load_pair(bottom_row + pair[j]);
        }
        float* const destination =
            tensor + image * 3 * static_cast<std::int64_t>(plane) + row * size + first;
        // @p fixed: the pair's first pixel is every left neighbour and its
        // second every right one, so each byte's place is a constant (one
        // byte conversion a sample instead of a 64-bit shift and one).
        auto emit = [&](auto fixed) {
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                float out[kColumns];
#pragma unroll
                for (int j = 0; j < kColumns; ++j) {
                    float sample;
                    if constexpr (decltype(fixed)::value) {
                        sample = blend(pair_byte_at(upper[j], c), pair_byte_at(upper[j], 3 + c),
                                       pair_byte_at(lower[j], c), pair_byte_at(lower[j], 3 + c), dx[j], dy);
                    } else {
                        sample = blend(pair_byte(upper[j], left[j], c), pair_byte(upper[j], right[j], c),
                                       pair_byte(lower[j], left[j], c), pair_byte(lower[j], right[j], c), dx[j],
                                       dy);
                    }
                    out[j] = normalise<kCorrected>(sample, geometry.mean[c], geometry.stddev[c], inverse.stddev[c]);
                }
                typedef float Run __attribute__((ext_vector_type(kColumns)));
                Run run;
#pragma unroll
                for (int j = 0; j < kColumns; ++j) {
                    run[j] = out[j];
                }
                *reinterpret_cast<Run*>(destination + static_cast<std::int64_t>(c) * plane) = run;
            }
        };
        if (interior) {
            emit(std::true_type{});
        } else {
            emit(std::false_type{});
        }
    }
}

template <bool kCorrected>
__global__ __launch_bounds__(kBlock) void preprocess_kernel(
    const std::uint8_t* __restrict__ pixels, int width, int height, float* __restrict__ tensor,
    int size, PreprocessGeometry geometry, Inverse inverse, int batch) {
#pragma clang fp contract(off)
    const int pixel = blockIdx.x * kBlock + threadIdx.x;
    const int plane = size * size;
    if (pixel >= plane) {
        return;
    }
    const int row = pixel / size;
    const int column = pixel - row * size;

    const float x = source_coordinate(geometry.origin_x, geometry.step, column);
    const float y = source_coordinate(geometry.origin_y, geometry.step, row);
    const int left = static_cast<int>(floorf(x));
    const int top = static_cast<int>(floorf(y));
    const float dx = x - static_cast<float>(left);
    const float dy = y - static_cast<float>(top);

    const int x0 = min(max(left, 0), width - 1);
    const int x1 = min(max(left + 1, 0), width - 1);
    const int y0 = min(max(top, 0), height - 1);
    const int y1 = min(max(top + 1, 0), height - 1);
    const std::int64_t row0 = static_cast<std::int64_t>(y0) * width;
    const std::int64_t row1 = static_cast<std::int64_t>(y1) * width;
    const std::int64_t i00 = (row0 + x0) * 3;
    const std::int64_t i01 = (row0 + x1) * 3;
    const std::int64_t i10 = (row1 + x0) * 3;
    const std::int64_t i11 = (row1 + x1) * 3;

    const std::int64_t image_bytes = static_cast<std::int64_t>(width) * height * 3;
    for (std::int64_t image = blockIdx.y; image < batch; image += gridDim.y) {
        const std::uint8_t* const source = pixels + image * image_bytes;
        float* const destination = tensor + image * 3 * static_cast<std::int64_t>(plane) + pixel;
#pragma unroll
        for (int channel = 0; channel < 3; ++channel) {
            const float sample = blend(static_cast<float>(source[i00 + channel]),
                                       static_cast<float>(source[i01 + channel]),
                                       static_cast<float>(source[i10 + channel]),
                                       static_cast<float>(source[i11 + channel]), dx, dy);
            destination[static_cast<std::int64_t>(channel) * plane] = normalise<kCorrected>(
                sample, geometry.mean[channel], geometry.stddev[channel], inverse.stddev[channel]);
        }
    }
}

} // namespace

hipError_t preprocess_u8(const std::uint8_t* pixels, int batch, int width, int height,
                         float* tensor, int size, const PreprocessGeometry& geometry,
                         hipStream_t stream) {
    const std::int64_t plane = static_cast<std::int64_t>(size) * size;
    const unsigned int images = static_cast<unsigned int>(batch < kMaxGridY ? batch : kMaxGridY);
    // The corrected divisions where their residuals stay normal: a standard
    // deviation of magnitude in [2^-20, 2^20] and a mean of 0 or of magnitude
    // in [2^-60, 2^60] keep (sample / 255 - mean) zero or at least 2^-61 in
    // magnitude, and its residual above 2^-100. Other settings (and NaN or
    // infinite ones) take the division operator.
    bool corrected = true;
    Inverse inverse{};
    for (int c = 0; c < 3; ++c) {
        const float mean = std::fabs(geometry.mean[c]);
        const float stddev = std::fabs(geometry.stddev[c]);
        corrected = corrected && stddev >= 0x1p-20F && stddev <= 0x1p20F &&
                    (mean == 0.0F || (mean >= 0x1p-60F && mean <= 0x1p60F));
        inverse.stddev[c] = 1.0F / geometry.stddev[c];
    }
    auto run = [&](auto with_correction) {
        constexpr bool kCorrected = decltype(with_correction)::value;
        if (size % kColumns == 0 && aligned16(tensor) && width >= 2) {
            const std::int64_t blocks = (plane / kColumns + kBlock - 1) / kBlock;
            preprocess_vector_kernel<kCorrected><<<dim3(static_cast<unsigned int>(blocks), images), kBlock, 0,
                                                   stream>>>(pixels, width, height, tensor, size, geometry,
                                                             inverse, batch);
        } else {
            const std::int64_t blocks = (plane + kBlock - 1) / kBlock;
            preprocess_kernel<kCorrected><<<dim3(static_cast<unsigned int>(blocks), images), kBlock, 0, stream>>>(
                pixels, width, height, tensor, size, geometry, inverse, batch);
        }
        return hipGetLastError();
    };
    return corrected ? run(std::true_type{}) : run(std::false_type{});
}

} // namespace cuvit::detail
