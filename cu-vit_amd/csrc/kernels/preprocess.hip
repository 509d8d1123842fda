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
// contraction, IEEE division), which is how the reference's host code
// evaluates it, so the tensor is bit-identical to it.
//
// Vector path (size a multiple of 4, 16-byte aligned tensor, images at least
// two pixels wide): one thread computes four consecutive output pixels of a
// row for all three channels. The row's y, top and dy are worked out once.
// The two horizontal neighbours of a sample are adjacent pixels, 6 contiguous
// bytes starting at pixel clamp(left, 0, W-2), so each (row, column) is one
// unaligned 4-byte and one 2-byte load (the edge clamps pick which of the two
// pixels each neighbour is) instead of six byte loads; neighbouring threads
// read neighbouring bytes, served from cache. The results go out as one
// 16-byte store per channel plane. Measured at 32 images of 320 x 240 to 224:
// 14.3 us with one pixel per thread and byte loads, 12.2 us like this; more
// columns or images per thread, or aligned 12-byte windows, were slower.
// Other shapes run one pixel per thread with byte loads. The grid covers
// (pixels, image); images beyond gridDim.y loop.
#include "device_common.hpp"
#include "launch.hpp"

namespace cuvit::detail {
namespace {

using cuvit::device::aligned16;

constexpr int kBlock = 256;
constexpr std::int64_t kMaxGridY = 65535;

/// Output pixels per thread on the vector path.
constexpr int kColumns = 4;

/// Bilinear sample of one channel: the reference's order of operations,
/// x weights first, each product and sum rounded on its own.
__device__ __forceinline__ float blend(float p00, float p01, float p10, float p11, float dx,
                                       float dy) {
#pragma clang fp contract(off)
    const float upper = p00 * (1.0F - dx) + p01 * dx;
    const float lower = p10 * (1.0F - dx) + p11 * dx;
    return upper * (1.0F - dy) + lower * dy;
}

/// (sample / 255 - mean) / stddev, two IEEE divisions.
__device__ __forceinline__ float normalise(float sample, float mean, float stddev) {
#pragma clang fp contract(off)
    return (sample / 255.0F - mean) / stddev;
}

/// Source coordinate of output index @p i along one axis.
__device__ __forceinline__ float source_coordinate(float origin, float step, int i) {
#pragma clang fp contract(off)
    return origin + (static_cast<float>(i) + 0.5F) * step - 0.5F;
}

/// Two adjacent RGB pixels (6 bytes from @p p, any alignment), little-endian
/// in the low 48 bits.
__device__ __forceinline__ std::uint64_t load_pair(const std::uint8_t* p) {
    std::uint32_t low = 0;
    std::uint16_t high = 0;
    __builtin_memcpy(&low, p, sizeof(low));
    __builtin_memcpy(&high, p + 4, sizeof(high));
    return static_cast<std::uint64_t>(low) | (static_cast<std::uint64_t>(high) << 32);
}

/// Channel @p channel of pixel @p pixel (0 or 1) of a pair, as a float.
__device__ __forceinline__ float pair_byte(std::uint64_t pair, int pixel, int channel) {
    return static_cast<float>(static_cast<std::uint8_t>(pair >> (8 * (pixel * 3 + channel))));
}

__global__ __launch_bounds__(kBlock) void preprocess_vector_kernel(
    const std::uint8_t* __restrict__ pixels, int width, int height, float* __restrict__ tensor,
    int size, PreprocessGeometry geometry, int batch) {
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

    const std::int64_t image_bytes = static_cast<std::int64_t>(width) * height * 3;
    for (std::int64_t image = blockIdx.y; image < batch; image += gridDim.y) {
        const std::uint8_t* const top_row = pixels + image * image_bytes + row0 * 3;
        const std::uint8_t* const bottom_row = pixels + image * image_bytes + row1 * 3;
        std::uint64_t upper[kColumns];
        std::uint64_t lower[kColumns];
#pragma unroll
        for (int j = 0; j < kColumns; ++j) {
            upper[j] = load_pair(top_row + pair[j]);
            lower[j] = load_pair(bottom_row + pair[j]);
        }
        float* const destination =
            tensor + image * 3 * static_cast<std::int64_t>(plane) + row * size + first;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float out[kColumns];
#pragma unroll
            for (int j = 0; j < kColumns; ++j) {
                const float sample = blend(pair_byte(upper[j], left[j], c),
                                           pair_byte(upper[j], right[j], c),
                                           pair_byte(lower[j], left[j], c),
                                           pair_byte(lower[j], right[j], c), dx[j], dy);
                out[j] = normalise(sample, geometry.mean[c], geometry.stddev[c]);
            }
            *reinterpret_cast<float4*>(destination + static_cast<std::int64_t>(c) * plane) =
                make_float4(out[0], out[1], out[2], out[3]);
        }
    }
}

__global__ __launch_bounds__(kBlock) void preprocess_kernel(
    const std::uint8_t* __restrict__ pixels, int width, int height, float* __restrict__ tensor,
    int size, PreprocessGeometry geometry, int batch) {
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
            destination[static_cast<std::int64_t>(channel) * plane] =
                normalise(sample, geometry.mean[channel], geometry.stddev[channel]);
        }
    }
}

} // namespace

hipError_t preprocess_u8(const std::uint8_t* pixels, int batch, int width, int height,
                         float* tensor, int size, const PreprocessGeometry& geometry,
                         hipStream_t stream) {
    const std::int64_t plane = static_cast<std::int64_t>(size) * size;
    const unsigned int images = static_cast<unsigned int>(batch < kMaxGridY ? batch : kMaxGridY);
    if (size % kColumns == 0 && aligned16(tensor) && width >= 2) {
        const std::int64_t blocks = (plane / kColumns + kBlock - 1) / kBlock;
        preprocess_vector_kernel<<<dim3(static_cast<unsigned int>(blocks), images), kBlock, 0,
                                   stream>>>(pixels, width, height, tensor, size, geometry, batch);
    } else {
        const std::int64_t blocks = (plane + kBlock - 1) / kBlock;
        preprocess_kernel<<<dim3(static_cast<unsigned int>(blocks), images), kBlock, 0, stream>>>(
            pixels, width, height, tensor, size, geometry, batch);
    }
    return hipGetLastError();
}

} // namespace cuvit::detail
