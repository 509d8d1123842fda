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
// One thread computes one output pixel for all three channels: the bilinear
// coordinates are shared, the four neighbours are 12 byte loads served from
// cache (neighbouring threads read neighbouring pixels), and the three stores
// go to three planes, each coalesced across the wavefront. The grid covers
// (pixel, image); images beyond gridDim.y loop.
#include "device_common.hpp"
#include "launch.hpp"

namespace cuvit::detail {
namespace {

constexpr int kBlock = 256;
constexpr std::int64_t kMaxGridY = 65535;

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

    const float x =
        geometry.origin_x + (static_cast<float>(column) + 0.5F) * geometry.step - 0.5F;
    const float y = geometry.origin_y + (static_cast<float>(row) + 0.5F) * geometry.step - 0.5F;
    const float fx = floorf(x);
    const float fy = floorf(y);
    const int left = static_cast<int>(fx);
    const int top = static_cast<int>(fy);
    const float dx = x - static_cast<float>(left);
    const float dy = y - static_cast<float>(top);
    const float wx = 1.0F - dx;
    const float wy = 1.0F - dy;

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
            const float p00 = static_cast<float>(source[i00 + channel]);
            const float p01 = static_cast<float>(source[i01 + channel]);
            const float p10 = static_cast<float>(source[i10 + channel]);
            const float p11 = static_cast<float>(source[i11 + channel]);
            const float upper = p00 * wx + p01 * dx;
            const float lower = p10 * wx + p11 * dx;
            const float sample = upper * wy + lower * dy;
            const float value = sample / 255.0F;
            destination[static_cast<std::int64_t>(channel) * plane] =
                (value - geometry.mean[channel]) / geometry.stddev[channel];
        }
    }
}

} // namespace

hipError_t preprocess_u8(const std::uint8_t* pixels, int batch, int width, int height,
                         float* tensor, int size, const PreprocessGeometry& geometry,
                         hipStream_t stream) {
    const std::int64_t plane = static_cast<std::int64_t>(size) * size;
    const std::int64_t blocks = (plane + kBlock - 1) / kBlock;
    const std::int64_t images = batch < kMaxGridY ? batch : kMaxGridY;
    preprocess_kernel<<<dim3(static_cast<unsigned int>(blocks), static_cast<unsigned int>(images)),
                        kBlock, 0, stream>>>(pixels, width, height, tensor, size, geometry, batch);
    return hipGetLastError();
}

} // namespace cuvit::detail
