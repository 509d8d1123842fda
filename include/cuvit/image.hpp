// Images: binary PPM loading and the preprocessing that turns an RGB image
// into the planar [channels, size, size] float tensor the model reads.
//
// Same types, functions, defaults and errors as the reference's
// include/cuvit/image.hpp:10-52 (src/runtime/image.cpp:57-135). load_ppm runs
// on the host (file parsing). preprocess runs on the GPU: the image goes up,
// one kernel resamples, crops and normalises it, the tensor comes back, and
// the values are bit-identical to the reference's host loop. launch_preprocess
// is the device-pointer form for callers whose pixels are already on the GPU,
// for a batch of equally sized images, writing straight into a model's input.
#pragma once

#include <hip/hip_runtime.h>

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace cuvit {

/// An 8-bit RGB image in interleaved order (image.hpp:12-19).
struct RgbImage {
    int width = 0;
    int height = 0;
    std::vector<std::uint8_t> pixels; // width * height * 3

    [[nodiscard]] bool empty() const noexcept { return pixels.empty(); }
};

/// Reads a binary PPM (P6) with an 8-bit maximum (image.cpp:57-93). Header
/// fields may be separated by whitespace and '#' comment lines; exactly one
/// whitespace byte separates the maximum from the payload. Throws
/// std::runtime_error, with the path in the message, for a file that cannot
/// be opened, another magic, a malformed header, a non-positive extent, a
/// maximum other than 255 or a short payload.
[[nodiscard]] RgbImage load_ppm(const std::string& path);

/// How a model's preprocessing maps pixels to tensor values (image.hpp:30-38).
struct Preprocessing {
    int size = 224;
    /// Fraction of the shorter side kept before the centre crop (timm's
    /// crop_pct): 0.9 resizes the shorter side to round(224 / 0.9) = 249 and
    /// crops the middle 224.
    float crop_fraction = 0.9F;
    std::array<float, 3> mean = {0.5F, 0.5F, 0.5F};
    std::array<float, 3> stddev = {0.5F, 0.5F, 0.5F};
};

/// The [3, size, size] tensor of @p image (image.cpp:95-135): bilinear
/// resampling of the shorter side to round(size / crop_fraction) with the
/// aspect ratio kept, the centre size x size crop, values scaled to [0, 1] and
/// normalised per channel. Computed on the current GPU and returned on the
/// host. Throws std::invalid_argument for an empty image, a non-positive
/// size, a crop fraction outside (0, 1] or a zero standard deviation.
[[nodiscard]] std::vector<float> preprocess(const RgbImage& image,
                                            const Preprocessing& settings = {});

/// Device form of preprocess (an extension): @p pixels holds @p batch images
/// of width x height, interleaved RGB, back to back; @p tensor receives
/// [batch, 3, size, size] floats. Enqueue-only on @p stream, like the kernel
/// launchers; same validation as preprocess plus null and negative-batch
/// checks, and a batch of zero returns at once.
void launch_preprocess(const std::uint8_t* pixels, int batch, int width, int height,
                       float* tensor, const Preprocessing& settings = {},
                       hipStream_t stream = nullptr);

} // namespace cuvit
