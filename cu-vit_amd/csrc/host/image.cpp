// Binary PPM loading (host) and image preprocessing (device), the reference's
// include/cuvit/image.hpp:10-52 and src/runtime/image.cpp:57-135.
//
// load_ppm reads the whole file and walks its header with a cursor. The
// header grammar is the reference's: the magic is the first
// whitespace-delimited token; each of width, height and maximum is found by
// skipping whitespace and '#' comment lines, and must then start with a
// digit; a value too large for an int reads as INT_MAX and makes the next
// field malformed (the behaviour of a failed stream extraction); exactly one
// byte follows the maximum. The payload length is checked against the file
// before anything is allocated for it.
//
// preprocess uploads the pixels, runs cuvit_preprocess_u8 (one kernel) and
// copies the tensor back on a stream of its own.
#include "cuvit/image.hpp"

#include "cuvit/capi.h"
#include "cuvit/device_buffer.hpp"
#include "cuvit/kernels.hpp"
#include "cuvit/stream.hpp"

#include "../capi/status.hpp"

#include <climits>
#include <fstream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <vector>

namespace cuvit {
namespace {

/// Whitespace and digits in the "C" locale, as the reference's stream reads
/// them.
bool is_space(unsigned char c) {
    return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r';
}
bool is_digit(unsigned char c) { return c >= '0' && c <= '9'; }

class HeaderCursor {
  public:
    explicit HeaderCursor(const std::vector<unsigned char>& bytes) : bytes_(bytes) {}

    /// The next whitespace-delimited token ("" at the end of the file).
    std::string token() {
        while (position_ < bytes_.size() && is_space(bytes_[position_])) {
            ++position_;
        }
        std::string text;
        while (position_ < bytes_.size() && !is_space(bytes_[position_])) {
            text.push_back(static_cast<char>(bytes_[position_++]));
        }
        return text;
    }

    /// The next header number (image.cpp:15-35).
    int field() {
        while (!failed_ && position_ < bytes_.size()) {
            const unsigned char c = bytes_[position_];
            if (c == '#') {
                while (position_ < bytes_.size() && bytes_[position_] != '\n') {
                    ++position_;
                }
                if (position_ < bytes_.size()) {
                    ++position_; // the newline ends the comment
                } else {
                    failed_ = true; // a comment running into the end of the file
                }
                continue;
            }
            if (is_space(c)) {
                ++position_;
                continue;
            }
            if (!is_digit(c)) {
                break;
            }
            long long value = 0;
            while (position_ < bytes_.size() && is_digit(bytes_[position_])) {
                if (value <= INT_MAX) {
                    value = value * 10 + (bytes_[position_] - '0');
                }
                ++position_;
            }
            if (value > INT_MAX) {
                failed_ = true;
                return INT_MAX;
            }
            return static_cast<int>(value);
        }
        throw std::runtime_error("Malformed PPM header");
    }

    /// Steps over the single byte between the maximum and the payload.
    void skip_byte() { ++position_; }

    [[nodiscard]] std::size_t position() const noexcept { return position_; }

  private:
    const std::vector<unsigned char>& bytes_;
    std::size_t position_ = 0;
    bool failed_ = false;
};

std::vector<unsigned char> read_file(const std::string& path) {
    std::ifstream stream(path, std::ios::binary);
    if (!stream) {
        throw std::runtime_error("Cannot open image: " + path);
    }
    return std::vector<unsigned char>(std::istreambuf_iterator<char>(stream),
                                      std::istreambuf_iterator<char>());
}

cuvit_preprocessing to_c(const Preprocessing& settings) {
    cuvit_preprocessing c{};
    c.size = settings.size;
    c.crop_fraction = settings.crop_fraction;
    for (std::size_t channel = 0; channel < 3; ++channel) {
        c.mean[channel] = settings.mean[channel];
        c.stddev[channel] = settings.stddev[channel];
    }
    return c;
}

} // namespace

RgbImage load_ppm(const std::string& path) {
    const std::vector<unsigned char> bytes = read_file(path);
    HeaderCursor cursor(bytes);
    if (cursor.token() != "P6") {
        throw std::runtime_error("Only binary PPM (P6) images are supported: " + path);
    }
    RgbImage image;
    image.width = cursor.field();
    image.height = cursor.field();
    const int maximum = cursor.field();
    if (image.width <= 0 || image.height <= 0) {
        throw std::runtime_error("PPM image has no extent: " + path);
    }
    if (maximum != 255) {
        throw std::runtime_error("Only 8-bit PPM images are supported: " + path);
    }
    cursor.skip_byte();

    const std::size_t payload = static_cast<std::size_t>(image.width) *
                                static_cast<std::size_t>(image.height) * 3;
    const std::size_t start = cursor.position();
    if (start > bytes.size() || bytes.size() - start < payload) {
        throw std::runtime_error("PPM image ends before its payload does: " + path);
    }
    image.pixels.assign(bytes.begin() + static_cast<std::ptrdiff_t>(start),
                        bytes.begin() + static_cast<std::ptrdiff_t>(start + payload));
    return image;
}

void launch_preprocess(const std::uint8_t* pixels, int batch, int width, int height,
                       float* tensor, const Preprocessing& settings, hipStream_t stream) {
    const cuvit_preprocessing c = to_c(settings);
    throw_on_error(cuvit_preprocess_u8(pixels, batch, width, height, &c, tensor,
                                       reinterpret_cast<cuvit_stream_t>(stream)));
}

std::vector<float> preprocess(const RgbImage& image, const Preprocessing& settings) {
    if (image.empty()) {
        throw std::invalid_argument("Cannot preprocess an empty image");
    }
    // Settings are checked before any device work, in the reference's order.
    throw_on_error(capi::check_preprocess_settings(image.width, image.height, to_c(settings)));
    const std::size_t needed = static_cast<std::size_t>(image.width) *
                               static_cast<std::size_t>(image.height) * 3;
    if (image.pixels.size() < needed) {
        throw std::invalid_argument("The image holds fewer pixels than its extents need");
    }

    const std::size_t elements = static_cast<std::size_t>(settings.size) * settings.size * 3;
    std::vector<float> tensor(elements);
    Stream stream;
    DeviceBuffer<std::uint8_t> device_pixels(needed);
    DeviceBuffer<float> device_tensor(elements);
    device_pixels.copy_from_host_async(image.pixels.data(), needed, stream.get());
    launch_preprocess(device_pixels.data(), 1, image.width, image.height, device_tensor.data(),
                      settings, stream.get());
    device_tensor.copy_to_host_async(tensor.data(), elements, stream.get());
    stream.synchronize();
    return tensor;
}

} // namespace cuvit
