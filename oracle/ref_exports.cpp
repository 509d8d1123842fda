// C exports over the reference's own CPU code, compiled in place from
// /root/reference by oracle/Makefile into oracle/_ref/libref.so. TEST
// INFRASTRUCTURE ONLY: it lets the tests check the oracle's restatement
// bit-for-bit against the reference's tests/reference/linear_algebra.hpp and
// elementwise.hpp, the weight-file code against src/runtime/weights.cpp and
// the image code against src/runtime/image.cpp.
// Nothing here is a stand-in for reference code: every computation below is
// a direct call into the reference's headers and sources.
#include "cuvit/image.hpp"
#include "cuvit/weights.hpp"
#include "reference/elementwise.hpp"
#include "reference/linear_algebra.hpp"

#include <cstdint>
#include <cstring>
#include <exception>
#include <string>
#include <vector>

namespace {
thread_local std::string last_error;
}

extern "C" {

void ref_layer_norm(const float* in, const float* gamma, const float* beta, float* out, int rows,
                    int columns, float epsilon) {
    cuvit::reference::layer_norm(in, gamma, beta, out, rows, columns, epsilon);
}

void ref_softmax(const float* in, float* out, int rows, int columns) {
    cuvit::reference::softmax(in, out, rows, columns);
}

void ref_gelu(const float* in, float* out, int64_t count) {
    cuvit::reference::gelu(in, out, static_cast<std::size_t>(count));
}

void ref_gemm(const float* a, const float* b, const float* bias, float* c, int m, int n, int k,
              float alpha) {
    cuvit::reference::gemm(a, b, bias, c, m, n, k, alpha);
}

void ref_gemm_transposed(const float* a, const float* b, const float* bias, float* c, int m, int n,
                         int k, float alpha) {
    cuvit::reference::gemm_transposed(a, b, bias, c, m, n, k, alpha);
}

void ref_gemm_term_magnitudes(const float* a, const float* b, float* scale, int m, int n, int k,
                              int transposed, float alpha) {
    const std::vector<float> s =
        cuvit::reference::gemm_term_magnitudes(a, b, m, n, k, transposed != 0, alpha);
    std::memcpy(scale, s.data(), s.size() * sizeof(float));
}

void ref_vector_add(const float* left, const float* right, float* out, int64_t count) {
    cuvit::reference::vector_add(left, right, out, static_cast<std::size_t>(count));
}

const char* ref_last_error(void) { return last_error.c_str(); }

// Writes a weight file with the reference's WeightFileWriter. extents_flat holds
// the extents of every tensor back to back. Returns 0 on success.
int ref_weights_write(const char* path, int count, const char* const* names, const int* ranks,
                      const int64_t* extents_flat, const float* const* data) {
    try {
        cuvit::WeightFileWriter writer;
        const int64_t* cursor = extents_flat;
        for (int i = 0; i < count; ++i) {
            std::vector<cuvit::Extent> extents(cursor, cursor + ranks[i]);
            cursor += ranks[i];
            writer.add(names[i], extents, data[i]);
        }
        writer.write(path);
        return 0;
    } catch (const std::exception& error) {
        last_error = error.what();
        return 1;
    }
}

// Loads @p path with the reference's WeightFile and copies tensor @p name,
// shape-checked against @p extents, into @p out. Returns 0 on success.
int ref_weights_read(const char* path, const char* name, int rank, const int64_t* extents,
                     float* out, int64_t capacity) {
    try {
        const cuvit::WeightFile file = cuvit::WeightFile::load(path);
        const std::vector<cuvit::Extent> shape(extents, extents + rank);
        const float* data = file.float_data(name, shape);
        int64_t count = 1;
        for (const cuvit::Extent e : shape) {
            count *= e;
        }
        if (count > capacity) {
            last_error = "output too small";
            return 1;
        }
        std::memcpy(out, data, static_cast<std::size_t>(count) * sizeof(float));
        return 0;
    } catch (const std::exception& error) {
        last_error = error.what();
        return 1;
    }
}

// Loads @p path with the reference's WeightFile; 0 when it loads, 1 with the
// reason in ref_last_error() when the reference rejects it.
int ref_weights_check(const char* path) {
    try {
        static_cast<void>(cuvit::WeightFile::load(path));
        return 0;
    } catch (const std::exception& error) {
        last_error = error.what();
        return 1;
    }
}

// preprocess() of src/runtime/image.cpp on one interleaved RGB image. Returns
// 0, or 1 with the reference's message in ref_last_error().
int ref_preprocess(const uint8_t* pixels, int width, int height, int size, float crop_fraction,
                   const float* mean, const float* stddev, float* tensor) {
    try {
        cuvit::RgbImage image;
        image.width = width;
        image.height = height;
        if (width > 0 && height > 0) {
            image.pixels.assign(pixels, pixels + static_cast<std::size_t>(width) * height * 3);
        }
        cuvit::Preprocessing settings;
        settings.size = size;
        settings.crop_fraction = crop_fraction;
        for (std::size_t c = 0; c < 3; ++c) {
            settings.mean[c] = mean[c];
            settings.stddev[c] = stddev[c];
        }
        const std::vector<float> out = cuvit::preprocess(image, settings);
        std::memcpy(tensor, out.data(), out.size() * sizeof(float));
        return 0;
    } catch (const std::exception& error) {
        last_error = error.what();
        return 1;
    }
}

// load_ppm() of src/runtime/image.cpp. Returns 0 with the extents and, when
// @p capacity allows, the pixels; 1 with the reference's message otherwise.
int ref_load_ppm(const char* path, int* width, int* height, uint8_t* pixels, int64_t capacity) {
    try {
        const cuvit::RgbImage image = cuvit::load_ppm(path);
        *width = image.width;
        *height = image.height;
        if (static_cast<int64_t>(image.pixels.size()) <= capacity) {
            std::memcpy(pixels, image.pixels.data(), image.pixels.size());
        }
        return 0;
    } catch (const std::exception& error) {
        last_error = error.what();
        return 1;
    }
}

} // extern "C"
