// cu-vit: the command-line classifier, with the reference's options, output
// and exit codes (src/main.cpp:21-206).
//
//   cu-vit --weights FILE.cvw (--image FILE.ppm | --raw FILE.bin)
//          [--top N] [--benchmark ITERATIONS] [--batch N] [--precision f32|bf16]
//
// The image never takes a host round trip after it is read: the PPM's pixels
// go to the GPU, the preprocessing kernel writes the model's input buffer in
// place, and only the logits come back. --benchmark replicates the input on
// the device to --batch images and times a HIP graph of one forward pass,
// replayed ITERATIONS times after ten warm-up passes. --precision (an
// extension) picks the model's storage type; the reference runs fp32.
#include "cuvit/capi.h"
#include "cuvit/device_buffer.hpp"
#include "cuvit/hip_check.hpp"
#include "cuvit/image.hpp"
#include "cuvit/kernels.hpp"
#include "cuvit/stream.hpp"
#include "cuvit/vit.hpp"
#include "cuvit/weights.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <exception>
#include <fstream>
#include <iostream>
#include <memory>
#include <numeric>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace {

struct Options {
    std::string weights;
    std::string image;
    std::string raw;
    int top = 5;
    int benchmark = 0;
    int batch = 1;
    cuvit::Precision precision = cuvit::Precision::kFloat32;
};

const char* const kUsage =
    "Usage: cu-vit --weights FILE.cvw (--image FILE.ppm | --raw FILE.bin)\n"
    "              [--top N] [--benchmark ITERATIONS] [--batch N] [--precision f32|bf16]\n\n"
    "  --weights   Weight file (.cvw)\n"
    "  --image     Binary PPM (P6). Convert with:\n"
    "                ffmpeg -i photo.jpg -pix_fmt rgb24 photo.ppm\n"
    "  --raw       Preprocessed float32 tensor, 3x224x224, planar\n"
    "  --top       Number of classes to report (default 5)\n"
    "  --benchmark Time this many forward passes after a warm-up\n"
    "  --batch     Replicate the input to this batch size when benchmarking\n"
    "  --precision f32 (default) or bf16 storage for weights and activations\n";

/// Parses the command line; --help prints the usage and exits with 0.
Options parse(int argc, char** argv) {
    Options options;
    auto value = [&](int& index, const std::string& flag) -> std::string {
        if (index + 1 >= argc) {
            throw std::runtime_error(flag + " needs a value");
        }
        return argv[++index];
    };
    for (int index = 1; index < argc; ++index) {
        const std::string flag = argv[index];
        if (flag == "--help" || flag == "-h") {
            std::cout << kUsage;
            std::exit(0);
        } else if (flag == "--weights") {
            options.weights = value(index, flag);
        } else if (flag == "--image") {
            options.image = value(index, flag);
        } else if (flag == "--raw") {
            options.raw = value(index, flag);
        } else if (flag == "--top") {
            options.top = std::stoi(value(index, flag));
        } else if (flag == "--benchmark") {
            options.benchmark = std::stoi(value(index, flag));
        } else if (flag == "--batch") {
            options.batch = std::stoi(value(index, flag));
        } else if (flag == "--precision") {
            const std::string name = value(index, flag);
            if (name == "f32") {
                options.precision = cuvit::Precision::kFloat32;
            } else if (name == "bf16") {
                options.precision = cuvit::Precision::kBFloat16;
            } else {
                throw std::runtime_error("--precision takes f32 or bf16, not " + name);
            }
        } else {
            throw std::runtime_error("Unknown argument: " + flag);
        }
    }
    return options;
}

std::vector<float> read_raw(const std::string& path, std::size_t count) {
    std::ifstream stream(path, std::ios::binary);
    if (!stream) {
        throw std::runtime_error("Cannot open tensor: " + path);
    }
    std::vector<float> values(count);
    stream.read(reinterpret_cast<char*>(values.data()),
                static_cast<std::streamsize>(count * sizeof(float)));
    if (static_cast<std::size_t>(stream.gcount()) != count * sizeof(float)) {
        throw std::runtime_error("Tensor is shorter than the model's input: " + path);
    }
    return values;
}

/// The @p count largest logits with their softmax probabilities (the softmax
/// in double, over every class, only for the report).
void print_top(const std::vector<float>& logits, int count) {
    const int shown = std::max(0, std::min(count, static_cast<int>(logits.size())));
    std::vector<int> labels(logits.size());
    std::iota(labels.begin(), labels.end(), 0);
    std::partial_sort(labels.begin(), labels.begin() + shown, labels.end(),
                      [&](int a, int b) { return logits[static_cast<std::size_t>(a)] >
                                                 logits[static_cast<std::size_t>(b)]; });
    const float peak = *std::max_element(logits.begin(), logits.end());
    double denominator = 0.0;
    for (const float logit : logits) {
        denominator += std::exp(static_cast<double>(logit) - peak);
    }
    std::printf("\nTop %d:\n", shown);
    for (int rank = 0; rank < shown; ++rank) {
        const int label = labels[static_cast<std::size_t>(rank)];
        const float logit = logits[static_cast<std::size_t>(label)];
        const double probability = std::exp(static_cast<double>(logit) - peak) / denominator;
        std::printf("  %4d  %9.4f  %6.2f%%\n", label, logit, probability * 100.0);
    }
    std::fflush(stdout);
}

/// Times @p iterations forward passes over @p batch copies of the image in
/// slot 0 of @p images, as replays of one captured HIP graph.
void benchmark(cuvit::VisionTransformer& model, cuvit::DeviceBuffer<float>& images,
               cuvit::DeviceBuffer<float>& logits, int iterations, int batch,
               const cuvit::Stream& stream) {
    const std::int64_t elements = static_cast<std::int64_t>(model.image_elements());
    // Slot 0 to slots 1..batch-1: the broadcast launcher with a slot stride of
    // one image.
    cuvit::launch_broadcast(images.data() + elements, images.data(), elements, elements,
                            batch - 1, stream.get());
    for (int pass = 0; pass < 10; ++pass) {
        model.forward(images.data(), logits.data(), batch, stream.get());
    }
    stream.synchronize();

    hipGraph_t captured = nullptr;
    CUVIT_HIP_CHECK(hipStreamBeginCapture(stream.get(), hipStreamCaptureModeThreadLocal));
    model.forward(images.data(), logits.data(), batch, stream.get());
    CUVIT_HIP_CHECK(hipStreamEndCapture(stream.get(), &captured));
    const std::unique_ptr<std::remove_pointer_t<hipGraph_t>, hipError_t (*)(hipGraph_t)> graph(
        captured, hipGraphDestroy);
    hipGraphExec_t instantiated = nullptr;
    CUVIT_HIP_CHECK(hipGraphInstantiate(&instantiated, graph.get(), nullptr, nullptr, 0));
    const std::unique_ptr<std::remove_pointer_t<hipGraphExec_t>, hipError_t (*)(hipGraphExec_t)>
        executable(instantiated, hipGraphExecDestroy);
    CUVIT_HIP_CHECK(hipGraphLaunch(executable.get(), stream.get()));
    stream.synchronize();

    const auto start = std::chrono::steady_clock::now();
    for (int pass = 0; pass < iterations; ++pass) {
        CUVIT_HIP_CHECK(hipGraphLaunch(executable.get(), stream.get()));
    }
    stream.synchronize();
    const auto finish = std::chrono::steady_clock::now();

    const double ms = std::chrono::duration<double, std::milli>(finish - start).count() / iterations;
    std::printf("\nBatch %d: %.3f ms per pass, %.3f ms per image (%.1f images/s over %d "
                "iterations)\n",
                batch, ms, ms / batch, 1000.0 * batch / ms, iterations);
}

int run(const Options& options) {
    if (options.weights.empty() || (options.image.empty() && options.raw.empty())) {
        std::cout << kUsage;
        return 1;
    }
    int device = 0;
    CUVIT_HIP_CHECK(hipGetDevice(&device));
    hipDeviceProp_t properties{};
    CUVIT_HIP_CHECK(hipGetDeviceProperties(&properties, device));
    std::printf("Cu-Vit\nGPU: %s (%s, %d CUs)\n", properties.name, properties.gcnArchName,
                properties.multiProcessorCount);

    const cuvit::WeightFile weights = cuvit::WeightFile::load(options.weights);
    const cuvit::VitConfig config;
    if (options.batch < 1) {
        throw std::runtime_error("--batch must be at least one");
    }
    cuvit::VisionTransformer model(config, weights, options.batch, options.precision);
    std::printf("Weights: %zu tensors, %.2f MiB; activations %.2f MiB\n", weights.size(),
                static_cast<double>(model.weight_bytes()) / (1024.0 * 1024.0),
                static_cast<double>(model.activation_bytes()) / (1024.0 * 1024.0));

    const std::size_t elements = model.image_elements();
    cuvit::Stream stream;
    cuvit::DeviceBuffer<float> images(elements * static_cast<std::size_t>(options.batch));
    cuvit::DeviceBuffer<float> logits(static_cast<std::size_t>(options.batch) * config.classes);
    if (!options.raw.empty()) {
        const std::vector<float> tensor = read_raw(options.raw, elements);
        images.copy_from_host_async(tensor.data(), elements, stream.get());
        std::printf("Input:   %s (preprocessed tensor)\n", options.raw.c_str());
    } else {
        const cuvit::RgbImage image = cuvit::load_ppm(options.image);
        cuvit::Preprocessing settings;
        settings.size = config.image_size;
        cuvit::DeviceBuffer<std::uint8_t> pixels(image.pixels.size());
        pixels.copy_from_host_async(image.pixels.data(), image.pixels.size(), stream.get());
        cuvit::launch_preprocess(pixels.data(), 1, image.width, image.height, images.data(),
                                 settings, stream.get());
        stream.synchronize(); // pixels is released at the end of this scope
        std::printf("Input:   %s (%dx%d)\n", options.image.c_str(), image.width, image.height);
    }

    model.forward(images.data(), logits.data(), 1, stream.get());
    std::vector<float> scores(static_cast<std::size_t>(config.classes));
    logits.copy_to_host_async(scores.data(), scores.size(), stream.get());
    stream.synchronize();
    print_top(scores, options.top);

    if (options.benchmark > 0) {
        benchmark(model, images, logits, options.benchmark, options.batch, stream);
    }
    return 0;
}

} // namespace

int main(int argc, char** argv) {
    try {
        return run(parse(argc, argv));
    } catch (const std::exception& error) {
        std::fflush(stdout);
        std::cerr << "cu-vit failed: " << error.what() << '\n';
        return 1;
    }
}
