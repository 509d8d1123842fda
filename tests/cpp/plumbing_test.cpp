// C++ tests of the host-side plumbing and launcher API, one executable with two
// groups: `host` needs no GPU (TensorView, launcher validation and exception
// mapping, weight files, VitConfig, arena sizing); `device` needs one
// (DeviceBuffer, HostBuffer, Stream, DeviceArena, and VisionTransformer in
// both precisions through the C++ API). The cases follow the reference's
// tests/tensor_test.cu, device_buffer_test.cu, host_buffer_test.cu,
// stream_test.cu, device_arena_test.cu, weights_test.cu, vit_test.cu and
// image_test.cu (PPM loading and argument checks on the host, preprocessing on
// the device).
#include "cuvit/device_arena.hpp"
#include "cuvit/device_buffer.hpp"
#include "cuvit/hip_check.hpp"
#include "cuvit/host_buffer.hpp"
#include "cuvit/image.hpp"
#include "cuvit/kernels.hpp"
#include "cuvit/stream.hpp"
#include "cuvit/tensor.hpp"
#include "cuvit/vit.hpp"
#include "cuvit/weights.hpp"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <iostream>
#include <iterator>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

namespace {

using cuvit::Extent;
using cuvit::TensorView;

struct Failure : std::runtime_error {
    explicit Failure(const std::string& message) : std::runtime_error(message) {}
};

void require(bool condition, const std::string& message) {
    if (!condition) {
        throw Failure(message);
    }
}

/// Runs @p body and requires that it throws exactly @p E.
template <typename E, typename Body> void require_throws(Body&& body, const std::string& message) {
    try {
        body();
    } catch (const E&) {
        return;
    } catch (const std::exception& other) {
        throw Failure(message + " (threw something else: " + other.what() + ")");
    }
    throw Failure(message + " (did not throw)");
}

float* scratch() {
    static float storage[256] = {};
    return storage;
}

// -- host: TensorView (reference tests/tensor_test.cu) -------------------------

void tensor_contiguous_layout() {
    const TensorView<float> v(scratch(), {2, 3, 4});
    require(v.rank() == 3 && v.size() == 24 && v.bytes() == 96, "rank / size / bytes");
    require(v.is_contiguous(), "a packed view is contiguous");
    require(v.stride(2) == 1 && v.stride(1) == 4 && v.stride(0) == 12, "row-major strides");
    require(v.offset_of({0, 0, 0}) == 0 && v.offset_of({1, 2, 3}) == 23, "offsets");
    require(v.shape_string() == "[2, 3, 4]", "shape string");
}

void tensor_rank_and_index_validation() {
    const TensorView<float> v(scratch(), {2, 3});
    require_throws<std::out_of_range>([&] { (void)v.extent(2); }, "axis past the rank");
    require_throws<std::invalid_argument>([&] { (void)v.offset_of({0}); }, "index of the wrong rank");
    require_throws<std::out_of_range>([&] { (void)v.offset_of({0, 3}); }, "index past an extent");
    require_throws<std::invalid_argument>([&] { TensorView<float> t(scratch(), {1, 1, 1, 1, 1}); },
                                          "rank above the maximum");
    require_throws<std::invalid_argument>([&] { TensorView<float> t(nullptr, {2}); },
                                          "non-empty view of null");
    const TensorView<float> empty(nullptr, {0, 3});
    require(empty.empty(), "an empty view may be null");
}

void tensor_slice_and_select() {
    const TensorView<float> v(scratch(), {4, 8});
    const auto rows = v.slice(0, 1, 2);
    require(rows.rank() == 2 && rows.extent(0) == 2 && rows.extent(1) == 8, "row slice shape");
    require(rows.data() == scratch() + 8 && rows.is_contiguous(), "row slice start / packing");
    const auto cols = v.slice(1, 2, 3);
    require(cols.extent(1) == 3 && cols.stride(0) == 8 && !cols.is_contiguous(), "column slice");
    require_throws<std::out_of_range>([&] { (void)v.slice(0, 3, 2); }, "slice past the end");

    const TensorView<float> cube(scratch(), {2, 3, 4});
    const auto plane = cube.select(0, 1);
    require(plane.rank() == 2 && plane.extent(0) == 3 && plane.data() == scratch() + 12 &&
                plane.is_contiguous(),
            "leading select");
    const auto middle = cube.select(1, 2);
    require(middle.extent(0) == 2 && middle.stride(0) == 12 && !middle.is_contiguous(),
            "middle select");
}

void tensor_attention_layout() {
    const Extent tokens = 197, heads = 3, head_dim = 64;
    std::vector<float> activation(static_cast<std::size_t>(tokens * heads * head_dim));
    const TensorView<float> packed(activation.data(), {tokens, heads, head_dim});
    const auto per_head = packed.transpose(0, 1);
    require(per_head.extent(0) == heads && per_head.extent(1) == tokens, "transpose swaps axes");
    require(per_head.data() == packed.data() && !per_head.is_contiguous(), "transpose moves nothing");
    require(packed.offset_of({5, 2, 7}) == per_head.offset_of({2, 5, 7}), "same element");
    const auto head = per_head.select(0, 1);
    require(head.stride(0) == heads * head_dim, "one head keeps the token stride");

    std::vector<float> qkv(static_cast<std::size_t>(tokens * 3 * 192));
    const TensorView<float> split(qkv.data(), {tokens, 3, 192});
    for (Extent part = 0; part < 3; ++part) {
        const auto view = split.select(1, part);
        require(view.data() == qkv.data() + part * 192 && view.stride(0) == 3 * 192 &&
                    !view.is_contiguous(),
                "a QKV part");
    }
}

void tensor_reshape_and_strides() {
    const TensorView<float> v(scratch(), {6, 4});
    const auto flat = v.reshape({24});
    require(flat.rank() == 1 && flat.size() == 24 && flat.data() == v.data(), "reshape");
    require_throws<std::invalid_argument>([&] { (void)v.reshape({5, 5}); }, "reshape changing size");
    require_throws<std::invalid_argument>([&] { (void)v.transpose(0, 1).reshape({24}); },
                                          "reshape of a strided view");
    const TensorView<float> unit(scratch(), {1, 8, 4});
    require(unit.is_contiguous() && unit.transpose(0, 1).is_contiguous(), "degenerate axes");
    const auto strided = TensorView<float>::strided(scratch(), {2, 3}, {16, 2});
    require(strided.offset_of({1, 2}) == 20 && !strided.is_contiguous(), "explicit strides");
    const TensorView<const float> readable = strided.as_const();
    require(readable.data() == strided.data() && readable.stride(0) == 16, "as_const");
    static_assert(std::is_const<TensorView<const float>::value_type>::value, "const view");
    require_throws<std::invalid_argument>(
        [&] { (void)TensorView<float>::strided(scratch(), {2, 3}, {6}); }, "stride count");
    require_throws<std::invalid_argument>(
        [&] { (void)TensorView<float>::strided(scratch(), {2, 3}, {6, -1}); }, "negative stride");
}

// -- host: launcher validation and exception mapping --------------------------

float* fake() { return reinterpret_cast<float*>(static_cast<std::uintptr_t>(0x1000)); }

void launchers_validate_before_any_hip_call() {
    // Empty problems are no-ops even with null operands (normalization.cu:226-228).
    float* const none = nullptr;
    cuvit::launch_layer_norm(none, none, none, none, 0, 192);
    cuvit::launch_softmax(none, none, 4, 0);
    cuvit::launch_gelu(none, none, 0);
    cuvit::launch_extract_patches(none, none, 0, 3, 224, 224, 16);
    cuvit::launch_broadcast(none, none, 0, 0, 3);
    cuvit::launch_add(none, none, 0);
    cuvit::launch_add_broadcast(none, none, 4, 0);
    cuvit::launch_gemm(none, none, none, none,
                       cuvit::gemm_problem(0, 4, 4, cuvit::GemmLayout::kNoTranspose));

    require_throws<std::invalid_argument>(
        [] { cuvit::launch_layer_norm(fake(), fake(), fake(), fake(), -1, 4); }, "negative rows");
    require_throws<std::invalid_argument>(
        [&] { cuvit::launch_layer_norm(fake(), none, fake(), fake(), 2, 4); }, "null gamma");
    require_throws<std::invalid_argument>([&] { cuvit::launch_softmax(none, fake(), 2, 2); },
                                          "null softmax input");
    require_throws<std::invalid_argument>(
        [] { cuvit::launch_extract_patches(fake(), fake(), 1, 3, 18, 16, 4); }, "partial patches");
    require_throws<std::invalid_argument>([] { cuvit::launch_broadcast(fake(), fake(), 8, 4, 2); },
                                          "stride below count");
    require_throws<std::length_error>(
        [] { cuvit::launch_gelu(fake(), fake(), std::int64_t{1} << 40); }, "grid limit");
    cuvit::GemmProblem split = cuvit::gemm_problem(4, 4, 4, cuvit::GemmLayout::kTransposed);
    split.batch.count = 6;
    split.batch.inner = 4;
    require_throws<std::invalid_argument>(
        [&] { cuvit::launch_gemm(fake(), fake(), none, fake(), split); }, "split batch");
    cuvit::GemmProblem narrow = cuvit::gemm_problem(4, 4, 4, cuvit::GemmLayout::kNoTranspose);
    narrow.lda = 3;
    require_throws<std::invalid_argument>(
        [&] { cuvit::launch_gemm(fake(), fake(), none, fake(), narrow); }, "narrow lda");
    try {
        cuvit::launch_softmax(fake(), none, 1, 1);
        throw Failure("a null softmax output was accepted");
    } catch (const std::invalid_argument& error) {
        require(std::string(error.what()) == "Softmax operands cannot be null",
                "the message is the reference launcher's");
    }
}

void hip_check_reports_the_error() {
    try {
        CUVIT_HIP_CHECK(hipErrorInvalidValue);
        throw Failure("CUVIT_HIP_CHECK did not throw");
    } catch (const cuvit::HipError& error) {
        require(error.code() == hipErrorInvalidValue, "HipError keeps the code");
        const std::string text = error.what();
        require(text.find("hipErrorInvalidValue") != std::string::npos, "message names the error");
        require(text.find("plumbing_test.cpp") != std::string::npos, "message names the file");
    }
}

// -- host: weight files and configuration ------------------------------------

void weights_round_trip_and_checks() {
    const std::string path = "cuvit_plumbing_weights.cvw";
    std::vector<float> patch(192 * 3 * 16 * 16);
    for (std::size_t i = 0; i < patch.size(); ++i) {
        patch[i] = static_cast<float>(i) * 0.25F;
    }
    std::vector<float> twelve(12, 0.5F);
    cuvit::WeightFileWriter writer;
    writer.add("patch_embed.weight", {192, 3, 16, 16}, patch.data());
    writer.add("weight", {3, 4}, twelve.data());
    require_throws<std::invalid_argument>([&] { writer.add("weight", {12}, twelve.data()); },
                                          "duplicate name");
    writer.write(path);
    const auto file = cuvit::WeightFile::load(path);
    std::remove(path.c_str());
    require(file.size() == 2 && file.contains("weight") && !file.contains("absent"), "entries");
    const float* data = file.float_data("patch_embed.weight", {192, 3, 16, 16});
    require(std::memcmp(data, patch.data(), patch.size() * sizeof(float)) == 0, "payload");
    for (const auto& entry : file.entries()) {
        require(entry.offset % 64 == 0, "payloads are 64-byte aligned");
    }
    try {
        (void)file.float_data("weight", {4, 3});
        throw Failure("a transposed shape was accepted");
    } catch (const std::runtime_error& error) {
        require(std::string(error.what()).find("[3, 4]") != std::string::npos, "shape message");
    }
    require_throws<std::runtime_error>([] { (void)cuvit::WeightFile::load("no_such_file.cvw"); },
                                       "missing file");
}

void vit_config_validation() {
    cuvit::VitConfig config;
    require(config.token_count() == 197 && config.head_dim() == 64 && config.patch_elements() == 768,
            "ViT-Tiny derived dimensions");
    config.validate();
    config.embed_dim = 25;
    config.heads = 4;
    require_throws<std::invalid_argument>([&] { config.validate(); }, "embed not divisible by heads");
    config = cuvit::VitConfig{};
    config.image_size = 30;
    require_throws<std::invalid_argument>([&] { config.validate(); }, "image not divisible by patch");
    const auto names = cuvit::VisionTransformer::expected_tensor_names(cuvit::VitConfig{});
    require(names.size() == 152 && names.front() == "cls_token" && names.back() == "head.bias",
            "expected names");
}

void arena_sizing() {
    require(cuvit::DeviceArena::kAlignment == 256, "alignment");
    require(cuvit::DeviceArena::reserved_bytes<float>(1) == 256, "one float pads to 256");
    require(cuvit::DeviceArena::reserved_bytes<float>(64) == 256, "64 floats fit 256");
    require(cuvit::DeviceArena::reserved_bytes<float>(65) == 512, "65 floats need 512");
    require(cuvit::DeviceArena::reserved_bytes<float>(0) == 0, "empty");
}

// -- device: DeviceBuffer (reference device_buffer_test.cu) --------------------

void device_buffer_copies_and_bounds() {
    std::vector<float> host(1000);
    for (std::size_t i = 0; i < host.size(); ++i) {
        host[i] = static_cast<float>(i);
    }
    cuvit::DeviceBuffer<float> buffer(host.size());
    require(buffer.size() == 1000 && buffer.bytes() == 4000 && !buffer.empty(), "size");
    int device = -1;
    CUVIT_HIP_CHECK(hipGetDevice(&device));
    require(buffer.device() == device, "records its device");
    buffer.copy_from_host(host.data(), host.size());
    std::vector<float> back(host.size());
    buffer.copy_to_host(back.data(), back.size());
    require(back == host, "round trip");
    std::vector<float> part(10);
    buffer.copy_to_host(part.data(), 10, 990);
    require(part[0] == 990.0F && part[9] == 999.0F, "offset copy");

    require_throws<std::out_of_range>([&] { buffer.copy_to_host(part.data(), 11, 990); },
                                      "read past the end");
    require_throws<std::invalid_argument>([&] { buffer.copy_from_host(nullptr, 4); }, "null host");
    require_throws<std::invalid_argument>([&] { buffer.copy_from_device(buffer, 10, 0, 5); },
                                          "overlapping self copy");
    buffer.copy_from_device(buffer, 10, 0, 500);
    buffer.copy_to_host(part.data(), 10, 500);
    require(part[0] == 0.0F && part[9] == 9.0F, "disjoint self copy");
    buffer.copy_from_device(buffer, 10, 500, 510);  // adjacent ranges touch but do not overlap
    buffer.copy_from_device(buffer, 10, 520, 510);
    require_throws<std::invalid_argument>([&] { buffer.copy_from_device(buffer, 10, 519, 510); },
                                          "self copy overlapping by one element");
    require_throws<std::out_of_range>([&] { buffer.copy_from_device(buffer, 1, 1000, 0); },
                                      "source offset at the end");
    buffer.copy_from_device(buffer, 0, 1000, 1000);  // empty copies at the end are fine
    buffer.copy_to_host(nullptr, 0, 1000);

    cuvit::DeviceBuffer<float> moved(std::move(buffer));
    require(buffer.empty() && buffer.data() == nullptr && buffer.device() == -1, "moved-from");
    require(moved.size() == 1000, "moved-to");
    moved.fill_zero();
    moved.copy_to_host(back.data(), back.size());
    for (const float v : back) {
        require(v == 0.0F, "zero fill");
    }
    float* const before = moved.data();
    moved.allocate(1000);
    require(moved.data() == before, "same size keeps the allocation");
    moved.reset();
    require(moved.empty(), "reset");
    require(moved.data() == nullptr && moved.device() == -1, "reset releases the allocation");
    moved.allocate(3);
    require(moved.size() == 3 && moved.device() == device, "allocate after reset");
    moved.allocate(0);
    require(moved.empty() && moved.data() == nullptr, "allocate(0) releases");
}

// -- device: HostBuffer (reference host_buffer_test.cu) -----------------------

void host_buffer_is_pinned_and_usable() {
    cuvit::HostBuffer<float> pinned(4096);
    hipPointerAttribute_t attributes{};
    CUVIT_HIP_CHECK(hipPointerGetAttributes(&attributes, pinned.data()));
    require(attributes.type == hipMemoryTypeHost, "allocation is page-locked host memory");
    for (std::size_t i = 0; i < pinned.size(); ++i) {
        pinned[i] = static_cast<float>(i) * 2.0F;
    }
    require(pinned.at(4095) == 8190.0F, "element access");
    require_throws<std::out_of_range>([&] { (void)pinned.at(4096); }, "at() bounds");
    float* const before = pinned.data();
    pinned.allocate(4096);
    require(pinned.data() == before && pinned[7] == 14.0F, "same size keeps contents");
    cuvit::HostBuffer<float> moved(std::move(pinned));
    require(pinned.empty() && moved.size() == 4096, "move");
    cuvit::HostBuffer<float> other(8);
    other = std::move(moved);
    require(moved.empty() && moved.data() == nullptr && other.size() == 4096 && other[7] == 14.0F,
            "move assignment");
    moved = std::move(other);
    require(std::distance(moved.begin(), moved.end()) == 4096, "iteration covers the elements");
    other.allocate(0);
    require(other.empty() && other.data() == nullptr, "allocate(0) keeps nothing");

    cuvit::DeviceBuffer<float> device(moved.size());
    cuvit::Stream stream;
    device.copy_from_host_async(moved.data(), moved.size(), stream.get());
    cuvit::HostBuffer<float> back(moved.size());
    back.fill_zero();
    device.copy_to_host_async(back.data(), back.size(), stream.get());
    stream.synchronize();
    require(std::memcmp(back.data(), moved.data(), moved.bytes()) == 0, "round trip via device");
}

// -- device: Stream (reference stream_test.cu) --------------------------------

void stream_pipeline() {
    cuvit::Stream stream;
    require(!stream.empty() && stream.query(), "a new stream is idle");
    const std::size_t count = 1 << 16;
    cuvit::HostBuffer<float> a(count), b(count), out(count);
    for (std::size_t i = 0; i < count; ++i) {
        a[i] = static_cast<float>(i);
        b[i] = 0.5F;
    }
    cuvit::DeviceBuffer<float> da(count), db(count);
    da.copy_from_host_async(a.data(), count, stream.get());
    db.copy_from_host_async(b.data(), count, stream.get());
    cuvit::launch_add(da.data(), db.data(), static_cast<std::int64_t>(count), stream.get());
    da.copy_to_host_async(out.data(), count, stream.get());
    stream.synchronize();
    require(stream.query(), "idle after synchronize");
    for (std::size_t i = 0; i < count; ++i) {
        require(out[i] == static_cast<float>(i) + 0.5F, "H2D -> add -> D2H on one stream");
    }

    cuvit::DeviceBuffer<float> copy(count);
    copy.copy_from_device_async(da, count, stream.get());
    std::vector<float> check(count);
    stream.synchronize();
    copy.copy_to_host(check.data(), count);
    require(check[count - 1] == static_cast<float>(count - 1) + 0.5F, "async device copy");

    cuvit::Stream other;
    cuvit::DeviceBuffer<float> x(count), y(count);
    x.fill_zero_async(stream.get());
    y.fill_zero_async(other.get());
    cuvit::launch_gelu(x.data(), x.data(), static_cast<std::int64_t>(count), stream.get());
    cuvit::launch_gelu(y.data(), y.data(), static_cast<std::int64_t>(count), other.get());
    stream.synchronize();
    other.synchronize();
    cuvit::Stream moved(std::move(other));
    require(other.empty() && other.get() == nullptr && !moved.empty(), "stream move");
}

// -- device: DeviceArena (reference device_arena_test.cu) ---------------------

void arena_carving() {
    cuvit::DeviceArena arena(1 << 20);
    require(arena.capacity() == (1u << 20) && arena.used() == 0, "capacity");
    auto a = arena.allocate<float>({3, 5});
    auto b = arena.allocate<float>({7});
    float* c = arena.allocate_raw<float>(100);
    for (const void* p : {static_cast<const void*>(a.data()), static_cast<const void*>(b.data()),
                          static_cast<const void*>(c)}) {
        require(reinterpret_cast<std::uintptr_t>(p) % 256 == 0, "every carve is 256-aligned");
    }
    require(b.data() >= a.data() + 15 && c >= b.data() + 7, "carves do not overlap");
    require(arena.used() == 256 + 256 + 512, "used() counts padding");
    require(a.extent(0) == 3 && a.extent(1) == 5 && a.is_contiguous(), "multi-dimensional view");
    const std::size_t used = arena.used();
    require_throws<std::runtime_error>([&] { (void)arena.allocate_raw<float>(1 << 20); },
                                       "exhaustion");
    require(arena.used() == used, "a failed carve does not move the cursor");
    arena.fill_zero();
    std::vector<float> back(100, 1.0F);
    CUVIT_HIP_CHECK(hipMemcpy(back.data(), c, 400, hipMemcpyDeviceToHost));
    for (const float v : back) {
        require(v == 0.0F, "fill_zero covers the arena");
    }
    arena.reset();
    require(arena.used() == 0 && arena.remaining() == arena.capacity(), "reset");
}

// -- device: the model through the C++ API (reference vit_test.cu) -----------

/// The vit_test configuration (vit_test.cu:36-47).
cuvit::VitConfig small_config() {
    cuvit::VitConfig config;
    config.image_size = 32;
    config.patch_size = 8;
    config.embed_dim = 24;
    config.depth = 2;
    config.heads = 4;
    config.mlp_hidden = 48;
    config.classes = 7;
    return config;
}

/// Deterministic weights in expected-name order (LN gamma near 1), as float32
/// or, for the GEMM matrices, bf16 (truncated bits are as good as any here).
void write_model(const cuvit::VitConfig& config, const std::string& path, bool bf16_matrices) {
    cuvit::WeightFileWriter writer;
    std::uint32_t state = 12345U;
    auto next = [&state] {
        state = state * 1664525U + 1013904223U;
        return (static_cast<float>(state >> 8) / 16777216.0F - 0.5F) * 0.4F;
    };
    const cuvit::Extent e = config.embed_dim;
    const cuvit::Extent t = config.token_count();
    const cuvit::Extent h = config.mlp_hidden;
    const cuvit::Extent c = config.classes;
    for (const std::string& name : cuvit::VisionTransformer::expected_tensor_names(config)) {
        std::vector<Extent> shape;
        const bool matrix = name.find("qkv.weight") != std::string::npos ||
                            name.find("proj.weight") != std::string::npos ||
                            name.find("fc1.weight") != std::string::npos ||
                            name.find("fc2.weight") != std::string::npos || name == "head.weight";
        if (name == "cls_token") shape = {1, 1, e};
        else if (name == "pos_embed") shape = {1, t, e};
        else if (name == "patch_embed.proj.weight")
            shape = {e, config.channels, config.patch_size, config.patch_size};
        else if (name.find("qkv.weight") != std::string::npos) shape = {3 * e, e};
        else if (name.find("qkv.bias") != std::string::npos) shape = {3 * e};
        else if (name.find("fc1.weight") != std::string::npos) shape = {h, e};
        else if (name.find("fc1.bias") != std::string::npos) shape = {h};
        else if (name.find("fc2.weight") != std::string::npos) shape = {e, h};
        else if (name.find("proj.weight") != std::string::npos) shape = {e, e};
        else if (name == "head.weight") shape = {c, e};
        else if (name == "head.bias") shape = {c};
        else shape = {e}; // biases of width e, LN gamma and beta
        Extent count = 1;
        for (const Extent x : shape) count *= x;
        const bool gamma = name.find("norm") != std::string::npos &&
                           name.find("weight") != std::string::npos;
        std::vector<float> values(static_cast<std::size_t>(count));
        for (float& v : values) v = (gamma ? 1.0F : 0.0F) + next();
        if (bf16_matrices && matrix) { // "proj.weight" covers patch_embed.proj.weight
            std::vector<std::uint16_t> bits(values.size());
            for (std::size_t i = 0; i < values.size(); ++i) {
                std::uint32_t word = 0;
                std::memcpy(&word, &values[i], sizeof(word));
                bits[i] = static_cast<std::uint16_t>(word >> 16);
            }
            writer.add_bf16(name, shape, bits.data());
        } else {
            writer.add(name, shape, values.data());
        }
    }
    writer.write(path);
}

void model_through_the_cpp_api() {
    const cuvit::VitConfig config = small_config();
    write_model(config, "model.cvw", false);
    write_model(config, "model_bf16.cvw", true);
    const cuvit::WeightFile file = cuvit::WeightFile::load("model.cvw");
    const cuvit::WeightFile file_bf16 = cuvit::WeightFile::load("model_bf16.cvw");
    require(file.version() == 1 && file_bf16.version() == 2, "weight file versions");

    const std::size_t per_image = static_cast<std::size_t>(config.channels) * config.image_size *
                                  config.image_size;
    std::vector<float> images(3 * per_image);
    for (std::size_t i = 0; i < images.size(); ++i) {
        images[i] = std::sin(0.37F * static_cast<float>(i));
    }
    const std::vector<float> first(images.begin(), images.begin() + static_cast<long>(per_image));

    for (const cuvit::Precision precision : {cuvit::Precision::kFloat32, cuvit::Precision::kBFloat16}) {
        cuvit::VisionTransformer model(config, file, 3, precision);
        require(model.precision() == precision, "precision is kept");
        const std::vector<float> batch = model.forward(images);
        const std::vector<float> alone = model.forward(first);
        require(batch.size() == 3 * static_cast<std::size_t>(config.classes), "logit count");
        for (const float v : batch) {
            require(std::isfinite(v), "finite logits");
        }
        require(std::memcmp(batch.data(), alone.data(), alone.size() * sizeof(float)) == 0,
                "an image in a batch equals the image alone (bitwise)");
        require_throws<std::invalid_argument>(
            [&] { (void)model.forward(std::vector<float>(4 * per_image)); }, "batch above max_batch");
        require_throws<std::invalid_argument>(
            [&] { (void)model.forward(std::vector<float>(per_image + 1)); }, "partial image");
    }

    // bf16 weights: loaded into either precision they match the float32 file
    // holding the same (widened) values, bitwise.
    cuvit::VisionTransformer from_bf16(config, file_bf16, 3, cuvit::Precision::kBFloat16);
    const std::vector<float> reduced = from_bf16.forward(images);
    cuvit::VisionTransformer fp32_of_bf16(config, file_bf16, 3);
    const std::vector<float> widened = fp32_of_bf16.forward(images);
    cuvit::VisionTransformer reference_fp32(config, file, 3);
    const std::vector<float> full = reference_fp32.forward(images);
    double diff = 0.0;
    double norm = 0.0;
    for (std::size_t i = 0; i < full.size(); ++i) {
        diff += (static_cast<double>(reduced[i]) - full[i]) * (static_cast<double>(reduced[i]) - full[i]);
        diff += (static_cast<double>(widened[i]) - full[i]) * (static_cast<double>(widened[i]) - full[i]);
        norm += 2.0 * static_cast<double>(full[i]) * full[i];
    }
    require(std::sqrt(diff / norm) < 5.0e-2, "bf16 weights stay within bf16 error of float32");
    std::remove("model.cvw");
    std::remove("model_bf16.cvw");
}

int run(const std::vector<std::pair<std::string, std::function<void()>>>& cases) {
    int failures = 0;
    for (const auto& [name, body] : cases) {
        try {
            body();
            std::cout << name << ": PASS" << std::endl;
        } catch (const std::exception& error) {
            std::cout << name << ": FAIL: " << error.what() << std::endl;
            ++failures;
        }
    }
    return failures == 0 ? 0 : 1;
}

// -- images (reference tests/image_test.cu) ----------------------------------

void write_ppm(const std::string& path, int width, int height,
               const std::vector<std::uint8_t>& pixels, const char* comment = nullptr) {
    std::ofstream stream(path, std::ios::binary);
    stream << "P6\n";
    if (comment != nullptr) {
        stream << '#' << comment << '\n';
    }
    stream << width << ' ' << height << "\n255\n";
    stream.write(reinterpret_cast<const char*>(pixels.data()),
                 static_cast<std::streamsize>(pixels.size()));
}

std::vector<std::uint8_t> ramp(int width, int height) {
    std::vector<std::uint8_t> pixels(static_cast<std::size_t>(width) * height * 3);
    for (int row = 0; row < height; ++row) {
        for (int column = 0; column < width; ++column) {
            const std::size_t at = (static_cast<std::size_t>(row) * width + column) * 3;
            pixels[at] = static_cast<std::uint8_t>(column * 255 / (width - 1));
            pixels[at + 1] = static_cast<std::uint8_t>(row * 255 / (height - 1));
            pixels[at + 2] = 128;
        }
    }
    return pixels;
}

void image_ppm_round_trip() {
    const std::vector<std::uint8_t> pixels = ramp(7, 5);
    write_ppm("plumbing_round_trip.ppm", 7, 5, pixels, " written by the test suite");
    const cuvit::RgbImage image = cuvit::load_ppm("plumbing_round_trip.ppm");
    require(image.width == 7 && image.height == 5, "the PPM header was misread");
    require(image.pixels == pixels, "the PPM payload changed on the way through");
    std::remove("plumbing_round_trip.ppm");
}

void image_malformed_files_are_rejected() {
    require_throws<std::runtime_error>([] { static_cast<void>(cuvit::load_ppm("absent.ppm")); },
                                       "a missing image was accepted");
    {
        std::ofstream ascii("plumbing_ascii.ppm");
        ascii << "P3\n2 2\n255\n0 0 0 0 0 0 0 0 0 0 0 0\n";
    }
    require_throws<std::runtime_error>(
        [] { static_cast<void>(cuvit::load_ppm("plumbing_ascii.ppm")); },
        "an ASCII PPM was accepted as binary");
    write_ppm("plumbing_short.ppm", 8, 8, std::vector<std::uint8_t>(8 * 8 * 3 - 32, 0));
    require_throws<std::runtime_error>(
        [] { static_cast<void>(cuvit::load_ppm("plumbing_short.ppm")); },
        "a truncated image was accepted");
    std::remove("plumbing_ascii.ppm");
    std::remove("plumbing_short.ppm");
}

void image_invalid_settings_are_rejected() {
    // Checked before any device work, so this runs without a GPU.
    cuvit::RgbImage image;
    image.width = 32;
    image.height = 32;
    image.pixels.assign(32 * 32 * 3, 100);
    cuvit::Preprocessing settings;
    settings.crop_fraction = 0.0F;
    require_throws<std::invalid_argument>([&] { static_cast<void>(cuvit::preprocess(image, settings)); },
                                          "a zero crop fraction was accepted");
    settings = cuvit::Preprocessing{};
    settings.stddev = {1.0F, 0.0F, 1.0F};
    require_throws<std::invalid_argument>([&] { static_cast<void>(cuvit::preprocess(image, settings)); },
                                          "a zero standard deviation was accepted");
    settings = cuvit::Preprocessing{};
    settings.size = 0;
    require_throws<std::invalid_argument>([&] { static_cast<void>(cuvit::preprocess(image, settings)); },
                                          "a zero size was accepted");
    require_throws<std::invalid_argument>(
        [] { static_cast<void>(cuvit::preprocess(cuvit::RgbImage{})); },
        "an empty image was accepted");
    require_throws<std::invalid_argument>(
        [] { cuvit::launch_preprocess(nullptr, -1, 4, 4, nullptr); },
        "a negative batch was accepted");
    cuvit::launch_preprocess(nullptr, 0, 4, 4, nullptr); // an empty batch returns at once
}

void image_uniform_grey_normalises_to_one_value() {
    cuvit::RgbImage image;
    image.width = 300;
    image.height = 300;
    image.pixels.assign(300 * 300 * 3, 128);
    const std::vector<float> tensor = cuvit::preprocess(image);
    require(tensor.size() == 3U * 224 * 224, "the preprocessed tensor has the wrong size");
    const float expected = (128.0F / 255.0F - 0.5F) / 0.5F;
    for (const float value : tensor) {
        require(std::fabs(value - expected) < 1.0e-5F,
                "a uniform image did not normalize to a uniform value");
    }
}

void image_channels_stay_planar() {
    cuvit::RgbImage image;
    image.width = 256;
    image.height = 256;
    image.pixels.resize(256 * 256 * 3);
    for (std::size_t pixel = 0; pixel < 256U * 256; ++pixel) {
        image.pixels[pixel * 3] = 255;
        image.pixels[pixel * 3 + 1] = 0;
        image.pixels[pixel * 3 + 2] = 128;
    }
    const std::vector<float> tensor = cuvit::preprocess(image);
    const std::size_t plane = 224 * 224;
    for (std::size_t i = 0; i < plane; ++i) {
        require(std::fabs(tensor[i] - 1.0F) < 1.0e-5F, "the red plane is not saturated");
        require(std::fabs(tensor[plane + i] + 1.0F) < 1.0e-5F, "the green plane is not empty");
        require(std::fabs(tensor[2 * plane + i] - (128.0F / 255.0F - 0.5F) / 0.5F) < 1.0e-5F,
                "the blue plane has the wrong value");
    }
}

void image_centre_crop_keeps_the_middle() {
    cuvit::RgbImage image;
    image.width = 600;
    image.height = 200;
    image.pixels.assign(600 * 200 * 3, 0);
    for (int row = 0; row < 200; ++row) {
        for (int column = 250; column < 350; ++column) {
            const std::size_t at = (static_cast<std::size_t>(row) * 600 + column) * 3;
            image.pixels[at] = image.pixels[at + 1] = image.pixels[at + 2] = 255;
        }
    }
    const std::vector<float> tensor = cuvit::preprocess(image);
    require(tensor[112 * 224 + 112] > 0.9F, "the centre of the crop is not the centre of the image");
    require(tensor[0] < -0.9F && tensor[224 * 224 - 1] < -0.9F, "the crop reached past the band");
}

void image_batch_equals_single_images() {
    // launch_preprocess over two images in one launch, straight into a
    // model-shaped input, gives each image's preprocess() bits.
    cuvit::RgbImage first;
    first.width = 320;
    first.height = 240;
    first.pixels = ramp(320, 240);
    cuvit::RgbImage second = first;
    for (std::size_t i = 0; i < second.pixels.size(); ++i) {
        second.pixels[i] = static_cast<std::uint8_t>(second.pixels[i] * 7 + i);
    }
    const std::size_t bytes = first.pixels.size();
    cuvit::DeviceBuffer<std::uint8_t> pixels(2 * bytes);
    pixels.copy_from_host(first.pixels.data(), bytes);
    pixels.copy_from_host(second.pixels.data(), bytes, bytes);
    const std::size_t elements = 3 * 224 * 224;
    cuvit::DeviceBuffer<float> tensor(2 * elements);
    cuvit::Stream stream;
    cuvit::launch_preprocess(pixels.data(), 2, 320, 240, tensor.data(), {}, stream.get());
    stream.synchronize();
    std::vector<float> both(2 * elements);
    tensor.copy_to_host(both.data(), both.size());
    const std::vector<float> a = cuvit::preprocess(first);
    const std::vector<float> b = cuvit::preprocess(second);
    require(std::memcmp(both.data(), a.data(), elements * sizeof(float)) == 0,
            "image 0 of the batch differs from preprocess()");
    require(std::memcmp(both.data() + elements, b.data(), elements * sizeof(float)) == 0,
            "image 1 of the batch differs from preprocess()");
}

} // namespace

int main(int argc, char** argv) {
    const std::string group = argc > 1 ? argv[1] : "host";
    if (group == "host") {
        return run({{"tensor_contiguous_layout", tensor_contiguous_layout},
                    {"tensor_rank_and_index_validation", tensor_rank_and_index_validation},
                    {"tensor_slice_and_select", tensor_slice_and_select},
                    {"tensor_attention_layout", tensor_attention_layout},
                    {"tensor_reshape_and_strides", tensor_reshape_and_strides},
                    {"launchers_validate_before_any_hip_call", launchers_validate_before_any_hip_call},
                    {"hip_check_reports_the_error", hip_check_reports_the_error},
                    {"weights_round_trip_and_checks", weights_round_trip_and_checks},
                    {"vit_config_validation", vit_config_validation},
                    {"arena_sizing", arena_sizing},
                    {"image_ppm_round_trip", image_ppm_round_trip},
                    {"image_malformed_files_are_rejected", image_malformed_files_are_rejected},
                    {"image_invalid_settings_are_rejected", image_invalid_settings_are_rejected}});
    }
    if (group == "device") {
        const int status = run({{"device_buffer_copies_and_bounds", device_buffer_copies_and_bounds},
                                {"host_buffer_is_pinned_and_usable", host_buffer_is_pinned_and_usable},
                                {"stream_pipeline", stream_pipeline},
                                {"arena_carving", arena_carving},
                                {"model_through_the_cpp_api", model_through_the_cpp_api},
                                {"image_uniform_grey_normalises_to_one_value",
                                 image_uniform_grey_normalises_to_one_value},
                                {"image_channels_stay_planar", image_channels_stay_planar},
                                {"image_centre_crop_keeps_the_middle", image_centre_crop_keeps_the_middle},
                                {"image_batch_equals_single_images", image_batch_equals_single_images}});
        // A kernel that faulted asynchronously would surface here.
        const hipError_t sync = hipDeviceSynchronize();
        if (sync != hipSuccess) {
            std::cout << "device synchronize: FAIL: " << hipGetErrorName(sync) << std::endl;
            return 1;
        }
        return status;
    }
    std::cerr << "usage: plumbing_test host|device" << std::endl;
    return 2;
}
