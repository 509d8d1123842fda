// Patch gather, class-token broadcast and positional-embedding add for gfx950.
//
// extract_patches (reference: include/cuvit/kernels.hpp:125-138,
// src/kernels/normalization.cu:159-192, CPU order tests/reference/vit.hpp:65-87)
// rewrites planar [B, C, H, W] images as [B * (H/P) * (W/P), C * P * P] patch
// rows, channel-major inside a row:
//   patches[(b*NP + py*NX + px) * C*P*P + c*P*P + ly*P + lx]
//     = images[((b*C + c)*H + py*P + ly)*W + px*P + lx]
// It is a permutation, so the kernels move opaque 16-byte vectors and the
// result is bit-exact by construction for any element type.
//
// Fast path: one workgroup per (image, channel, patch-row) strip. The strip's
// source is P whole image rows, one contiguous span of P*W elements; its
// destination is NX patch blocks of P*P contiguous elements each. Consecutive
// threads write consecutive 16-byte vectors of a patch block (fully coalesced
// stores); each quad of threads reads one 16-element run of an image row, and
// the workgroup as a whole reads every byte of its span once, so every cache
// line fetched from HBM is consumed by the same workgroup. The patch matrix is
// written with streaming (non-temporal) stores.
//
// bf16 images 224 wide in 16 x 16 patches (ViT/16) take a variant that moves
// whole strips through LDS, so that both its loads and its stores cover whole
// 128-byte lines (extract_patches_staged_bf16_kernel).
//
// broadcast / add_broadcast (normalization.cu:194-212) are 2-D grids over
// (slot, vector) with float4 traffic when counts and pointers allow it. The
// positional add reads and rewrites each token line once, with non-temporal
// loads and stores (3.9 -> 3.4 us at ViT-Tiny batch 32). The gather keeps
// plain loads: non-temporal ones measured slower for it (9.7 -> 10.2 us).
#include "device_common.hpp"
#include "launch.hpp"

#include <type_traits>

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

constexpr int kBlock = 256;

/// Vectors each thread of the strip kernel moves per round: with their loads
/// in flight together the b32 fp32 gather measured 9.04 us against 9.45 us for
/// one at a time.
constexpr int kUnroll = 4;

/// @tparam ElementSize bytes per element (4 fp32, 2 bf16).
/// @tparam PV 16-byte vectors per patch row (P = PV * 16 / ElementSize).
template <int ElementSize, int PV>
__global__ __launch_bounds__(kBlock) void extract_patches_strip_kernel(
    const unsigned char* __restrict__ images, unsigned char* __restrict__ patches, int channels,
    int height, int width, std::int64_t strips) {
    constexpr int kVec = 16 / ElementSize;     // elements per vector
    constexpr int kPatch = PV * kVec;          // P
    constexpr int kChunkVectors = kPatch * PV; // vectors in one P x P block
    using Word = Vec16;

    const int patches_across = width / kPatch;
    const int patches_down = height / kPatch;
    const int strip_vectors = patches_across * kChunkVectors; // = P * W / kVec
    const std::int64_t row_elements = static_cast<std::int64_t>(channels) * kPatch * kPatch;

    for (std::int64_t strip = blockIdx.x; strip < strips; strip += gridDim.x) {
        // strip = (image * channels + channel) * patches_down + patch_row
        const std::int64_t plane = strip / patches_down; // image * channels + channel
        const int patch_row = static_cast<int>(strip - plane * patches_down);
        const std::int64_t image = plane / channels;
        const int channel = static_cast<int>(plane - image * channels);

        const unsigned char* const source =
            images + ((plane * height + static_cast<std::int64_t>(patch_row) * kPatch) * width) *
                         ElementSize;
        const std::int64_t first_patch =
            (image * patches_down + patch_row) * static_cast<std::int64_t>(patches_across);
        unsigned char* const destination =
            patches + (first_patch * row_elements + static_cast<std::int64_t>(channel) * kPatch *
                                                        kPatch) *
                          ElementSize;

        // kUnroll vectors per thread, all loads issued before the first store.
        for (int first = threadIdx.x; first < strip_vectors; first += kBlock * kUnroll) {
            Word value[kUnroll];
            std::int64_t destination_element[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int v = first + u * kBlock;
                const int patch_column = v / kChunkVectors; // power-of-two divisor
                const int q = v % kChunkVectors;
                const int local_row = q / PV;
                const int local_vector = q % PV;
                const std::int64_t source_element =
                    static_cast<std::int64_t>(local_row) * width + patch_column * kPatch +
                    local_vector * kVec;
                destination_element[u] = static_cast<std::int64_t>(patch_column) * row_elements +
                                         static_cast<std::int64_t>(q) * kVec;
                if (v < strip_vectors) {
                    value[u] = load16(source + source_element * ElementSize);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                if (first + u * kBlock < strip_vectors) {
                    store16_streaming(destination + destination_element[u] * ElementSize,
                                      value[u]);
                }
            }
        }
    }
}

/// The bf16 model's first step in one pass: fp32 images gathered into bf16
/// patch rows, each value rounded once to nearest-even (float_to_bf16's
/// rounding, as the conversion kernel does). A value's rounding does not
/// depend on where it moves, so the result is bitwise the conversion followed
/// by the bf16 strip gather, without the bf16 image written and read back.
/// A unit is 8 elements: 32 bytes read (two 16-byte loads), 16 written.
/// @tparam PV 16-byte output vectors per patch row (P = 8 PV).
template <int PV>
__global__ __launch_bounds__(kBlock) void extract_patches_strip_f32_to_bf16_kernel(
    const float* __restrict__ images, std::uint16_t* __restrict__ patches, int channels,
    int height, int width, std::int64_t strips) {
    constexpr int kVec = 8;
    constexpr int kPatch = PV * kVec;
    constexpr int kChunkVectors = kPatch * PV;

    const int patches_across = width / kPatch;
    const int patches_down = height / kPatch;
    const int strip_vectors = patches_across * kChunkVectors;
    const std::int64_t row_elements = static_cast<std::int64_t>(channels) * kPatch * kPatch;

    for (std::int64_t strip = blockIdx.x; strip < strips; strip += gridDim.x) {
        const std::int64_t plane = strip / patches_down; // image * channels + channel
        const int patch_row = static_cast<int>(strip - plane * patches_down);
        const std::int64_t image = plane / channels;
        const int channel = static_cast<int>(plane - image * channels);

        const float* const source =
            images + (plane * height + static_cast<std::int64_t>(patch_row) * kPatch) * width;
        const std::int64_t first_patch =
            (image * patches_down + patch_row) * static_cast<std::int64_t>(patches_across);
        std::uint16_t* const destination =
            patches + first_patch * row_elements + static_cast<std::int64_t>(channel) * kPatch * kPatch;

        for (int first = threadIdx.x; first < strip_vectors; first += kBlock * kUnroll) {
            Vec16 low[kUnroll];
            Vec16 high[kUnroll];
            std::int64_t destination_element[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                const int v = first + u * kBlock;
                const int patch_column = v / kChunkVectors; // power-of-two divisor
                const int q = v % kChunkVectors;
                const int local_row = q / PV;
                const int local_vector = q % PV;
                const std::int64_t source_element =
                    static_cast<std::int64_t>(local_row) * width + patch_column * kPatch +
                    local_vector * kVec;
                destination_element[u] = static_cast<std::int64_t>(patch_column) * row_elements +
                                         static_cast<std::int64_t>(q) * kVec;
                if (v < strip_vectors) {
                    low[u] = load16(source + source_element);
                    high[u] = load16(source + source_element + 4);
                }
            }
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
                if (first + u * kBlock < strip_vectors) {
                    const Vec16 packed{{pack_bf16x2(__uint_as_float(low[u].w[0]), __uint_as_float(low[u].w[1])),
                                        pack_bf16x2(__uint_as_float(low[u].w[2]), __uint_as_float(low[u].w[3])),
                                        pack_bf16x2(__uint_as_float(high[u].w[0]), __uint_as_float(high[u].w[1])),
                                        pack_bf16x2(__uint_as_float(high[u].w[2]), __uint_as_float(high[u].w[3]))}};
                    store16_streaming(destination + destination_element[u], packed);
                }
            }
        }
    }
}

/// Pair kernel: fp32, three channels, 16 x 16 patches, an even number of patch
/// columns (ViT/16 at 224). One wavefront per task, a task being (image, patch
/// row, pair of adjacent patch columns). The task's source is 48 row units
/// (channel c, line ly) of 32 floats, the two patches' lines side by side: one
/// whole 128-byte cache line, read by the 8 lanes of one unit. Lane l reads 16
/// bytes of unit (8 j + l / 8) at 16 (l % 8) bytes; its destination is the same
/// line of one of the two patches, so each load instruction moves 8 whole
/// cache lines and each store writes two runs of 512 contiguous bytes.
///
/// bf16 keeps the strip kernel: there a unit is half a cache line, whose other
/// half belongs to the next task, which the dispatcher gives to another XCD,
/// so both XCDs fetch the line (11.1-11.8 us against 9.1 us for the strip
/// kernel at ViT-Base batch 64, where the strip's workgroup reads both halves).
///
/// The grid is half the task count and each wavefront takes tasks t and
/// t + grid, with the second task's loads issued before the first task's
/// stores. The compiler then paces each store on the completion of an older
/// load or store (at most five outstanding after the twelve loads of an fp32
/// pair), which keeps the read stream ahead of the write stream: at ViT-Tiny
/// batch 32 this took the gather from 8.87 us (strip kernel) to 7.52 us on one
/// MI355X, where a same-bytes copy took 7.72 us. The same loads and stores
/// issued in one batch (all loads, then all stores) took 8.25-8.60 us.
///
/// @tparam kHeight, kWidth the image geometry when known at compile time (224 x 224,
///   ViT/16's), 0 for the runtime arguments: with constants the task's index
///   math becomes shifts and multiplies by constants instead of divisions and
///   32-bit multiplies by runtime values, all of it ahead of the first loads.
template <int kHeight, int kWidth>
__global__ __launch_bounds__(kWave) void extract_patches_pair_kernel(
    const unsigned char* __restrict__ images, unsigned char* __restrict__ patches,
    int height_argument, int width_argument, int tasks) {
    const int height = kHeight > 0 ? kHeight : height_argument;
    const int width = kWidth > 0 ? kWidth : width_argument;
    constexpr int kChannels = 3;
    constexpr int kPatch = 16;
    constexpr int kElement = 4;
    constexpr int kLanesPerUnit = 8;  // 2 patches x 4 vectors of one line
    constexpr int kUnitsPerLoad = kWave / kLanesPerUnit;
    constexpr int kLoads = kChannels * kPatch / kUnitsPerLoad;

    const int lane = static_cast<int>(threadIdx.x);
    const int k = lane % kLanesPerUnit;
    const int half = k / 4;
    const int vector = k % 4;
    const int unit_in_load = lane / kLanesPerUnit;
    const int across = width / kPatch;
    const int down = height / kPatch;
    const int pairs = across / 2;
    const std::int64_t row_bytes = static_cast<std::int64_t>(width) * kElement;
    const std::int64_t patch_row_bytes = static_cast<std::int64_t>(kChannels) * kPatch * kPatch *
                                         kElement;

    std::int64_t source[kLoads];
    std::int64_t target[kLoads];
    auto locate = [&](int task, std::int64_t* from, std::int64_t* to) {
        const int band = task / pairs;  // image * down + patch row
        const int pair = task - band * pairs;
        const int image = band / down;
        const int patch_row = band - image * down;
        const std::int64_t patch = static_cast<std::int64_t>(band) * across + 2 * pair + half;
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            const int unit = j * kUnitsPerLoad + unit_in_load;
            const int channel = unit / kPatch;
            const int line = unit % kPatch;
            from[j] = ((static_cast<std::int64_t>(image) * kChannels + channel) * height +
                       patch_row * kPatch + line) *
                          row_bytes +
                      static_cast<std::int64_t>(2 * pair) * kPatch * kElement + k * 16;
            to[j] = patch * patch_row_bytes + (channel * kPatch + line) * kPatch * kElement +
                    vector * 16;
        }
    };

    int task = static_cast<int>(blockIdx.x);
    if (task >= tasks) {
        return;
    }
    Vec16 value[kLoads];
    locate(task, source, target);
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
        value[j] = load16(images + source[j]);
    }
    for (;;) {
        const int next = task + static_cast<int>(gridDim.x);  // tasks < 2^31 - grid
        const bool more = next < tasks;
        std::int64_t next_source[kLoads];
        std::int64_t next_target[kLoads];
        Vec16 next_value[kLoads];
        if (more) {
            locate(next, next_source, next_target);
#pragma unroll
            for (int j = 0; j < kLoads; ++j) {
                next_value[j] = load16(images + next_source[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            store16_streaming(patches + target[j], value[j]);
        }
        if (!more) {
            break;
        }
#pragma unroll
        for (int j = 0; j < kLoads; ++j) {
            value[j] = next_value[j];
            target[j] = next_target[j];
        }
        task = next;
    }
}

/// The gather of 224-wide bf16 images in 16 x 16 patches (ViT/16's bf16
/// input) through LDS. A strip (image, channel, patch row) is 16 image rows,
/// one contiguous line-aligned span of 7 KiB, and its destination is 14 patch
/// blocks of 512 contiguous bytes: thread t loads vector t of the strip (each
/// load instruction eight whole 128-byte lines), writes it to its block's
/// place in LDS, and after a barrier stores vector t of the blocks (four whole
/// lines per block). The strip kernel reads 64-byte halves of 16 lines per
/// instruction, at half the per-CU load rate, and at ViT-Base batch 64 took
/// 9.1 us against 8.1 us for a same-bytes copy. LDS blocks are padded to 34
/// vectors, which spreads a wavefront's scattered 16-byte writes over the
/// banks. Workgroups are persistent and take kStrips strips per turn; the next
/// turn's loads are issued before this turn's stores (LDS double-buffered), so
/// each CU keeps reading while it writes. Measured at ViT-Base batch 64 over
/// cold buffers, one box, strips per turn x workgroups per CU (45.7 KiB of LDS
/// a workgroup at three strips): 3 x 3 7.7 us, 4 x 2 8.0, 3 x 4 8.4, 1 x 6-8
/// 8.8, 2 x 2-5 8.7-9.1, 3 x 2 9.5, 5 x 1 10.8; earlier, plain loads instead
/// of non-temporal ones 8.4 against 7.8-7.9 us at 4 x 2.
template <int kStrips>
__global__ __launch_bounds__(448) void extract_patches_staged_bf16_kernel(
    const unsigned char* __restrict__ images, unsigned char* __restrict__ patches, int channels,
    int patches_down, std::int64_t strips) {
    constexpr int kPatch = 16;
    constexpr int kWidth = 224;
    constexpr int kVec = 8;                               // bf16 per 16-byte vector
    constexpr int kPatchVectors = kPatch / kVec;          // 2 per patch row
    constexpr int kRowVectors = kWidth / kVec;            // 28 per image row
    constexpr int kStripVectors = kPatch * kRowVectors;   // 448 = the workgroup
    constexpr int kBlockVectors = kPatch * kPatchVectors; // 32 per 16 x 16 block
    constexpr int kPitch = kBlockVectors + 2;
    constexpr int kAcross = kWidth / kPatch;              // 14 blocks per strip
    __shared__ Vec16 staged[2][kStrips][kAcross * kPitch];

    const int t = static_cast<int>(threadIdx.x);
    const int row = t / kRowVectors;
    const int x = t - row * kRowVectors;
    const int slot = (x / kPatchVectors) * kPitch + row * kPatchVectors + x % kPatchVectors;
    const int block = t / kBlockVectors;
    const int q = t - block * kBlockVectors;
    const std::int64_t row_bytes = static_cast<std::int64_t>(channels) * kPatch * kPatch * 2;
    const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * kStrips;

    // A strip's source is strip * 16 image rows from the start: the planes'
    // rows follow one another and each plane holds its strips in order.
    Vec16 value[kStrips];
    auto load = [&](std::int64_t first) {
#pragma unroll
        for (int s = 0; s < kStrips; ++s) {
            if (first + s < strips) {
                value[s] = load16_streaming(images + ((first + s) * kStripVectors + t) * 16);
            }
        }
    };
    std::int64_t first = static_cast<std::int64_t>(blockIdx.x) * kStrips;
    if (first >= strips) {
        return;  // the whole workgroup, before any barrier
    }
    load(first);
    for (int buffer = 0; first < strips; first += stride, buffer ^= 1) {
#pragma unroll
        for (int s = 0; s < kStrips; ++s) {
            staged[buffer][s][slot] = value[s];
        }
        // Everyone's writes of this turn in; the other buffer's reads (the
        // previous turn) done before the turn after rewrites it.
        __syncthreads();
        if (first + stride < strips) {
            load(first + stride);
        }
#pragma unroll
        for (int s = 0; s < kStrips; ++s) {
            const std::int64_t strip = first + s;
            if (strip < strips) {
                const std::int64_t plane = strip / patches_down;  // image * channels + channel
                const std::int64_t patch_row = strip - plane * patches_down;
                const std::int64_t image = plane / channels;
                const std::int64_t channel = plane - image * channels;
                const std::int64_t patch = (image * patches_down + patch_row) * kAcross + block;
                store16_streaming(patches + patch * row_bytes + channel * (kPatch * kPatch * 2) + q * 16,
                                  staged[buffer][s][block * kPitch + q]);
            }
        }
    }
}

/// Stores one gathered value: as it is, or an fp32 value rounded to bf16 bits.
__device__ __forceinline__ void store_value(std::uint32_t* out, std::uint32_t word) { *out = word; }
__device__ __forceinline__ void store_value(std::uint16_t* out, std::uint16_t word) { *out = word; }
__device__ __forceinline__ void store_value(std::uint16_t* out, float value) {
    *out = float_to_bf16(value);
}

/// One element per iteration, any geometry and alignment. @p In and @p Out
/// are the same word (a bit-exact move) or fp32 in and bf16 bits out.
template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void extract_patches_element_kernel(
    const In* __restrict__ images, Out* __restrict__ patches, int channels, int height,
    int width, int patch, std::int64_t total) {
    const std::int64_t patch_area = static_cast<std::int64_t>(patch) * patch;
    const std::int64_t row_length = channels * patch_area;
    const int patches_across = width / patch;
    const int patches_per_image = (height / patch) * patches_across;
    const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * kBlock;

    for (std::int64_t index = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
         index < total; index += stride) {
        const std::int64_t global_patch = index / row_length;
        const std::int64_t element = index - global_patch * row_length;
        const std::int64_t image = global_patch / patches_per_image;
        const int patch_index = static_cast<int>(global_patch - image * patches_per_image);
        const int channel = static_cast<int>(element / patch_area);
        const int within = static_cast<int>(element - channel * patch_area);
        const int local_row = within / patch;
        const int local_column = within - local_row * patch;
        const int patch_row = patch_index / patches_across;
        const int patch_column = patch_index - patch_row * patches_across;

        const std::int64_t source =
            ((image * channels + channel) * height + patch_row * patch + local_row) *
                static_cast<std::int64_t>(width) +
            patch_column * patch + local_column;
        store_value(patches + index, images[source]);
    }
}

__global__ __launch_bounds__(kBlock) void broadcast_vector_kernel(
    float4* __restrict__ destination, const float4* __restrict__ source, std::int64_t vectors,
    std::int64_t destination_stride_vectors, int batch) {
    for (std::int64_t slot = blockIdx.y; slot < batch; slot += gridDim.y) {
        float4* const target = destination + slot * destination_stride_vectors;
        for (std::int64_t v = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
             v < vectors; v += static_cast<std::int64_t>(gridDim.x) * kBlock) {
            target[v] = source[v];
        }
    }
}

template <typename Word>
__global__ __launch_bounds__(kBlock) void broadcast_element_kernel(
    Word* __restrict__ destination, const Word* __restrict__ source, std::int64_t count,
    std::int64_t destination_stride, int batch) {
    for (std::int64_t slot = blockIdx.y; slot < batch; slot += gridDim.y) {
        Word* const target = destination + slot * destination_stride;
        for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
             i < count; i += static_cast<std::int64_t>(gridDim.x) * kBlock) {
            target[i] = source[i];
        }
    }
}

__global__ __launch_bounds__(kBlock) void add_broadcast_vector_kernel(
    float4* __restrict__ accumulator, const float4* __restrict__ addend, std::int64_t vectors,
    int batch) {
    for (std::int64_t v = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
         v < vectors; v += static_cast<std::int64_t>(gridDim.x) * kBlock) {
        const float4 a = addend[v];
        for (std::int64_t slot = blockIdx.y; slot < batch; slot += gridDim.y) {
            float4* const target = accumulator + slot * vectors + v;
            Vec16 t = load16_streaming(target);
            t.w[0] = __float_as_uint(__uint_as_float(t.w[0]) + a.x);
            t.w[1] = __float_as_uint(__uint_as_float(t.w[1]) + a.y);
            t.w[2] = __float_as_uint(__uint_as_float(t.w[2]) + a.z);
            t.w[3] = __float_as_uint(__uint_as_float(t.w[3]) + a.w);
            store16_streaming(target, t);
        }
    }
}

__global__ __launch_bounds__(kBlock) void add_broadcast_element_kernel(
    float* __restrict__ accumulator, const float* __restrict__ addend, std::int64_t count,
    int batch) {
    for (std::int64_t i = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < count;
         i += static_cast<std::int64_t>(gridDim.x) * kBlock) {
        const float a = addend[i];
        for (std::int64_t slot = blockIdx.y; slot < batch; slot += gridDim.y) {
            accumulator[slot * count + i] += a;
        }
    }
}

constexpr int kStripBlocksPerCu = 8;
constexpr std::int64_t kMaxGridY = 65535;

/// (x, y) grid for the slot kernels: x covers the @p units of one slot, y the
/// slots, with x * y bounded by a few dozen blocks per compute unit. Both
/// kernels loop over whatever the grid does not cover.
dim3 slot_grid(std::int64_t units, int batch) {
    const std::int64_t budget = static_cast<std::int64_t>(compute_units()) * 32;
    std::int64_t x = (units + kBlock - 1) / kBlock;
    x = x < budget ? x : budget;
    std::int64_t y = budget / x;
    y = y < batch ? y : batch;
    y = y < kMaxGridY ? y : kMaxGridY;
    y = y > 0 ? y : 1;
    return dim3(static_cast<unsigned int>(x), static_cast<unsigned int>(y));
}

template <int ElementSize, int PV>
hipError_t launch_strips(const void* images, void* patches, int batch, int channels, int height,
                         int width, hipStream_t stream) {
    constexpr int kPatch = PV * 16 / ElementSize;
    const std::int64_t strips =
        static_cast<std::int64_t>(batch) * channels * (height / kPatch);
    const unsigned int grid = stride_grid(strips, 1, kStripBlocksPerCu);
    extract_patches_strip_kernel<ElementSize, PV><<<grid, kBlock, 0, stream>>>(
        static_cast<const unsigned char*>(images), static_cast<unsigned char*>(patches), channels,
        height, width, strips);
    return hipGetLastError();
}

template <int ElementSize>
hipError_t dispatch_patches(const void* images, void* patches, int batch, int channels, int height,
                            int width, int patch, hipStream_t stream) {
    constexpr int kVec = 16 / ElementSize;
    if (ElementSize == 4 && aligned16(images) && aligned16(patches) && channels == 3 &&
        patch == 16 && (width / 16) % 2 == 0) {
        const std::int64_t tasks = static_cast<std::int64_t>(batch) * (height / 16) * (width / 32);
        // Task indices, and a task plus the grid, stay below 2^31.
        if (tasks <= 0x3fffffff) {
            const std::int64_t grid = (tasks + 1) / 2;  // two tasks per wavefront
            auto kernel = height == 224 && width == 224 ? extract_patches_pair_kernel<224, 224>
                                                        : extract_patches_pair_kernel<0, 0>;
            kernel<<<static_cast<unsigned int>(grid), kWave, 0, stream>>>(
                static_cast<const unsigned char*>(images), static_cast<unsigned char*>(patches),
                height, width, static_cast<int>(tasks));
            return hipGetLastError();
        }
    }
    if (ElementSize == 2 && aligned16(images) && aligned16(patches) && patch == 16 && width == 224) {
        constexpr int kStrips = 3;
        const std::int64_t strips = static_cast<std::int64_t>(batch) * channels * (height / 16);
        const std::int64_t groups = (strips + kStrips - 1) / kStrips;
        const std::int64_t cap = static_cast<std::int64_t>(compute_units()) * 3;
        const unsigned int grid = static_cast<unsigned int>(groups < cap ? groups : cap);
        extract_patches_staged_bf16_kernel<kStrips><<<grid, 448, 0, stream>>>(
            static_cast<const unsigned char*>(images), static_cast<unsigned char*>(patches), channels,
            height / 16, strips);
        return hipGetLastError();
    }
    if (aligned16(images) && aligned16(patches) && patch % kVec == 0) {
        switch (patch / kVec) {
        case 1: return launch_strips<ElementSize, 1>(images, patches, batch, channels, height, width, stream);
        case 2: return launch_strips<ElementSize, 2>(images, patches, batch, channels, height, width, stream);
        case 4: return launch_strips<ElementSize, 4>(images, patches, batch, channels, height, width, stream);
        case 8: return launch_strips<ElementSize, 8>(images, patches, batch, channels, height, width, stream);
        default: break;
        }
    }
    using Word = std::conditional_t<ElementSize == 4, std::uint32_t, std::uint16_t>;
    const std::int64_t total = static_cast<std::int64_t>(batch) * channels * height * width;
    const unsigned int grid = stride_grid(total, kBlock, 16);
    extract_patches_element_kernel<Word, Word><<<grid, kBlock, 0, stream>>>(
        static_cast<const Word*>(images), static_cast<Word*>(patches), channels, height, width,
        patch, total);
    return hipGetLastError();
}

} // namespace

hipError_t extract_patches_f32_to_bf16(const float* images, std::uint16_t* patches, int batch,
                                      int channels, int height, int width, int patch,
                                      hipStream_t stream) {
    if (!aligned16(images) || !aligned16(patches) || patch % 8 != 0 || width % 8 != 0) {
        return hipErrorNotSupported;
    }
    const std::int64_t strips = static_cast<std::int64_t>(batch) * channels * (height / patch);
    const unsigned int grid = stride_grid(strips, 1, kStripBlocksPerCu);
    auto run = [&](auto kernel) {
        kernel<<<grid, kBlock, 0, stream>>>(images, patches, channels, height, width, strips);
        return hipGetLastError();
    };
    switch (patch / 8) {
    case 1: return run(extract_patches_strip_f32_to_bf16_kernel<1>);
    case 2: return run(extract_patches_strip_f32_to_bf16_kernel<2>);
    case 4: return run(extract_patches_strip_f32_to_bf16_kernel<4>);
    case 8: return run(extract_patches_strip_f32_to_bf16_kernel<8>);
    default: return hipErrorNotSupported;
    }
}

hipError_t extract_patches_f32_to_bf16_any(const float* images, std::uint16_t* patches, int batch,
                                          int channels, int height, int width, int patch,
                                          hipStream_t stream) {
    const hipError_t strips = extract_patches_f32_to_bf16(images, patches, batch, channels, height,
                                                          width, patch, stream);
    if (strips != hipErrorNotSupported) {
        return strips;
    }
    const std::int64_t total = static_cast<std::int64_t>(batch) * channels * height * width;
    const unsigned int grid = stride_grid(total, kBlock, 16);
    extract_patches_element_kernel<float, std::uint16_t><<<grid, kBlock, 0, stream>>>(
        images, patches, channels, height, width, patch, total);
    return hipGetLastError();
}

hipError_t extract_patches(const void* images, void* patches, int element_size, int batch,
                           int channels, int height, int width, int patch, hipStream_t stream) {
    if (element_size == 4) {
        return dispatch_patches<4>(images, patches, batch, channels, height, width, patch, stream);
    }
    return dispatch_patches<2>(images, patches, batch, channels, height, width, patch, stream);
}

namespace {

/// The broadcast is a copy, so it is typed only by the element (Word).
template <typename Word>
hipError_t broadcast(Word* destination, const Word* source, std::int64_t count,
                     std::int64_t destination_stride, int batch, hipStream_t stream) {
    constexpr std::int64_t kVec = 16 / sizeof(Word);
    if (count % kVec == 0 && destination_stride % kVec == 0 && aligned16(destination) &&
        aligned16(source)) {
        const std::int64_t vectors = count / kVec;
        const dim3 grid = slot_grid(vectors, batch);
        broadcast_vector_kernel<<<grid, kBlock, 0, stream>>>(
            reinterpret_cast<float4*>(destination), reinterpret_cast<const float4*>(source),
            vectors, destination_stride / kVec, batch);
    } else {
        const dim3 grid = slot_grid(count, batch);
        broadcast_element_kernel<Word><<<grid, kBlock, 0, stream>>>(destination, source, count,
                                                                    destination_stride, batch);
    }
    return hipGetLastError();
}

} // namespace

hipError_t broadcast_f32(float* destination, const float* source, std::int64_t count,
                         std::int64_t destination_stride, int batch, hipStream_t stream) {
    return broadcast(destination, source, count, destination_stride, batch, stream);
}

hipError_t broadcast_bf16(std::uint16_t* destination, const std::uint16_t* source,
                          std::int64_t count, std::int64_t destination_stride, int batch,
                          hipStream_t stream) {
    return broadcast(destination, source, count, destination_stride, batch, stream);
}

hipError_t add_broadcast_f32(float* accumulator, const float* addend, std::int64_t count, int batch,
                             hipStream_t stream) {
    if (count % 4 == 0 && aligned16(accumulator) && aligned16(addend)) {
        const std::int64_t vectors = count / 4;
        const dim3 grid = slot_grid(vectors, batch);
        add_broadcast_vector_kernel<<<grid, kBlock, 0, stream>>>(
            reinterpret_cast<float4*>(accumulator), reinterpret_cast<const float4*>(addend),
            vectors, batch);
    } else {
        const dim3 grid = slot_grid(count, batch);
        add_broadcast_element_kernel<<<grid, kBlock, 0, stream>>>(accumulator, addend, count,
                                                                  batch);
    }
    return hipGetLastError();
}

} // namespace cuvit::detail
