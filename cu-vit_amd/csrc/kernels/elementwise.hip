// Residual add, erf GELU and fp32 <-> bf16 conversion for gfx950.
//
// add:  accumulator[i] += addend[i]                (normalization.cu:148-154)
// gelu: 0.5 * x * (1 + erf(x / sqrt(2)))           (normalization.cu:138-146,
//       the erf form of nn.GELU(approximate='none'); CPU path
//       tests/reference/linear_algebra.hpp:120-129)
// A single fp32 add rounds identically everywhere, so add is bit-exact against
// the CPU. GELU is device_common.hpp's branch-free erfc form, shared with the
// GEMM epilogue so both give the same bits.
// convert: fp32 -> bf16 to nearest even, bf16 -> fp32 exactly; no counterpart
//       in the reference, used by the bf16 model at its fp32 input and output.
//
// All run as grid-stride loops over 16-byte vectors when the pointers are
// aligned, with the tail (count % elements-per-vector) handled by the first
// threads of the grid; unaligned pointers take a scalar loop.
#include "device_common.hpp"
#include "launch.hpp"

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

constexpr int kBlock = 256;
constexpr int kBlocksPerCu = 8;

__global__ __launch_bounds__(kBlock) void add_kernel(float* __restrict__ accumulator,
                                                     const float* __restrict__ addend,
                                                     std::int64_t count, bool vectorized) {
    const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * kBlock;
    const std::int64_t first = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    std::int64_t done = 0;
    if (vectorized) {
        const std::int64_t vectors = count / 4;
        for (std::int64_t v = first; v < vectors; v += stride) {
            float4 a = reinterpret_cast<float4*>(accumulator)[v];
            const float4 b = reinterpret_cast<const float4*>(addend)[v];
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
            reinterpret_cast<float4*>(accumulator)[v] = a;
        }
        done = vectors * 4;
    }
    for (std::int64_t i = done + first; i < count; i += stride) {
        accumulator[i] += addend[i];
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void gelu_kernel(const T* __restrict__ input,
                                                      T* __restrict__ output, std::int64_t count,
                                                      bool vectorized) {
    constexpr int E = Elem<T>::kPerVec;
    const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * kBlock;
    const std::int64_t first = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    std::int64_t done = 0;
    if (vectorized) {
        const std::int64_t vectors = count / E;
        for (std::int64_t v = first; v < vectors; v += stride) {
            const Vec16 x = load16(input + v * E);
            Vec16 y;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                Elem<T>::set(y, e, gelu(Elem<T>::get(x, e)));
            }
            store16(output + v * E, y);
        }
        done = vectors * E;
    }
    for (std::int64_t i = done + first; i < count; i += stride) {
        Elem<T>::store(output + i, gelu(Elem<T>::load(input + i)));
    }
}

/// output[i] = input[i] converted between fp32 and bf16 (round to nearest
/// even going down, exact going up). Eight elements per iteration when the
/// pointers are 16-byte aligned: one or two 16-byte loads in, two or one out.
template <typename In, typename Out>
__global__ __launch_bounds__(kBlock) void convert_kernel(const In* __restrict__ input,
                                                         Out* __restrict__ output,
                                                         std::int64_t count, bool vectorized) {
    constexpr int kGroup = 8;
    constexpr int kInVec = Elem<In>::kPerVec;
    constexpr int kOutVec = Elem<Out>::kPerVec;
    const std::int64_t stride = static_cast<std::int64_t>(gridDim.x) * kBlock;
    const std::int64_t first = static_cast<std::int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    std::int64_t done = 0;
    if (vectorized) {
        const std::int64_t groups = count / kGroup;
        for (std::int64_t g = first; g < groups; g += stride) {
            Vec16 x[kGroup / kInVec];
#pragma unroll
            for (int i = 0; i < kGroup / kInVec; ++i) {
                x[i] = load16(input + g * kGroup + i * kInVec);
            }
            Vec16 y[kGroup / kOutVec];
#pragma unroll
            for (int e = 0; e < kGroup; ++e) {
                Elem<Out>::set(y[e / kOutVec], e % kOutVec, Elem<In>::get(x[e / kInVec], e % kInVec));
            }
#pragma unroll
            for (int o = 0; o < kGroup / kOutVec; ++o) {
                store16(output + g * kGroup + o * kOutVec, y[o]);
            }
        }
        done = groups * kGroup;
    }
    for (std::int64_t i = done + first; i < count; i += stride) {
        Elem<Out>::store(output + i, Elem<In>::load(input + i));
    }
}

template <typename In, typename Out>
hipError_t convert(const In* input, Out* output, std::int64_t count, hipStream_t stream) {
    const bool vectorized = aligned16(input) && aligned16(output);
    const unsigned int grid = stride_grid(vectorized ? (count + 7) / 8 : count, kBlock, kBlocksPerCu);
    convert_kernel<In, Out><<<grid, kBlock, 0, stream>>>(input, output, count, vectorized);
    return hipGetLastError();
}

} // namespace

hipError_t convert_f32_to_bf16(const float* input, std::uint16_t* output, std::int64_t count,
                               hipStream_t stream) {
    return convert(input, output, count, stream);
}

hipError_t convert_bf16_to_f32(const std::uint16_t* input, float* output, std::int64_t count,
                               hipStream_t stream) {
    return convert(input, output, count, stream);
}

hipError_t add_f32(float* accumulator, const float* addend, std::int64_t count,
                   hipStream_t stream) {
    const bool vectorized = aligned16(accumulator) && aligned16(addend);
    const unsigned int grid = stride_grid(vectorized ? (count + 3) / 4 : count, kBlock, kBlocksPerCu);
    add_kernel<<<grid, kBlock, 0, stream>>>(accumulator, addend, count, vectorized);
    return hipGetLastError();
}

hipError_t gelu_f32(const float* input, float* output, std::int64_t count, hipStream_t stream) {
    const bool vectorized = aligned16(input) && aligned16(output);
    const unsigned int grid = stride_grid(vectorized ? (count + 3) / 4 : count, kBlock, kBlocksPerCu);
    gelu_kernel<float><<<grid, kBlock, 0, stream>>>(input, output, count, vectorized);
    return hipGetLastError();
}

hipError_t gelu_bf16(const std::uint16_t* input, std::uint16_t* output, std::int64_t count,
                     hipStream_t stream) {
    const bool vectorized = aligned16(input) && aligned16(output);
    const unsigned int grid = stride_grid(vectorized ? (count + 7) / 8 : count, kBlock, kBlocksPerCu);
    gelu_kernel<std::uint16_t><<<grid, kBlock, 0, stream>>>(input, output, count, vectorized);
    return hipGetLastError();
}

} // namespace cuvit::detail
