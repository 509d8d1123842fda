// Row softmax for gfx950.
//
// Semantics follow the reference launcher (include/cuvit/kernels.hpp:120-123)
// and its CPU path (tests/reference/linear_algebra.hpp:98-118): per row,
// exp(x - max) / sum(exp(x - max)). input == output is allowed; the model runs
// it in place over the attention logits (src/model/vit.cu:225).
//
// Register path (rows up to 64 * kMaxTerms columns). One wavefront owns a row
// at a time: lane l holds columns l, l + 64, l + 128, ... as its terms, loaded
// straight from HBM (consecutive lanes read consecutive elements, so each load
// instruction is one contiguous 256-byte span for fp32). The row stays in
// registers from the max through the exponentials to the scaled store, so HBM
// sees exactly one read and one write per element. Rows of 197 floats are not
// 16-byte aligned, and measured on MI355X this per-element layout beats both
// staging 4-row blocks through LDS as aligned dwordx4 traffic and one block of
// rows per single-wave workgroup, because it keeps more rows in flight per CU.
//
// The reduction order is fixed by column index alone: column c is lane
// c % 64's (c / 64)-th term, then the fixed wavefront tree combines the lanes.
// A row therefore gives the same bits wherever it sits in a launch, which is
// what keeps a batch bitwise equal to its images run one at a time.
//
// Exponentials are exp2((x - max) * log2(e)) on the hardware exp2. x - max is
// exact at x = max, where the largest outputs sit, and the relative error of an
// exponential grows only with |x - max| (about |x - max| * 2^-23 plus the exp2
// unit's ~1 ulp), so it is largest where the output is smallest: under 1e-6
// absolute for every output, far inside the reference test's 1e-4 relative
// tolerance (tests/elementwise_test.cu:254-255).
//
// Streaming path (rows wider than the register path holds): one wavefront per
// row with an online max: a single streaming pass keeps a running (max, sum)
// per lane, rescaling the sum when the max grows, the lanes are merged, and a
// second pass writes the result.
#include "device_common.hpp"
#include "launch.hpp"

#include <cmath>

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;
constexpr float kLog2e = 1.4426950408889634F;

/// Rows the register path holds: up to 64 * kMaxTerms columns.
constexpr int kMaxTerms = 16;

/// exp(x - max).
__device__ __forceinline__ float shifted_exp(float x, float max) {
    return __builtin_amdgcn_exp2f((x - max) * kLog2e);
}

template <typename T, int J>
__global__ __launch_bounds__(kBlock) void softmax_rows_kernel(const T* input, T* output, int rows,
                                                              int columns) {
    const int lane = lane_id();
    const std::int64_t waves = static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock;

    for (std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock +
                            threadIdx.x / kWave;
         row < rows; row += waves) {
        const T* const source = input + row * columns;
        T* const destination = output + row * columns;

        float x[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int column = lane + kWave * j;
            x[j] = column < columns ? Elem<T>::load(source + column) : -INFINITY;
        }

        float maximum = x[0];
#pragma unroll
        for (int j = 1; j < J; ++j) {
            maximum = fmaxf(maximum, x[j]);
        }
        const float row_maximum = wave_allreduce(maximum, Max{});

        float sum = 0.F;
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int column = lane + kWave * j;
            x[j] = column < columns ? shifted_exp(x[j], row_maximum) : 0.F;
            sum += x[j];
        }
        const float inverse = 1.0F / wave_allreduce(sum, Sum{});

#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int column = lane + kWave * j;
            if (column < columns) {
                Elem<T>::store(destination + column, x[j] * inverse);
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void softmax_online_kernel(const T* input, T* output, int rows,
                                                                int columns) {
    const int lane = lane_id();
    const std::int64_t waves = static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock;
    for (std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock +
                            threadIdx.x / kWave;
         row < rows; row += waves) {
        const T* const source = input + row * columns;
        T* const destination = output + row * columns;

        float maximum = -INFINITY;
        float sum = 0.F;
        for (int column = lane; column < columns; column += kWave) {
            const float value = Elem<T>::load(source + column);
            if (value > maximum) {
                sum = sum * shifted_exp(maximum, value) + 1.0F;
                maximum = value;
            } else if (value != -INFINITY) {
                sum += shifted_exp(value, maximum);
            }
        }
        const float row_maximum = wave_allreduce(maximum, Max{});
        const float scaled = sum == 0.F ? 0.F : sum * shifted_exp(maximum, row_maximum);
        const float inverse = 1.0F / wave_allreduce(scaled, Sum{});

        for (int column = lane; column < columns; column += kWave) {
            const float value = Elem<T>::load(source + column);
            Elem<T>::store(destination + column, shifted_exp(value, row_maximum) * inverse);
        }
    }
}

/// Workgroups per compute unit before the grid loops: 32 waves, the most a CU
/// holds at this kernel's register use, measured fastest at ViT shapes.
constexpr int kBlocksPerCu = 8;

template <typename T, int J>
hipError_t launch_rows(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    const unsigned int grid = stride_grid(rows, kWavesPerBlock, kBlocksPerCu);
    softmax_rows_kernel<T, J><<<grid, kBlock, 0, stream>>>(input, output, rows, columns);
    return hipGetLastError();
}

template <typename T>
hipError_t dispatch(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    if (columns <= kWave * kMaxTerms) {
        switch ((columns + kWave - 1) / kWave) {
        case 1: return launch_rows<T, 1>(input, output, rows, columns, stream);
        case 2: return launch_rows<T, 2>(input, output, rows, columns, stream);
        case 3: return launch_rows<T, 3>(input, output, rows, columns, stream);
        case 4: return launch_rows<T, 4>(input, output, rows, columns, stream);
        case 5:
        case 6: return launch_rows<T, 6>(input, output, rows, columns, stream);
        case 7:
        case 8: return launch_rows<T, 8>(input, output, rows, columns, stream);
        case 9:
        case 10:
        case 11:
        case 12: return launch_rows<T, 12>(input, output, rows, columns, stream);
        default: return launch_rows<T, 16>(input, output, rows, columns, stream);
        }
    }
    const unsigned int grid = stride_grid(rows, kWavesPerBlock, kBlocksPerCu);
    softmax_online_kernel<T><<<grid, kBlock, 0, stream>>>(input, output, rows, columns);
    return hipGetLastError();
}

} // namespace

hipError_t softmax_f32(const float* input, float* output, int rows, int columns,
                       hipStream_t stream) {
    return dispatch<float>(input, output, rows, columns, stream);
}

hipError_t softmax_bf16(const std::uint16_t* input, std::uint16_t* output, int rows, int columns,
                        hipStream_t stream) {
    return dispatch<std::uint16_t>(input, output, rows, columns, stream);
}

} // namespace cuvit::detail
