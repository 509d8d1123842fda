// Row softmax for gfx950.
//
// Semantics follow the reference launcher (include/cuvit/kernels.hpp:120-123)
// and its CPU path (tests/reference/linear_algebra.hpp:98-118): per row,
// exp(x - max) / sum(exp(x - max)). input == output is allowed; the model runs
// it in place over the attention logits (src/model/vit.cu:225).
//
// Fast path. A 197-wide fp32 row is 788 bytes, so rows do not start on 16-byte
// boundaries, but four consecutive rows are 197 float4 exactly (eight rows for
// bf16). One wavefront owns such a block: it reads it with aligned dwordx4
// loads into LDS, reduces each row out of LDS and writes the block back with
// dwordx4 stores. The row stays in registers between the max and the sum, so
// HBM sees one read and one write per element.
//
// The reduction order is fixed by column index alone: column c is handled by
// lane c % 64 as its (c / 64)-th term, then the fixed wavefront tree combines
// the lanes. A row therefore gives the same bits wherever it sits in a launch,
// which is what keeps a batch bitwise equal to its images run one at a time.
//
// Generic path (unaligned pointers or rows wider than the fast path holds):
// one wavefront per row with an online max: a single streaming pass keeps a
// running (max, sum) per lane, rescaling the sum when the max grows, the lanes
// are merged, and a second pass writes the result.
#include "device_common.hpp"
#include "launch.hpp"

#include <cmath>

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

/// Exponential used for each element: the accurate one for fp32 output, the
/// hardware exp2 for bf16, whose output rounding dominates either way.
template <typename T> __device__ __forceinline__ float element_exp(float x);
template <> __device__ __forceinline__ float element_exp<float>(float x) { return expf(x); }
template <> __device__ __forceinline__ float element_exp<std::uint16_t>(float x) {
    return __expf(x);
}

/// Rows whose softmax fits the fast path: up to 64 * kMaxTerms columns.
constexpr int kMaxTerms = 16;

template <typename T, int J>
__global__ __launch_bounds__(kWave) void softmax_block_kernel(const T* input, T* output,
                                                              int rows, int columns) {
    constexpr int E = Elem<T>::kPerVec;
    constexpr int R = E; // rows per block: R rows of any width are `columns` vectors
    extern __shared__ Vec16 tile[];
    T* const tile_elements = reinterpret_cast<T*>(tile);

    const int lane = lane_id();
    const std::int64_t blocks = (static_cast<std::int64_t>(rows) + R - 1) / R;

    for (std::int64_t block = blockIdx.x; block < blocks; block += gridDim.x) {
        const std::int64_t first_row = block * R;
        const int rows_here = static_cast<int>(
            rows - first_row < R ? rows - first_row : static_cast<std::int64_t>(R));
        const T* const source = input + first_row * columns;
        T* const destination = output + first_row * columns;

        if (rows_here == R) {
            for (int v = lane; v < columns; v += kWave) {
                tile[v] = load16(source + static_cast<std::int64_t>(v) * E);
            }
        } else {
            for (int i = lane; i < rows_here * columns; i += kWave) {
                tile_elements[i] = source[i];
            }
        }
        __syncthreads();

        float x[R][J];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = lane + kWave * j;
                x[r][j] = (r < rows_here && column < columns)
                              ? Elem<T>::load(tile_elements + r * columns + column)
                              : -INFINITY;
            }
        }

        float inverse[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float maximum = x[r][0];
#pragma unroll
            for (int j = 1; j < J; ++j) {
                maximum = fmaxf(maximum, x[r][j]);
            }
            maximum = wave_allreduce(maximum, Max{});

            float sum = 0.F;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = lane + kWave * j;
                x[r][j] = column < columns ? element_exp<T>(x[r][j] - maximum) : 0.F;
                sum += x[r][j];
            }
            inverse[r] = 1.0F / wave_allreduce(sum, Sum{});
        }

#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (r < rows_here) {
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int column = lane + kWave * j;
                    if (column < columns) {
                        Elem<T>::store(tile_elements + r * columns + column, x[r][j] * inverse[r]);
                    }
                }
            }
        }
        __syncthreads();

        if (rows_here == R) {
            for (int v = lane; v < columns; v += kWave) {
                store16(destination + static_cast<std::int64_t>(v) * E, tile[v]);
            }
        } else {
            for (int i = lane; i < rows_here * columns; i += kWave) {
                destination[i] = tile_elements[i];
            }
        }
        __syncthreads();
    }
}

template <typename T>
__global__ __launch_bounds__(kWave) void softmax_online_kernel(const T* input, T* output, int rows,
                                                               int columns) {
    const int lane = lane_id();
    for (std::int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const T* const source = input + row * columns;
        T* const destination = output + row * columns;

        float maximum = -INFINITY;
        float sum = 0.F;
        for (int column = lane; column < columns; column += kWave) {
            const float value = Elem<T>::load(source + column);
            if (value > maximum) {
                sum = sum * element_exp<T>(maximum - value) + 1.0F;
                maximum = value;
            } else if (value != -INFINITY) {
                sum += element_exp<T>(value - maximum);
            }
        }
        const float row_maximum = wave_allreduce(maximum, Max{});
        const float scaled = sum == 0.F ? 0.F : sum * element_exp<T>(maximum - row_maximum);
        const float inverse = 1.0F / wave_allreduce(scaled, Sum{});

        for (int column = lane; column < columns; column += kWave) {
            const float value = Elem<T>::load(source + column);
            Elem<T>::store(destination + column, element_exp<T>(value - row_maximum) * inverse);
        }
    }
}

/// Single-wave workgroups resident per compute unit before the grid loops.
constexpr int kBlocksPerCu = 32;

template <typename T, int J>
hipError_t launch_block(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    constexpr int R = Elem<T>::kPerVec;
    const std::int64_t blocks = (static_cast<std::int64_t>(rows) + R - 1) / R;
    const unsigned int grid = stride_grid(blocks, 1, kBlocksPerCu);
    const std::size_t lds = static_cast<std::size_t>(columns) * sizeof(Vec16);
    softmax_block_kernel<T, J><<<grid, kWave, lds, stream>>>(input, output, rows, columns);
    return hipGetLastError();
}

template <typename T>
hipError_t dispatch(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    if (aligned16(input) && aligned16(output) && columns <= kWave * kMaxTerms) {
        switch ((columns + kWave - 1) / kWave) {
        case 1: return launch_block<T, 1>(input, output, rows, columns, stream);
        case 2: return launch_block<T, 2>(input, output, rows, columns, stream);
        case 3: return launch_block<T, 3>(input, output, rows, columns, stream);
        case 4: return launch_block<T, 4>(input, output, rows, columns, stream);
        case 5:
        case 6: return launch_block<T, 6>(input, output, rows, columns, stream);
        case 7:
        case 8: return launch_block<T, 8>(input, output, rows, columns, stream);
        case 9:
        case 10:
        case 11:
        case 12: return launch_block<T, 12>(input, output, rows, columns, stream);
        default: return launch_block<T, 16>(input, output, rows, columns, stream);
        }
    }
    const unsigned int grid = stride_grid(rows, 1, kBlocksPerCu);
    softmax_online_kernel<T><<<grid, kWave, 0, stream>>>(input, output, rows, columns);
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
