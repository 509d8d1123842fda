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
// Staged path (the same rows at large row counts). R rows of any width are
// `columns` 16-byte vectors (R = 4 fp32, 8 bf16), so each wavefront moves an
// R-row block between HBM and a wave-private LDS tile with aligned dwordx4
// traffic and reduces each row out of LDS in the same lane / term order and
// with the same arithmetic as the register path, so both paths give the same
// bits for a row. Which one runs depends only on the row count (measured:
// the register path wins at ViT-Tiny batch 32, the staged path from ViT-Base
// batch 64 up, 43 us vs 55 us for [151296, 197] bf16).
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

template <typename T, int J>
__global__ __launch_bounds__(kBlock) void softmax_staged_kernel(const T* input, T* output, int rows,
                                                                int columns) {
    constexpr int R = Elem<T>::kPerVec;
    extern __shared__ Vec16 lds[];
    const int lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    Vec16* const tile = lds + wave * columns;
    T* const tile_elements = reinterpret_cast<T*>(tile);
    const std::int64_t blocks = (static_cast<std::int64_t>(rows) + R - 1) / R;

    // Every wavefront of the workgroup runs the same iterations (a block past
    // the end is simply empty), so the barriers below are uniform.
    for (std::int64_t base = static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock; base < blocks;
         base += static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock) {
        const std::int64_t block = base + wave;
        const std::int64_t first_row = block * R;
        const int rows_here =
            block < blocks ? static_cast<int>(rows - first_row < R ? rows - first_row : R) : 0;
        const T* const source = input + first_row * columns;
        T* const destination = output + first_row * columns;

        if (rows_here == R) {
            for (int v = lane; v < columns; v += kWave) {
                tile[v] = load16(source + static_cast<std::int64_t>(v) * R);
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
            const float row_maximum = wave_allreduce(maximum, Max{});
            float sum = 0.F;
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = lane + kWave * j;
                x[r][j] = column < columns ? shifted_exp(x[r][j], row_maximum) : 0.F;
                sum += x[r][j];
            }
            inverse[r] = 1.0F / wave_allreduce(sum, Sum{});
        }
        __syncthreads();

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
                store16(destination + static_cast<std::int64_t>(v) * R, tile[v]);
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

/// Row counts from which the staged path is used: more than four rows per
/// wavefront once every compute unit is full.
std::int64_t staged_threshold() { return static_cast<std::int64_t>(compute_units()) * 128; }

template <typename T, int J>
hipError_t launch_rows(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    constexpr int R = Elem<T>::kPerVec;
    if (rows >= staged_threshold() && aligned16(input) && aligned16(output)) {
        const std::int64_t blocks = (static_cast<std::int64_t>(rows) + R - 1) / R;
        const unsigned int grid = stride_grid(blocks, kWavesPerBlock, kBlocksPerCu);
        const std::size_t lds = static_cast<std::size_t>(kWavesPerBlock) * columns * sizeof(Vec16);
        softmax_staged_kernel<T, J><<<grid, kBlock, lds, stream>>>(input, output, rows, columns);
        return hipGetLastError();
    }
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
