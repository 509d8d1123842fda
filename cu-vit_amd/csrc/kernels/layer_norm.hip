// Row-wise LayerNorm for gfx950.
//
// Semantics follow the reference launcher (include/cuvit/kernels.hpp:101-109)
// and its CPU path (tests/reference/linear_algebra.hpp:70-96):
//   out[r][c] = (in[r][c] - mean) / sqrt(var + eps) * gamma[c] + beta[c]
// with the biased variance.
//
// Fast path (the ViT shapes): a team of 16 or 64 lanes owns one row and keeps
// it in registers as 16-byte vectors, so the row is read from HBM once and
// written once (non-temporal loads and stores through the C ABI, plain ones
// inside the model, whose next GEMM reads the rows from the caches); the two
// statistics passes run over VGPRs.
// A 192-wide fp32 row is 16 lanes x 3 float4, four rows per wavefront.
//
// Numerics: deviations are taken from the row's first element (d = x - x0),
// which is exact for values within a factor of two of x0, and the centred value
// is kept as d - mean(d) rather than x - (x0 + mean(d)), so a large common
// offset never has to be represented next to the small spread. This is the
// same remedy the reference kernel applies (normalization.cu:59-70), carried
// one rounding further.
//
// Generic path (odd widths, unaligned pointers, very wide rows): one wavefront
// per row, three strided passes over the row (the second and third hit cache).
#include "device_common.hpp"
#include "launch.hpp"

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

template <int Lanes, typename Op> __device__ __forceinline__ float team_allreduce(float v, Op op) {
    if constexpr (Lanes == 16) {
        return row16_allreduce(v, op);
    } else {
        return wave_allreduce(v, op);
    }
}

/// Value of lane @p source_lane broadcast to the calling lane.
__device__ __forceinline__ float lane_broadcast(float v, int source_lane) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(source_lane << 2, __float_as_int(v)));
}

/// @tparam Streaming non-temporal loads and stores (input read once, output
/// read later from HBM: 3.60 -> 3.37 us at [6304, 192] with the loads too);
/// plain ones leave the output in the caches for a kernel that reads it next,
/// and read an input a kernel has just written.
/// @tparam kColumns the row width when it is fixed at compile time (the ViT
/// widths), 0 otherwise: the width's divisions, the column masks and the row
/// offsets then fold to constants ahead of the first load, the same values.
/// @tparam Strided input rows @p input_stride elements apart; otherwise packed
/// (the stride is the row width, compile-time with @p kColumns).
template <typename T, int Lanes, int V, bool Streaming, int kColumns = 0, bool Strided = false>
__global__ __launch_bounds__(kBlock) void layer_norm_vector_kernel(
    const T* __restrict__ input, const float* __restrict__ gamma, const float* __restrict__ beta,
    T* __restrict__ output, int rows, int columns_argument, float epsilon,
    std::int64_t input_stride) {
    constexpr int E = Elem<T>::kPerVec;
    const int columns = kColumns > 0 ? kColumns : columns_argument;
    constexpr int kTeams = kWave / Lanes;

    const int lane = lane_id();
    const int team = lane / Lanes;
    const int team_lane = lane % Lanes;
    const int vectors = columns / E;

    bool valid[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
        valid[j] = team_lane + Lanes * j < vectors;
    }

    // gamma and beta for this lane's columns, held in registers for every row
    // the wavefront processes when they fit (fp32 rows up to 64 vectors per
    // lane-set); otherwise fetched at the store. Holding them keeps a dependent
    // cache round trip off the path between the statistics and the store.
    constexpr bool kHoist = V * E <= 16;
    float g[kHoist ? V : 1][kHoist ? E : 1];
    float b[kHoist ? V : 1][kHoist ? E : 1];
    if constexpr (kHoist) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const int column = (team_lane + Lanes * j) * E;
#pragma unroll
            for (int e = 0; e < E; e += 4) {
                float4 gv = make_float4(0.F, 0.F, 0.F, 0.F);
                float4 bv = gv;
                if (valid[j]) {
                    gv = *reinterpret_cast<const float4*>(gamma + column + e);
                    bv = *reinterpret_cast<const float4*>(beta + column + e);
                }
                g[j][e] = gv.x;
                g[j][e + 1] = gv.y;
                g[j][e + 2] = gv.z;
                g[j][e + 3] = gv.w;
                b[j][e] = bv.x;
                b[j][e + 1] = bv.y;
                b[j][e + 2] = bv.z;
                b[j][e + 3] = bv.w;
            }
        }
    }

    // Rows too wide for that at a fixed width (bf16 at 768: 48 columns a
    // lane) take gamma and beta from LDS, staged once per workgroup. Their
    // loads are issued right behind the first row's, so the two round trips
    // overlap instead of the parameters' following the row statistics.
    constexpr bool kStage = !kHoist && kColumns > 0;
    constexpr int kParamQuads = kStage ? 2 * kColumns / 4 : 1;  // gamma's float4s, then beta's
    __shared__ float4 staged_params[kParamQuads];

    const float inverse_columns = 1.0F / static_cast<float>(columns);
    const std::int64_t groups = (static_cast<std::int64_t>(rows) + kTeams - 1) / kTeams;
    const std::int64_t wave_count = static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock;
    const std::int64_t first_wave =
        static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;

    // A group's rows into registers (zeros past the last row); the next
    // group's are read at the end of the current one.
    Vec16 raw[V];
    auto load_group = [&](std::int64_t group) {
        const std::int64_t row = group * kTeams + team;
        const T* const source = input + row * (Strided ? input_stride : columns);
#pragma unroll
        for (int j = 0; j < V; ++j) {
            raw[j] = Vec16{{0U, 0U, 0U, 0U}};
            if (row < rows && valid[j]) {
                raw[j] = Streaming ? load16_streaming(source + (team_lane + Lanes * j) * E)
                                   : load16(source + (team_lane + Lanes * j) * E);
            }
        }
    };
    load_group(first_wave);
    if constexpr (kStage) {
        // Thread t holds quads t and t + kBlock (two named registers: an
        // array here is placed in LDS by the compiler).
        static_assert(kParamQuads > kBlock && kParamQuads <= 2 * kBlock,
                      "gamma and beta in two rounds, the first whole");
        auto param = [&](int index) {
            return index < kColumns / 4 ? reinterpret_cast<const float4*>(gamma)[index]
                                        : reinterpret_cast<const float4*>(beta)[index - kColumns / 4];
        };
        const int first = static_cast<int>(threadIdx.x);
        const int second = first + kBlock;
        const float4 first_quad = param(first);
        float4 second_quad = make_float4(0.F, 0.F, 0.F, 0.F);
        if (second < kParamQuads) {
            second_quad = param(second);
        }
        staged_params[first] = first_quad;
        if (second < kParamQuads) {
            staged_params[second] = second_quad;
        }
        __syncthreads();
    }

    for (std::int64_t group = first_wave; group < groups; group += wave_count) {
        const std::int64_t row = group * kTeams + team;
        const bool row_valid = row < rows;

        // x0 lives in element 0 of the team's first lane.
        const float x0 =
            lane_broadcast(Elem<T>::get(raw[0], 0), (lane / Lanes) * Lanes);

        float d[V][E];
        float partial = 0.F;
#pragma unroll
        for (int j = 0; j < V; ++j) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                d[j][e] = valid[j] ? Elem<T>::get(raw[j], e) - x0 : 0.F;
                partial += d[j][e];
            }
        }
        const float mean_deviation = team_allreduce<Lanes>(partial, Sum{}) * inverse_columns;

        float squares = 0.F;
#pragma unroll
        for (int j = 0; j < V; ++j) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                d[j][e] = valid[j] ? d[j][e] - mean_deviation : 0.F;
                squares += d[j][e] * d[j][e];
            }
        }
        const float variance = team_allreduce<Lanes>(squares, Sum{}) * inverse_columns;
        const float inverse_deviation = rsqrtf(variance + epsilon);

        if (row_valid) {
            T* const destination = output + row * columns;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                if (valid[j]) {
                    const int column = (team_lane + Lanes * j) * E;
                    Vec16 result{{0U, 0U, 0U, 0U}};
#pragma unroll
                    for (int e = 0; e < E; e += 4) {
                        float gv[4];
                        float bv[4];
                        if constexpr (kHoist) {
                            for (int i = 0; i < 4; ++i) {
                                gv[i] = g[j][e + i];
                                bv[i] = b[j][e + i];
                            }
                        } else {
                            float4 gq;
                            float4 bq;
                            if constexpr (kStage) {
                                gq = staged_params[(column + e) / 4];
                                bq = staged_params[kColumns / 4 + (column + e) / 4];
                            } else {
                                gq = *reinterpret_cast<const float4*>(gamma + column + e);
                                bq = *reinterpret_cast<const float4*>(beta + column + e);
                            }
                            gv[0] = gq.x; gv[1] = gq.y; gv[2] = gq.z; gv[3] = gq.w;
                            bv[0] = bq.x; bv[1] = bq.y; bv[2] = bq.z; bv[3] = bq.w;
                        }
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            Elem<T>::set(result, e + i, d[j][e + i] * inverse_deviation * gv[i] + bv[i]);
                        }
                    }
                    if constexpr (Streaming) {
                        store16_streaming(destination + (team_lane + Lanes * j) * E, result);
                    } else {
                        store16(destination + (team_lane + Lanes * j) * E, result);
                    }
                }
            }
        }
        if (group + wave_count < groups) {
            load_group(group + wave_count);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void layer_norm_generic_kernel(
    const T* __restrict__ input, const float* __restrict__ gamma, const float* __restrict__ beta,
    T* __restrict__ output, int rows, int columns, float epsilon, std::int64_t input_stride) {
    const int lane = lane_id();
    const float inverse_columns = 1.0F / static_cast<float>(columns);
    const std::int64_t wave_count = static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock;

    for (std::int64_t row = static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock +
                            threadIdx.x / kWave;
         row < rows; row += wave_count) {
        const T* const source = input + row * input_stride;
        const float x0 = Elem<T>::load(source);

        float partial = 0.F;
        for (int column = lane; column < columns; column += kWave) {
            partial += Elem<T>::load(source + column) - x0;
        }
        const float mean_deviation = wave_allreduce(partial, Sum{}) * inverse_columns;

        float squares = 0.F;
        for (int column = lane; column < columns; column += kWave) {
            const float centred = (Elem<T>::load(source + column) - x0) - mean_deviation;
            squares += centred * centred;
        }
        const float variance = wave_allreduce(squares, Sum{}) * inverse_columns;
        const float inverse_deviation = rsqrtf(variance + epsilon);

        T* const destination = output + row * columns;
        for (int column = lane; column < columns; column += kWave) {
            const float centred = (Elem<T>::load(source + column) - x0) - mean_deviation;
            Elem<T>::store(destination + column,
                           centred * inverse_deviation * gamma[column] + beta[column]);
        }
    }
}

/// Waves each compute unit is given before the kernels start looping.
constexpr int kWavesPerCu = 16;

template <typename T, int Lanes, int V, int kColumns = 0, bool Strided = false>
hipError_t launch_vector(const T* input, const float* gamma, const float* beta, T* output, int rows,
                         int columns, float epsilon, bool streaming, std::int64_t input_stride,
                         hipStream_t stream) {
    constexpr int kTeams = kWave / Lanes;
    const std::int64_t groups = (static_cast<std::int64_t>(rows) + kTeams - 1) / kTeams;
    const unsigned int grid = stride_grid(groups, kWavesPerBlock, kWavesPerCu / kWavesPerBlock);
    auto kernel = streaming ? layer_norm_vector_kernel<T, Lanes, V, true, kColumns, Strided>
                            : layer_norm_vector_kernel<T, Lanes, V, false, kColumns, Strided>;
    kernel<<<grid, kBlock, 0, stream>>>(input, gamma, beta, output, rows, columns, epsilon,
                                        input_stride);
    return hipGetLastError();
}

template <typename T>
hipError_t dispatch(const T* input, const float* gamma, const float* beta, T* output, int rows,
                    int columns, float epsilon, bool streaming, std::int64_t input_stride,
                    hipStream_t stream) {
    constexpr int E = Elem<T>::kPerVec;
    const bool vectorizable = columns % E == 0 && input_stride % E == 0 && aligned16(input) &&
                              aligned16(output) && aligned16(gamma) && aligned16(beta);
    const int vectors = columns / E;
    if (input_stride != columns) {
        // Strided rows (the model's class-token rows): the ViT widths, else
        // the one-wavefront-per-row kernel.
        if (vectorizable && columns == 192) {
            return launch_vector<T, 16, (192 / E + 15) / 16, 192, true>(
                input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        }
        if (vectorizable && columns == 768) {
            constexpr int kLanes = 768 / E <= 16 * 8 ? 16 : kWave;
            return launch_vector<T, kLanes, (768 / E + kLanes - 1) / kLanes, 768, true>(
                input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        }
        const unsigned int grid = stride_grid(rows, kWavesPerBlock, kWavesPerCu / kWavesPerBlock);
        layer_norm_generic_kernel<T><<<grid, kBlock, 0, stream>>>(input, gamma, beta, output, rows,
                                                                  columns, epsilon, input_stride);
        return hipGetLastError();
    }
    // The ViT widths with the width fixed at compile time, each on the team and
    // vector count the switch below picks ([6304, 192] fp32 3.37 -> 3.31 us,
    // [12608, 768] bf16 9.36 -> 8.56 us).
    if (vectorizable && columns == 192) {
        return launch_vector<T, 16, (192 / E + 15) / 16, 192>(input, gamma, beta, output, rows, columns,
                                                              epsilon, streaming, input_stride, stream);
    }
    if (vectorizable && columns == 768) {
        constexpr bool kNarrow = 768 / E <= 16 * 8;
        constexpr int kLanes = kNarrow ? 16 : kWave;
        return launch_vector<T, kLanes, (768 / E + kLanes - 1) / kLanes, 768>(
            input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
    }
    if (vectorizable && vectors <= 16 * 8) {
        switch ((vectors + 15) / 16) {
        case 1: return launch_vector<T, 16, 1>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 2: return launch_vector<T, 16, 2>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 3: return launch_vector<T, 16, 3>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 4: return launch_vector<T, 16, 4>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 5: return launch_vector<T, 16, 5>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 6: return launch_vector<T, 16, 6>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 7: return launch_vector<T, 16, 7>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        default: return launch_vector<T, 16, 8>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        }
    }
    if (vectorizable && vectors <= kWave * 8) {
        switch ((vectors + kWave - 1) / kWave) {
        case 3: return launch_vector<T, 64, 3>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 4: return launch_vector<T, 64, 4>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 5: return launch_vector<T, 64, 5>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 6: return launch_vector<T, 64, 6>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        case 7: return launch_vector<T, 64, 7>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        default: return launch_vector<T, 64, 8>(input, gamma, beta, output, rows, columns, epsilon, streaming, input_stride, stream);
        }
    }
    const unsigned int grid = stride_grid(rows, kWavesPerBlock, kWavesPerCu / kWavesPerBlock);
    layer_norm_generic_kernel<T><<<grid, kBlock, 0, stream>>>(input, gamma, beta, output, rows,
                                                              columns, epsilon, input_stride);
    return hipGetLastError();
}

} // namespace

hipError_t layer_norm_f32(const float* input, const float* gamma, const float* beta, float* output,
                          int rows, int columns, float epsilon, hipStream_t stream, bool streaming,
                          std::int64_t input_stride) {
    return dispatch<float>(input, gamma, beta, output, rows, columns, epsilon, streaming,
                           input_stride > 0 ? input_stride : columns, stream);
}

hipError_t layer_norm_bf16(const std::uint16_t* input, const float* gamma, const float* beta,
                           std::uint16_t* output, int rows, int columns, float epsilon,
                           hipStream_t stream, bool streaming, std::int64_t input_stride) {
    return dispatch<std::uint16_t>(input, gamma, beta, output, rows, columns, epsilon, streaming,
                                   input_stride > 0 ? input_stride : columns, stream);
}

} // namespace cuvit::detail
