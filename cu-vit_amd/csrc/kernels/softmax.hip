// Row softmax for gfx950.
//
// Semantics follow the reference launcher (include/cuvit/kernels.hpp:120-123)
// and its CPU path (tests/reference/linear_algebra.hpp:98-118): per row,
// exp(x - max) / sum(exp(x - max)). input == output is allowed; the model runs
// it in place over the attention logits (src/model/vit.cu:225).
//
// Each row is reduced by a team of L lanes: column c is lane c % L's
// (c / L)-th term, the lane folds its terms in order, then a fixed DPP tree
// combines the team. The team width depends only on the row width: rows up to
// 256 wide use 16-lane teams (four rows per wavefront, one quarter of the
// reduction instructions per row), wider rows a full 64-lane wavefront.
// Measured on MI355X, the 16-lane teams cut the [151296, 197] bf16 softmax
// from 41.9 us to 27 us and the fp32 [18912, 197] one from 7.8 to 6.6 us. Both
// paths below give a row the same bits for a given (type, width), wherever the
// row sits in a launch, which is what keeps a batch bitwise equal to its
// images run one at a time.
//
// Register path: each team loads its row's terms straight from HBM, keeps
// them in registers from the max through the exponentials to the scaled
// store, so HBM sees one read and one write per element. It takes wide rows
// below the staged path's row count, and team-of-16 rows whose pointers are
// not 16-byte aligned.
//
// Both paths read and write HBM with non-temporal loads and stores: every
// line is read once and written once, and the pair skips allocating and
// writing back lines the kernel will not touch again (fp32 [18912, 197] in
// place on full wavefronts: 8.5 -> 7.8 us; the bf16 [151296, 197]: 28 ->
// 26 us). Plain loads with non-temporal stores were slower than plain ones.
//
// Staged path: R rows of any width are `columns` 16-byte vectors (R = 4 fp32,
// 8 bf16), so each wavefront moves an R-row block between HBM and a
// wave-private LDS tile with aligned dwordx4 traffic, and prefetches its next
// block into registers while it reduces the current one out of LDS. It runs
// for every team-of-16 row when the pointers allow and for wider rows from a
// row count that fills the chip several times over.
//
// Exponentials are exp2((x - max) * log2(e)) on the hardware exp2. x - max is
// exact at x = max, where the largest outputs sit, and the relative error of an
// exponential grows only with |x - max| (about |x - max| * 2^-23 plus the exp2
// unit's ~1 ulp), so it is largest where the output is smallest: under 1e-6
// absolute for every output, far inside the reference test's 1e-4 relative
// tolerance (tests/elementwise_test.cu:254-255). bf16 rows of the register and
// staged paths take exp2(fma(x, log2 e, -(max * log2 e))) instead, one
// instruction a term fewer (the fused bf16 attention does the same, so the two
// stay bitwise equal): the shift's rounding moves an exponent by at most an
// ulp of max * log2 e, a relative change of about 1e-7 in the output against
// bf16's 4e-3 spacing.
//
// Streaming path (rows wider than the register path holds): one wavefront per
// row with an online max: a single streaming pass keeps a running (max, sum)
// per lane, rescaling the sum when the max grows, the lanes are merged, and a
// second pass writes the result.
#include "device_common.hpp"
#include "launch.hpp"
#include "softmax_terms.hpp"

#include <cmath>

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

/// Terms per lane the register and staged paths hold.
constexpr int kMaxTerms = 16;
/// Widest row a 16-lane team takes.
constexpr int kTeamColumns = 16 * kMaxTerms;

template <typename T, int L, int J>
__global__ __launch_bounds__(kBlock) void softmax_rows_kernel(const T* input, T* output, int rows,
                                                              int columns) {
    constexpr int kTeams = kWave / L;
    const int lane = lane_id();
    const int t = lane % L;
    const std::int64_t groups = (static_cast<std::int64_t>(rows) + kTeams - 1) / kTeams;
    const std::int64_t waves = static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock;

    for (std::int64_t group = static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock +
                              threadIdx.x / kWave;
         group < groups; group += waves) {
        const std::int64_t row = group * kTeams + lane / L;
        const bool here = row < rows;
        const T* const source = input + row * columns;
        T* const destination = output + row * columns;

        float x[J];
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int column = t + L * j;
            x[j] = here && column < columns ? Elem<T>::load_streaming(source + column) : -INFINITY;
        }
        softmax_terms<L, J, sizeof(T) == 2>(x, t, columns);
        if (here) {
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = t + L * j;
                if (column < columns) {
                    Elem<T>::store_streaming(destination + column, x[j]);
                }
            }
        }
    }
}

/// 16-byte vectors of an R-row block each lane prefetches: blocks up to
/// 64 * kPrefetch vectors, which covers every row the staged path takes.
constexpr int kPrefetch = 4;

/// Block row a team reduces in a pass. With four teams over the eight rows
/// of a bf16 block, the passes take rows (0, 4, 1, 5), then (2, 6, 3, 7): at
/// 197 columns the four teams' 16-element reads then fall on disjoint LDS
/// banks (SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE of the [151296, 197]
/// softmax 0.406 -> 0.000), where rows (0, 1, 2, 3) put teams 0 and 2, and
/// 1 and 3, on common banks. Which team takes a row changes none of its bits.
/// The four-row fp32 blocks have no such order: 197 * r mod 64 for four
/// rows of a block never spreads four 16-bank runs apart.
template <int kTeams, int R> __device__ __forceinline__ int team_row(int pass, int team) {
    if constexpr (kTeams == 4 && R == 8) {
        return 2 * pass + (team >> 1) + 4 * (team & 1);
    } else {
        return pass * kTeams + team;
    }
}

/// @tparam kColumns the row width when it is fixed at compile time (the ViT
/// token count), 0 otherwise: the loops over a block's vectors and the tile
/// offsets then run on constants, the same values.
template <typename T, int L, int J, int kColumns = 0>
__global__ __launch_bounds__(kBlock) void softmax_staged_kernel(const T* input, T* output, int rows,
                                                                int columns_argument) {
    constexpr int R = Elem<T>::kPerVec;
    const int columns = kColumns > 0 ? kColumns : columns_argument;
    constexpr int kTeams = kWave / L;
    constexpr int kPasses = (R + kTeams - 1) / kTeams;
    extern __shared__ Vec16 lds[];
    const int lane = lane_id();
    const int t = lane % L;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    Vec16* const tile = lds + wave * columns;
    T* const tile_elements = reinterpret_cast<T*>(tile);
    const std::int64_t blocks = (static_cast<std::int64_t>(rows) + R - 1) / R;
    const std::int64_t step = static_cast<std::int64_t>(gridDim.x) * kWavesPerBlock;

    // The next full block of this wavefront, held in registers while the
    // current one is reduced.
    Vec16 ahead[kPrefetch];
    auto prefetch = [&](std::int64_t block) {
        if (block < blocks && (block + 1) * R <= rows) {
            const T* const source = input + block * R * columns;
#pragma unroll
            for (int i = 0; i < kPrefetch; ++i) {
                const int v = lane + kWave * i;
                if (v < columns) {
                    ahead[i] = load16_streaming(source + static_cast<std::int64_t>(v) * R);
                }
            }
        }
    };
    prefetch(static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock + wave);

    // Every wavefront of the workgroup runs the same iterations (a block past
    // the end is simply empty), so the barriers below are uniform.
    for (std::int64_t base = static_cast<std::int64_t>(blockIdx.x) * kWavesPerBlock; base < blocks;
         base += step) {
        const std::int64_t block = base + wave;
        const std::int64_t first_row = block * R;
        const int rows_here =
            block < blocks ? static_cast<int>(rows - first_row < R ? rows - first_row : R) : 0;
        const T* const source = input + first_row * columns;
        T* const destination = output + first_row * columns;

        if (rows_here == R) {
#pragma unroll
            for (int i = 0; i < kPrefetch; ++i) {
                const int v = lane + kWave * i;
                if (v < columns) {
                    tile[v] = ahead[i];
                }
            }
        } else {
            for (int i = lane; i < rows_here * columns; i += kWave) {
                tile_elements[i] = source[i];
            }
        }
        __syncthreads();
        prefetch(block + step);

        // Each lane writes back exactly the elements it read, so the
        // reductions need no barrier between them.
#pragma unroll
        for (int pass = 0; pass < kPasses; ++pass) {
            const int r = team_row<kTeams, R>(pass, lane / L);
            const bool here = r < rows_here;
            float x[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = t + L * j;
                x[j] = here && column < columns ? Elem<T>::load(tile_elements + r * columns + column)
                                                : -INFINITY;
            }
            softmax_terms<L, J, sizeof(T) == 2>(x, t, columns);
            if (here) {
#pragma unroll
                for (int j = 0; j < J; ++j) {
                    const int column = t + L * j;
                    if (column < columns) {
                        Elem<T>::store(tile_elements + r * columns + column, x[j]);
                    }
                }
            }
        }
        __syncthreads();

        if (rows_here == R) {
            for (int v = lane; v < columns; v += kWave) {
                store16_streaming(destination + static_cast<std::int64_t>(v) * R, tile[v]);
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
/// holds at the register path's register use, measured fastest at ViT shapes.
constexpr int kBlocksPerCu = 8;
/// The staged path keeps a prefetched block in registers: 16 waves per CU
/// measured fastest ([151296, 197] bf16: 27.0 us against 29.8 us at 32).
constexpr int kStagedBlocksPerCu = 4;

/// Row counts from which full-wavefront rows take the staged path: more than
/// four rows per wavefront once every compute unit is full.
std::int64_t staged_threshold() { return static_cast<std::int64_t>(compute_units()) * 128; }

template <typename T, int L, int J, int kColumns = 0>
hipError_t launch_rows(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    constexpr int R = Elem<T>::kPerVec;
    const bool staged = L < kWave || rows >= staged_threshold();
    if (staged && columns <= kWave * kPrefetch && aligned16(input) && aligned16(output)) {
        const std::int64_t blocks = (static_cast<std::int64_t>(rows) + R - 1) / R;
        const unsigned int grid = stride_grid(blocks, kWavesPerBlock, kStagedBlocksPerCu);
        const std::size_t lds = static_cast<std::size_t>(kWavesPerBlock) * columns * sizeof(Vec16);
        softmax_staged_kernel<T, L, J, kColumns><<<grid, kBlock, lds, stream>>>(input, output, rows,
                                                                               columns);
        return hipGetLastError();
    }
    const std::int64_t teams = kWave / L;
    const unsigned int grid = stride_grid((rows + teams - 1) / teams, kWavesPerBlock, kBlocksPerCu);
    softmax_rows_kernel<T, L, J><<<grid, kBlock, 0, stream>>>(input, output, rows, columns);
    return hipGetLastError();
}

/// Picks J, the terms per lane, for a team of L lanes. Rounding J up adds
/// terms that are -inf before and 0 after the exponential, which changes no
/// bit of the max or the sum, so the choice never changes a result.
template <typename T, int L>
hipError_t launch_team(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    switch ((columns + L - 1) / L) {
    case 1: return launch_rows<T, L, 1>(input, output, rows, columns, stream);
    case 2: return launch_rows<T, L, 2>(input, output, rows, columns, stream);
    case 3: return launch_rows<T, L, 3>(input, output, rows, columns, stream);
    case 4: return launch_rows<T, L, 4>(input, output, rows, columns, stream);
    case 5:
    case 6: return launch_rows<T, L, 6>(input, output, rows, columns, stream);
    case 7:
    case 8: return launch_rows<T, L, 8>(input, output, rows, columns, stream);
    case 9:
    case 10: return launch_rows<T, L, 10>(input, output, rows, columns, stream);
    case 11:
    case 12:
    case 13: return launch_rows<T, L, 13>(input, output, rows, columns, stream);
    default: return launch_rows<T, L, 16>(input, output, rows, columns, stream);
    }
}

template <typename T>
hipError_t dispatch(const T* input, T* output, int rows, int columns, hipStream_t stream) {
    // The ViT token count (197) with the width fixed at compile time, on the
    // team and term count launch_team picks for it ([18912, 197] fp32 6.84 ->
    // 6.77 us, [151296, 197] bf16 25.7 -> 24.7 us); the register path of that
    // instance keeps its runtime loops.
    if (columns == 197 && kTeamColumns >= 197) {
        return launch_rows<T, 16, 13, 197>(input, output, rows, columns, stream);
    }
    if (columns <= kTeamColumns) {
        return launch_team<T, 16>(input, output, rows, columns, stream);
    }
    if (columns <= kWave * kMaxTerms) {
        return launch_team<T, kWave>(input, output, rows, columns, stream);
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
