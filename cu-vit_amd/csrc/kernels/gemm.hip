// Batched GEMM with the bias / GELU / accumulate epilogue, on gfx950 MFMA.
//
// Semantics are the reference's launch_gemm (include/cuvit/kernels.hpp:61-99,
// src/kernels/gemm.cu:44-242):
//   C[i][m][n] = epilogue(alpha * sum_k A[i][m][k] * B_layout[i][k][n] + bias[n])
// where the epilogue applies, in this order, alpha, the bias, the erf GELU and
// finally either C = value or C += value (gemm.cu:153-162). Batches are flat
// (entry * stride) or split into (entry / inner, entry % inner) with outer
// strides (gemm.cu:58-72); every operand has its own leading dimension.
//
// fp32: v_mfma_f32_32x32x2_f32, A staged k-major in LDS so each lane reads one
// float per MFMA. bf16: v_mfma_f32_32x32x16_bf16 (gfx950's doubled-K form),
// A staged row-major so each lane reads 8 consecutive k as one 16-byte LDS read;
// accumulation is fp32 and the result is rounded to bf16 once.
//
// Every tile shape uses the same MFMA instruction and walks K strictly in
// order with no split-K, so a given output element is computed by the same
// sequence of operations whatever the tile, the problem height or the batch.
// That keeps results independent of the tile choice (the property the
// reference states at gemm.cu:233-235) and batched rows bitwise equal to the
// same rows computed alone. Zero padding past M, N or K adds exact zeros.
#include "device_common.hpp"
#include "launch.hpp"

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256; // 4 wavefronts in a 2 x 2 arrangement

struct Offsets {
    std::int64_t a;
    std::int64_t b;
    std::int64_t c;
};

/// Element offsets of batch entry @p entry (gemm.cu:58-72).
__device__ __forceinline__ Offsets entry_offsets(const GemmArgs& args, int entry) {
    if (args.inner > 0) {
        const std::int64_t outer = entry / args.inner;
        const std::int64_t index = entry - outer * args.inner;
        return {outer * args.outer_stride_a + index * args.stride_a,
                outer * args.outer_stride_b + index * args.stride_b,
                outer * args.outer_stride_c + index * args.stride_c};
    }
    return {entry * args.stride_a, entry * args.stride_b, entry * args.stride_c};
}

__device__ __forceinline__ float gelu(float x) {
    return 0.5F * x * (1.0F + erff(x * 0.7071067811865475F));
}

/// The store of one output element: alpha, bias, GELU, then overwrite or add.
template <typename T>
__device__ __forceinline__ void epilogue_store(T* c, std::int64_t offset, float sum,
                                               const float* bias, int column,
                                               const GemmArgs& args) {
    float value = args.alpha * sum;
    if (bias != nullptr) {
        value += bias[column];
    }
    if (args.gelu) {
        value = gelu(value);
    }
    if (args.accumulate) {
        value = Elem<T>::load(c + offset) + value;
    }
    Elem<T>::store(c + offset, value);
}

/// Writes a wave's 32 x 32 accumulator tile. Lane l holds column l % 32 and,
/// in register r, row 8 * (r / 4) + 4 * (l / 32) + r % 4 of the tile.
template <typename T>
__device__ __forceinline__ void store_tile(T* c, const floatx16& acc, int row_origin,
                                           int column_origin, const float* bias,
                                           const GemmArgs& args) {
    const int lane = lane_id();
    const int column = column_origin + (lane & 31);
    if (column >= args.n) {
        return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = row_origin + 8 * (r / 4) + 4 * (lane >> 5) + (r & 3);
        if (row < args.m) {
            epilogue_store(c, static_cast<std::int64_t>(row) * args.ldc + column, acc[r], bias,
                           column, args);
        }
    }
}

// -- fp32 ---------------------------------------------------------------------

template <int BM, int BN> struct F32Shape {
    static constexpr int kBK = 16;
    static constexpr int kPad = 4;
    static constexpr int kTM = BM / 64; // 32 x 32 MFMA tiles per wave, along M
    static constexpr int kTN = BN / 64;
    static constexpr int kAQuads = BM * kBK / 4 / kThreads;
    static constexpr int kBQuads = BN * kBK / 4 / kThreads;
    static_assert(kAQuads >= 1 && kBQuads >= 1, "tile too small for the block");
};

/// Four consecutive elements of row @p row from column @p column of a
/// row-major matrix, zero outside [rows, columns). Vector when allowed.
template <bool Vector>
__device__ __forceinline__ float4 load_quad(const float* matrix, int ld, int row, int rows,
                                            int column, int columns) {
    float4 q = make_float4(0.F, 0.F, 0.F, 0.F);
    if (row >= rows) {
        return q;
    }
    const float* p = matrix + static_cast<std::int64_t>(row) * ld + column;
    if (Vector && column + 3 < columns) {
        return *reinterpret_cast<const float4*>(p);
    }
    if (column < columns) q.x = p[0];
    if (column + 1 < columns) q.y = p[1];
    if (column + 2 < columns) q.z = p[2];
    if (column + 3 < columns) q.w = p[3];
    return q;
}

template <int BM, int BN, bool VecA, bool VecB, bool TransB>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const float* __restrict__ a,
                                                            const float* __restrict__ b,
                                                            const float* __restrict__ bias,
                                                            float* c, GemmArgs args) {
    using S = F32Shape<BM, BN>;
    constexpr int BK = S::kBK;
    __shared__ __attribute__((aligned(16))) float tile_a[BK][BM + S::kPad];
    __shared__ __attribute__((aligned(16))) float tile_b[BK][BN + S::kPad];

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = t / kWave;
    const int wave_m = wave >> 1;
    const int wave_n = wave & 1;

    const int tiles_n = (args.n + BN - 1) / BN;
    const int tiles_m = (args.m + BM - 1) / BM;
    const std::int64_t tiles = static_cast<std::int64_t>(tiles_m) * tiles_n;

    for (int entry = blockIdx.y; entry < args.count; entry += gridDim.y) {
        const Offsets off = entry_offsets(args, entry);
        const float* const a_entry = a + off.a;
        const float* const b_entry = b + off.b;
        float* const c_entry = c + off.c;

        for (std::int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
            const int row0 = static_cast<int>(tile / tiles_n) * BM;
            const int col0 = static_cast<int>(tile % tiles_n) * BN;

            floatx16 acc[S::kTM][S::kTN];
#pragma unroll
            for (int i = 0; i < S::kTM; ++i)
#pragma unroll
                for (int j = 0; j < S::kTN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.F;

            float4 ra[S::kAQuads];
            float4 rb[S::kBQuads];
            auto fetch = [&](int k0) {
#pragma unroll
                for (int p = 0; p < S::kAQuads; ++p) {
                    const int q = t + kThreads * p;
                    ra[p] = load_quad<VecA>(a_entry, args.lda, row0 + q / (BK / 4), args.m,
                                            k0 + 4 * (q % (BK / 4)), args.k);
                }
#pragma unroll
                for (int p = 0; p < S::kBQuads; ++p) {
                    const int q = t + kThreads * p;
                    if constexpr (TransB) {
                        rb[p] = load_quad<VecB>(b_entry, args.ldb, col0 + q / (BK / 4), args.n,
                                                k0 + 4 * (q % (BK / 4)), args.k);
                    } else {
                        rb[p] = load_quad<VecB>(b_entry, args.ldb, k0 + q / (BN / 4), args.k,
                                                col0 + 4 * (q % (BN / 4)), args.n);
                    }
                }
            };
            auto stage = [&]() {
#pragma unroll
                for (int p = 0; p < S::kAQuads; ++p) {
                    const int q = t + kThreads * p;
                    const int row = q / (BK / 4);
                    const int kq = 4 * (q % (BK / 4));
                    tile_a[kq][row] = ra[p].x;
                    tile_a[kq + 1][row] = ra[p].y;
                    tile_a[kq + 2][row] = ra[p].z;
                    tile_a[kq + 3][row] = ra[p].w;
                }
#pragma unroll
                for (int p = 0; p < S::kBQuads; ++p) {
                    const int q = t + kThreads * p;
                    if constexpr (TransB) {
                        const int column = q / (BK / 4);
                        const int kq = 4 * (q % (BK / 4));
                        tile_b[kq][column] = rb[p].x;
                        tile_b[kq + 1][column] = rb[p].y;
                        tile_b[kq + 2][column] = rb[p].z;
                        tile_b[kq + 3][column] = rb[p].w;
                    } else {
                        const int kk = q / (BN / 4);
                        const int nq = 4 * (q % (BN / 4));
                        *reinterpret_cast<float4*>(&tile_b[kk][nq]) = rb[p];
                    }
                }
            };

            if (args.k > 0) {
                fetch(0);
            }
            for (int k0 = 0; k0 < args.k; k0 += BK) {
                __syncthreads();
                stage();
                __syncthreads();
                if (k0 + BK < args.k) {
                    fetch(k0 + BK);
                }
#pragma unroll
                for (int kk = 0; kk < BK; kk += 2) {
                    const int kr = kk + (lane >> 5);
                    float fa[S::kTM];
                    float fb[S::kTN];
#pragma unroll
                    for (int i = 0; i < S::kTM; ++i) {
                        fa[i] = tile_a[kr][wave_m * (BM / 2) + 32 * i + (lane & 31)];
                    }
#pragma unroll
                    for (int j = 0; j < S::kTN; ++j) {
                        fb[j] = tile_b[kr][wave_n * (BN / 2) + 32 * j + (lane & 31)];
                    }
#pragma unroll
                    for (int i = 0; i < S::kTM; ++i)
#pragma unroll
                        for (int j = 0; j < S::kTN; ++j)
                            acc[i][j] =
                                __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i], fb[j], acc[i][j], 0, 0, 0);
                }
            }

#pragma unroll
            for (int i = 0; i < S::kTM; ++i)
#pragma unroll
                for (int j = 0; j < S::kTN; ++j)
                    store_tile(c_entry, acc[i][j], row0 + wave_m * (BM / 2) + 32 * i,
                               col0 + wave_n * (BN / 2) + 32 * j, bias, args);
        }
    }
}

// -- bf16 ---------------------------------------------------------------------

template <int BM, int BN> struct Bf16Shape {
    static constexpr int kBK = 32;
    static constexpr int kPad = 8; // bf16 elements of padding per LDS row
    static constexpr int kTM = BM / 64;
    static constexpr int kTN = BN / 64;
    static constexpr int kAOcts = BM * kBK / 8 / kThreads;
    static constexpr int kBOcts = BN * kBK / 8 / kThreads;
    static_assert(kAOcts >= 1 && kBOcts >= 1, "tile too small for the block");
};

/// Eight consecutive bf16 of row @p row from column @p column, zero outside.
template <bool Vector>
__device__ __forceinline__ Vec16 load_oct(const std::uint16_t* matrix, int ld, int row, int rows,
                                          int column, int columns) {
    Vec16 v{{0U, 0U, 0U, 0U}};
    if (row >= rows) {
        return v;
    }
    const std::uint16_t* p = matrix + static_cast<std::int64_t>(row) * ld + column;
    if (Vector && column + 7 < columns) {
        return load16(p);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        if (column + e < columns) {
            const std::uint32_t bits = p[e];
            v.w[e >> 1] |= (e & 1) ? (bits << 16) : bits;
        }
    }
    return v;
}

template <int BM, int BN, bool VecA, bool VecB, bool TransB>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(const std::uint16_t* __restrict__ a,
                                                             const std::uint16_t* __restrict__ b,
                                                             const float* __restrict__ bias,
                                                             std::uint16_t* c, GemmArgs args) {
    using S = Bf16Shape<BM, BN>;
    constexpr int BK = S::kBK;
    constexpr int kRow = BK + S::kPad;
    __shared__ __attribute__((aligned(16))) std::uint16_t tile_a[BM * kRow];
    __shared__ __attribute__((aligned(16))) std::uint16_t tile_b[BN * kRow];

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = t / kWave;
    const int wave_m = wave >> 1;
    const int wave_n = wave & 1;

    const int tiles_n = (args.n + BN - 1) / BN;
    const int tiles_m = (args.m + BM - 1) / BM;
    const std::int64_t tiles = static_cast<std::int64_t>(tiles_m) * tiles_n;

    for (int entry = blockIdx.y; entry < args.count; entry += gridDim.y) {
        const Offsets off = entry_offsets(args, entry);
        const std::uint16_t* const a_entry = a + off.a;
        const std::uint16_t* const b_entry = b + off.b;
        std::uint16_t* const c_entry = c + off.c;

        for (std::int64_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
            const int row0 = static_cast<int>(tile / tiles_n) * BM;
            const int col0 = static_cast<int>(tile % tiles_n) * BN;

            floatx16 acc[S::kTM][S::kTN];
#pragma unroll
            for (int i = 0; i < S::kTM; ++i)
#pragma unroll
                for (int j = 0; j < S::kTN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.F;

            Vec16 ra[S::kAOcts];
            Vec16 rb[S::kBOcts];
            auto fetch = [&](int k0) {
#pragma unroll
                for (int p = 0; p < S::kAOcts; ++p) {
                    const int q = t + kThreads * p;
                    ra[p] = load_oct<VecA>(a_entry, args.lda, row0 + q / (BK / 8), args.m,
                                           k0 + 8 * (q % (BK / 8)), args.k);
                }
#pragma unroll
                for (int p = 0; p < S::kBOcts; ++p) {
                    const int q = t + kThreads * p;
                    if constexpr (TransB) {
                        rb[p] = load_oct<VecB>(b_entry, args.ldb, col0 + q / (BK / 8), args.n,
                                               k0 + 8 * (q % (BK / 8)), args.k);
                    } else {
                        rb[p] = load_oct<VecB>(b_entry, args.ldb, k0 + q / (BN / 8), args.k,
                                               col0 + 8 * (q % (BN / 8)), args.n);
                    }
                }
            };
            auto stage = [&]() {
#pragma unroll
                for (int p = 0; p < S::kAOcts; ++p) {
                    const int q = t + kThreads * p;
                    store16(&tile_a[(q / (BK / 8)) * kRow + 8 * (q % (BK / 8))], ra[p]);
                }
#pragma unroll
                for (int p = 0; p < S::kBOcts; ++p) {
                    const int q = t + kThreads * p;
                    if constexpr (TransB) {
                        store16(&tile_b[(q / (BK / 8)) * kRow + 8 * (q % (BK / 8))], rb[p]);
                    } else {
                        // B is [K, N]: scatter the 8 columns into k-contiguous rows.
                        const int kk = q / (BN / 8);
                        const int n8 = 8 * (q % (BN / 8));
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const std::uint32_t word = rb[p].w[e >> 1];
                            tile_b[(n8 + e) * kRow + kk] =
                                static_cast<std::uint16_t>((e & 1) ? (word >> 16) : (word & 0xFFFFU));
                        }
                    }
                }
            };

            if (args.k > 0) {
                fetch(0);
            }
            for (int k0 = 0; k0 < args.k; k0 += BK) {
                __syncthreads();
                stage();
                __syncthreads();
                if (k0 + BK < args.k) {
                    fetch(k0 + BK);
                }
#pragma unroll
                for (int kk = 0; kk < BK; kk += 16) {
                    const int kr = kk + 8 * (lane >> 5);
                    bf16x8 fa[S::kTM];
                    bf16x8 fb[S::kTN];
#pragma unroll
                    for (int i = 0; i < S::kTM; ++i) {
                        const int row = wave_m * (BM / 2) + 32 * i + (lane & 31);
                        fa[i] = __builtin_bit_cast(bf16x8, load16(&tile_a[row * kRow + kr]));
                    }
#pragma unroll
                    for (int j = 0; j < S::kTN; ++j) {
                        const int column = wave_n * (BN / 2) + 32 * j + (lane & 31);
                        fb[j] = __builtin_bit_cast(bf16x8, load16(&tile_b[column * kRow + kr]));
                    }
#pragma unroll
                    for (int i = 0; i < S::kTM; ++i)
#pragma unroll
                        for (int j = 0; j < S::kTN; ++j)
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j],
                                                                                acc[i][j], 0, 0, 0);
                }
            }

#pragma unroll
            for (int i = 0; i < S::kTM; ++i)
#pragma unroll
                for (int j = 0; j < S::kTN; ++j)
                    store_tile(c_entry, acc[i][j], row0 + wave_m * (BM / 2) + 32 * i,
                               col0 + wave_n * (BN / 2) + 32 * j, bias, args);
        }
    }
}

// -- dispatch -----------------------------------------------------------------

constexpr int kBlocksPerCu = 4;
constexpr int kMaxGridY = 65535;

/// True when every row of the operand starts on a 16-byte boundary.
template <typename T>
bool rows_aligned(const T* base, int ld, std::int64_t stride, std::int64_t outer_stride,
                  bool split) {
    constexpr int kPerVec = 16 / static_cast<int>(sizeof(T));
    return aligned16(base) && ld % kPerVec == 0 && stride % kPerVec == 0 &&
           (!split || outer_stride % kPerVec == 0);
}

template <typename T, int BM, int BN, bool VecA, bool VecB, bool TransB>
hipError_t launch_tile(const T* a, const T* b, const float* bias, T* c, const GemmArgs& args,
                       hipStream_t stream) {
    const std::int64_t tiles =
        static_cast<std::int64_t>((args.m + BM - 1) / BM) * ((args.n + BN - 1) / BN);
    const int entries = args.count < kMaxGridY ? args.count : kMaxGridY;
    std::int64_t budget = static_cast<std::int64_t>(compute_units()) * kBlocksPerCu * 64;
    budget = budget / entries > 0 ? budget / entries : 1;
    const unsigned int grid_x = static_cast<unsigned int>(tiles < budget ? tiles : budget);
    const dim3 grid(grid_x, static_cast<unsigned int>(entries));
    if constexpr (sizeof(T) == 4) {
        gemm_f32_kernel<BM, BN, VecA, VecB, TransB><<<grid, kThreads, 0, stream>>>(a, b, bias, c, args);
    } else {
        gemm_bf16_kernel<BM, BN, VecA, VecB, TransB><<<grid, kThreads, 0, stream>>>(a, b, bias, c, args);
    }
    return hipGetLastError();
}

template <typename T, int BM, int BN, bool VecA>
hipError_t pick_b(const T* a, const T* b, const float* bias, T* c, const GemmArgs& args, bool vec_b,
                  hipStream_t stream) {
    if (args.transposed) {
        return vec_b ? launch_tile<T, BM, BN, VecA, true, true>(a, b, bias, c, args, stream)
                     : launch_tile<T, BM, BN, VecA, false, true>(a, b, bias, c, args, stream);
    }
    return vec_b ? launch_tile<T, BM, BN, VecA, true, false>(a, b, bias, c, args, stream)
                 : launch_tile<T, BM, BN, VecA, false, false>(a, b, bias, c, args, stream);
}

template <typename T, int BM, int BN>
hipError_t pick_a(const T* a, const T* b, const float* bias, T* c, const GemmArgs& args, bool vec_a,
                  bool vec_b, hipStream_t stream) {
    return vec_a ? pick_b<T, BM, BN, true>(a, b, bias, c, args, vec_b, stream)
                 : pick_b<T, BM, BN, false>(a, b, bias, c, args, vec_b, stream);
}

template <typename T>
hipError_t dispatch(const T* a, const T* b, const float* bias, T* c, const GemmArgs& args,
                    hipStream_t stream) {
    const bool split = args.inner > 0;
    const bool vec_a = rows_aligned(a, args.lda, args.stride_a, args.outer_stride_a, split);
    const bool vec_b = rows_aligned(b, args.ldb, args.stride_b, args.outer_stride_b, split);
    // Tall problems get the 128 x 128 tile; the result does not depend on it.
    const std::int64_t tall_tiles =
        static_cast<std::int64_t>((args.m + 127) / 128) * ((args.n + 127) / 128) * args.count;
    if (args.m >= 256 && args.n >= 128 && tall_tiles >= compute_units()) {
        return pick_a<T, 128, 128>(a, b, bias, c, args, vec_a, vec_b, stream);
    }
    return pick_a<T, 64, 64>(a, b, bias, c, args, vec_a, vec_b, stream);
}

} // namespace

hipError_t gemm_f32(const float* a, const float* b, const float* bias, float* c,
                    const GemmArgs& args, hipStream_t stream) {
    return dispatch<float>(a, b, bias, c, args, stream);
}

hipError_t gemm_bf16(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                     std::uint16_t* c, const GemmArgs& args, hipStream_t stream) {
    return dispatch<std::uint16_t>(a, b, bias, c, args, stream);
}

} // namespace cuvit::detail
