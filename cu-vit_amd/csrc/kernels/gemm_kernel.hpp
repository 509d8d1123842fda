// The batched GEMM kernel behind launch_gemm, for gfx950 MFMA.
//
// Semantics are the reference's launch_gemm (include/cuvit/kernels.hpp:61-99,
// src/kernels/gemm.cu:44-242):
//   C[i][m][n] = epilogue(alpha * sum_k A[i][m][k] * B_layout[i][k][n] + bias[n])
// where the epilogue applies, in this order, alpha, the bias, the erf GELU and
// finally either C = value or C += value (gemm.cu:153-162). Internally an
// [m, n] addend may follow the bias (the model's positional add). Batches are flat
// (entry * stride) or split into (entry / inner, entry % inner) with outer
// strides (gemm.cu:58-72); every operand has its own leading dimension.
//
// Structure. A workgroup of WM x WN wavefronts (four, or twelve for the
// largest bf16 tile) owns a BM x BN tile of C; each
// wavefront owns (TM * E) x (TN * E) of it as TM x TN MFMA tiles of edge E.
// K is walked in BK-wide stages. Both operand tiles sit in LDS as
// [rows][BK] (k contiguous), rows padded by 16 bytes so that the sixteen
// lanes reading one fragment column hit sixteen different bank quads. Stages
// are double-buffered in LDS and fetched from global memory into registers
// two stages ahead, so a global load has two stages of MFMA work to land and
// each stage costs one barrier.
//
// MFMA. fp32 uses v_mfma_f32_16x16x4_f32 (E = 16) and bf16
// v_mfma_f32_32x32x16_bf16 (E = 32); measured on MI355X with an in-kernel
// cycle counter, the fp32 one issues every 32 core cycles even as a single
// dependent chain (the full rate; 32 x 32 x 2 takes 64 for twice the work),
// and bf16's 32 x 32 form reaches 2.1 PFLOP/s where its 16 x 16 form reaches
// only 1.2; fp32's fine 16 x 16 tiles fit ViT-Tiny's 192- and 197-wide shapes. Lane l reads one 16-byte fragment per operand per k-block:
// row l % E of its operand and k chunk l / E, so a k-block is 16 consecutive
// k for both types. bf16 feeds the chunk to one MFMA. fp32 feeds element s of
// the chunk to the s-th of four MFMAs, so MFMA s of a k-block sums
// k = kb + s, kb + 4 + s, kb + 8 + s, kb + 12 + s. The B fragment goes in the
// MFMA's first operand and the A fragment in its second, which computes the
// transposed tile: lane l ends up holding row l % E of C in runs of four
// consecutive columns, so the epilogue stores 16 (fp32) or 8 (bf16)
// contiguous bytes at a time.
//
// Determinism. Every tile shape of a type uses the same MFMA and walks K in
// the same order, over the same number of k-blocks, with no split-K, so an
// output element is computed by the same operations whatever the tile, the
// problem height or the batch. That
// keeps results independent of the tile choice (the property the reference
// states at gemm.cu:233-235) and batched rows bitwise equal to the same rows
// computed alone. Operand elements outside the problem read as zero, so
// padding past K adds exact zeros, and results past M or N are never stored.
#pragma once

#include "device_common.hpp"
#include "launch.hpp"


namespace cuvit::detail::gemm {

using namespace cuvit::device;

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

/// Threads of a four-wavefront workgroup (the wide and tiled bf16 kernels).
constexpr int kThreads = 256;

/// The MFMA of each storage type. kEdge is the MFMA tile's edge; a lane's
/// accumulator holds kRuns runs of four consecutive columns of row
/// lane % kEdge, run q starting at column column(lane, q) of the tile.
template <typename T> struct Mma;

template <> struct Mma<float> {
    static constexpr int kEdge = 16;
    static constexpr int kPerVec = 4; // elements per 16-byte fragment
    static constexpr int kRuns = 1;
    using Acc = floatx4;
    __device__ __forceinline__ static int column(int lane, int) { return 4 * (lane >> 4); }
    __device__ __forceinline__ static void run(Acc& acc, const Vec16& b, const Vec16& a) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(b.w[s]), __uint_as_float(a.w[s]),
                                                       acc, 0, 0, 0);
        }
    }
};

template <> struct Mma<std::uint16_t> {
    static constexpr int kEdge = 32;
    static constexpr int kPerVec = 8;
    static constexpr int kRuns = 4;
    using Acc = floatx16;
    __device__ __forceinline__ static int column(int lane, int q) { return 8 * q + 4 * (lane >> 5); }
    __device__ __forceinline__ static void run(Acc& acc, const Vec16& b, const Vec16& a) {
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, b),
                                                      __builtin_bit_cast(bf16x8, a), acc, 0, 0, 0);
    }
};

/// Consecutive k covered by one 16-byte fragment column of a wavefront.
template <typename T> constexpr int kKBlock = (kWave / Mma<T>::kEdge) * Mma<T>::kPerVec;

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

/// alpha, bias, the optional addend, GELU: everything of the epilogue before
/// the store, with the bias term already loaded (@p with_bias false: none).
__device__ __forceinline__ float epilogue_value(float sum, bool with_bias, float bias_value, int row,
                                                int column, const GemmArgs& args) {
    // alpha * sum and each addition round on their own (no fused multiply-add),
    // the reference's order, in every GEMM kernel alike.
#pragma clang fp contract(off)
    float value = args.alpha * sum;
    if (with_bias) {
        value += bias_value;
    }
    if (args.addend != nullptr) {
        value += args.addend[static_cast<std::int64_t>(row) * args.ld_addend + column];
    }
    if (args.gelu) {
        value = gelu(value);
    }
    return value;
}

// -- operand loads ------------------------------------------------------------
//
// The vector path reads operands with raw buffer loads. A buffer resource
// covers a tile's operand rows from their first element; any byte offset at or
// past kRecords reads as zero in hardware. Elements outside the problem (rows
// past M or N, k past K) are given the offset kOutside, so a tail needs no
// branch and no select on loaded data: the compiler can keep every stage's
// loads in flight and count them exactly.

constexpr int kRecords = 0x7FFFFFF0;
constexpr unsigned int kOutside = 0x7FFFFFF0U;
/// Largest tile span, in bytes, the vector path addresses from one base.
constexpr std::int64_t kMaxSpan = std::int64_t{1} << 30;

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_resource(const void* base) {
    // 0x00020000: the gfx9 descriptor word 3 for untyped 32-bit access.
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             kRecords, 0x00020000);
}

__device__ __forceinline__ Vec16 buffer_load16(__amdgpu_buffer_rsrc_t resource,
                                               unsigned int offset) {
    return __builtin_bit_cast(Vec16, __builtin_amdgcn_raw_buffer_load_b128(resource, offset, 0, 0));
}

/// Byte offset of element (row, k) of a row-major operand whose resource
/// starts at its row 0, or kOutside when the element lies outside.
template <typename T>
__device__ __forceinline__ unsigned int chunk_offset(int row, int rows, int ld, int k, int depth) {
    return row < rows && k < depth
               ? static_cast<unsigned int>((row * ld + k) * static_cast<int>(sizeof(T)))
               : kOutside;
}

/// Scalar path: one 16-byte chunk of a row-major [rows][depth] operand, row
/// @p row, elements @p k .. + kPerVec, zero outside.
template <typename T>
__device__ __forceinline__ Vec16 load_chunk_scalar(const T* matrix, int ld, int row, int rows, int k,
                                                   int depth) {
    Vec16 v{{0U, 0U, 0U, 0U}};
    if (row < rows) {
        const T* p = matrix + static_cast<std::int64_t>(row) * ld;
#pragma unroll
        for (int e = 0; e < Mma<T>::kPerVec; ++e) {
            if (k + e < depth) {
                Elem<T>::put_bits(v, e, p + k + e);
            }
        }
    }
    return v;
}

/// The accumulating epilogue's C + value, rounded on its own: the add never
/// fuses with the multiply that ends the GELU before it, in any kernel, so
/// every kernel gives the same bits.
__device__ __forceinline__ float add_unfused(float c, float value) {
#pragma clang fp contract(off)
    return c + value;
}

/// Four consecutive elements of C as one load: 16 bytes for fp32, 8 for bf16.
template <typename T> struct Quad;
template <> struct Quad<float> {
    using Type = floatx4;
};
template <> struct Quad<std::uint16_t> {
    using Type = uint2;
};

/// Stores four consecutive results (C = value, or C = @p old + value when
/// accumulating, @p old being the four elements read beforehand); @p p is
/// aligned to the four elements' size.
__device__ __forceinline__ void store4(float* p, const float (&value)[4], bool accumulate,
                                       const floatx4& old) {
    floatx4 v{value[0], value[1], value[2], value[3]};
    if (accumulate) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
            v[r] = add_unfused(old[r], v[r]);
    }
    *reinterpret_cast<floatx4*>(p) = v;
}

__device__ __forceinline__ void store4(std::uint16_t* p, const float (&value)[4], bool accumulate,
                                       const uint2& old) {
    float v[4] = {value[0], value[1], value[2], value[3]};
    if (accumulate) {
        v[0] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.x & 0xFFFFU)), v[0]);
        v[1] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.x >> 16)), v[1]);
        v[2] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.y & 0xFFFFU)), v[2]);
        v[3] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.y >> 16)), v[3]);
    }
    uint2 bits;
    bits.x = static_cast<std::uint32_t>(float_to_bf16(v[0])) |
             (static_cast<std::uint32_t>(float_to_bf16(v[1])) << 16);
    bits.y = static_cast<std::uint32_t>(float_to_bf16(v[2])) |
             (static_cast<std::uint32_t>(float_to_bf16(v[3])) << 16);
    *reinterpret_cast<uint2*>(p) = bits;
}

/// Compile-time shape of one kernel instance.
template <typename T, int WM, int WN, int TM, int TN, int BK> struct Shape {
    static_assert(WM * WN == 4 || WM * WN == 12, "four or twelve wavefronts per workgroup");
    static constexpr int kThreads = kWave * WM * WN;
    static constexpr int kE = Mma<T>::kEdge;
    static constexpr int kBM = WM * TM * kE;
    static constexpr int kBN = WN * TN * kE;
    static constexpr int kV = Mma<T>::kPerVec;
    static constexpr int kKBlock = gemm::kKBlock<T>;
    static_assert(BK % kKBlock == 0, "stages hold whole k-blocks");
    /// Rows of four 16-byte chunks (bf16 at BK = 32) are stored unpadded with
    /// chunk c of row r at c ^ ((r >> 2) & 3). Measured with
    /// SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE on gfx950 for the two access
    /// patterns here, a stage write (lane l: row l / 4, chunk l % 4) and a
    /// fragment read (lane l: row l % 32, chunk kb + l / 32):
    ///   16-byte pad (80-byte rows)       reads 0,    writes 0.5
    ///   unpadded, c ^ ((r >> 1) & 3)     reads 0.5,  writes 0
    ///   unpadded, c ^ ((r >> 2) & 3)     reads 0,    writes 0
    /// Rows of eight chunks keep the 16-byte pad (144-byte rows), which
    /// measured 0 for both.
    static constexpr bool kSwizzle = BK / kV == 4;
    static_assert(!kSwizzle || kE % 16 == 0, "fragment rows keep their placement across MFMA tiles");
    static constexpr int kPitch = kSwizzle ? BK : BK + kV; // elements per LDS row
    static constexpr int kChunksPerRow = BK / kV;     // 16-byte chunks per operand row of a stage
    static constexpr int kAChunks = kBM * kChunksPerRow;
    static constexpr int kBChunks = kBN * kChunksPerRow;
    static constexpr int kAPerThread = (kAChunks + kThreads - 1) / kThreads;
    static constexpr int kBPerThread = (kBChunks + kThreads - 1) / kThreads;
    static constexpr int kStage = (kBM + kBN) * kPitch; // elements per LDS stage
    static constexpr std::size_t kLdsBytes = 2 * kStage * sizeof(T);

    /// Where chunk @p chunk of operand row @p row sits in its LDS row.
    __device__ __forceinline__ static int place(int row, int chunk) {
        if constexpr (kSwizzle) {
            return chunk ^ ((row >> 2) & 3);
        } else {
            return chunk;
        }
    }
};

/// Which tile a workgroup computes. With px * py == 8 the tile grid of an
/// entry is split into px x py blocks and workgroup x goes to block x % 8:
/// the MI355X dispatcher hands consecutive workgroups to its 8 XCDs in turn,
/// so each XCD's L2 then serves one block, its A rows and its B columns,
/// instead of every XCD streaming all of A. With px == 0 the tiles are in
/// plain row-major order.
struct TileMap {
    int px;
    int py;
};

/// Start of part @p i of @p n split into @p parts near-equal parts.
__device__ __forceinline__ int split_point(int n, int parts, int i) { return n * i / parts; }

/// K walked per type in whole spans: every tile shape of a type runs the same
/// number of k-blocks (those past K add 0 * 0), so even the sign of an exact
/// zero result does not depend on the tile. fp32 stages are 32 deep and run
/// in pairs; bf16 stages are 32 or 64 deep and run to a multiple of 128.
template <typename T> constexpr int kSpan = sizeof(T) == 2 ? 128 : 64;

/// @tparam MinWaves wavefronts per SIMD the register allocation must allow
/// (amdgpu_waves_per_eu); 1 leaves the compiler free.
template <typename T, int WM, int WN, int TM, int TN, int BK, bool VecA, bool VecB, bool TransB,
          int MinWaves>
__global__ __launch_bounds__(kWave * WM * WN) __attribute__((amdgpu_waves_per_eu(MinWaves))) void gemm_kernel(const T* __restrict__ a,
                                                        const T* __restrict__ b,
                                                        const float* __restrict__ bias, T* c,
                                                        GemmArgs args, TileMap map, bool vector_c) {
    using S = Shape<T, WM, WN, TM, TN, BK>;
    // Explicit MFMA / memory interleave for the bf16 tiles whose stages are
    // whole 16-byte chunks written as such (vector A and B, B as [N, K]).
    constexpr bool kInterleave = sizeof(T) == 2 && VecA && VecB && TransB && TM * TN >= 4;
    constexpr int BM = S::kBM;
    constexpr int BN = S::kBN;
    constexpr int P = S::kPitch;
    constexpr int V = S::kV;
    extern __shared__ Vec16 lds_vectors[];
    T* const lds = reinterpret_cast<T*>(lds_vectors);

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = t / kWave;
    const int wave_m = wave / WN;
    const int wave_n = wave % WN;
    constexpr int E = S::kE;
    const int fragment_row = lane % E;
    const int fragment_chunk = lane / E;

    const int tiles_n = (args.n + BN - 1) / BN;
    int tile_m = static_cast<int>(blockIdx.x) / tiles_n;
    int tile_n = static_cast<int>(blockIdx.x) % tiles_n;
    if (map.px > 0) {
        const int tiles_m = (args.m + BM - 1) / BM;
        const int block = static_cast<int>(blockIdx.x) % 8;
        const int index = static_cast<int>(blockIdx.x) / 8;
        const int m_lo = split_point(tiles_m, map.px, block / map.py);
        const int m_hi = split_point(tiles_m, map.px, block / map.py + 1);
        const int n_lo = split_point(tiles_n, map.py, block % map.py);
        const int n_hi = split_point(tiles_n, map.py, block % map.py + 1);
        const int width = n_hi - n_lo;
        if (index >= (m_hi - m_lo) * width) {
            return; // this block has fewer tiles than the grid allows; no barrier is skipped
        }
        tile_m = m_lo + index / width;
        tile_n = n_lo + index % width;
    }
    const int row0 = tile_m * BM;
    const int col0 = tile_n * BN;
    static_assert(kSpan<T> % (2 * BK) == 0, "a span is a whole number of stage pairs");
    const int steps = (args.k + kSpan<T> - 1) / kSpan<T> * (kSpan<T> / BK);

    for (int entry = blockIdx.y; entry < args.count; entry += gridDim.y) {
        const Offsets off = entry_offsets(args, entry);
        const T* const a_entry = a + off.a;
        const T* const b_entry = b + off.b;
        T* const c_entry = c + off.c;

        typename Mma<T>::Acc acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4 * Mma<T>::kRuns; ++r)
                    acc[i][j][r] = 0.F;

        Vec16 ra0[S::kAPerThread], rb0[S::kBPerThread];
        Vec16 ra1[S::kAPerThread], rb1[S::kBPerThread];

        // Global -> registers for stage @p step. Offsets are relative to the
        // tile: A from its row row0, B [N, K] from its row col0, B [K, N]
        // from its column col0.
        const T* const a_tile = a_entry + static_cast<std::int64_t>(row0) * args.lda;
        const T* const b_tile =
            TransB ? b_entry + static_cast<std::int64_t>(col0) * args.ldb : b_entry + col0;
        const auto a_resource = buffer_resource(a_tile);
        const auto b_resource = buffer_resource(b_tile);
        const int a_rows = args.m - row0;
        const int b_rows = args.n - col0;
        auto fetch = [&](Vec16 (&ra)[S::kAPerThread], Vec16 (&rb)[S::kBPerThread], int step) {
            const int k0 = step * BK;
#pragma unroll
            for (int p = 0; p < S::kAPerThread; ++p) {
                const int q = t + S::kThreads * p;
                if (S::kAChunks % S::kThreads == 0 || q < S::kAChunks) {
                    const int row = q / S::kChunksPerRow;
                    const int k = k0 + V * (q % S::kChunksPerRow);
                    if constexpr (VecA) {
                        ra[p] = buffer_load16(a_resource,
                                              chunk_offset<T>(row, a_rows, args.lda, k, args.k));
                    } else {
                        ra[p] = load_chunk_scalar(a_tile, args.lda, row, a_rows, k, args.k);
                    }
                }
            }
#pragma unroll
            for (int p = 0; p < S::kBPerThread; ++p) {
                const int q = t + S::kThreads * p;
                if (S::kBChunks % S::kThreads == 0 || q < S::kBChunks) {
                    if constexpr (TransB) {
                        const int row = q / S::kChunksPerRow;
                        const int k = k0 + V * (q % S::kChunksPerRow);
                        if constexpr (VecB) {
                            rb[p] = buffer_load16(b_resource,
                                                  chunk_offset<T>(row, b_rows, args.ldb, k, args.k));
                        } else {
                            rb[p] = load_chunk_scalar(b_tile, args.ldb, row, b_rows, k, args.k);
                        }
                    } else {
                        // [BK][BN] in global order: chunk q is k row q / (BN / V),
                        // i.e. row k of the [K, N] matrix from column col0 + n.
                        const int k = k0 + q / (BN / V);
                        const int n = V * (q % (BN / V));
                        if constexpr (VecB) {
                            rb[p] = buffer_load16(b_resource,
                                                  chunk_offset<T>(k, args.k, args.ldb, n, b_rows));
                        } else {
                            rb[p] = load_chunk_scalar(b_tile, args.ldb, k, args.k, n, b_rows);
                        }
                    }
                }
            }
        };

        // Registers -> LDS stage @p buffer.
        auto stage = [&](const Vec16 (&ra)[S::kAPerThread], const Vec16 (&rb)[S::kBPerThread],
                         int buffer) {
            T* const tile_a = lds + buffer * S::kStage;
            T* const tile_b = tile_a + BM * P;
#pragma unroll
            for (int p = 0; p < S::kAPerThread; ++p) {
                const int q = t + S::kThreads * p;
                if (S::kAChunks % S::kThreads == 0 || q < S::kAChunks) {
                    const int row = q / S::kChunksPerRow;
                    store16(tile_a + row * P + V * S::place(row, q % S::kChunksPerRow), ra[p]);
                }
            }
#pragma unroll
            for (int p = 0; p < S::kBPerThread; ++p) {
                const int q = t + S::kThreads * p;
                if (S::kBChunks % S::kThreads == 0 || q < S::kBChunks) {
                    if constexpr (TransB) {
                        const int row = q / S::kChunksPerRow;
                        store16(tile_b + row * P + V * S::place(row, q % S::kChunksPerRow), rb[p]);
                    } else {
                        // Scatter the chunk's V columns into k-contiguous rows.
                        const int kk = q / (BN / V);
                        const int n = V * (q % (BN / V));
#pragma unroll
                        for (int e = 0; e < V; ++e) {
                            const int row = n + e;
                            Elem<T>::store_bits(tile_b + row * P + V * S::place(row, kk / V) + kk % V,
                                                rb[p], e);
                        }
                    }
                }
            }
        };

        // MFMAs over LDS stage @p buffer.
        auto compute = [&](int buffer) {
            const T* const tile_a = lds + buffer * S::kStage + (wave_m * TM * E + fragment_row) * P;
            const T* const tile_b =
                lds + buffer * S::kStage + (BM + wave_n * TN * E + fragment_row) * P;
#pragma unroll
            for (int kb = 0; kb < BK; kb += S::kKBlock) {
                // Every fragment row is fragment_row modulo E, a multiple of
                // the placement's 16-row period, so the lane's placement
                // depends on fragment_row alone.
                const int k = V * S::place(fragment_row, kb / V + fragment_chunk);
                Vec16 fa[TM];
                Vec16 fb[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    fa[i] = load16(tile_a + i * E * P + k);
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    fb[j] = load16(tile_b + j * E * P + k);
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        Mma<T>::run(acc[i][j], fb[j], fa[i]);
            }
        };

        // One stage of the loop: the MFMAs over LDS buffer @p buffer, the
        // next stage's registers into the other buffer, and the loads of the
        // stage two further on into the registers just freed. With
        // kInterleave the MFMA stream is ordered explicitly: the first
        // k-block's fragments, then one MFMA per fragment read for the
        // following k-blocks, and the LDS writes and global loads spread
        // over the last k-block's MFMAs (measured on the ViT-Base bf16
        // GEMMs: FC1 + GELU 165 -> 147 us, FC2 107 -> 94 us). The order of
        // the MFMAs, and so every result bit, is the same either way.
        auto advance = [&](const Vec16 (&ra)[S::kAPerThread], const Vec16 (&rb)[S::kBPerThread],
                           Vec16 (&la)[S::kAPerThread], Vec16 (&lb)[S::kBPerThread], int buffer,
                           int next_fetch) {
            if constexpr (kInterleave) {
                compute(buffer);
                stage(ra, rb, buffer ^ 1);
                fetch(la, lb, next_fetch);
                constexpr int kBlocks = BK / S::kKBlock;
                constexpr int kMfma = TM * TN * kBlocks;
                constexpr int kReads = (TM + TN) * kBlocks;
                constexpr int kPaired = kReads - (TM + TN);
                constexpr int kRest = kMfma - kPaired;
                constexpr int kWrites = (S::kAPerThread + S::kBPerThread + kRest - 1) / kRest;
                static_assert(kRest > 0, "more MFMAs than fragment reads");
                __builtin_amdgcn_sched_group_barrier(0x100, TM + TN, 0); // DS reads
#pragma unroll
                for (int i = 0; i < kPaired; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
                }
#pragma unroll
                for (int i = 0; i < kRest; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x200, kWrites, 0);  // DS write
                    __builtin_amdgcn_sched_group_barrier(0x020, kWrites, 0);  // VMEM read
                }
            } else {
                stage(ra, rb, buffer ^ 1);
                fetch(la, lb, next_fetch);
                compute(buffer);
            }
        };

        // Stage s sits in LDS buffer s % 2. Register set 0 carries even
        // stages and set 1 odd ones, each loaded two stages before use. The
        // loop body runs unconditionally, two stages per trip: a stage past
        // K reads as zero and its MFMAs add products 0 * 0 to accumulators
        // that started at +0, which changes no bit of them. So every path
        // through the loop has the same loads in flight, each LDS write waits
        // only for its own set, and the accumulators stay in place.
        if (steps > 0) {
            fetch(ra0, rb0, 0);
            stage(ra0, rb0, 0);
            fetch(ra1, rb1, 1);
            // Keep set 1's loads ahead of set 0's, the order the loop keeps.
            __builtin_amdgcn_sched_barrier(0);
            fetch(ra0, rb0, 2);
            __syncthreads();
            for (int step = 0; step < steps; step += 2) {
                advance(ra1, rb1, ra1, rb1, 0, step + 3);
                __syncthreads();
                advance(ra0, rb0, ra0, rb0, 1, step + 4);
                __syncthreads();
            }
        }

        // Epilogue: lane holds row fragment_row of each MFMA tile in runs of
        // four consecutive columns. The bias of each whole run (inside N) is
        // read once for all the tile's rows, all runs' loads in flight
        // together; a run that N cuts reads its bias element by element.
        float run_bias[TN][Mma<T>::kRuns][4] = {};
        if (bias != nullptr) {
            // The resource ends at N: a run past N reads zeros, with no select
            // on the offset (a run that N cuts is not read from here).
            const auto bias_resource = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(bias), static_cast<short>(0), args.n * 4, 0x00020000);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
#pragma unroll
                for (int q = 0; q < Mma<T>::kRuns; ++q) {
                    const int col = col0 + wave_n * TN * E + j * E + Mma<T>::column(lane, q);
                    const Vec16 v = buffer_load16(bias_resource, static_cast<unsigned int>(col) * 4U);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        run_bias[j][q][r] = __uint_as_float(v.w[r]);
                    }
                }
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = row0 + wave_m * TM * E + i * E + fragment_row;
            if (row >= args.m) {
                continue;
            }
            // Batch entries run as one problem: the entry's own row.
            int local = row;
            std::int64_t c_offset = static_cast<std::int64_t>(row) * args.ldc;
            if (args.rows_per_entry > 0) {
                const int entry_index = row / args.rows_per_entry;
                local = row - entry_index * args.rows_per_entry;
                c_offset = entry_index * args.stride_c + static_cast<std::int64_t>(local) * args.ldc;
            }
            T* const c_row = c_entry + c_offset;
            // C may alias nothing the kernel reads, but the compiler cannot
            // know it: read the row's old values for all runs before the
            // first store, so the loads overlap instead of each waiting
            // behind the store before it.
            typename Quad<T>::Type old[TN][Mma<T>::kRuns] = {};
            if (vector_c && args.accumulate) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
#pragma unroll
                    for (int q = 0; q < Mma<T>::kRuns; ++q) {
                        const int col = col0 + wave_n * TN * E + j * E + Mma<T>::column(lane, q);
                        if (col + 3 < args.n) {
                            old[j][q] = *reinterpret_cast<const typename Quad<T>::Type*>(c_row + col);
                        }
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
#pragma unroll
                for (int q = 0; q < Mma<T>::kRuns; ++q) {
                    const int col = col0 + wave_n * TN * E + j * E + Mma<T>::column(lane, q);
                    if (col >= args.n) {
                        continue;
                    }
                    const bool whole_run = col + 3 < args.n;
                    float value[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        value[r] = 0.F;
                        if (col + r < args.n) {
                            const float bias_value =
                                bias == nullptr ? 0.F : whole_run ? run_bias[j][q][r] : bias[col + r];
                            value[r] = epilogue_value(acc[i][j][4 * q + r], bias != nullptr, bias_value,
                                                      local, col + r, args);
                        }
                    }
                    if (vector_c && whole_run) {
                        store4(c_row + col, value, args.accumulate, old[j][q]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (col + r < args.n) {
                                float v = value[r];
                                if (args.accumulate) {
                                    v = add_unfused(Elem<T>::load(c_row + col + r), v);
                                }
                                Elem<T>::store(c_row + col + r, v);
                            }
                        }
                    }
                }
            }
        }
        // The k loop ended on a barrier, so the next entry may refill LDS.
    }
}

} // namespace cuvit::detail::gemm
