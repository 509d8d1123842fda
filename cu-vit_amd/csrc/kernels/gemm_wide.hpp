// The bf16 GEMM for large problems without accumulation (ViT-Base FC1 with
// GELU, QKV), B given as [N, K]: wider wavefront tiles than gemm_kernel.hpp's
// and an epilogue staged through LDS.
//
// Tile. A workgroup of four wavefronts owns a (2 TM 32) x (2 TN 32) tile of C;
// each wavefront owns TM x TN MFMA tiles of 32 x 32. With TM = 2, TN = 4
// (128 x 256 per workgroup, 64 x 128 per wavefront) a k-block costs a
// wavefront 6 fragment reads of 16 bytes per lane for 8 MFMAs, against 4 for
// 4 with gemm_kernel.hpp's 64 x 64 wavefront tiles: a quarter less LDS
// traffic per MFMA, which is what bounds that kernel. Stages are 32 deep
// (rows of four 16-byte chunks, chunk c of row r at c ^ ((r >> 2) & 3), free of
// bank conflicts for both the stage writes and the fragment reads), double
// buffered in LDS, loaded into registers one stage ahead; two workgroups fit
// a CU (200 VGPRs, 64 KiB of LDS each).
//
// The MFMA sequence per output element is gemm_kernel.hpp's exactly: the same
// v_mfma_f32_32x32x16_bf16 with B in the first operand, over the same k-blocks
// in the same order (K rounded up to a multiple of 128, zeros beyond it), from
// an accumulator starting at +0. So the two kernels give bitwise the same C,
// and which one runs depends on the shape only.
//
// Epilogue. alpha, the bias and GELU are applied in registers (the tile's
// bias staged into LDS before the k loop, read from there; the flags, and
// whether alpha differs from 1, as template parameters: 1 * x is x, bit for
// bit), each
// value rounded once to bf16 and written into the LDS as a [BM][BN] tile with
// 16-byte chunk c of row r at c ^ (r % chunks_per_row); after a barrier each
// wavefront reads whole rows back and stores them with 16-byte non-temporal
// stores, so every 128-byte line of C is written by one instruction.
// Measured at ViT-Base FC1 + GELU (12608 x 3072 x 768) on one MI355X:
// 110 us against 137 us for gemm_kernel.hpp's 128 x 128 tiles, same bits.
// The epilogue there is still about a third of the time: 38.7 M erf
// evaluations are ~27 us of the whole GPU's VALU issue, and the two
// workgroups of a CU reach their epilogues together.
#pragma once

#include "gemm_kernel.hpp"

#include <type_traits>

namespace cuvit::detail::gemm {

template <int TM, int TN> struct WideShape {
    static constexpr int kE = 32;
    static constexpr int kBM = 2 * TM * kE;
    static constexpr int kBN = 2 * TN * kE;
    static constexpr int kBK = 32;
    static constexpr int kRowChunks = kBK / 8;  // 16-byte chunks per stage row
    static constexpr int kAPerThread = kBM * kRowChunks / kThreads;
    static constexpr int kBPerThread = kBN * kRowChunks / kThreads;
    static constexpr int kStageChunks = (kBM + kBN) * kRowChunks;
    static constexpr std::size_t kStageBytes = 2 * static_cast<std::size_t>(kStageChunks) * 16;
    static constexpr std::size_t kTileBytes = static_cast<std::size_t>(kBM) * kBN * 2;
    static constexpr std::size_t kCoreBytes = kStageBytes > kTileBytes ? kStageBytes : kTileBytes;
    /// The stages or the C tile, then the tile's bias (kBN floats).
    static constexpr std::size_t kLdsBytes = kCoreBytes + static_cast<std::size_t>(kBN) * 4;
    static_assert(kBM * kRowChunks % kThreads == 0 && kBN * kRowChunks % kThreads == 0,
                  "whole stage chunks per thread");

    /// LDS chunk of stage row @p r, chunk @p c.
    __device__ __forceinline__ static int stage_chunk(int r, int c) {
        return r * kRowChunks + (c ^ ((r >> 2) & 3));
    }
};

template <int TM, int TN, bool kBias, bool kGelu, bool kAlpha>
__global__ __launch_bounds__(kThreads, 2) void gemm_wide_kernel(const std::uint16_t* __restrict__ a,
                                                               const std::uint16_t* __restrict__ b,
                                                               const float* __restrict__ bias,
                                                               std::uint16_t* c, GemmArgs args,
                                                               TileMap map) {
    using S = WideShape<TM, TN>;
    constexpr int E = S::kE;
    constexpr int BM = S::kBM;
    constexpr int BN = S::kBN;
    constexpr int RC = S::kRowChunks;
    extern __shared__ Vec16 lds_vectors[];
    Vec16* const lds = lds_vectors;

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = t / kWave;
    const int wave_m = wave / 2;
    const int wave_n = wave % 2;
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
            return;  // this block has fewer tiles than the grid allows; no barrier is skipped
        }
        tile_m = m_lo + index / width;
        tile_n = n_lo + index % width;
    }
    const int row0 = tile_m * BM;
    const int col0 = tile_n * BN;
    const int steps = (args.k + kSpan<std::uint16_t> - 1) / kSpan<std::uint16_t> *
                      (kSpan<std::uint16_t> / S::kBK);

    // The tile's bias into LDS once, ahead of every k loop, columns past N
    // reading as zero: the epilogue then reads it from LDS instead of waiting
    // on global loads after the k loop.
    float* const tile_bias = reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(lds_vectors) +
                                                      S::kCoreBytes);
    if constexpr (kBias) {
        if (threadIdx.x < BN / 4) {
            const int col = col0 + 4 * static_cast<int>(threadIdx.x);
            // N is a multiple of 8 here, so a run of four starts and ends inside
            const Vec16 v = buffer_load16(buffer_resource(bias),
                                          col < args.n ? static_cast<unsigned int>(col) * 4U : kOutside);
            store16(tile_bias + 4 * threadIdx.x, v);
        }
        __syncthreads();
    }

    for (int entry = blockIdx.y; entry < args.count; entry += gridDim.y) {
        const Offsets off = entry_offsets(args, entry);
        const std::uint16_t* const a_tile = a + off.a + static_cast<std::int64_t>(row0) * args.lda;
        const std::uint16_t* const b_tile = b + off.b + static_cast<std::int64_t>(col0) * args.ldb;
        std::uint16_t* const c_entry = c + off.c;
        const auto a_resource = buffer_resource(a_tile);
        const auto b_resource = buffer_resource(b_tile);
        const int a_rows = args.m - row0;
        const int b_rows = args.n - col0;

        floatx16 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[i][j][r] = 0.F;

        Vec16 ra[S::kAPerThread];
        Vec16 rb[S::kBPerThread];
        auto fetch = [&](int step) {
            const int k0 = step * S::kBK;
#pragma unroll
            for (int p = 0; p < S::kAPerThread; ++p) {
                const int q = t + kThreads * p;
                ra[p] = buffer_load16(a_resource, chunk_offset<std::uint16_t>(
                                                      q / RC, a_rows, args.lda, k0 + 8 * (q % RC), args.k));
            }
#pragma unroll
            for (int p = 0; p < S::kBPerThread; ++p) {
                const int q = t + kThreads * p;
                rb[p] = buffer_load16(b_resource, chunk_offset<std::uint16_t>(
                                                      q / RC, b_rows, args.ldb, k0 + 8 * (q % RC), args.k));
            }
        };
        auto stage = [&](int buffer) {
            Vec16* const base = lds + buffer * S::kStageChunks;
#pragma unroll
            for (int p = 0; p < S::kAPerThread; ++p) {
                const int q = t + kThreads * p;
                base[S::stage_chunk(q / RC, q % RC)] = ra[p];
            }
#pragma unroll
            for (int p = 0; p < S::kBPerThread; ++p) {
                const int q = t + kThreads * p;
                base[BM * RC + S::stage_chunk(q / RC, q % RC)] = rb[p];
            }
        };
        auto compute = [&](int buffer) {
            const Vec16* const base = lds + buffer * S::kStageChunks;
#pragma unroll
            for (int kb = 0; kb < S::kBK / 16; ++kb) {
                Vec16 fa[TM];
                Vec16 fb[TN];
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    fa[i] = base[S::stage_chunk(wave_m * TM * E + i * E + fragment_row,
                                                2 * kb + fragment_chunk)];
                }
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    fb[j] = base[BM * RC + S::stage_chunk(wave_n * TN * E + j * E + fragment_row,
                                                          2 * kb + fragment_chunk)];
                }
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        Mma<std::uint16_t>::run(acc[i][j], fb[j], fa[i]);
            }
        };

        // Stage s in LDS buffer s % 2; the registers carry stage s + 1 while
        // stage s is multiplied. The loop always runs whole: a stage past K
        // reads as zero and its MFMAs add exact zeros. The scheduling
        // barriers keep the next stage's loads ahead of the MFMAs and the
        // LDS writes after them (110 us for FC1 against 126 us with the
        // compiler's own order, which sank the loads to the stage's end).
        fetch(0);
        stage(0);
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            fetch(s + 1);
            __builtin_amdgcn_sched_barrier(0);
            compute(s & 1);
            __builtin_amdgcn_sched_barrier(0);
            stage((s + 1) & 1);
            __syncthreads();
        }

        // Epilogue through LDS: the k loop ended on a barrier, so the stage
        // buffers are free. The bias of the lane's 64 columns (tile j, run q
        // of four columns) comes from the tile's bias in LDS (held in
        // registers over the k loop it would cost the registers of a second
        // workgroup).
        float column_bias[TN][4][4];
        if constexpr (kBias) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const Vec16 v =
                        load16(tile_bias + wave_n * TN * E + j * E + Mma<std::uint16_t>::column(lane, q));
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        column_bias[j][q][e] = __uint_as_float(v.w[e]);
                    }
                }
        }
        constexpr int kTileChunks = BN / 8;  // 16-byte chunks per row of the C tile
        unsigned char* const tile = reinterpret_cast<unsigned char*>(lds);
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int r = wave_m * TM * E + i * E + fragment_row;
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        // The order of gemm_kernel.hpp's epilogue_value: alpha * sum,
                        // then the bias, each rounded on its own.
#pragma clang fp contract(off)
                        float x = kAlpha ? args.alpha * acc[i][j][4 * q + e] : acc[i][j][4 * q + e];
                        if constexpr (kBias) {
                            x += column_bias[j][q][e];
                        }
                        v[e] = kGelu ? gelu(x) : x;
                    }
                    uint2 bits;
                    bits.x = pack_bf16x2(v[0], v[1]);
                    bits.y = pack_bf16x2(v[2], v[3]);
                    const int chunk = (wave_n * TN * E + j * E) / 8 + q;
                    *reinterpret_cast<uint2*>(tile + r * (BN * 2) +
                                              ((chunk ^ (r % kTileChunks)) * 16) + (lane / 32) * 8) =
                        bits;
                }
        }
        __syncthreads();
        constexpr int kRowsPerStore = kWave / kTileChunks;
        constexpr int kStoreRounds = BM / (4 * kRowsPerStore);
        // Four rounds' LDS reads issued together, then their stores: a read
        // per store, each waited on before its store, left the LDS latency
        // exposed sixteen times a tile.
        constexpr int kBatch = kStoreRounds % 4 == 0 ? 4 : 1;
        const int chunk = lane % kTileChunks;
        const int col = col0 + 8 * chunk;
#pragma unroll 1
        for (int it0 = 0; it0 < kStoreRounds; it0 += kBatch) {
            Vec16 v[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int r = ((it0 + u) * 4 + wave) * kRowsPerStore + lane / kTileChunks;
                v[u] = *reinterpret_cast<const Vec16*>(tile + r * (BN * 2) +
                                                       ((chunk ^ (r % kTileChunks)) * 16));
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int row = row0 + ((it0 + u) * 4 + wave) * kRowsPerStore + lane / kTileChunks;
                if (row < args.m && col < args.n) {  // N is a multiple of 8 on this path
                    store16_streaming(c_entry + static_cast<std::int64_t>(row) * args.ldc + col, v[u]);
                }
            }
        }
        __syncthreads();  // the next entry refills the LDS
    }
}

} // namespace cuvit::detail::gemm
