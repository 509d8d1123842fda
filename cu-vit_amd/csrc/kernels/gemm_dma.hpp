// The bf16 GEMM for the large products with B given as [N, K] (the ViT-Base
// linear layers): one persistent workgroup of eight wavefronts per CU, BM x 256
// tiles, operands brought into LDS by direct-to-LDS loads.
//
// Why this shape, measured on MI355X. A CU's memory pipeline moves about
// 1 KiB per 21 cycles into LDS, and a wavefront issuing a load waits its turn
// there (about 85 cycles with four wavefronts loading), so a stage's loads
// cost as much issue time as its MFMAs unless a tile brings at least
// 256 x 256 outputs per 64-deep stage; and with two wavefronts per SIMD one
// wavefront's MFMAs run while the other waits to issue a load. So all eight
// wavefronts walk the same tile (each (BM / 2) x 64 of it); one wavefront per
// SIMD issues the next stage's loads right after each stage barrier while the
// other keeps the MFMAs going; and the tile sizes
// (320 x 256 for FC1, 256 x 256 for QKV, 192 x 256 for FC2 and the
// projection at ViT-Base b64) give one or two nearly full rounds on 256 CUs.
//
// Operands. 64-deep LDS stages, rows of 128 bytes: B in a ring of two, A in
// a ring of three where LDS allows (192-row tiles: A's loads then go out two
// stages ahead, which took FC2 from 82 to 72-74 us with A from HBM). One
// buffer_load_dwordx4 ... lds moves eight whole 128-byte rows, lane
// l's 16 bytes landing at the instruction's LDS base + 16 l; those loads are
// issued from inline assembly and waited for by hand (s_waitcnt vmcnt before
// each stage's barrier, leaving the newest stage's A loads in flight when A
// runs two ahead), so the compiler neither waits for them early nor drains
// them at other barriers. Chunk c of stage row r sits in 16-byte
// slot c ^ ((r >> 1) & 7): conflict-free for the stage writes and for the
// fragment reads (lane l: row l % 32, chunk 2 kb + l / 32). The last stage of
// a tile brings the next tile's first stage.
//
// Epilogue. Each wavefront finishes its accumulator tiles in pairs (i, 0) and
// (i, 1), 32 rows by 64 columns: alpha, bias, GELU, + old C, one rounding to
// bf16, written in the MFMA layout into its own 4 KiB area of the B slot just
// consumed, then read back as whole 128-byte rows and stored eight lanes per
// row (old C comes in the same way). Stores that cover 32 bytes of 32 rows
// each, straight from the MFMA layout, measured several times slower.
//
// Arithmetic. Each output is the sum gemm_kernel.hpp computes: the same
// v_mfma_f32_32x32x16_bf16 with B in the first operand, over K rounded up to
// a multiple of 128 in order, from +0; then alpha * sum, + bias, + addend,
// GELU, + old C (unfused, in that order) and one rounding. So this kernel is bitwise equal
// to the other bf16 kernels and which one runs depends on the shape only.
#pragma once

#include "gemm_kernel.hpp"

#include <type_traits>
#include <utility>

namespace cuvit::detail::gemm {

/// Calls @p f with std::integral_constant<int, 0> .. <N - 1>, in order.
template <typename F, int... I>
__device__ __forceinline__ void static_for_each(F& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F> __device__ __forceinline__ void static_for(F&& f) {
    static_for_each(f, std::make_integer_sequence<int, N>{});
}

typedef int sgpr4 __attribute__((ext_vector_type(4)));

/// A raw buffer descriptor in SGPRs: @p bytes records from @p base, 32-bit
/// untyped; offsets at or past @p bytes read as zero.
__device__ __forceinline__ sgpr4 scalar_resource(const void* base, unsigned int bytes) {
    const auto address = reinterpret_cast<std::uint64_t>(base);
    sgpr4 d;
    d.x = __builtin_amdgcn_readfirstlane(static_cast<int>(address & 0xFFFFFFFFU));
    d.y = __builtin_amdgcn_readfirstlane(static_cast<int>((address >> 32) & 0xFFFFU));
    d.z = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
    d.w = 0x00020000;
    return d;
}

/// The LDS byte address of a shared-memory pointer.
__device__ __forceinline__ unsigned int lds_address(const void* p) {
    return static_cast<unsigned int>(
        reinterpret_cast<std::size_t>((__attribute__((address_space(3))) const char*)p));
}

/// Sixteen bytes per lane from @p resource at byte @p offset into LDS at
/// @p m0 + 16 lane; not tracked by the compiler (waited for by hand).
__device__ __forceinline__ void load_to_lds(unsigned int m0, unsigned int offset, sgpr4 resource) {
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(m0), "v"(offset), "s"(resource)
                 : "memory", "m0");
}

/// This wavefront's memory operations (when @p memory) and LDS reads done,
/// then the workgroup.
__device__ __forceinline__ void stage_barrier(bool memory) {
    if (memory) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" : : : "memory");
    } else {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory");
    }
}

template <int BM> struct DmaShape {
    static constexpr int kThreads = 512;
    static constexpr int kBN = 256;
    static constexpr int kTM = BM / 64;  // MFMA tiles per wavefront: 2 x 4 wavefronts
    static constexpr int kTN = 2;
    static_assert(kBN / 4 == 64, "one wavefront loads the tile's bias, four columns per lane");
    // A stage is BM rows of A and 256 of B, 64 bf16 of k (128 bytes) per row,
    // in two rings: B's holds two stages, A's three where LDS allows (192-row
    // tiles), so that A's loads go out two stages ahead of their use.
    static constexpr int kASlotBytes = BM * 128;
    static constexpr int kBSlotBytes = kBN * 128;
    static constexpr int kASlots = 3 * kASlotBytes + 2 * kBSlotBytes + 1024 + 32 <= 160 * 1024 ? 3 : 2;
    static constexpr int kAhead = kASlots - 1;  // stages A's loads run ahead
    static constexpr int kBOffset = kASlots * kASlotBytes;
    static constexpr int kBiasOffset = kBOffset + 2 * kBSlotBytes;

    static constexpr int kLoads = (BM + kBN) / 32;  // load instructions per loading wavefront per stage
    static constexpr int kLoadsA = BM / 32;
    static constexpr int kRoleOffset = kBiasOffset + kBN * 4;  // eight SIMD ids at start-up
    static constexpr int kLdsBytes = kRoleOffset + 8 * 4;
    static_assert(BM % 64 == 0, "whole MFMA tiles per wavefront");
    static_assert(kBSlotBytes >= 8 * 4096, "a consumed B slot holds every wavefront's staging");
    static_assert(kLdsBytes <= 160 * 1024, "LDS");
};

/// @tparam kAddend an [m, n] fp32 term added after the bias (args.addend; the
///   model's positional add in the patch embedding), its row the output row
///   within its batch entry; this instance also takes batch entries run as one
///   problem (args.rows_per_entry > 0), each row stored back in its entry (the
///   others keep that arithmetic out of their epilogue: FC1's instance, at
///   256 VGPRs, measured 75 -> 86 us with it).
template <int BM, bool kBias, bool kGelu, bool kAlpha, bool kAccumulate, bool kAddend = false>
__global__ __launch_bounds__(512, 1) void gemm_dma_kernel(const std::uint16_t* __restrict__ a,
                                                          const std::uint16_t* __restrict__ b,
                                                          const float* __restrict__ bias,
                                                          std::uint16_t* c, GemmArgs args, TileMap map) {
    using S = DmaShape<BM>;
    constexpr int BN = S::kBN;
    constexpr int TM = S::kTM;
    constexpr int TN = S::kTN;
    extern __shared__ Vec16 lds_vectors[];
    unsigned char* const lds = reinterpret_cast<unsigned char*>(lds_vectors);
    const unsigned int lds_base = __builtin_amdgcn_readfirstlane(lds_address(lds));

    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
    const int wave_m = wave / 4;
    const int wave_n = wave % 4;

    // One wavefront per SIMD loads the stages: it issues a whole stage right
    // after the barrier (waiting its turn at the memory pipeline) while the
    // other wavefront of its SIMD keeps the MFMAs going. HW_ID bits 5:4 give
    // the SIMD; if the eight are not two per SIMD, wavefronts 0-3 load.
    int* const simd_of = reinterpret_cast<int*>(lds + S::kRoleOffset);
    const int my_simd = __builtin_amdgcn_readfirstlane(
        static_cast<int>((__builtin_amdgcn_s_getreg(4 | (4 << 6) | (1 << 11))) & 3));
    if (lane == 0) {
        simd_of[wave] = my_simd;
    }
    __syncthreads();
    bool loader = wave < 4;
    int loader_index = wave % 4;
    {
        int ids[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            ids[w] = simd_of[w];
        }
        int rank = 0;
        bool pairs = true;
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            int same = 0;
#pragma unroll
            for (int v = 0; v < 8; ++v) {
                same += ids[v] == ids[w] ? 1 : 0;
            }
            pairs = pairs && same == 2;
            rank += (w < wave && ids[w] == my_simd) ? 1 : 0;
        }
        if (pairs) {
            loader = rank == 0;
            loader_index = my_simd;
        }
    }
    loader = __builtin_amdgcn_readfirstlane(loader ? 1 : 0) != 0;
    loader_index = __builtin_amdgcn_readfirstlane(loader_index);

    // This workgroup's tiles: its XCD's block of the tile grid, taken in turn
    // by the XCD's workgroups, row-major within the block.
    const int tiles_m = (args.m + BM - 1) / BM;
    const int tiles_n = (args.n + BN - 1) / BN;
    const int xcd = static_cast<int>(blockIdx.x) % 8;
    const int first = static_cast<int>(blockIdx.x) / 8;
    const int turns = static_cast<int>(gridDim.x) / 8;
    const int m_lo = split_point(tiles_m, map.px, xcd / map.py);
    const int m_hi = split_point(tiles_m, map.px, xcd / map.py + 1);
    const int n_lo = split_point(tiles_n, map.py, xcd % map.py);
    const int n_hi = split_point(tiles_n, map.py, xcd % map.py + 1);
    const int width = n_hi - n_lo;
    const int block_tiles = (m_hi - m_lo) * width;
    const int tiles = first < block_tiles ? (block_tiles - first + turns - 1) / turns : 0;
    if (tiles == 0) {
        return;  // the whole workgroup leaves before any barrier
    }
    auto origin = [&](int j, int& row0, int& col0) {
        const int index = first + j * turns;
        row0 = __builtin_amdgcn_readfirstlane((m_lo + index / width) * BM);
        col0 = __builtin_amdgcn_readfirstlane((n_lo + index % width) * BN);
    };
    const int stages = (args.k + 127) / 128 * 2;
    const int total_stages = tiles * stages;

    // -- stage loads. Instruction p of loader w fills stage rows
    // 32 p + 8 w .. + 8 (A rows for p < BM / 32, then B rows); lane l lands in
    // row + l / 8, slot l % 8, which holds chunk (l % 8) ^ ((row >> 1) & 7).
    const int load_chunk = (lane & 7) ^ ((4 * (loader_index & 1) + (lane >> 4)) & 7);
    const int load_row = 8 * loader_index + (lane >> 3);
    // Stage g's A goes to A slot g % kASlots, its B to B slot g % 2.
    struct StageLoads {
        sgpr4 resource;
        unsigned int m0;
        int k;
        bool active;
    };
    auto stage_loads = [&](int g, bool operand_a) {
        // Past the last stage the descriptors of the last tile are built and
        // nothing is issued (no branch around them: they stay in SGPRs).
        StageLoads l;
        l.active = g < total_stages;
        const int gc = l.active ? g : total_stages - 1;
        int row0, col0;
        origin(gc / stages, row0, col0);
        if (operand_a) {
            const int rows_a = min(args.m - row0, BM);
            l.resource = scalar_resource(a + static_cast<std::int64_t>(row0) * args.lda,
                                         static_cast<unsigned int>(rows_a * args.lda * 2));
            l.m0 = lds_base + static_cast<unsigned int>((gc % S::kASlots) * S::kASlotBytes + loader_index * 1024);
        } else {
            const int rows_b = min(args.n - col0, BN);
            l.resource = scalar_resource(b + static_cast<std::int64_t>(col0) * args.ldb,
                                         static_cast<unsigned int>(rows_b * args.ldb * 2));
            l.m0 = lds_base +
                   static_cast<unsigned int>(S::kBOffset + (gc & 1) * S::kBSlotBytes + loader_index * 1024);
        }
        l.k = (gc % stages) * 64 + 8 * load_chunk;
        return l;
    };
    // Row 32 p + load_row of an operand at k: the lane's byte offset for row
    // load_row plus p steps of 32 rows (a scalar), added per load. One
    // offset per row, held across the k loop, took 18 VGPRs: the compiler
    // spilled, and a reload between a stage's loads waited for all of them.
    // Past K the offset starts at kOutside, which stays past the descriptor's
    // range with any step, so the hardware returns zeros; rows past M fall
    // past it through the row offset itself.
    const unsigned int a_step = static_cast<unsigned int>(__builtin_amdgcn_readfirstlane(64 * args.lda));
    const unsigned int b_step = static_cast<unsigned int>(__builtin_amdgcn_readfirstlane(64 * args.ldb));
    auto issue_rows = [&](const StageLoads& l, int ld, unsigned int step, auto count) {
        if (!l.active) {
            return;
        }
        const unsigned int offset = l.k < args.k ? static_cast<unsigned int>((load_row * ld + l.k) * 2) : kOutside;
#pragma unroll
        for (int p = 0; p < decltype(count)::value; ++p) {
            load_to_lds(l.m0 + static_cast<unsigned int>(p * 4096), offset + static_cast<unsigned int>(p) * step,
                        l.resource);
        }
    };
    auto issue_a = [&](int g) {
        issue_rows(stage_loads(g, true), args.lda, a_step, std::integral_constant<int, S::kLoadsA>{});
    };
    auto issue_b = [&](int g) {
        issue_rows(stage_loads(g, false), args.ldb, b_step, std::integral_constant<int, S::kLoads - S::kLoadsA>{});
    };

    // -- fragments: A tile i at A slot row wave_m BM/2 + 32 i + lane % 32, B
    // tile j at B slot row 64 wave_n + 32 j + lane % 32; k chunk 2 kb + lane / 32.
    const int swizzle = ((lane & 31) >> 1) & 7;
    const unsigned int a_fragment = static_cast<unsigned int>((wave_m * (BM / 2) + (lane & 31)) * 128);
    const unsigned int b_fragment = static_cast<unsigned int>((wave_n * 64 + (lane & 31)) * 128);
    unsigned int fragment_column[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        fragment_column[kb] = static_cast<unsigned int>(((2 * kb + (lane >> 5)) ^ swizzle) * 16);
    }

    floatx16 acc[TM][TN];
    // The fragments of k-block kb + 1 are read while the MFMAs of kb run (two
    // register sets); scheduling barriers keep that order.
    auto compute = [&](int g) {
        const unsigned char* const base_a = lds + (g % S::kASlots) * S::kASlotBytes;
        const unsigned char* const base_b = lds + S::kBOffset + (g & 1) * S::kBSlotBytes;
        Vec16 fa[2][TM];
        Vec16 fb[2][TN];
        auto read = [&](int kb, int set) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                fa[set][i] = *reinterpret_cast<const Vec16*>(base_a + a_fragment + i * 4096 + fragment_column[kb]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                fb[set][j] = *reinterpret_cast<const Vec16*>(base_b + b_fragment + j * 4096 + fragment_column[kb]);
            }
        };
        read(0, 0);
        static_for<4>([&](auto block) {
            constexpr int kb = decltype(block)::value;
            if constexpr (kb < 3) {
                read(kb + 1, (kb + 1) & 1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    Mma<std::uint16_t>::run(acc[i][j], fb[kb & 1][j], fa[kb & 1][i]);
            __builtin_amdgcn_sched_barrier(0);
        });
    };

    // -- epilogue through the wavefront's 4 KiB staging area: 32 rows of 128
    // bytes, chunk c of row r at slot c ^ ((r >> 1) & 7).
    Vec16 old_rows[4];
    auto pair_row = [&](int pair, int row0, int k) {
        return row0 + wave_m * (BM / 2) + 32 * pair + 8 * k + (lane >> 3);
    };
    const int pair_col = wave_n * 64 + 8 * (lane & 7);
    // Output row -> its element offset in C (in its batch entry when the
    // entries run as one problem) and its row within the entry.
    auto local_row = [&](int row) {
        return kAddend && args.rows_per_entry > 0 ? row - (row / args.rows_per_entry) * args.rows_per_entry
                                                  : row;
    };
    auto c_offset = [&](int row) -> std::int64_t {
        if (kAddend && args.rows_per_entry > 0) {
            const int entry = row / args.rows_per_entry;
            return entry * args.stride_c + static_cast<std::int64_t>(row - entry * args.rows_per_entry) * args.ldc;
        }
        return static_cast<std::int64_t>(row) * args.ldc;
    };
    auto load_old = [&](int pair, int row0, int col0) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int row = pair_row(pair, row0, k);
            const int col = col0 + pair_col;
            old_rows[k] = row < args.m && col < args.n ? load16(c + c_offset(row) + col)
                                                       : Vec16{{0U, 0U, 0U, 0U}};
        }
    };
    auto finish_pair = [&](auto pair_c, unsigned char* staging, int row0, int col0) {
        constexpr int pair = decltype(pair_c)::value;
        auto staged = [&](int r, int chunk) {
            return staging + r * 128 + ((chunk ^ ((r >> 1) & 7)) * 16);
        };
        if constexpr (kAccumulate) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                *reinterpret_cast<Vec16*>(staged(8 * k + (lane >> 3), lane & 7)) = old_rows[k];
            }
            if (pair + 1 < TM) {
                load_old(pair + 1, row0, col0);  // the next pair's old C, in flight meanwhile
            }
        }
        const unsigned char* const bias_slot = lds + S::kBiasOffset;
        const int r = lane & 31;
        // The addend's four values of each run (j, q) of this lane's row,
        // all loads in flight before the first is used.
        Vec16 addend_runs[kAddend ? TN * 4 : 1];
        if constexpr (kAddend) {
            const int row = row0 + wave_m * (BM / 2) + 32 * pair + r;
            const int local = row < args.m ? local_row(row) : 0;
            const float* const addend_row = args.addend + static_cast<std::int64_t>(local) * args.ld_addend;
            static_for<TN>([&](auto tile_j) {
                constexpr int j = decltype(tile_j)::value;
                static_for<4>([&](auto run) {
                    constexpr int q = decltype(run)::value;
                    const int col = col0 + wave_n * 64 + 32 * j + Mma<std::uint16_t>::column(lane, q);
                    addend_runs[4 * j + q] =
                        row < args.m && col < args.n ? load16(addend_row + col) : Vec16{{0U, 0U, 0U, 0U}};
                });
            });
        }
        static_for<TN>([&](auto tile_j) {
            constexpr int j = decltype(tile_j)::value;
            static_for<4>([&](auto run) {
                constexpr int q = decltype(run)::value;
                uint2* const at = reinterpret_cast<uint2*>(staged(r, 4 * j + q) + 8 * (lane >> 5));
                float bias_value[4] = {0.F, 0.F, 0.F, 0.F};
                if constexpr (kBias) {
                    const Vec16 raw = *reinterpret_cast<const Vec16*>(
                        bias_slot + (wave_n * 64 + 32 * j + Mma<std::uint16_t>::column(lane, q)) * 4);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        bias_value[e] = __uint_as_float(raw.w[e]);
                    }
                }
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
#pragma clang fp contract(off)
                    float x = kAlpha ? args.alpha * acc[pair][j][4 * q + e] : acc[pair][j][4 * q + e];
                    if constexpr (kBias) {
                        x += bias_value[e];
                    }
                    if constexpr (kAddend) {
                        x += __uint_as_float(addend_runs[4 * j + q].w[e]);
                    }
                    v[e] = kGelu ? gelu(x) : x;
                }
                if constexpr (kAccumulate) {
                    const uint2 old = *at;
                    v[0] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.x & 0xFFFFU)), v[0]);
                    v[1] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.x >> 16)), v[1]);
                    v[2] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.y & 0xFFFFU)), v[2]);
                    v[3] = add_unfused(bf16_to_float(static_cast<std::uint16_t>(old.y >> 16)), v[3]);
                }
                *at = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
            });
        });
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int row = pair_row(pair, row0, k);
            const int col = col0 + pair_col;
            const Vec16 v = *reinterpret_cast<const Vec16*>(staged(8 * k + (lane >> 3), lane & 7));
            if (row < args.m && col < args.n) {  // N is a multiple of 8 on this path
                store16_streaming(c + c_offset(row) + col, v);
            }
        }
    };

    // Stage 0, and A's stages up to kAhead - 1, before the loop. With A two
    // stages ahead a stage waits for vmcnt(kLoadsA): every load but the
    // newest stage's A loads has landed.
    if (loader) {
#pragma unroll
        for (int g = 0; g < S::kAhead; ++g) {
            issue_a(g);
            if (g == 0) {
                issue_b(0);
            }
        }
    }
    for (int tile = 0; tile < tiles; ++tile) {
        int row0, col0;
        origin(tile, row0, col0);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[i][j][r] = 0.F;
        for (int step = 0; step < stages; ++step) {
            const int g = tile * stages + step;
            // Stage g's loads landed (the loaders wait for their own; a tile's
            // first stage already did, at the barrier before the previous
            // epilogue), and stage g - 1's slots are free for the loads below.
            // The newest kLoadsA loads are stage g + 1's A, issued during stage
            // g - 1 (or before the loop), unless g + 1 is past the last stage:
            // then nothing may stay in flight.
            if (loader && (step > 0 || tile == 0)) {
                if (S::kAhead == 2 && g + 1 < total_stages) {
                    static_assert(S::kLoadsA <= 63, "vmcnt");
                    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(S::kLoadsA) : "memory");
                } else {
                    stage_barrier(true);
                }
            } else {
                stage_barrier(false);
            }
            if (loader) {
                issue_b(g + 1);
                if (kBias && step == 0 && loader_index == 0) {
                    // the tile's bias (four columns per lane, BN / 4 == 64 lanes),
                    // read by the epilogue after the k loop
                    const int col = col0 + 4 * lane;
                    const unsigned int offset = col < args.n ? static_cast<unsigned int>(col) * 4U : kOutside;
                    load_to_lds(lds_base + static_cast<unsigned int>(S::kBiasOffset), offset,
                                scalar_resource(bias, static_cast<unsigned int>(args.n) * 4U));
                }
                issue_a(g + S::kAhead);
            }
            compute(g);
        }
        // Every wavefront done with the last stage, the bias and the next
        // tile's first stages landed: the last stage's B slot becomes the
        // staging areas.
        stage_barrier(true);
        unsigned char* const staging =
            lds + S::kBOffset + ((tile * stages + stages - 1) & 1) * S::kBSlotBytes + wave * 4096;
        if constexpr (kAccumulate) {
            load_old(0, row0, col0);
        }
        static_for<TM>([&](auto pair) { finish_pair(pair, staging, row0, col0); });
    }
}

} // namespace cuvit::detail::gemm
