// fp32 GEMM for tall problems with B as [N, K] (the model's linear layers:
// 6304 rows against 192-768 columns at ViT-Tiny batch 32).
//
// A workgroup owns a panel of BN consecutive columns of C and a range of
// 16-row tiles. It stages B's panel rows into LDS once, the whole of K, and
// after that one barrier its wavefronts never wait on each other again: each
// wavefront walks its own (row tile, column part) items, loads its A
// fragments from global memory straight into the MFMA operand layout (no LDS
// round trip for A), and reads B fragments from the resident panel. A's
// fragments for the next register group are in flight while the current
// group's MFMAs run.
//
// Same arithmetic as gemm_kernel<float>: lane l holds row l % 16 of A and of
// the panel at k chunk l / 16, k-blocks of 16 are walked in ascending order
// over K rounded up to a multiple of 64, and element s of a fragment feeds the
// s-th of four v_mfma_f32_16x16x4_f32 (B fragment as the first operand). So
// every accumulator sees the same MFMAs with the same operands in the same
// order as in the LDS-tiled kernel, and the two give bitwise equal results;
// the epilogue (alpha, bias, GELU, store or accumulate) is the same function.
// Elements past M, N or K read as zero; results past M are not stored, and N
// is a multiple of 4 so a run of four columns is all in or all out.
#pragma once

#include "gemm_kernel.hpp"

namespace cuvit::detail::gemm {

/// @tparam KB k-blocks of 16 walked (K rounded up to a multiple of 64, / 16)
/// @tparam BN panel width (columns of C, rows of B)
/// @tparam TN 16-column MFMA tiles per wavefront item
/// @tparam KG k-blocks of A per register group
/// @tparam W wavefronts per workgroup
template <int KB, int BN, int TN, int KG, int W> struct PanelShape {
    static_assert(KB % 4 == 0, "K walked in spans of 64");
    static_assert(BN % (16 * TN) == 0, "a panel is whole wavefront items wide");
    static constexpr int kParts = BN / (16 * TN); // wavefronts sharing one row tile
    static_assert(W % kParts == 0, "every wavefront keeps one column part");
    static constexpr int kRowStride = W / kParts; // row tiles between a wavefront's items
    static_assert(KB % KG == 0, "register groups split K evenly");
    static constexpr int kGroups = KB / KG;
    static_assert(KG >= TN, "a step has a k-block for each epilogue slice");
    /// Floats per LDS panel row: 16 KB plus a 16-byte pad, so that the 16
    /// lanes reading one fragment column (16 rows, same k) hit 16 different
    /// bank quads (16 KB floats is a multiple of 64 banks).
    static constexpr int kPitch = 16 * KB + 4;
    static constexpr std::size_t kLdsBytes = static_cast<std::size_t>(BN) * kPitch * sizeof(float);
    static constexpr int kThreads = kWave * W;
    static constexpr int kChunks = BN * 4 * KB; // 16-byte chunks of the panel
    static constexpr int kChunksPerThread = (kChunks + kThreads - 1) / kThreads;
};

/// @p groups row-tile ranges per panel: workgroup x computes panel x / groups
/// over range x % groups. The epilogue's parts are compile-time; there is no
/// addend, and kAlpha false means alpha is 1 (1 * x is x, bit for bit).
template <int KB, int BN, int TN, int KG, int W, bool kAlpha, bool kBias, bool kGelu, bool kAccumulate>
__global__ __launch_bounds__(kWave * W) void gemm_panel_kernel(const float* __restrict__ a,
                                                             const float* __restrict__ b,
                                                             const float* __restrict__ bias,
                                                             float* c, GemmArgs args, int groups) {
    using S = PanelShape<KB, BN, TN, KG, W>;
    constexpr int G = S::kGroups;
    extern __shared__ Vec16 lds_vectors[];
    float* const panel = reinterpret_cast<float*>(lds_vectors);

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int fragment_row = lane % 16;
    const int fragment_chunk = lane / 16;

    const int panel_index = static_cast<int>(blockIdx.x) / groups;
    const int group = static_cast<int>(blockIdx.x) % groups;
    const int col0 = panel_index * BN;
    const int tiles_m = (args.m + 15) / 16;
    const int tile_hi = split_point(tiles_m, groups, group + 1);
    const int part = wave % S::kParts;
    const int first_tile = split_point(tiles_m, groups, group) + wave / S::kParts;
    const int tiles = first_tile < tile_hi ? (tile_hi - first_tile + S::kRowStride - 1) / S::kRowStride : 0;

    // Panel loads: B rows col0 .. col0 + BN, k 0 .. 16 KB; zero past N and K.
    const auto b_resource = buffer_resource(b + static_cast<std::int64_t>(col0) * args.ldb);
    const int b_rows = args.n - col0;
    Vec16 staged[S::kChunksPerThread];
#pragma unroll
    for (int p = 0; p < S::kChunksPerThread; ++p) {
        const int q = t + S::kThreads * p;
        if (S::kChunks % S::kThreads == 0 || q < S::kChunks) {
            const int row = q / (4 * KB);
            const int k = 4 * (q % (4 * KB));
            staged[p] = buffer_load16(b_resource, chunk_offset<float>(row, b_rows, args.ldb, k, args.k));
        }
    }

    // This lane's row of the wavefront's @p n-th tile.
    auto tile_row = [&](int n) { return (first_tile + n * S::kRowStride) * 16 + fragment_row; };

    // A fragments of group @p g of the wavefront's @p n-th tile; a tile past
    // the wavefront's last reads nothing.
    const auto a_resource = buffer_resource(a);
    auto fetch = [&](Vec16 (&ra)[KG], int n, int g) {
        const int row = tile_row(n);
        const int k0 = 16 * KG * g + 4 * fragment_chunk;
        const bool live = n < tiles && row < args.m;
        const unsigned int base = static_cast<unsigned int>((row * args.lda + k0) * 4);
#pragma unroll
        for (int kb = 0; kb < KG; ++kb) {
            const bool inside = live && k0 + 16 * kb < args.k;
            ra[kb] = buffer_load16(a_resource, inside ? base + 64U * kb : kOutside);
        }
    };

    Vec16 ra[2][KG];
    fetch(ra[0], 0, 0);

#pragma unroll
    for (int p = 0; p < S::kChunksPerThread; ++p) {
        const int q = t + S::kThreads * p;
        if (S::kChunks % S::kThreads == 0 || q < S::kChunks) {
            const int row = q / (4 * KB);
            store16(panel + row * S::kPitch + 4 * (q % (4 * KB)), staged[p]);
        }
    }

    // The bias of the wavefront's columns, loaded once: lane l's column run
    // of tile j starts at column(j).
    auto column = [&](int j) { return col0 + part * 16 * TN + 16 * j + 4 * fragment_chunk; };
    float bias_value[TN][4];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
            bias_value[j][r] = kBias && column(j) < args.n ? bias[column(j) + r] : 0.0F;

    __syncthreads();

    // A lane with nothing to store (row past M, columns past N) stores to an
    // offset the buffer resource drops, so the epilogue has no branch.
    const auto c_resource = buffer_resource(c);
    auto c_offset = [&](int row, int j) {
        return row < args.m && column(j) < args.n ? static_cast<unsigned int>((row * args.ldc + column(j)) * 4)
                                                  : kOutside;
    };

    const float* const fragments = panel + (part * 16 * TN + fragment_row) * S::kPitch + 4 * fragment_chunk;
    floatx4 acc[TN];
    floatx4 old[TN];

    // MFMAs of group @p g over the A fragments in @p ra. B fragments are read
    // one k-block ahead of their MFMAs, two sets live: the schedule barrier
    // keeps the compiler from hoisting every k-block's LDS reads to the top,
    // which would hold TN * KG fragments at once.
    auto multiply = [&](const Vec16 (&fa)[KG], int g) {
        const float* const base = fragments + 16 * KG * g;
        Vec16 fb[2][TN];
#pragma unroll
        for (int j = 0; j < TN; ++j)
            fb[0][j] = load16(base + j * 16 * S::kPitch);
#pragma unroll
        for (int kb = 0; kb < KG; ++kb) {
            if (kb + 1 < KG) {
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    fb[(kb + 1) & 1][j] = load16(base + j * 16 * S::kPitch + 16 * (kb + 1));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        __uint_as_float(fb[kb & 1][j].w[s]), __uint_as_float(fa[kb].w[s]),
                        g == 0 && kb == 0 && s == 0 ? floatx4{0.F, 0.F, 0.F, 0.F} : acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    auto finish = [&](int n) {
        const int row = tile_row(n);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            floatx4 value;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // epilogue_value's steps with its flags fixed: alpha, the
                // bias, GELU, each rounded on its own.
#pragma clang fp contract(off)
                float v = acc[j][r];
                if constexpr (kAlpha) {
                    v = args.alpha * v;
                }
                if constexpr (kBias) {
                    v += bias_value[j][r];
                }
                if constexpr (kGelu) {
                    v = gelu(v);
                }
                value[r] = v;
            }
            if constexpr (kAccumulate) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    value[r] = add_unfused(old[j][r], value[r]);
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, value), c_resource, c_offset(row, j), 0, 0);
        }
    };

    // Tile n, its groups in order; step s = G n + g uses register set s % 2,
    // and the set it frees is refilled for step s + 2. Two tiles per trip
    // keep every set index a compile-time constant.
    auto tile = [&](int n, int parity) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int set = (parity + g) & 1;
            if constexpr (kAccumulate) {
                if (g == G - 1) {
                    // the old C, loaded ahead of the last group's MFMAs
                    const int row = tile_row(n);
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        old[j] = __builtin_bit_cast(floatx4, buffer_load16(c_resource, c_offset(row, j)));
                }
            }
            // step s + 1 into the other set, then this step's MFMAs
            fetch(ra[set ^ 1], g + 1 < G ? n : n + 1, g + 1 < G ? g + 1 : 0);
            multiply(ra[set], g);
        }
        finish(n);
    };

    for (int n = 0; n < tiles; n += 2) {
        tile(n, 0);
        if (n + 1 < tiles) {
            tile(n + 1, G & 1);
        }
    }
}

} // namespace cuvit::detail::gemm
