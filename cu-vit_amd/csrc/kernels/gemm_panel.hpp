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
// over K (here a multiple of 64, as the tiled kernel rounds it), and element
// s of a fragment feeds the s-th of four v_mfma_f32_16x16x4_f32 (B fragment
// as the first operand). So every accumulator sees the same MFMAs with the
// same operands in the same order as in the LDS-tiled kernel, and the two
// give bitwise equal results; the epilogue (alpha, bias, GELU, store or
// accumulate) takes the same steps. Rows past M and panel rows past N read
// as zero; results past M are not stored, and N is a multiple of 4 so a run
// of four columns is all in or all out. An out-of-range offset (kOutside)
// plus a group's 64-byte steps stays past the buffer resource's record
// count, so it reads zero.
#pragma once

#include "gemm_kernel.hpp"

namespace cuvit::detail::gemm {

/// @tparam KB k-blocks of 16 (K = 16 KB, a multiple of 64)
/// @tparam BN panel width (columns of C, rows of B)
/// @tparam TN 16-column MFMA tiles of a full wavefront item (even: a half
///         item has TN / 2)
/// @tparam KG k-blocks of A per register group
/// @tparam W wavefronts per workgroup (a multiple of the 4 SIMDs)
template <int KB, int BN, int TN, int KG, int W> struct PanelShape {
    static_assert(KB % 4 == 0, "K walked in spans of 64");
    static_assert(TN % 2 == 0, "a full item splits into two halves");
    static_assert(BN % (16 * TN) == 0, "a panel is whole items wide");
    static constexpr int kParts = BN / (16 * TN); // full items across the panel
    static_assert(W % 4 == 0, "the same number of wavefronts on every SIMD");
    static constexpr int kPerSimd = W / 4;
    static_assert(KB % KG == 0, "register groups split K evenly");
    static constexpr int kGroups = KB / KG;
    /// Floats per LDS panel row: 16 KB plus a 16-byte pad, so that the 16
    /// lanes reading one fragment column (16 rows, same k) hit 16 different
    /// bank quads (16 KB floats is a multiple of 64 banks).
    static constexpr int kPitch = 16 * KB + 4;
    static constexpr int kPanelFloats = BN * kPitch;
    /// The panel, then the panel's BN bias values.
    static constexpr std::size_t kLdsBytes = static_cast<std::size_t>(kPanelFloats + BN) * sizeof(float);
    static constexpr int kThreads = kWave * W;
    static constexpr int kChunks = BN * 4 * KB; // 16-byte chunks of the panel
    static constexpr int kChunksPerThread = (kChunks + kThreads - 1) / kThreads;
};

/// @p groups row-tile ranges per panel: workgroup x computes panel x / groups
/// over range x % groups. The epilogue's parts are compile-time (kAddend: the
/// [m, n] addend after the bias, the model's positional add), and kAlpha
/// false means alpha is 1 (1 * x is x, bit for bit). With
/// args.rows_per_entry > 0 the rows are batch entries run as one problem:
/// row p is stored as row p % rows_per_entry of entry p / rows_per_entry.
///
/// Work split. A workgroup's R row tiles make U = R * kParts full items
/// (16 x 16 TN). The first 4 floor(U / 4) go round robin to the four SIMDs,
/// the rest are cut into half items (16 x 8 TN) dealt the same way, so no
/// SIMD carries more than half an item beyond another: the MFMA pipe is the
/// bound, and a whole item's difference would idle three SIMDs for its
/// length. The wavefronts of a SIMD take its items in turn; wavefronts w and
/// w + 4 share a SIMD (the CU places a workgroup's wavefronts on its SIMDs
/// in turn, read from the hardware id register on MI355X).
template <int KB, int BN, int TN, int KG, int W, bool kAlpha, bool kBias, bool kGelu, bool kAccumulate,
          bool kAddend = false>
__global__ __launch_bounds__(kWave * W) void gemm_panel_kernel(const float* __restrict__ a,
                                                             const float* __restrict__ b,
                                                             const float* __restrict__ bias,
                                                             float* c, GemmArgs args, int groups) {
    using S = PanelShape<KB, BN, TN, KG, W>;
    constexpr int G = S::kGroups;
    constexpr int kHalf = TN / 2;
    extern __shared__ Vec16 lds_vectors[];
    float* const panel = reinterpret_cast<float*>(lds_vectors);
    float* const panel_bias = panel + S::kPanelFloats;

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int fragment_row = lane % 16;
    const int fragment_chunk = lane / 16;

    const int panel_index = static_cast<int>(blockIdx.x) / groups;
    const int group = static_cast<int>(blockIdx.x) % groups;
    const int col0 = panel_index * BN;
    const int tiles_m = (args.m + 15) / 16;
    const int tile_lo = split_point(tiles_m, groups, group);
    const int units = (split_point(tiles_m, groups, group + 1) - tile_lo) * S::kParts;
    const int whole = units / 4 * 4;           // full items, dealt four at a time
    const int halves = 2 * (units - whole);    // the rest, as half items
    const int simd = wave % 4;
    const int slot = wave / 4;
    const int full_per_simd = whole / 4;
    const int simd_items = full_per_simd + (simd < halves ? (halves - simd + 3) / 4 : 0);
    const int items = slot < simd_items ? (simd_items - slot + S::kPerSimd - 1) / S::kPerSimd : 0;

    // Item n of this wavefront: its row tile, its first column within the
    // panel, and whether it is a full item.
    struct Item {
        int tile;
        int column;
        bool full;
    };
    auto item = [&](int n) -> Item {
        const int e = slot + S::kPerSimd * n;
        if (e < full_per_simd) {
            const int u = simd + 4 * e;
            return {tile_lo + u / S::kParts, (u % S::kParts) * 16 * TN, true};
        }
        const int q = simd + 4 * (e - full_per_simd);
        const int u = whole + q / 2;
        return {tile_lo + u / S::kParts, (u % S::kParts) * 16 * TN + (q % 2) * 16 * kHalf, false};
    };

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
    // The panel's bias (zero past N, or without a bias).
    Vec16 staged_bias{{0U, 0U, 0U, 0U}};
    if (kBias && t < BN / 4) {
        staged_bias = buffer_load16(buffer_resource(bias), col0 + 4 * t < args.n
                                                               ? static_cast<unsigned int>((col0 + 4 * t) * 4)
                                                               : kOutside);
    }

    // A fragments of group @p g of row tile @p tile; an item past the
    // wavefront's last (@p live false) or a row past M reads nothing. K is
    // exactly 16 KB, so every k-block is inside; the k-blocks of a group sit
    // 64 bytes apart, which the loads take as immediate offsets.
    const auto a_resource = buffer_resource(a);
    auto fetch = [&](Vec16 (&ra)[KG], int tile, bool live, int g) {
        const int row = tile * 16 + fragment_row;
        const unsigned int base =
            live && row < args.m ? static_cast<unsigned int>((row * args.lda + 16 * KG * g + 4 * fragment_chunk) * 4)
                                 : kOutside;
#pragma unroll
        for (int kb = 0; kb < KG; ++kb) {
            ra[kb] = buffer_load16(a_resource, base + 64U * kb);
        }
    };

    Vec16 ra[2][KG];
    fetch(ra[0], item(0).tile, items > 0, 0);

#pragma unroll
    for (int p = 0; p < S::kChunksPerThread; ++p) {
        const int q = t + S::kThreads * p;
        if (S::kChunks % S::kThreads == 0 || q < S::kChunks) {
            const int row = q / (4 * KB);
            store16(panel + row * S::kPitch + 4 * (q % (4 * KB)), staged[p]);
        }
    }
    if (t < BN / 4) {
        store16(panel_bias + 4 * t, staged_bias);
    }
    __syncthreads();

    // A lane with nothing to store (row past M, columns past N) stores to an
    // offset the buffer resource drops, so the epilogue has no branch.
    const auto c_resource = buffer_resource(c);
    // Row @p row's place: its element offset in C and its row of the addend
    // (the entry's own row when entries run as one problem).
    struct Place {
        int c_row;
        int local;
    };
    auto place = [&](int row) -> Place {
        if (args.rows_per_entry > 0) {
            const int entry = row / args.rows_per_entry;
            const int local = row - entry * args.rows_per_entry;
            return {static_cast<int>(entry * args.stride_c) + local * args.ldc, local};
        }
        return {row * args.ldc, row};
    };
    auto c_offset = [&](int row, const Place& at, int column) {
        return row < args.m && column < args.n ? static_cast<unsigned int>((at.c_row + column) * 4)
                                               : kOutside;
    };
    const auto addend_resource = buffer_resource(kAddend ? args.addend : c);

    floatx4 acc[TN];
    floatx4 old[TN];

    // MFMAs of group @p g over the A fragments in @p fa, for the Tiles
    // 16-column tiles from panel column @p column. B fragments are read
    // kLead k-blocks ahead of their MFMAs (kLead + 1 sets live); the schedule
    // barrier keeps the compiler from hoisting every k-block's LDS reads to
    // the top.
    constexpr int kLead = KG > 2 ? 2 : 1;
    auto multiply = [&](auto tiles, const Vec16 (&fa)[KG], int g, int column) {
        constexpr int Tiles = decltype(tiles)::value;
        const float* const base = panel + (column + fragment_row) * S::kPitch + 16 * KG * g + 4 * fragment_chunk;
        Vec16 fb[kLead + 1][Tiles];
#pragma unroll
        for (int kb = 0; kb < kLead; ++kb)
#pragma unroll
            for (int j = 0; j < Tiles; ++j)
                fb[kb][j] = load16(base + j * 16 * S::kPitch + 16 * kb);
#pragma unroll
        for (int kb = 0; kb < KG; ++kb) {
            if (kb + kLead < KG) {
#pragma unroll
                for (int j = 0; j < Tiles; ++j)
                    fb[(kb + kLead) % (kLead + 1)][j] = load16(base + j * 16 * S::kPitch + 16 * (kb + kLead));
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int j = 0; j < Tiles; ++j)
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        __uint_as_float(fb[kb % (kLead + 1)][j].w[s]), __uint_as_float(fa[kb].w[s]),
                        g == 0 && kb == 0 && s == 0 ? floatx4{0.F, 0.F, 0.F, 0.F} : acc[j], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    auto load_old = [&](auto tiles, int row, int column) {
        constexpr int Tiles = decltype(tiles)::value;
        const Place at = place(row);
#pragma unroll
        for (int j = 0; j < Tiles; ++j)
            old[j] = __builtin_bit_cast(
                floatx4, buffer_load16(c_resource, c_offset(row, at, col0 + column + 16 * j + 4 * fragment_chunk)));
    };

    auto finish = [&](auto tiles, int row, int column) {
        constexpr int Tiles = decltype(tiles)::value;
        const Place at = place(row);
#pragma unroll
        for (int j = 0; j < Tiles; ++j) {
            const int within = column + 16 * j + 4 * fragment_chunk;
            floatx4 bias_value{0.F, 0.F, 0.F, 0.F};
            if constexpr (kBias) {
                bias_value = __builtin_bit_cast(floatx4, load16(panel_bias + within));
            }
            floatx4 addend_value{0.F, 0.F, 0.F, 0.F};
            if constexpr (kAddend) {
                const int column_index = col0 + within;
                addend_value = __builtin_bit_cast(
                    floatx4, buffer_load16(addend_resource,
                                           row < args.m && column_index < args.n
                                               ? static_cast<unsigned int>(
                                                     (at.local * args.ld_addend + column_index) * 4)
                                               : kOutside));
            }
            floatx4 value;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // epilogue_value's steps with its flags fixed: alpha, the
                // bias, the addend, GELU, each rounded on its own.
#pragma clang fp contract(off)
                float v = acc[j][r];
                if constexpr (kAlpha) {
                    v = args.alpha * v;
                }
                if constexpr (kBias) {
                    v += bias_value[r];
                }
                if constexpr (kAddend) {
                    v += addend_value[r];
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
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4, value), c_resource,
                                                   c_offset(row, at, col0 + within), 0, 0);
        }
    };

    // Item n, its groups in order; step s = G n + g uses register set s % 2,
    // and the set it frees is refilled for step s + 1. Two items per trip
    // keep every set index a compile-time constant.
    auto run_item = [&](int n, int parity) {
        const Item it = item(n);
        const Item next = item(n + 1);
        const int row = it.tile * 16 + fragment_row;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int set = (parity + g) & 1;
            if constexpr (kAccumulate) {
                if (g == G - 1) {
                    // the old C, loaded ahead of the last group's MFMAs
                    if (it.full) {
                        load_old(std::integral_constant<int, TN>{}, row, it.column);
                    } else {
                        load_old(std::integral_constant<int, kHalf>{}, row, it.column);
                    }
                }
            }
            // step s + 1 into the other set, then this step's MFMAs
            if (g + 1 < G) {
                fetch(ra[set ^ 1], it.tile, true, g + 1);
            } else {
                fetch(ra[set ^ 1], next.tile, n + 1 < items, 0);
            }
            if (it.full) {
                multiply(std::integral_constant<int, TN>{}, ra[set], g, it.column);
            } else {
                multiply(std::integral_constant<int, kHalf>{}, ra[set], g, it.column);
            }
        }
        if (it.full) {
            finish(std::integral_constant<int, TN>{}, row, it.column);
        } else {
            finish(std::integral_constant<int, kHalf>{}, row, it.column);
        }
    };

    for (int n = 0; n < items; n += 2) {
        run_item(n, 0);
        if (n + 1 < items) {
            run_item(n + 1, G & 1);
        }
    }
}

} // namespace cuvit::detail::gemm
