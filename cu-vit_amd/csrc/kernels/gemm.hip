// Host dispatch of the batched GEMM. The kernels, all measured on MI355X at
// the ViT shapes and picked in this order:
//   fp32 (16 x 16 MFMA): the resident-panel kernel (gemm_panel.hpp) for
//        tall products with B as [N, K] and K of 192 or 768 (the ViT-Tiny
//        linear layers and patch embedding); else the tiled kernel
//        (gemm_kernel.hpp), 32 x 32 tiles, 64 x 64 once a problem has work
//        for more than 32 small tiles per compute unit.
//   bf16 (32 x 32 MFMA): the wide kernel (gemm_wide.hpp, 128 x 256 tiles)
//        for large products without accumulation (ViT-Base FC1, QKV); the
//        tiled kernel's twelve-wavefront 256 x 192 tile when one round of it
//        covers a product that 128 x 128 tiles would need more than two per
//        compute unit for (ViT-Base FC2, projection, patch embedding); else
//        128 x 128 once a problem fills every compute unit twice with it
//        (32-deep stages up to K = 1024), else 64 x 64.
// Every kernel of a type runs the same MFMA over K in the same order, so the
// choice never changes a result.
#include "gemm_dma.hpp"
#include "gemm_kernel.hpp"
#include "gemm_panel.hpp"
#include "gemm_wide.hpp"

namespace cuvit::detail {
namespace {

using cuvit::device::aligned16;
using gemm::kThreads;
using gemm::Shape;

constexpr int kMaxGridY = 65535;

/// True when every row of an operand starts on a 16-byte boundary and rows
/// of @p depth elements (the vector direction) hold whole 16-byte chunks.
template <typename T>
bool vector_operand(const T* base, int ld, int depth, std::int64_t stride, std::int64_t outer_stride,
                    bool split) {
    constexpr int V = gemm::Mma<T>::kPerVec;
    return aligned16(base) && ld % V == 0 && depth % V == 0 && stride % V == 0 &&
           (!split || outer_stride % V == 0);
}

/// True when the epilogue may store four results at once.
template <typename T> bool vector_output(const T* c, const GemmArgs& args) {
    const bool split = args.inner > 0;
    return (reinterpret_cast<std::uintptr_t>(c) % (4 * sizeof(T))) == 0 && args.ldc % 4 == 0 &&
           args.stride_c % 4 == 0 && (!split || args.outer_stride_c % 4 == 0);
}

/// The px x py split of an entry's tile grid among the 8 XCDs (px * py = 8)
/// that moves the fewest bytes into their L2 caches, A being read once per
/// column block and B once per row block, counting B double when its block
/// would not fit comfortably in one XCD's 4 MB L2. Measured on the ViT-Base
/// bf16 GEMMs: FC1 183 -> 173 us, FC2 129 -> 120 us. The fp32 ViT-Tiny GEMMs
/// (a few MB in all) gained nothing from it, so they keep row-major order.
gemm::TileMap tile_map(const GemmArgs& args, int bm, int bn, std::size_t element) {
    gemm::TileMap map{0, 0};
    const int tiles_m = (args.m + bm - 1) / bm;
    const int tiles_n = (args.n + bn - 1) / bn;
    if (element != 2 || static_cast<std::int64_t>(tiles_m) * tiles_n < 64) {
        return map;
    }
    const double a_bytes = static_cast<double>(tiles_m) * bm * args.k * element;
    const double b_bytes = static_cast<double>(tiles_n) * bn * args.k * element;
    constexpr double kL2Budget = 3.0 * (1 << 20);
    double best = 0.0;
    for (const int px : {8, 4, 2, 1}) {
        const int py = 8 / px;
        if (px > tiles_m || py > tiles_n) {
            continue;
        }
        double cost = py * a_bytes + px * b_bytes;
        if (b_bytes / py > kL2Budget) {
            cost *= 2.0;
        }
        if (map.px == 0 || cost < best) {
            best = cost;
            map = gemm::TileMap{px, py};
        }
    }
    return map;
}

template <typename T, int WM, int WN, int TM, int TN, int BK, int MinWaves, bool VecA, bool VecB,
          bool TransB>
hipError_t launch(const T* a, const T* b, const float* bias, T* c, const GemmArgs& args,
                  bool vector_c, hipStream_t stream) {
    using S = Shape<T, WM, WN, TM, TN, BK>;
    const gemm::TileMap map = tile_map(args, S::kBM, S::kBN, sizeof(T));
    const std::int64_t tiles_m = (args.m + S::kBM - 1) / S::kBM;
    const std::int64_t tiles_n = (args.n + S::kBN - 1) / S::kBN;
    // With the XCD split every block gets a workgroup slot per tile of the
    // largest block.
    const std::int64_t tiles = map.px > 0
                                   ? 8 * ((tiles_m + map.px - 1) / map.px) * ((tiles_n + map.py - 1) / map.py)
                                   : tiles_m * tiles_n;
    if (tiles > 0x7FFFFFFF) {
        return hipErrorInvalidConfiguration;
    }
    // The occupancy hint caps registers; the element-wise operand paths need
    // more than it leaves, so they take the default.
    constexpr int kMinWaves = VecA && VecB ? MinWaves : 1;
    auto kernel = gemm::gemm_kernel<T, WM, WN, TM, TN, BK, VecA, VecB, TransB, kMinWaves>;
    // Above 64 KiB of LDS a kernel has to opt in, once per device.
    static std::atomic<std::uint64_t> opted_in{0};
    if (const hipError_t opted = allow_lds(reinterpret_cast<const void*>(kernel), S::kLdsBytes, opted_in);
        opted != hipSuccess) {
        return opted;
    }
    const dim3 grid(static_cast<unsigned int>(tiles),
                    static_cast<unsigned int>(args.count < kMaxGridY ? args.count : kMaxGridY));
    kernel<<<grid, S::kThreads, S::kLdsBytes, stream>>>(a, b, bias, c, args, map, vector_c);
    return hipGetLastError();
}

template <typename T, int WM, int WN, int TM, int TN, int BK, int MinWaves = 1>
hipError_t pick_flags(const T* a, const T* b, const float* bias, T* c, const GemmArgs& args,
                      hipStream_t stream) {
    using S = Shape<T, WM, WN, TM, TN, BK>;
    const bool split = args.inner > 0;
    // Buffer offsets of a tile stay inside the span one descriptor addresses.
    bool vec_a = vector_operand(a, args.lda, args.k, args.stride_a, args.outer_stride_a, split) &&
                 static_cast<std::int64_t>(S::kBM) * args.lda * sizeof(T) < gemm::kMaxSpan;
    bool vec_b;
    if (args.transposed) {
        vec_b = vector_operand(b, args.ldb, args.k, args.stride_b, args.outer_stride_b, split) &&
                static_cast<std::int64_t>(S::kBN) * args.ldb * sizeof(T) < gemm::kMaxSpan;
    } else {
        vec_b = vector_operand(b, args.ldb, args.n, args.stride_b, args.outer_stride_b, split) &&
                static_cast<std::int64_t>(args.k) * args.ldb * sizeof(T) < gemm::kMaxSpan;
    }
    const bool vec_c = vector_output(c, args);
#define CUVIT_GEMM_LAUNCH(VA, VB)                                                                  \
    (args.transposed                                                                               \
         ? launch<T, WM, WN, TM, TN, BK, MinWaves, VA, VB, true>(a, b, bias, c, args, vec_c, stream) \
         : launch<T, WM, WN, TM, TN, BK, MinWaves, VA, VB, false>(a, b, bias, c, args, vec_c, stream))
    if (vec_a) {
        return vec_b ? CUVIT_GEMM_LAUNCH(true, true) : CUVIT_GEMM_LAUNCH(true, false);
    }
    return vec_b ? CUVIT_GEMM_LAUNCH(false, true) : CUVIT_GEMM_LAUNCH(false, false);
#undef CUVIT_GEMM_LAUNCH
}

/// @p args with a batch whose entries share B (stride 0) and whose A rows
/// follow one another run as one problem of all the entries' rows
/// (rows_per_entry: each output row goes back to its entry); @p args itself
/// otherwise. Every output is computed by the same operations either way.
GemmArgs as_one_problem(const GemmArgs& args) {
    GemmArgs whole = args;
    if (args.count > 1 && args.inner == 0 && args.stride_b == 0 && args.m > 0 &&
        args.stride_a == static_cast<std::int64_t>(args.m) * args.lda &&
        static_cast<std::int64_t>(args.m) * args.count <= 0x7FFFFFFF) {
        whole.m = args.m * args.count;
        whole.count = 1;
        whole.rows_per_entry = args.m;
    }
    return whole;
}

std::int64_t tile_count(const GemmArgs& args, int bm, int bn) {
    return static_cast<std::int64_t>((args.m + bm - 1) / bm) * ((args.n + bn - 1) / bn) * args.count;
}

} // namespace

/// The resident-panel kernel (gemm_panel.hpp) for a problem it covers: one
/// batch entry (or entries run as one, rows_per_entry), B as [N, K], K equal
/// to 16 KB, vector A and B, C written in 16-byte runs (N, ldc and the entry
/// stride multiples of 4, C 16-byte aligned), an addend only without GELU or
/// accumulation (and in 16-byte runs), every operand within one descriptor's
/// span, and at least eight wavefront items per compute unit. Returns
/// hipErrorNotSupported otherwise.
template <int KB, int BN, int TN, int KG, int W>
hipError_t launch_panel(const float* a, const float* b, const float* bias, float* c,
                        const GemmArgs& args, hipStream_t stream) {
    using S = gemm::PanelShape<KB, BN, TN, KG, W>;
    const std::int64_t tiles_m = (args.m + 15) / 16;
    const std::int64_t panels = (args.n + BN - 1) / BN;
    const bool with_addend = args.addend != nullptr;
    const std::int64_t c_span =
        args.rows_per_entry > 0
            ? ((args.m - 1) / args.rows_per_entry + 1) * args.stride_c
            : static_cast<std::int64_t>(args.m) * args.ldc;
    const bool eligible =
        args.count == 1 && args.transposed &&
        (!with_addend || (!args.gelu && !args.accumulate && aligned16(args.addend) &&
                          args.ld_addend % 4 == 0 &&
                          static_cast<std::int64_t>(args.m) * args.ld_addend * 4 < gemm::kMaxSpan)) &&
        args.k == 16 * KB && vector_operand(a, args.lda, args.k, 0, 0, false) &&
        vector_operand(b, args.ldb, args.k, 0, 0, false) && vector_output(c, args) && aligned16(c) &&
        args.n % 4 == 0 && static_cast<std::int64_t>(args.m) * args.lda * 4 < gemm::kMaxSpan &&
        c_span * 4 < gemm::kMaxSpan &&
        static_cast<std::int64_t>(BN) * args.ldb * 4 < gemm::kMaxSpan &&
        tiles_m * panels * S::kParts >= 8 * static_cast<std::int64_t>(compute_units());
    if (!eligible) {
        return hipErrorNotSupported;
    }
    // One workgroup per compute unit: the row tiles of a panel split into
    // as many ranges as there are compute units per panel.
    std::int64_t groups = compute_units() / panels;
    groups = groups < 1 ? 1 : groups > tiles_m ? tiles_m : groups;
    const dim3 grid(static_cast<unsigned int>(panels * groups));
    const int groups_argument = static_cast<int>(groups);
    auto run = [&](auto kernel) -> hipError_t {
        static std::atomic<std::uint64_t> opted_in{0};
        if (const hipError_t opted =
                allow_lds(reinterpret_cast<const void*>(kernel), S::kLdsBytes, opted_in);
            opted != hipSuccess) {
            return opted;
        }
        kernel<<<grid, S::kThreads, S::kLdsBytes, stream>>>(a, b, bias, c, args, groups_argument);
        return hipGetLastError();
    };
    // The epilogue's parts as template flags: alpha (when not 1), bias, GELU,
    // accumulate; the addend alone (the patch embedding's positional add).
    auto with_alpha = [&](auto alpha, auto with_bias, auto gelu, auto accumulate) -> hipError_t {
        return run(gemm::gemm_panel_kernel<KB, BN, TN, KG, W, decltype(alpha)::value,
                                           decltype(with_bias)::value, decltype(gelu)::value,
                                           decltype(accumulate)::value>);
    };
    if (with_addend) {
        auto with_bias = [&](auto alpha) -> hipError_t {
            constexpr bool kAlpha = decltype(alpha)::value;
            return bias != nullptr
                       ? run(gemm::gemm_panel_kernel<KB, BN, TN, KG, W, kAlpha, true, false, false, true>)
                       : run(gemm::gemm_panel_kernel<KB, BN, TN, KG, W, kAlpha, false, false, false, true>);
        };
        return args.alpha == 1.0F ? with_bias(std::false_type{}) : with_bias(std::true_type{});
    }
    auto with_accumulate = [&](auto with_bias, auto gelu) -> hipError_t {
        if (args.accumulate) {
            return args.alpha == 1.0F ? with_alpha(std::false_type{}, with_bias, gelu, std::true_type{})
                                      : with_alpha(std::true_type{}, with_bias, gelu, std::true_type{});
        }
        return args.alpha == 1.0F ? with_alpha(std::false_type{}, with_bias, gelu, std::false_type{})
                                  : with_alpha(std::true_type{}, with_bias, gelu, std::false_type{});
    };
    auto with_gelu = [&](auto with_bias) -> hipError_t {
        return args.gelu ? with_accumulate(with_bias, std::true_type{})
                         : with_accumulate(with_bias, std::false_type{});
    };
    return bias != nullptr ? with_gelu(std::true_type{}) : with_gelu(std::false_type{});
}

hipError_t gemm_f32(const float* a, const float* b, const float* bias, float* c,
                    const GemmArgs& args, hipStream_t stream) {
    // Tall single products with B as [N, K] (the model's linear layers): the
    // resident-panel kernel, bitwise equal to the tiles below. Measured at
    // ViT-Tiny batch 32 (6304 rows), against the tiled kernel: QKV 21.4 ->
    // 17.8 us, FC1 + GELU 27.9 -> 24.2, projection 10.7 -> 8.4, FC2 25.7 ->
    // 22.7. Wide panels with three wavefronts per SIMD suit the wide outputs,
    // 32-column panels the 192-wide ones.
    // A batch whose entries share B and whose A rows follow one another (the
    // patch embedding: 196 rows per image into rows 1.. of its 197) runs as
    // one problem of all its rows (ViT-Tiny b32 embedding 27 -> 22 us).
    const GemmArgs whole = as_one_problem(args);
    if (whole.n >= 512) {
        if (const hipError_t panel = launch_panel<12, 64, 2, 4, 12>(a, b, bias, c, whole, stream);
            panel != hipErrorNotSupported) {
            return panel;
        }
    } else if (const hipError_t panel = launch_panel<12, 32, 2, 4, 8>(a, b, bias, c, whole, stream);
               panel != hipErrorNotSupported) {
        return panel;
    }
    if (const hipError_t panel = launch_panel<48, 32, 2, 4, 12>(a, b, bias, c, whole, stream);
        panel != hipErrorNotSupported) {
        return panel;
    }
    if (tile_count(args, 32, 32) > static_cast<std::int64_t>(compute_units()) * 32) {
        return pick_flags<float, 2, 2, 2, 2, 32>(a, b, bias, c, args, stream);
    }
    return pick_flags<float, 2, 2, 1, 1, 32>(a, b, bias, c, args, stream);
}

/// The wide-tile kernel (gemm_wide.hpp) for a problem it covers: B as [N, K],
/// A and B vector operands within one descriptor's span, C written whole in
/// 16-byte pieces (N, ldc and the C strides multiples of 8, C 16-byte aligned),
/// no accumulation and no addend, and enough 128 x 256 tiles to fill every
/// CU's two slots. Returns hipErrorNotSupported otherwise.
template <int TM, int TN>
hipError_t launch_wide(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                       std::uint16_t* c, const GemmArgs& args, hipStream_t stream) {
    using S = gemm::WideShape<TM, TN>;
    const bool split = args.inner > 0;
    const bool eligible =
        args.transposed && !args.accumulate && args.addend == nullptr &&
        vector_operand(a, args.lda, args.k, args.stride_a, args.outer_stride_a, split) &&
        vector_operand(b, args.ldb, args.k, args.stride_b, args.outer_stride_b, split) &&
        static_cast<std::int64_t>(S::kBM) * args.lda * 2 < gemm::kMaxSpan &&
        static_cast<std::int64_t>(S::kBN) * args.ldb * 2 < gemm::kMaxSpan && aligned16(c) &&
        args.n % 8 == 0 && args.ldc % 8 == 0 && args.stride_c % 8 == 0 &&
        (!split || args.outer_stride_c % 8 == 0) &&
        tile_count(args, S::kBM, S::kBN) >= static_cast<std::int64_t>(compute_units()) * 2;
    if (!eligible) {
        return hipErrorNotSupported;
    }
    const gemm::TileMap map = tile_map(args, S::kBM, S::kBN, 2);
    const std::int64_t tiles_m = (args.m + S::kBM - 1) / S::kBM;
    const std::int64_t tiles_n = (args.n + S::kBN - 1) / S::kBN;
    const std::int64_t tiles = map.px > 0 ? 8 * ((tiles_m + map.px - 1) / map.px) *
                                                ((tiles_n + map.py - 1) / map.py)
                                          : tiles_m * tiles_n;
    if (tiles > 0x7FFFFFFF) {
        return hipErrorNotSupported;
    }
    const dim3 grid(static_cast<unsigned int>(tiles),
                    static_cast<unsigned int>(args.count < kMaxGridY ? args.count : kMaxGridY));
    auto run = [&](auto kernel) -> hipError_t {
        static std::atomic<std::uint64_t> opted_in{0};
        if (const hipError_t opted =
                allow_lds(reinterpret_cast<const void*>(kernel), S::kLdsBytes, opted_in);
            opted != hipSuccess) {
            return opted;
        }
        kernel<<<grid, kThreads, S::kLdsBytes, stream>>>(a, b, bias, c, args, map);
        return hipGetLastError();
    };
    auto pick = [&](auto with_alpha) -> hipError_t {
        constexpr bool kAlpha = decltype(with_alpha)::value;
        if (bias != nullptr) {
            return args.gelu ? run(gemm::gemm_wide_kernel<TM, TN, true, true, kAlpha>)
                             : run(gemm::gemm_wide_kernel<TM, TN, true, false, kAlpha>);
        }
        return args.gelu ? run(gemm::gemm_wide_kernel<TM, TN, false, true, kAlpha>)
                         : run(gemm::gemm_wide_kernel<TM, TN, false, false, kAlpha>);
    };
    return args.alpha == 1.0F ? pick(std::false_type{}) : pick(std::true_type{});
}

/// The XCD split for a persistent kernel whose @p turns workgroups per XCD
/// take an XCD's tiles in turn: fewest rounds (the largest block's tiles over
/// @p turns), then the fewest bytes moved into the L2 caches (tile_map's
/// measure). Measured at ViT-Base FC2 on 192 x 256 tiles: a byte-only choice
/// left one XCD 34 tiles for its 32 workgroups, 139 against 88 us.
gemm::TileMap balanced_map(const GemmArgs& args, int bm, int bn, int turns) {
    const int tiles_m = (args.m + bm - 1) / bm;
    const int tiles_n = (args.n + bn - 1) / bn;
    const double a_bytes = static_cast<double>(tiles_m) * bm * args.k * 2;
    const double b_bytes = static_cast<double>(tiles_n) * bn * args.k * 2;
    constexpr double kL2Budget = 3.0 * (1 << 20);
    gemm::TileMap best{0, 0};
    double best_cost = 0.0;
    int best_rounds = 0;
    for (const int px : {8, 4, 2, 1}) {
        const int py = 8 / px;
        if (px > tiles_m || py > tiles_n) {
            continue;
        }
        const int block = ((tiles_m + px - 1) / px) * ((tiles_n + py - 1) / py);
        const int rounds = (block + turns - 1) / turns;
        double cost = py * a_bytes + px * b_bytes;
        if (b_bytes / py > kL2Budget) {
            cost *= 2.0;
        }
        if (best.px == 0 || rounds < best_rounds || (rounds == best_rounds && cost < best_cost)) {
            best = gemm::TileMap{px, py};
            best_cost = cost;
            best_rounds = rounds;
        }
    }
    return best;
}

/// The direct-to-LDS kernel (gemm_dma.hpp) for a problem it covers: one batch
/// entry, B as [N, K], N a multiple of 256, K of at least 256, no addend,
/// vector A and B, C written in 16-byte pieces, every operand tile within one
/// descriptor's span, the CUs a multiple of 8 (one persistent workgroup per
/// CU, eight per XCD) and BM x 256 tiles for at least half the CUs. BM is the
/// height with the fewest rounds x BM (ViT-Base b64: 320 for FC1, 256 for QKV,
/// 192 for FC2 and the projection). Returns hipErrorNotSupported otherwise.
hipError_t launch_dma(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                      std::uint16_t* c, const GemmArgs& problem, hipStream_t stream) {
    const int units = compute_units();
    // A batch whose entries share B and follow one another in A runs as one
    // problem, each row stored back in its entry: the patch embedding, with
    // its positional addend (the instance that takes entries).
    const GemmArgs args = as_one_problem(problem);
    const bool with_addend = args.addend != nullptr;
    const bool entries = args.rows_per_entry > 0;
    // The addend only in the combination the model uses (bias, no alpha, no
    // GELU, no accumulation), 16-byte runs of it per lane.
    const bool addend_ok =
        !with_addend ||
        (bias != nullptr && args.alpha == 1.0F && !args.gelu && !args.accumulate && aligned16(args.addend) &&
         args.ld_addend % 4 == 0);
    const bool eligible =
        args.transposed && args.count == 1 && addend_ok && (!entries || (with_addend && args.stride_c % 8 == 0)) &&
        args.n % 256 == 0 && args.k >= 256 && units % 8 == 0 &&
        vector_operand(a, args.lda, args.k, 0, 0, false) && vector_operand(b, args.ldb, args.k, 0, 0, false) &&
        static_cast<std::int64_t>(320) * args.lda * 2 < gemm::kMaxSpan &&
        static_cast<std::int64_t>(256) * args.ldb * 2 < gemm::kMaxSpan && aligned16(c) &&
        args.ldc % 8 == 0 && static_cast<std::int64_t>(args.n) * 4 < gemm::kMaxSpan;
    if (!eligible) {
        return hipErrorNotSupported;
    }
    int bm = 0;
    std::int64_t best = 0;
    for (const int height : {192, 256, 320}) {
        if (with_addend && height == 320) {
            continue;  // the addend's registers would spill at 320 rows
        }
        const std::int64_t tiles = tile_count(args, height, 256);
        const std::int64_t cost = (tiles + units - 1) / units * height;
        if (bm == 0 || cost < best) {
            bm = height;
            best = cost;
        }
    }
    if (2 * tile_count(args, bm, 256) < units) {
        return hipErrorNotSupported;  // fewer tiles than half the CUs: the other kernels
    }
    const int turns = units / 8;
    const gemm::TileMap map = balanced_map(args, bm, 256, turns);
    auto run = [&](auto kernel, std::size_t lds_bytes) -> hipError_t {
        static std::atomic<std::uint64_t> opted_in{0};
        if (const hipError_t opted = allow_lds(reinterpret_cast<const void*>(kernel), lds_bytes, opted_in);
            opted != hipSuccess) {
            return opted;
        }
        kernel<<<units, 512, lds_bytes, stream>>>(a, b, bias, c, args, map);
        return hipGetLastError();
    };
    // The epilogue's parts as template flags: bias, GELU, alpha (when not 1),
    // accumulate.
    auto pick = [&](auto height) -> hipError_t {
        constexpr int BM = decltype(height)::value;
        constexpr std::size_t kLds = gemm::DmaShape<BM>::kLdsBytes;
        if (with_addend) {
            if constexpr (BM == 320) {
                return hipErrorNotSupported;  // not chosen for an addend (see above)
            } else {
                return run(gemm::gemm_dma_kernel<BM, true, false, false, false, true>, kLds);
            }
        }
        auto with_flags = [&](auto with_bias, auto with_gelu, auto with_alpha) -> hipError_t {
            constexpr bool kB = decltype(with_bias)::value;
            constexpr bool kG = decltype(with_gelu)::value;
            constexpr bool kA = decltype(with_alpha)::value;
            return args.accumulate ? run(gemm::gemm_dma_kernel<BM, kB, kG, kA, true>, kLds)
                                   : run(gemm::gemm_dma_kernel<BM, kB, kG, kA, false>, kLds);
        };
        auto with_alpha = [&](auto with_bias, auto with_gelu) -> hipError_t {
            return args.alpha == 1.0F ? with_flags(with_bias, with_gelu, std::false_type{})
                                      : with_flags(with_bias, with_gelu, std::true_type{});
        };
        auto with_gelu = [&](auto with_bias) -> hipError_t {
            return args.gelu ? with_alpha(with_bias, std::true_type{}) : with_alpha(with_bias, std::false_type{});
        };
        return bias != nullptr ? with_gelu(std::true_type{}) : with_gelu(std::false_type{});
    };
    switch (bm) {
    case 192: return pick(std::integral_constant<int, 192>{});
    case 256: return pick(std::integral_constant<int, 256>{});
    default: return pick(std::integral_constant<int, 320>{});
    }
}

hipError_t gemm_bf16(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                     std::uint16_t* c, const GemmArgs& args, hipStream_t stream) {
    // The direct-to-LDS kernel where it applies (ViT-Base b64 against the
    // kernels below, same bits, two input sets: FC1 + GELU 99 -> 87 us, QKV
    // 61 -> 50, FC2 accumulating 81 -> 67, the projection 38 -> 26; the patch
    // embedding 51 -> 29 inside the forward. With A from HBM now 78, 52, 68
    // and 27 us).
    if (const hipError_t dma = launch_dma(a, b, bias, c, args, stream); dma != hipErrorNotSupported) {
        return dma;
    }
    // 128 x 256 tiles with 64 x 128 per wavefront (ViT-Base FC1 + GELU 137 ->
    // 110 us), where they apply; bitwise the same results as the tiles below.
    if (const hipError_t wide = launch_wide<2, 4>(a, b, bias, c, args, stream);
        wide != hipErrorNotSupported) {
        return wide;
    }
    // One round of 256 x 192 tiles, twelve wavefronts of 64 x 64 (three per
    // SIMD), for products with B as [N, K] that would need more than two
    // 128 x 128 tiles per CU: each CU then streams one tile's whole K, with
    // three wavefronts per SIMD to cover the loads (ViT-Base FC2 12608 x 768 x
    // 3072, accumulating: 110 -> 81 us; the projection, K = 768: 43 -> 40 us).
    // Eight wavefronts of 64 x 96 ran FC2 in 92-95 us and the projection in
    // 49: two per SIMD left the waves waiting on their loads 54% of the time.
    // A batch whose entries' A rows follow one another and share B (the
    // model's patch embedding: 196 rows per image into rows 1.. of its 197)
    // runs as one problem of all the rows, so tiles do not stop at entry
    // boundaries (ViT-Base b64 embedding 53 -> 41 us).
    const std::int64_t units = compute_units();
    const GemmArgs whole = as_one_problem(args);
    if (whole.transposed && whole.k >= 512 && tile_count(whole, 256, 192) <= units &&
        tile_count(whole, 128, 128) > 2 * units) {
        using S = Shape<std::uint16_t, 4, 3, 2, 2, 64>;
        const bool split = whole.inner > 0;
        if (vector_operand(a, whole.lda, whole.k, whole.stride_a, whole.outer_stride_a, split) &&
            vector_operand(b, whole.ldb, whole.k, whole.stride_b, whole.outer_stride_b, split) &&
            static_cast<std::int64_t>(S::kBM) * whole.lda * 2 < gemm::kMaxSpan &&
            static_cast<std::int64_t>(S::kBN) * whole.ldb * 2 < gemm::kMaxSpan) {
            return launch<std::uint16_t, 4, 3, 2, 2, 64, 3, true, true, true>(
                a, b, bias, c, whole, vector_output(c, whole), stream);
        }
    }
    if (tile_count(args, 128, 128) >= units * 2) {
        // Up to K = 1024, 32-deep stages with registers for three workgroups
        // per CU beat 64-deep ones at two (ViT-Base FC1 + GELU 146 -> 136 us,
        // QKV 103 -> 96, projection 45.5 -> 38.4); FC2 (K = 3072) keeps the
        // 64-deep stages (95 against 99 us).
        if (args.k <= 1024) {
            return pick_flags<std::uint16_t, 2, 2, 2, 2, 32, 3>(a, b, bias, c, args, stream);
        }
        return pick_flags<std::uint16_t, 2, 2, 2, 2, 64>(a, b, bias, c, args, stream);
    }
    // 64 x 64: 32-deep stages for short K (ViT-Tiny FC1 6304 x 768 x 192 with
    // GELU: 13.4 against 16.1 us), 64-deep beyond (FC2, K = 768: 10.9 against
    // 11.7 us).
    if (args.k <= 512) {
        return pick_flags<std::uint16_t, 2, 2, 1, 1, 32>(a, b, bias, c, args, stream);
    }
    return pick_flags<std::uint16_t, 2, 2, 1, 1, 64>(a, b, bias, c, args, stream);
}

} // namespace cuvit::detail
