// Fused attention for the bf16 model: context = softmax(Q.K^T * scale).V per
// (image, head) from the packed bf16 QKV projection, without the
// [images, heads, tokens, tokens] logits in HBM.
//
// The bf16 model otherwise runs the reference's three launches
// (src/model/vit.cu:205-245) through this library's bf16 twins: the Q.K^T
// GEMM with alpha = 1/sqrt(head_dim) into bf16 logits, softmax in place, and
// the weights.V GEMM into the bf16 context. This kernel performs the same
// operations in the same order, including every rounding to bf16, so its
// output is bitwise equal to those three launches:
//   * logits: the GEMM's v_mfma_f32_32x32x16_bf16 over head_dim in k-blocks
//     of 16 with the same operand roles (K fragment first, Q fragment
//     second; lane l reads row l % 32 and k chunk 8 (l / 32)), then
//     alpha * sum rounded to bf16, as the GEMM epilogue stores it;
//   * softmax: the bf16 row softmax's own code (softmax_terms.hpp, teams of
//     16 lanes, column c on team lane c % 16) over the bf16 logits, each
//     probability rounded to bf16;
//   * weights.V: the GEMM's MFMA over keys in k-blocks of 16, the k loop
//     running over the same k-blocks as the GEMM's, keys past the
//     token count contributing exact zeros (the GEMM runs its 64-key stages
//     in pairs, and so does this loop), then the sum rounded to bf16.
//
// Layout: qkv is [images, tokens, 3, heads, 64] and context is
// [images, tokens, heads, 64], bf16. A workgroup owns one (image, head) and
// `waves` query tiles of 32 rows, one per wavefront. V of the (image, head)
// sits in LDS transposed, [64][keys], so a lane's weights.V B fragment is
// 16 contiguous bytes; each wavefront keeps its tile's logits, then
// probabilities, in a private [32][keys] LDS block. Q and K fragments are
// read straight from global memory (16 contiguous bytes each). Rows are
// padded by 8 elements, which makes the 16-byte fragment reads of 16
// consecutive rows hit distinct bank quads for every padded key count.
#include "device_common.hpp"
#include "gemm_kernel.hpp"
#include "launch.hpp"
#include "softmax_terms.hpp"

#include <cmath>

namespace cuvit::detail {
namespace {

using namespace cuvit::device;
using gemm::Mma;

using Bf16Mma = Mma<std::uint16_t>;
using Acc = Bf16Mma::Acc;

constexpr int kHeadDim = 64;
constexpr int kEdge = 32;        // MFMA tile edge: 32 queries x 32 keys (or dims)
constexpr int kKBlock = 16;      // k per MFMA
constexpr int kStage = 64;       // the GEMM's k stage: weights.V runs whole stages
constexpr int kMaxTokens = 256;
constexpr int kMaxWaves = 8;
constexpr std::size_t kMaxLds = 152 * 1024; // 256 tokens fit with 7 query tiles

/// Elements per padded LDS row for @p tokens keys.
__host__ __device__ constexpr int row_pitch(int tokens) {
    return (tokens + kEdge - 1) / kEdge * kEdge + 8;
}

__host__ __device__ constexpr std::size_t lds_bytes(int tokens, int waves) {
    return static_cast<std::size_t>(kHeadDim + waves * kEdge) * row_pitch(tokens) * 2;
}

/// 16 bytes at @p element of @p base, or zero when @p inside is false.
__device__ __forceinline__ Vec16 load_or_zero(const std::uint16_t* base, std::int64_t element,
                                              bool inside) {
    return inside ? load16(base + element) : Vec16{{0U, 0U, 0U, 0U}};
}

template <int J>
__global__ __launch_bounds__(kMaxWaves * kWave) void attention_bf16_kernel(
    const std::uint16_t* __restrict__ qkv, std::uint16_t* __restrict__ context, int heads,
    int tokens, float scale) {
    extern __shared__ Vec16 lds_vectors[];
    const int pitch = row_pitch(tokens);
    const int padded = pitch - 8; // keys rounded up to whole 32-key tiles
    std::uint16_t* const values = reinterpret_cast<std::uint16_t*>(lds_vectors); // [64][pitch]
    const int waves = static_cast<int>(blockDim.x) / kWave;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = lane_id();
    const int row = lane % kEdge;         // fragment row
    const int chunk = 8 * (lane / kEdge); // fragment k offset
    std::uint16_t* const tile = values + (kHeadDim + wave * kEdge) * pitch; // [32][pitch]

    const int pair = blockIdx.y;
    const int image = pair / heads;
    const int head = pair - image * heads;
    const int embed = heads * kHeadDim;
    const std::int64_t qkv_row = 3 * static_cast<std::int64_t>(embed);
    const std::uint16_t* const q_base =
        qkv + static_cast<std::int64_t>(image) * tokens * qkv_row + head * kHeadDim;
    const std::uint16_t* const k_base = q_base + embed;
    const std::uint16_t* const v_base = q_base + 2 * embed;

    // V transposed into LDS; keys past the tokens are zero.
    constexpr int kChunks = kHeadDim / 8;
    for (int c = threadIdx.x; c < padded * kChunks; c += blockDim.x) {
        const int key = c / kChunks;
        const int d0 = 8 * (c % kChunks);
        const Vec16 v = load_or_zero(v_base, key * qkv_row + d0, key < tokens);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            Elem<std::uint16_t>::store_bits(values + (d0 + e) * pitch + key, v, e);
        }
    }

    const int query0 = (static_cast<int>(blockIdx.x) * waves + wave) * kEdge;
    const bool active = query0 < tokens; // idle waves still meet every barrier

    // Logits: 32 queries x 32 keys per MFMA tile, rounded to bf16 into the
    // wavefront's LDS block.
    if (active) {
        const int query = query0 + row;
        Vec16 q[kHeadDim / kKBlock];
#pragma unroll
        for (int kb = 0; kb < kHeadDim / kKBlock; ++kb) {
            q[kb] = load_or_zero(q_base, query * qkv_row + kb * kKBlock + chunk, query < tokens);
        }
        for (int key0 = 0; key0 < padded; key0 += kEdge) {
            const int key = key0 + row;
            Acc acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[r] = 0.F;
            }
#pragma unroll
            for (int kb = 0; kb < kHeadDim / kKBlock; ++kb) {
                const Vec16 k =
                    load_or_zero(k_base, key * qkv_row + kb * kKBlock + chunk, key < tokens);
                Bf16Mma::run(acc, k, q[kb]);
            }
            // lane: query row, keys key0 + column(lane, run) + 0..3
#pragma unroll
            for (int run = 0; run < Bf16Mma::kRuns; ++run) {
                const int column = key0 + Bf16Mma::column(lane, run);
                uint2 bits;
                bits.x = static_cast<std::uint32_t>(float_to_bf16(scale * acc[4 * run])) |
                         (static_cast<std::uint32_t>(float_to_bf16(scale * acc[4 * run + 1])) << 16);
                bits.y = static_cast<std::uint32_t>(float_to_bf16(scale * acc[4 * run + 2])) |
                         (static_cast<std::uint32_t>(float_to_bf16(scale * acc[4 * run + 3])) << 16);
                *reinterpret_cast<uint2*>(tile + row * pitch + column) = bits;
            }
        }
    }
    __syncthreads();

    // Softmax of the wavefront's 32 rows, four 16-lane teams at a time;
    // probabilities go back in place, keys past the tokens as zero.
    if (active) {
        const int t = lane % 16;
        for (int base = 0; base < kEdge; base += kWave / 16) {
            std::uint16_t* const r = tile + (base + lane / 16) * pitch;
            float x[J];
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = t + 16 * j;
                x[j] = column < tokens ? bf16_to_float(r[column]) : -INFINITY;
            }
            softmax_terms<16, J>(x, t, tokens);
#pragma unroll
            for (int j = 0; j < J; ++j) {
                const int column = t + 16 * j;
                if (column < padded) {
                    r[column] = float_to_bf16(x[j]);
                }
            }
            for (int column = 16 * J + t; column < padded; column += 16) {
                r[column] = 0;
            }
        }
    }
    __syncthreads();

    // weights.V: two 32-wide tiles of head_dim, k over whole 64-key stages.
    if (active) {
        const int query = query0 + row;
        // the GEMM's loop runs its stages in pairs (a stage past K adds
        // products 0 * 0), so the same number of k-blocks runs here
        const int stages = (tokens + kStage - 1) / kStage;
        const int k_blocks = (stages + 1) / 2 * 2 * (kStage / kKBlock);
#pragma unroll
        for (int d0 = 0; d0 < kHeadDim; d0 += kEdge) {
            Acc acc;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                acc[r] = 0.F;
            }
            for (int kb = 0; kb < k_blocks; ++kb) {
                const int key = kb * kKBlock + chunk;
                const bool inside = key < padded;
                const Vec16 p = inside ? load16(tile + row * pitch + key) : Vec16{{0U, 0U, 0U, 0U}};
                const Vec16 v =
                    inside ? load16(values + (d0 + row) * pitch + key) : Vec16{{0U, 0U, 0U, 0U}};
                Bf16Mma::run(acc, v, p);
            }
            if (query < tokens) {
                std::uint16_t* const out = context +
                                           (static_cast<std::int64_t>(image) * tokens + query) * embed +
                                           head * kHeadDim + d0;
#pragma unroll
                for (int run = 0; run < Bf16Mma::kRuns; ++run) {
                    const int column = Bf16Mma::column(lane, run);
                    uint2 bits;
                    bits.x = static_cast<std::uint32_t>(float_to_bf16(1.0F * acc[4 * run])) |
                             (static_cast<std::uint32_t>(float_to_bf16(1.0F * acc[4 * run + 1])) << 16);
                    bits.y = static_cast<std::uint32_t>(float_to_bf16(1.0F * acc[4 * run + 2])) |
                             (static_cast<std::uint32_t>(float_to_bf16(1.0F * acc[4 * run + 3])) << 16);
                    *reinterpret_cast<uint2*>(out + column) = bits;
                }
            }
        }
    }
}

template <int J>
hipError_t launch(const std::uint16_t* qkv, std::uint16_t* context, int images, int heads,
                  int tokens, int waves, hipStream_t stream) {
    auto kernel = attention_bf16_kernel<J>;
    static std::atomic<std::uint64_t> opted_in{0};
    if (const hipError_t opted = allow_lds(reinterpret_cast<const void*>(kernel), kMaxLds, opted_in);
        opted != hipSuccess) {
        return opted;
    }
    const int query_tiles = (tokens + kEdge - 1) / kEdge;
    const dim3 grid(static_cast<unsigned int>((query_tiles + waves - 1) / waves),
                    static_cast<unsigned int>(images * heads));
    const float scale = 1.0F / std::sqrt(static_cast<float>(kHeadDim));
    kernel<<<grid, waves * kWave, lds_bytes(tokens, waves), stream>>>(qkv, context, heads, tokens,
                                                                       scale);
    return hipGetLastError();
}

} // namespace

bool attention_bf16_supported(int tokens, int head_dim) {
    return head_dim == kHeadDim && tokens > 0 && tokens <= kMaxTokens;
}

hipError_t attention_bf16(const std::uint16_t* qkv, std::uint16_t* context, int images, int heads,
                          int tokens, int head_dim, hipStream_t stream) {
    if (!attention_bf16_supported(tokens, head_dim)) {
        return hipErrorInvalidValue;
    }
    // Query tiles per workgroup: as many as LDS holds, fewer when that would
    // leave the grid under two workgroups per compute unit.
    const int query_tiles = (tokens + kEdge - 1) / kEdge;
    const std::int64_t pairs = static_cast<std::int64_t>(images) * heads;
    int waves = query_tiles < kMaxWaves ? query_tiles : kMaxWaves;
    while (waves > 1 && lds_bytes(tokens, waves) > kMaxLds) {
        --waves;
    }
    const std::int64_t target = 2 * static_cast<std::int64_t>(compute_units());
    while (waves > 1 && pairs * ((query_tiles + waves - 1) / waves) < target) {
        --waves;
    }
    // J as the bf16 softmax picks it for rows of `tokens` (any J that covers
    // the row gives the same bits).
    switch ((tokens + 15) / 16) {
    case 1:
    case 2: return launch<2>(qkv, context, images, heads, tokens, waves, stream);
    case 3:
    case 4: return launch<4>(qkv, context, images, heads, tokens, waves, stream);
    case 5:
    case 6:
    case 7:
    case 8: return launch<8>(qkv, context, images, heads, tokens, waves, stream);
    case 9:
    case 10:
    case 11:
    case 12:
    case 13: return launch<13>(qkv, context, images, heads, tokens, waves, stream);
    default: return launch<16>(qkv, context, images, heads, tokens, waves, stream);
    }
}

} // namespace cuvit::detail
