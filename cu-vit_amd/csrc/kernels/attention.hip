// Fused attention for the ViT block: context = softmax(Q.K^T * scale).V per
// (image, head), from the packed QKV projection, without materializing the
// [images, heads, tokens, tokens] logits.
//
// The reference runs this as three launches (src/model/vit.cu:205-245): the
// Q.K^T GEMM with alpha = 1/sqrt(head_dim) into the logits, softmax in place,
// and the weights.V GEMM into the context. This kernel computes the very same
// floating-point operations in the same order, so its output is bitwise equal
// to those three launches of this library:
//   * logits: the GEMM's v_mfma_f32_16x16x4_f32 over head_dim in k-blocks of
//     16 (MFMA s of a block sums k = kb + s, kb + 4 + s, kb + 8 + s,
//     kb + 12 + s), then alpha * sum, exactly as in the GEMM epilogue;
//   * softmax: the max is exact in any order; the exponentials are the same
//     exp2((x - max) * log2 e); the sum reproduces the softmax kernel's
//     16-lane team (rows up to 256 wide): team lane t sums the columns
//     t + 16 j in order from +0, then the DPP tree (pair, quad, half-row
//     mirror, row mirror). Here the 16 partial sums sit four to a lane in
//     the four lanes that hold a query row, and the tree is replayed with
//     two cross-lane swaps; probabilities are e * (1 / sum) as there;
//   * weights.V: the GEMM's MFMA over keys in k-blocks of 16, keys past the
//     token count contributing exact zeros.
// The probabilities never leave registers: a lane of the logits tile holds
// row l % 16 and keys 4 (l / 16) .. + 3 of each 16-key tile, which is
// exactly the A fragment the weights.V MFMA consumes.
//
// Layout: qkv is [images, tokens, 3, heads, head_dim] and context is
// [images, tokens, heads, head_dim] (src/model/vit.cu:199-245). A workgroup
// owns one (image, head) and up to kWaves query tiles of 16 rows; K and V of
// that (image, head) sit in LDS as [key][head_dim + 4] fp32 (padded rows give
// conflict-free 16-byte fragment reads).
#include "device_common.hpp"
#include "gemm_kernel.hpp"
#include "launch.hpp"

#include <cmath>

namespace cuvit::detail {
namespace {

using namespace cuvit::device;

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kHeadDim = 64;          // head_dim this kernel handles
constexpr int kPitch = kHeadDim + 4;  // floats per LDS row
constexpr int kMaxKeyTiles = 16;      // up to 256 tokens
constexpr float kLog2e = 1.4426950408889634F;

/// op(value of lanes 16 k + i, value of lanes 16 (k + 1) + i) for k = 0 and
/// k = 2, in both lanes of each pair (@p kRows 16: rows of 16 lanes, by
/// v_permlane16_swap), or op(lower half, upper half) (@p kRows 32, by
/// v_permlane32_swap): a swap of the value with itself leaves each lane its
/// own value and its partner's, the lower one first in both lanes, with no LDS
/// round trip. op is max or + here, which give the same bits as
/// op(own, partner) in either order.
template <int kRows, typename Op> __device__ __forceinline__ float combine_rows(float value, Op op) {
    const std::uint32_t bits = __float_as_uint(value);
    if constexpr (kRows == 16) {
        const auto swapped = __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
        return op(__uint_as_float(swapped[0]), __uint_as_float(swapped[1]));
    } else {
        static_assert(kRows == 32, "rows of 16 or halves of 32 lanes");
        const auto swapped = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
        return op(__uint_as_float(swapped[0]), __uint_as_float(swapped[1]));
    }
}

template <int KT, int Waves>
__global__ __launch_bounds__(Waves * kWave) void attention_kernel(const float* __restrict__ qkv,
                                                                  float* __restrict__ context,
                                                                  int heads, int tokens, float scale) {
    extern __shared__ Vec16 lds_vectors[];
    float* const keys = reinterpret_cast<float*>(lds_vectors);
    float* const values = keys + KT * 16 * kPitch;

    const int t = threadIdx.x;
    const int lane = lane_id();
    const int wave = t / kWave;
    const int row_in_tile = lane & 15;
    const int group = lane >> 4;

    const int pair = blockIdx.y;
    const int image = pair / heads;
    const int head = pair - image * heads;
    const int embed = heads * kHeadDim;
    const std::int64_t qkv_row = 3 * static_cast<std::int64_t>(embed);
    const float* const q_base = qkv + static_cast<std::int64_t>(image) * tokens * qkv_row + head * kHeadDim;
    const float* const k_base = q_base + embed; // V follows K by embed in every token's row

    const int query_tile = blockIdx.x * Waves + wave;
    const int q0 = query_tile * 16;
    const bool live = q0 < tokens; // wavefronts past the tokens still stage K and V

    // Q fragments: row q0 + l % 16 (clamped), head_dim chunk 4 (l / 16) of
    // each k-block, loaded first so that their latency overlaps K's and V's.
    const int q_row = q0 + row_in_tile < tokens ? q0 + row_in_tile : tokens - 1;
    const auto q_resource = gemm::buffer_resource(q_base);
    Vec16 qf[kHeadDim / 16];
#pragma unroll
    for (int kb = 0; kb < kHeadDim / 16; ++kb) {
        qf[kb] = gemm::buffer_load16(q_resource, static_cast<unsigned int>((q_row * qkv_row + 16 * kb + 4 * group) * 4));
    }

    // K and V of this (image, head), all loads in flight at once, K's first
    // (rows past the tokens read as zero). K goes to LDS as its loads land;
    // V's stores wait until the logits and the softmax are done, so V's loads
    // land meanwhile.
    constexpr int kQuadsPerRow = kHeadDim / 4;
    constexpr int kQuads = KT * 16 * kQuadsPerRow;
    constexpr int kPerThread = (kQuads + Waves * kWave - 1) / (Waves * kWave);
    const auto kv_resource = gemm::buffer_resource(k_base);
    Vec16 kreg[kPerThread];
    Vec16 vreg[kPerThread];
    auto kv_offset = [&](int i) -> unsigned int {
        const int q = t + i * Waves * kWave;
        const int row = q / kQuadsPerRow;
        const bool inside = q < kQuads && row < tokens;
        return inside ? static_cast<unsigned int>((row * qkv_row + 4 * (q % kQuadsPerRow)) * 4) : gemm::kOutside;
    };
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        kreg[i] = gemm::buffer_load16(kv_resource, kv_offset(i));
    }
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const unsigned int offset = kv_offset(i);
        vreg[i] = gemm::buffer_load16(kv_resource, offset == gemm::kOutside ? offset : offset + 4U * embed);
    }
    auto stage = [&](float* tile, const Vec16 (&reg)[kPerThread]) {
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
            const int q = t + i * Waves * kWave;
            if (kQuads % (Waves * kWave) == 0 || q < kQuads) {
                store16(tile + (q / kQuadsPerRow) * kPitch + 4 * (q % kQuadsPerRow), reg[i]);
            }
        }
    };
    // Logits: lane holds row q0 + l % 16, keys 16 jt + 4 (l / 16) + r. The
    // first MFMA of a tile takes its zero accumulator as a constant. K goes
    // to LDS one load round at a time (kTilesPerRound key tiles), each behind
    // a barrier, so the first MFMAs wait for the first round only (ViT-Tiny
    // b32: 20.9-21.4 -> 20.5-20.9 us, same bits).
    constexpr int kTilesPerRound = Waves * kWave / kQuadsPerRow / 16;
    static_assert(kTilesPerRound >= 1, "a load round holds whole key tiles");
    floatx4 s[KT];
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int q = t + i * Waves * kWave;
        if (kQuads % (Waves * kWave) == 0 || q < kQuads) {
            store16(keys + (q / kQuadsPerRow) * kPitch + 4 * (q % kQuadsPerRow), kreg[i]);
        }
        __syncthreads();
        if (live) {
#pragma unroll
            for (int jt = i * kTilesPerRound; jt < (i + 1) * kTilesPerRound && jt < KT; ++jt) {
#pragma unroll
                for (int kb = 0; kb < kHeadDim / 16; ++kb) {
                    const Vec16 kf = load16(keys + (16 * jt + row_in_tile) * kPitch + 16 * kb + 4 * group);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        s[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kf.w[e]),
                                                                     __uint_as_float(qf[kb].w[e]),
                                                                     kb == 0 && e == 0 ? floatx4{0.F, 0.F, 0.F, 0.F} : s[jt],
                                                                     0, 0, 0);
                    }
                }
            }
        }
    }
    if (live) {

    // alpha * sum, rounded on its own as the GEMM epilogue stores it (never
    // fused into the subtraction below), then the row max over the valid
    // keys (exact in any order); only the last key tile holds keys past the
    // tokens.
    float maximum = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < KT; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma clang fp contract(off)
            s[jt][r] = scale * s[jt][r];
            if (jt < KT - 1 || 16 * jt + 4 * group + r < tokens) {
                maximum = fmaxf(maximum, s[jt][r]);
            }
        }
    }
    const auto larger = [](float a, float b) { return fmaxf(a, b); };
    maximum = combine_rows<32>(combine_rows<16>(maximum, larger), larger);

    // Exponentials; keys past the tokens become exact zeros.
#pragma unroll
    for (int jt = 0; jt < KT; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float e = __builtin_amdgcn_exp2f((s[jt][r] - maximum) * kLog2e);
            s[jt][r] = jt < KT - 1 || 16 * jt + 4 * group + r < tokens ? e : 0.F;
        }
    }

    // The softmax's sum (16-lane teams, softmax_terms.hpp): team lane t sums
    // columns t + 16 j in order from +0, i.e. tile j, element t of the tile,
    // which this lane holds for t = 4 g + r. Then the team's DPP tree:
    // pairs (t ^ 1), quads (t ^ 2), quad 0 + quad 1 and quad 2 + quad 3 (the
    // half-row mirror), and the two halves (the row mirror); here the quad
    // totals sit in the four lanes of a query row, one exchange per level.
    // Tiles past the row (up to the softmax kernel's 16) would add +0.
    float partial[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float sum = 0.F;
#pragma unroll
        for (int jt = 0; jt < KT; ++jt) {
            sum += s[jt][r];
        }
        partial[r] = sum;
    }
    const float quad = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const auto add = [](float a, float b) { return a + b; };
    const float inverse = 1.0F / combine_rows<32>(combine_rows<16>(quad, add), add);
#pragma unroll
    for (int jt = 0; jt < KT; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[jt][r] *= inverse;
        }
    }

    } // live

    stage(values, vreg);
    __syncthreads();
    if (!live) {
        return; // no barrier follows
    }

    // weights.V: lane provides weights[row][keys 16 jt + 4 g + e] (its own
    // registers) and V[keys 16 jt + 4 g + e][16 dt + l % 16].
    floatx4 out[kHeadDim / 16];
#pragma unroll
    for (int jt = 0; jt < KT; ++jt) {
        const float* const v_rows = values + (16 * jt + 4 * group) * kPitch + row_in_tile;
#pragma unroll
        for (int dt = 0; dt < kHeadDim / 16; ++dt) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                out[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                    v_rows[e * kPitch + 16 * dt], s[jt][e],
                    jt == 0 && e == 0 ? floatx4{0.F, 0.F, 0.F, 0.F} : out[dt], 0, 0, 0);
            }
        }
    }

    // Lane holds context[row][16 dt + 4 (l / 16) .. + 3].
    const int row = q0 + row_in_tile;
    if (row < tokens) {
        float* const destination = context +
                                   (static_cast<std::int64_t>(image) * tokens + row) * embed +
                                   head * kHeadDim + 4 * group;
#pragma unroll
        for (int dt = 0; dt < kHeadDim / 16; ++dt) {
            *reinterpret_cast<floatx4*>(destination + 16 * dt) = out[dt];
        }
    }
}

constexpr int kWaves = 8;

template <int KT>
hipError_t launch(const float* qkv, float* context, int images, int heads, int tokens,
                  hipStream_t stream) {
    constexpr std::size_t kLds = 2 * static_cast<std::size_t>(KT) * 16 * kPitch * sizeof(float);
    auto kernel = attention_kernel<KT, kWaves>;
    static std::atomic<std::uint64_t> opted_in{0};
    if (const hipError_t opted = allow_lds(reinterpret_cast<const void*>(kernel), kLds, opted_in);
        opted != hipSuccess) {
        return opted;
    }
    const dim3 grid(static_cast<unsigned int>((KT + kWaves - 1) / kWaves),
                    static_cast<unsigned int>(images * heads));
    const float scale = 1.0F / std::sqrt(static_cast<float>(kHeadDim));
    kernel<<<grid, kWaves * kWave, kLds, stream>>>(qkv, context, heads, tokens, scale);
    return hipGetLastError();
}

} // namespace

bool attention_supported(int tokens, int head_dim) {
    return head_dim == kHeadDim && tokens > 0 && tokens <= 16 * kMaxKeyTiles;
}

hipError_t attention_f32(const float* qkv, float* context, int images, int heads, int tokens,
                         int head_dim, hipStream_t stream) {
    if (!attention_supported(tokens, head_dim)) {
        return hipErrorInvalidValue;
    }
    // One instance per key-tile count: the tiles are compile-time, and only
    // the last one carries keys past the tokens.
    switch ((tokens + 15) / 16) {
    case 1: return launch<1>(qkv, context, images, heads, tokens, stream);
    case 2: return launch<2>(qkv, context, images, heads, tokens, stream);
    case 3: return launch<3>(qkv, context, images, heads, tokens, stream);
    case 4: return launch<4>(qkv, context, images, heads, tokens, stream);
    case 5: return launch<5>(qkv, context, images, heads, tokens, stream);
    case 6: return launch<6>(qkv, context, images, heads, tokens, stream);
    case 7: return launch<7>(qkv, context, images, heads, tokens, stream);
    case 8: return launch<8>(qkv, context, images, heads, tokens, stream);
    case 9: return launch<9>(qkv, context, images, heads, tokens, stream);
    case 10: return launch<10>(qkv, context, images, heads, tokens, stream);
    case 11: return launch<11>(qkv, context, images, heads, tokens, stream);
    case 12: return launch<12>(qkv, context, images, heads, tokens, stream);
    case 13: return launch<13>(qkv, context, images, heads, tokens, stream);
    case 14: return launch<14>(qkv, context, images, heads, tokens, stream);
    case 15: return launch<15>(qkv, context, images, heads, tokens, stream);
    default: return launch<kMaxKeyTiles>(qkv, context, images, heads, tokens, stream);
    }
}

} // namespace cuvit::detail
