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
//     two cross-lane exchanges; probabilities are e * (1 / sum) as there;
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

__device__ __forceinline__ float shuffle_xor(float value, int mask) {
    return __shfl_xor(value, mask, kWave);
}

template <int Waves>
__global__ __launch_bounds__(Waves * kWave) void attention_kernel(const float* __restrict__ qkv,
                                                                  float* __restrict__ context,
                                                                  int heads, int tokens, float scale) {
    extern __shared__ Vec16 lds_vectors[];
    float* const keys = reinterpret_cast<float*>(lds_vectors);
    const int key_tiles = (tokens + 15) / 16;
    float* const values = keys + key_tiles * 16 * kPitch;

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
    const float* const k_base = q_base + embed;
    const float* const v_base = q_base + 2 * embed;

    // K and V of this (image, head) into LDS; rows past the tokens are zero.
    constexpr int kQuadsPerRow = kHeadDim / 4;
    for (int q = t; q < key_tiles * 16 * kQuadsPerRow; q += Waves * kWave) {
        const int row = q / kQuadsPerRow;
        const int quad = q - row * kQuadsPerRow;
        float4 k4 = make_float4(0.F, 0.F, 0.F, 0.F);
        float4 v4 = k4;
        if (row < tokens) {
            k4 = *reinterpret_cast<const float4*>(k_base + row * qkv_row + 4 * quad);
            v4 = *reinterpret_cast<const float4*>(v_base + row * qkv_row + 4 * quad);
        }
        *reinterpret_cast<float4*>(keys + row * kPitch + 4 * quad) = k4;
        *reinterpret_cast<float4*>(values + row * kPitch + 4 * quad) = v4;
    }
    __syncthreads();

    const int query_tile = blockIdx.x * Waves + wave;
    const int q0 = query_tile * 16;
    if (q0 >= tokens) {
        return; // no barrier follows
    }

    // Q fragments: row q0 + l % 16 (clamped), head_dim chunk 4 (l / 16) of
    // each k-block.
    const int q_row = q0 + row_in_tile < tokens ? q0 + row_in_tile : tokens - 1;
    Vec16 qf[kHeadDim / 16];
#pragma unroll
    for (int kb = 0; kb < kHeadDim / 16; ++kb) {
        qf[kb] = load16(q_base + q_row * qkv_row + 16 * kb + 4 * group);
    }

    // Logits: lane holds row q0 + l % 16, keys 16 jt + 4 (l / 16) + r.
    floatx4 s[kMaxKeyTiles];
#pragma unroll
    for (int jt = 0; jt < kMaxKeyTiles; ++jt) {
        s[jt] = floatx4{0.F, 0.F, 0.F, 0.F};
        if (jt < key_tiles) {
#pragma unroll
            for (int kb = 0; kb < kHeadDim / 16; ++kb) {
                const Vec16 kf = load16(keys + (16 * jt + row_in_tile) * kPitch + 16 * kb + 4 * group);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(kf.w[e]),
                                                                 __uint_as_float(qf[kb].w[e]), s[jt],
                                                                 0, 0, 0);
                }
            }
        }
    }

    // Row max over the valid keys (exact in any order).
    float maximum = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < kMaxKeyTiles; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * jt + 4 * group + r;
            s[jt][r] = scale * s[jt][r];
            if (key < tokens) {
                maximum = fmaxf(maximum, s[jt][r]);
            }
        }
    }
    maximum = fmaxf(maximum, shuffle_xor(maximum, 16));
    maximum = fmaxf(maximum, shuffle_xor(maximum, 32));

    // Exponentials; keys past the tokens become exact zeros.
#pragma unroll
    for (int jt = 0; jt < kMaxKeyTiles; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = 16 * jt + 4 * group + r;
            s[jt][r] = key < tokens ? __builtin_amdgcn_exp2f((s[jt][r] - maximum) * kLog2e) : 0.F;
        }
    }

    // The softmax's sum (16-lane teams, softmax_terms.hpp): team lane t sums
    // columns t + 16 j in order from +0, i.e. tile j, element t of the tile,
    // which this lane holds for t = 4 g + r. Then the team's DPP tree:
    // pairs (t ^ 1), quads (t ^ 2), quad 0 + quad 1 and quad 2 + quad 3 (the
    // half-row mirror), and the two halves (the row mirror); here the quad
    // totals sit in the four lanes of a query row, one exchange per level.
    float partial[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float sum = 0.F;
#pragma unroll
        for (int jt = 0; jt < kMaxKeyTiles; ++jt) {
            sum += s[jt][r];
        }
        partial[r] = sum;
    }
    const float quad = (partial[0] + partial[1]) + (partial[2] + partial[3]);
    const float half = quad + shuffle_xor(quad, 16);
    const float inverse = 1.0F / (half + shuffle_xor(half, 32));
#pragma unroll
    for (int jt = 0; jt < kMaxKeyTiles; ++jt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s[jt][r] *= inverse;
        }
    }

    // weights.V: lane provides weights[row][keys 16 jt + 4 g + e] (its own
    // registers) and V[keys 16 jt + 4 g + e][16 dt + l % 16].
    floatx4 out[kHeadDim / 16];
#pragma unroll
    for (int dt = 0; dt < kHeadDim / 16; ++dt) {
        out[dt] = floatx4{0.F, 0.F, 0.F, 0.F};
    }
#pragma unroll
    for (int jt = 0; jt < kMaxKeyTiles; ++jt) {
        if (jt < key_tiles) {
            const float* const v_rows = values + (16 * jt + 4 * group) * kPitch + row_in_tile;
#pragma unroll
            for (int dt = 0; dt < kHeadDim / 16; ++dt) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    out[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(v_rows[e * kPitch + 16 * dt], s[jt][e],
                                                                   out[dt], 0, 0, 0);
                }
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

} // namespace

bool attention_supported(int tokens, int head_dim) {
    return head_dim == kHeadDim && tokens > 0 && tokens <= 16 * kMaxKeyTiles;
}

hipError_t attention_f32(const float* qkv, float* context, int images, int heads, int tokens,
                         int head_dim, hipStream_t stream) {
    if (!attention_supported(tokens, head_dim)) {
        return hipErrorInvalidValue;
    }
    const int key_tiles = (tokens + 15) / 16;
    const std::size_t lds = 2 * static_cast<std::size_t>(key_tiles) * 16 * kPitch * sizeof(float);
    static std::atomic<std::uint64_t> opted_in{0};
    if (const hipError_t opted =
            allow_lds(reinterpret_cast<const void*>(attention_kernel<kWaves>),
                      2 * 16 * kMaxKeyTiles * kPitch * sizeof(float), opted_in);
        opted != hipSuccess) {
        return opted;
    }
    const dim3 grid(static_cast<unsigned int>((key_tiles + kWaves - 1) / kWaves),
                    static_cast<unsigned int>(images * heads));
    const float scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
    attention_kernel<kWaves><<<grid, kWaves * kWave, lds, stream>>>(qkv, context, heads, tokens, scale);
    return hipGetLastError();
}

} // namespace cuvit::detail
