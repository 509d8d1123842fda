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
//     alpha * sum rounded to bf16, as the GEMM epilogue stores it (alpha =
//     1/8 enters as a factor of the exponential's constant, which gives
//     the same bits);
//   * softmax: the bf16 row softmax's own code (softmax_terms.hpp, teams of
//     16 lanes, column c on team lane c % 16) over the bf16 logits, each
//     probability rounded to bf16;
//   * weights.V: the GEMM's MFMA over keys in k-blocks of 16, the k loop
//     running over the same k-blocks as the GEMM's, keys past the
//     token count contributing exact zeros (the GEMM runs its 64-key stages
//     in pairs, and so does this loop), then the sum rounded to bf16.
//
// The logits and probabilities never touch LDS. A lane of a 32 x 32 logits
// tile holds query row l % 32 and, for each of four runs q, the keys
// 8 q + 4 (l / 32) + 0..3, so the two lanes l and l ^ 32 hold a query's whole
// row. The bf16 softmax's team lane t (column c on lane c % 16, its columns
// summed in order c = t, t + 16, ...) corresponds to residue t = 8 (q % 2) +
// 4 (l / 32) + r of a lane's runs: each lane keeps eight of the sixteen
// partial sums in the same order, the DPP tree (t ^ 1, t ^ 2, half-row
// mirror, row mirror) becomes (Q0 + Q1) + (Q2 + Q3) over the quad totals Qa
// with one swap between l and l ^ 32, and the probabilities, rounded to
// bf16, are swapped by halves between l and l ^ 32 into the weights.V A
// fragments (8 consecutive keys per lane).
//
// Layout: qkv is [images, tokens, 3, heads, 64] and context is
// [images, tokens, heads, 64], bf16. A workgroup owns one (image, head) and
// `waves` query tiles of 32 rows, one per wavefront. K of the (image, head)
// sits in LDS as [keys][64 + 8]; with the padding, 16 consecutive rows hit
// distinct bank quads. V sits as [keys][64], unpadded, its 16-byte chunk m of
// key k at chunk m ^ 4 ((k >> 1) & 1), and a lane's weights.V B fragment (8
// consecutive keys of one dim) comes from two ds_read_b64_tr_b16, the LDS
// read that transposes 16-bit elements within each 16 lanes: lane i of a
// group receives element i % 4 of the 8 bytes lane 4 e + i / 4 addressed, as
// its element e. With lane j of a group addressing key base + j / 4, dims
// 4 (j % 4) + 0..3, lane i gets dim i of keys base + 0..3. The 32 lanes of
// a half-wavefront read four keys' 32 dims, which the placement spreads over
// all 64 banks, and the stores from global memory write whole 16-byte chunks
// (the transposed layout this replaces took eight 2-byte stores a chunk,
// about half of the kernel's LDS cycles lost to bank conflicts). Q fragments
// are read straight from global memory (16 contiguous bytes).
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
constexpr int kStage = 64;       // the GEMM's k stage
constexpr int kMaxTokens = 256;
constexpr int kMaxKeyTiles = kMaxTokens / kEdge;
constexpr int kMaxWaves = 8;
constexpr int kWavesPerGroup = 4;
/// log2 e / sqrt(head_dim): the logits' scale, 1/8 (a power of two), folded
/// into the exponential's base-2 constant.
constexpr float kScaledLog2e = kLog2e * 0.125F;
static_assert(kHeadDim == 64, "the logits' scale is 1/8");

/// Elements per LDS row of K ([key][head_dim + 8]).
constexpr int kKeyPitch = kHeadDim + 8;
/// 16-byte chunks of one key's K or V row.
constexpr int kChunksPerKey = kHeadDim / 8;

/// V ([key][head_dim]), then K.
__host__ __device__ constexpr std::size_t lds_bytes(int key_tiles) {
    return static_cast<std::size_t>(key_tiles) * kEdge * (kHeadDim + kKeyPitch) * 2;
}

/// Element offset of V[key][dim] in its LDS tile: 16-byte chunk dim / 8 of
/// the key's row sits at chunk (dim / 8) ^ 4 ((key >> 1) & 1).
__device__ __forceinline__ int value_slot(int key, int dim) {
    return key * kHeadDim + 8 * ((dim >> 3) ^ (4 * ((key >> 1) & 1))) + (dim & 7);
}

/// Four 16-bit elements in LDS, the operand type of ds_read_b64_tr_b16.
typedef short Short4 __attribute__((vector_size(4 * sizeof(short))));
using Lds4x16 = __attribute__((address_space(3))) Short4;

/// The weights.V B fragment of k-block @p kb, dims @p d0 + 0..31: lane l
/// holds dim d0 + l % 32, keys 16 kb + 8 (l / 32) + 0..7, the layout a
/// 16-byte row of transposed V would give it.
__device__ __forceinline__ Vec16 value_fragment(const std::uint16_t* values, int kb, int d0,
                                                int lane) {
    const int j = lane & 15;
    const int dim = d0 + 16 * ((lane >> 4) & 1) + 4 * (j & 3);
    Vec16 fragment;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
        const int key = kb * 16 + 8 * (lane >> 5) + 4 * s + (j >> 2);
        // `values` points into LDS; the C-style cast is the address-space
        // conversion the builtin's operand needs.
        const auto part =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((Lds4x16*)(values + value_slot(key, dim)));
        fragment.w[2 * s] = static_cast<std::uint16_t>(part[0]) |
                            (static_cast<std::uint32_t>(static_cast<std::uint16_t>(part[1])) << 16);
        fragment.w[2 * s + 1] = static_cast<std::uint16_t>(part[2]) |
                                (static_cast<std::uint32_t>(static_cast<std::uint16_t>(part[3])) << 16);
    }
    return fragment;
}

/// 16 bytes at @p element of the pair's packed projection, through the
/// buffer resource @p resource (based at that element 0), or zero when
/// @p inside is false: the offset is then one the resource drops, so the load
/// needs no branch. Element offsets stay far inside 32 bits (at most 256
/// tokens of 3 * heads * 64 elements).
__device__ __forceinline__ Vec16 load_or_zero(__amdgpu_buffer_rsrc_t resource, std::int64_t element,
                                              bool inside) {
    return gemm::buffer_load16(resource, inside ? static_cast<unsigned int>(element * 2) : gemm::kOutside);
}

/// op(the lower half's value, the upper half's value) in lanes l and l ^ 32
/// alike: one v_permlane32_swap of the value with itself leaves a lane of the
/// lower half its own value and its partner's, and a lane of the upper half
/// its partner's and its own, lower half first in both (no LDS round trip).
/// The two halves then hold the same bits; op is max or + here, which give
/// the same bits as op(own, partner) in either order.
template <typename Op> __device__ __forceinline__ float combine_halves(float value, Op op) {
    const std::uint32_t bits = __float_as_uint(value);
    const auto swapped = __builtin_amdgcn_permlane32_swap(bits, bits, false, false);
    return op(__uint_as_float(swapped[0]), __uint_as_float(swapped[1]));
}

__device__ __forceinline__ std::uint32_t pack_bf16(float low, float high) {
    return pack_bf16x2(low, high);
}

/// The (image, head) pair's query, key and value bases in the packed
/// [images, tokens, 3, heads, 64] projection.
struct PairBases {
    const std::uint16_t* q;
    const std::uint16_t* k;
    const std::uint16_t* v;
    int image;
    int head;
};

__device__ __forceinline__ PairBases pair_bases(const std::uint16_t* qkv, int pair, int heads,
                                                int tokens) {
    const int image = pair / heads;
    const int head = pair - image * heads;
    const std::int64_t qkv_row = 3 * static_cast<std::int64_t>(heads) * kHeadDim;
    const std::uint16_t* const q =
        qkv + static_cast<std::int64_t>(image) * tokens * qkv_row + head * kHeadDim;
    return {q, q + heads * kHeadDim, q + 2 * heads * kHeadDim, image, head};
}

/// @tparam KT 32-key tiles covering the tokens.
/// @tparam Chunks per thread of a pair's K and V (ceil(2 * KT * 32 * 8 / threads)) when the
///   workgroup loops over several pairs and prefetches the next pair's K and V into
///   registers while it works on the current one; 0 for one pair per workgroup.
/// @tparam kTokens the token count when it is fixed at compile time (197,
///   the ViT/16 count at 224), 0 otherwise: the runs of the last key tile
///   that lie wholly past it are then known to be zero, and their logits
///   skip the max, the exponential, the sum and the probability (a sum of
///   non-negative terms from +0 is unchanged by adding +0).
template <int KT, int Chunks, int kTokens = 0>
__global__ __launch_bounds__(kMaxWaves * kWave) void attention_bf16_kernel(
    const std::uint16_t* __restrict__ qkv, std::uint16_t* __restrict__ context, int heads,
    int tokens_argument, int pairs) {
    const int tokens = kTokens > 0 ? kTokens : tokens_argument;
    // Run q of key tile kt holds keys kt * 32 + 8 q + 4 half + 0..3: with
    // the token count known, a run whose first key is past it is all past it.
    auto run_past = [](int kt, int q) { return kTokens > 0 && kt * kEdge + 8 * q >= kTokens; };
    constexpr int kPadded = KT * kEdge;
    constexpr int kBufferElements = kPadded * (kHeadDim + kKeyPitch);
    extern __shared__ Vec16 lds_vectors[];
    std::uint16_t* const lds = reinterpret_cast<std::uint16_t*>(lds_vectors);
    const int waves = static_cast<int>(blockDim.x) / kWave;
    const int wave = static_cast<int>(threadIdx.x) / kWave;
    const int lane = lane_id();
    const int row = lane % kEdge;  // fragment row: query (logits) or dim (V)
    const int half = lane / kEdge; // which half of a run pair the lane holds
    const int chunk = 8 * half;    // fragment k offset
    const int embed = heads * kHeadDim;
    const std::int64_t qkv_row = 3 * static_cast<std::int64_t>(embed);
    constexpr int kChunks = kHeadDim / 8;

    // V and K of a pair into LDS buffer `buffer` ([kPadded][64] V, then
    // [kPadded][72] K), straight from global memory; keys past the tokens are zero.
    auto load_direct = [&](const PairBases& b, int buffer) {
        std::uint16_t* const values = lds + buffer * kBufferElements;
        std::uint16_t* const keys = values + kPadded * kHeadDim;
        const auto resource = gemm::buffer_resource(b.k);
        // Rounds of kRound chunks per thread: a round's loads all go out
        // before its stores, one latency per round.
        constexpr int kRound = 4;
        const int threads = static_cast<int>(blockDim.x);
        for (int c0 = threadIdx.x; c0 < kPadded * kChunks; c0 += kRound * threads) {
            Vec16 v[kRound];
            Vec16 k[kRound];
#pragma unroll
            for (int r = 0; r < kRound; ++r) {
                const int c = c0 + r * threads;
                const int key = c / kChunks;
                const int d0 = 8 * (c % kChunks);
                const bool inside = c < kPadded * kChunks && key < tokens;
                v[r] = load_or_zero(resource, key * qkv_row + d0 + embed, inside);
                k[r] = load_or_zero(resource, key * qkv_row + d0, inside);
            }
#pragma unroll
            for (int r = 0; r < kRound; ++r) {
                const int c = c0 + r * threads;
                if (c < kPadded * kChunks) {
                    const int key = c / kChunks;
                    const int d0 = 8 * (c % kChunks);
                    store16(values + value_slot(key, d0), v[r]);
                    store16(keys + key * kKeyPitch + d0, k[r]);
                }
            }
        }
    };
    // The same through registers: chunk c of the pair's 2 * kPadded * 8 is
    // thread (c % threads)'s element c / threads; V's chunks first.
    Vec16 ahead[Chunks > 0 ? Chunks : 1];
    auto prefetch = [&](const PairBases& b) {
        // V sits embed elements after K in every token's row.
        const auto resource = gemm::buffer_resource(b.k);
#pragma unroll
        for (int i = 0; i < Chunks; ++i) {
            const int c = static_cast<int>(threadIdx.x) + i * static_cast<int>(blockDim.x);
            const bool is_key = c >= kPadded * kChunks;
            const int cc = is_key ? c - kPadded * kChunks : c;
            const int key = cc / kChunks;
            const int d0 = 8 * (cc % kChunks);
            ahead[i] = load_or_zero(resource, key * qkv_row + d0 + (is_key ? 0 : embed),
                                    c < 2 * kPadded * kChunks && key < tokens);
        }
    };
    auto commit = [&](int buffer) {
        std::uint16_t* const values = lds + buffer * kBufferElements;
        std::uint16_t* const keys = values + kPadded * kHeadDim;
#pragma unroll
        for (int i = 0; i < Chunks; ++i) {
            const int c = static_cast<int>(threadIdx.x) + i * static_cast<int>(blockDim.x);
            if (c < 2 * kPadded * kChunks) {
                const bool is_key = c >= kPadded * kChunks;
                const int cc = is_key ? c - kPadded * kChunks : c;
                const int key = cc / kChunks;
                const int d0 = 8 * (cc % kChunks);
                if (is_key) {
                    store16(keys + key * kKeyPitch + d0, ahead[i]);
                } else {
                    store16(values + value_slot(key, d0), ahead[i]);
                }
            }
        }
    };

    // This wavefront's query tile, the same in every pair; its Q fragments
    // (16 contiguous bytes of row query, k chunk 8 half) straight from global
    // memory, the next pair's loaded while the current one is worked on.
    const int query0 = (static_cast<int>(blockIdx.x) * waves + wave) * kEdge;
    const int query = query0 + row;
    auto load_queries = [&](const PairBases& b, Vec16 (&q)[kHeadDim / kKBlock]) {
        const auto resource = gemm::buffer_resource(b.q);
#pragma unroll
        for (int kb = 0; kb < kHeadDim / kKBlock; ++kb) {
            q[kb] = load_or_zero(resource, query * qkv_row + kb * kKBlock + chunk, query < tokens);
        }
    };

    int pair = static_cast<int>(blockIdx.y);
    int buffer = 0;
    Vec16 q[kHeadDim / kKBlock];
    Vec16 q_ahead[kHeadDim / kKBlock];
    // The first pair: its Q, then (with a prefetch register set) all of its
    // K and V loads in flight before the first LDS store, one latency in all
    // (the strided loop below waits for each round of loads in turn).
    load_queries(pair_bases(qkv, pair, heads, tokens), q);
    if constexpr (Chunks > 0) {
        prefetch(pair_bases(qkv, pair, heads, tokens));
        commit(0);
    } else {
        load_direct(pair_bases(qkv, pair, heads, tokens), 0);
    }
    __syncthreads();
    for (;;) {
    const int next = pair + static_cast<int>(gridDim.y);
    const bool more = Chunks > 0 && next < pairs;
    if (more) {
        prefetch(pair_bases(qkv, next, heads, tokens));
        load_queries(pair_bases(qkv, next, heads, tokens), q_ahead);
    }
    const PairBases bases = pair_bases(qkv, pair, heads, tokens);
    const int image = bases.image;
    const int head = bases.head;
    const std::uint16_t* const values = lds + buffer * kBufferElements;
    const std::uint16_t* const keys = values + kPadded * kHeadDim;
    if (query0 < tokens) {

    // Logits tiles: the GEMM's MFMA and operand roles, alpha * sum rounded
    // to bf16 as the GEMM stores it, then read back as the softmax reads it.
    // The first k-block's MFMA takes its zero accumulator as an inline
    // constant (the same +0 the GEMM starts from, without 16 moves a tile).
    Acc x[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int key = kt * kEdge + row;
#pragma unroll
        for (int kb = 0; kb < kHeadDim / kKBlock; ++kb) {
            const Vec16 k = load16(keys + key * kKeyPitch + kb * kKBlock + chunk);
            x[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gemm::bf16x8, k),
                                                           __builtin_bit_cast(gemm::bf16x8, q[kb]),
                                                           kb == 0 ? Acc{} : x[kt], 0, 0, 0);
        }
    }

    // The GEMM stores alpha * sum rounded to bf16, alpha = 1/8. A power of
    // two commutes with rounding to nearest (bf16 or float), with the max and
    // with a difference of two such values, and log2 e / 8 is as exact as
    // log2 e: the softmax's exponent (round(sum / 8) - round(max / 8)) * log2 e
    // is (round(sum) - round(max)) * (log2 e / 8), bit for bit, whenever the
    // scaled values are normal floats. (Below 2^-126 the two differ only by
    // less than an exponent of 2^-120, which exp2 returns as 1 either way.)
    // So the sums are rounded unscaled, two per conversion (the same rounding
    // as one at a time), and the 1/8 rides in the exponent's constant. The
    // row max over the valid keys is exact in any order, and rounding to
    // nearest never reverses an order, so the max of the rounded logits is
    // the rounded max of the unrounded ones: it is taken over the products,
    // which need no canonicalizing.
    float maximum = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key = kt * kEdge + Bf16Mma::column(lane, i / 4) + i % 4;
            // Only the last key tile holds keys past the tokens.
            if (!run_past(kt, i / 4) && (kt < KT - 1 || key < tokens)) {
                maximum = fmaxf(maximum, x[kt][i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
            if (run_past(kt, i / 4)) {
                continue;
            }
            const std::uint32_t bits = pack_bf16x2(x[kt][i], x[kt][i + 1]);
            x[kt][i] = __uint_as_float(bits << 16);
            x[kt][i + 1] = __uint_as_float(bits & 0xFFFF0000U);
        }
    }
    maximum = bf16_to_float(float_to_bf16(maximum));
    maximum = combine_halves(maximum, [](float a, float b) { return fmaxf(a, b); });

    // Exponentials in the bf16 softmax's fused form (softmax_terms.hpp),
    // exp2(x * c + shift) with shift = -(max * c) rounded once, where c
    // carries the 1/8; keys past the tokens are 0, as the softmax sets them.
    const float shift = -(maximum * kScaledLog2e);
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int key = kt * kEdge + Bf16Mma::column(lane, i / 4) + i % 4;
            x[kt][i] = !run_past(kt, i / 4) && (kt < KT - 1 || key < tokens)
                           ? __builtin_amdgcn_exp2f(fmaf(x[kt][i], kScaledLog2e, shift))
                           : 0.F;
        }
    }

    // Team lane t = 8 g + 4 half + r sums columns t + 16 j, j = 0, 1, ...:
    // column t + 16 j is run q = g + 2 (j % 2), element r, of key tile j / 2.
    float quad[2];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        float part[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float sum = 0.F;
#pragma unroll
            for (int j = 0; j < 2 * KT; ++j) {
                if (!run_past(j / 2, g + 2 * (j % 2))) {
                    sum += x[j / 2][4 * (g + 2 * (j % 2)) + r];
                }
            }
            part[r] = sum;
        }
        // DPP steps t ^ 1 and t ^ 2 inside the quad
        quad[g] = (part[0] + part[1]) + (part[2] + part[3]);
    }
    // half-row mirror pairs quads 0-1 and 2-3, row mirror the two results:
    // (Q0 + Q1) + (Q2 + Q3), the same bits in both lanes of the row
    const auto add = [](float a, float b) { return a + b; };
    const float total = combine_halves(quad[0], add) + combine_halves(quad[1], add);
    const float inverse = 1.0F / total;

    // Probabilities rounded to bf16 and packed by runs: p[kt][q] = keys
    // kt * 32 + 8 q + 4 half + 0..3.
    std::uint32_t p[KT][4][2];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int run = 0; run < 4; ++run) {
            if (run_past(kt, run)) {
                p[kt][run][0] = 0U;  // 0 * inverse, rounded: +0
                p[kt][run][1] = 0U;
                continue;
            }
            p[kt][run][0] = pack_bf16(x[kt][4 * run] * inverse, x[kt][4 * run + 1] * inverse);
            p[kt][run][1] = pack_bf16(x[kt][4 * run + 2] * inverse, x[kt][4 * run + 3] * inverse);
        }
    }
    // A fragment of k-block 2 kt + s: keys kt * 32 + 16 s + 8 half + 0..7.
    // Half 0 needs its own run 2 s and its partner's; half 1 its partner's
    // run 2 s + 1 and its own. v_permlane32_swap of (run 2 s, run 2 s + 1)
    // trades the upper lanes of the first with the lower lanes of the second
    // (new first[32 + i] = second[i], new second[i] = first[32 + i]), which
    // leaves exactly that in (first, second) in every lane.
    Vec16 fragment[2 * KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            Vec16& f = fragment[2 * kt + s];
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const auto swapped = __builtin_amdgcn_permlane32_swap(p[kt][2 * s][w], p[kt][2 * s + 1][w],
                                                                     false, false);
                f.w[w] = swapped[0];
                f.w[2 + w] = swapped[1];
            }
        }
    }

    // weights.V over the GEMM's k-blocks: its 64-key stages run in pairs.
    constexpr int kStages = (kPadded + kStage - 1) / kStage;
    constexpr int kBlocks = (kStages + 1) / 2 * 2 * (kStage / kKBlock);
    // The two 32-dim halves accumulate side by side (two independent MFMA
    // chains); each keeps the k-block order above.
    Acc acc2[2];
#pragma unroll
    for (int kb = 0; kb < kBlocks; ++kb) {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            if (kb == 0) {
                const Vec16 v = value_fragment(values, kb, d * kEdge, lane);
                acc2[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(gemm::bf16x8, v),
                                                                 __builtin_bit_cast(gemm::bf16x8, fragment[0]),
                                                                 Acc{}, 0, 0, 0);
            } else if (kb < 2 * KT) {
                const Vec16 v = value_fragment(values, kb, d * kEdge, lane);
                Bf16Mma::run(acc2[d], v, fragment[kb]);
            } else {
                const Vec16 zero{{0U, 0U, 0U, 0U}};
                Bf16Mma::run(acc2[d], zero, zero);
            }
        }
    }
#pragma unroll
    for (int d0 = 0; d0 < kHeadDim; d0 += kEdge) {
        const Acc& acc = acc2[d0 / kEdge];
        if (query < tokens) {
            std::uint16_t* const out = context +
                                       (static_cast<std::int64_t>(image) * tokens + query) * embed +
                                       head * kHeadDim + d0;
#pragma unroll
            for (int run = 0; run < Bf16Mma::kRuns; ++run) {
                uint2 bits;
                bits.x = pack_bf16(1.0F * acc[4 * run], 1.0F * acc[4 * run + 1]);
                bits.y = pack_bf16(1.0F * acc[4 * run + 2], 1.0F * acc[4 * run + 3]);
                *reinterpret_cast<uint2*>(out + Bf16Mma::column(lane, run)) = bits;
            }
        }
    }
    }  // query0 < tokens
    if (!more) {
        break;
    }
    commit(buffer ^ 1);
    // Every wavefront is done with this pair's buffer and the next one's is whole.
    __syncthreads();
    buffer ^= 1;
    pair = next;
    static_assert(kHeadDim / kKBlock == 4, "four Q fragments");
    q[0] = q_ahead[0];
    q[1] = q_ahead[1];
    q[2] = q_ahead[2];
    q[3] = q_ahead[3];
    }
}

template <int KT>
hipError_t launch(const std::uint16_t* qkv, std::uint16_t* context, int images, int heads,
                  int tokens, hipStream_t stream) {
    // Query tiles per workgroup, measured on MI355X at 197 tokens: all of
    // them (one K/V load per (image, head)) once there are two (image, head)
    // pairs per compute unit (ViT-Base b64: 47.1 us against 49.9 with four),
    // four below that (ViT-Tiny b32: 11.4 us against 14.8 with seven).
    const int query_tiles = (tokens + kEdge - 1) / kEdge;
    const std::int64_t pairs = static_cast<std::int64_t>(images) * heads;
    const bool many = pairs >= 2 * static_cast<std::int64_t>(compute_units());
    const int per_group = many ? kMaxWaves : kWavesPerGroup;
    const int waves = query_tiles < per_group ? query_tiles : per_group;
    // (Up to 7 key tiles, 224 tokens: with 8 the prefetch registers spill.)
    if constexpr (KT <= 7) {
    if (many && pairs <= 0x7FFFFFFF) {
        // One workgroup per CU (the kernel's registers allow one of KT
        // wavefronts) looping over pairs, the next pair's K and V loaded into
        // registers during the current pair's work and into the second LDS
        // buffer after it: each CU's later pairs do not wait for their loads.
        // With waves = KT, a thread's share of a pair's K and V is 8 chunks.
        constexpr int kChunksPerThread = 2 * kEdge * kChunksPerKey / kWave;
        const std::int64_t groups = compute_units() < pairs ? compute_units() : pairs;
        auto run = [&](auto kernel, std::atomic<std::uint64_t>& opted_in) -> hipError_t {
            if (const hipError_t opted =
                    allow_lds(reinterpret_cast<const void*>(kernel), 2 * lds_bytes(KT), opted_in);
                opted != hipSuccess) {
                return opted;
            }
            kernel<<<dim3(1, static_cast<unsigned int>(groups)), query_tiles * kWave,
                     2 * lds_bytes(KT), stream>>>(qkv, context, heads, tokens, static_cast<int>(pairs));
            return hipGetLastError();
        };
        // 197 tokens (ViT/16 at 224) with the count as a constant: the last
        // key tile's runs past it cost nothing.
        if constexpr (KT == 7) {
            if (tokens == 197) {
                static std::atomic<std::uint64_t> opted_in{0};
                return run(attention_bf16_kernel<KT, kChunksPerThread, 197>, opted_in);
            }
        }
        static std::atomic<std::uint64_t> opted_in{0};
        return run(attention_bf16_kernel<KT, kChunksPerThread>, opted_in);
    }
    }
    // Above 64 KiB (256 tokens) the kernel opts in to more LDS, once per device.
    auto kernel = attention_bf16_kernel<KT, 0>;
    static std::atomic<std::uint64_t> opted_in{0};
    if (const hipError_t opted = allow_lds(reinterpret_cast<const void*>(kernel), lds_bytes(KT),
                                           opted_in);
        opted != hipSuccess) {
        return opted;
    }
    const dim3 grid(static_cast<unsigned int>((query_tiles + waves - 1) / waves),
                    static_cast<unsigned int>(pairs));
    kernel<<<grid, waves * kWave, lds_bytes(KT), stream>>>(qkv, context, heads, tokens,
                                                          static_cast<int>(pairs));
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
    switch ((tokens + kEdge - 1) / kEdge) {
    case 1: return launch<1>(qkv, context, images, heads, tokens, stream);
    case 2: return launch<2>(qkv, context, images, heads, tokens, stream);
    case 3: return launch<3>(qkv, context, images, heads, tokens, stream);
    case 4: return launch<4>(qkv, context, images, heads, tokens, stream);
    case 5: return launch<5>(qkv, context, images, heads, tokens, stream);
    case 6: return launch<6>(qkv, context, images, heads, tokens, stream);
    case 7: return launch<7>(qkv, context, images, heads, tokens, stream);
    default: return launch<kMaxKeyTiles>(qkv, context, images, heads, tokens, stream);
    }
}

} // namespace cuvit::detail
