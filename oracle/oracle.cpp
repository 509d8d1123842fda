// CPU oracle for the layer-kernel path. TEST INFRASTRUCTURE ONLY (see
// oracle.h): what the tests compare the HIP library against, never part of it.
//
// How each function is pinned (beyond restating the reference's loops):
//   layer_norm, softmax, gelu, gemm, gemm_transposed, gemm_term_magnitudes
//     - bit-exact against the reference's own tests/reference/linear_algebra.hpp
//       compiled from /root/reference into oracle/_ref (tests/test_oracle_ref.py);
//     - closed forms and invariants (zero mean / unit variance, rows summing to
//       one, one-hot saturation, GELU landmarks, textbook triple loop).
//   gemm_problem_run - reduces to gemm / gemm_transposed per entry, and the
//     epilogue order is checked against a deliberately wrong order.
//   extract_patches - iota known answer (every output equals its source index)
//     and the permutation property; brute-force index map at small geometry.
//   add, add_broadcast, broadcast - closed forms.
//   vit_forward - assembled from the pinned pieces; cross-checked against a
//     numpy restatement of tests/reference/vit.hpp at a small configuration.
//   vit_forward_bf16 - the same code with rounding inserted (no reference: the
//     bf16 model is an extension); pinned by reducing to vit_forward on
//     bf16-exact data with rounding as the only difference, by its rounding
//     agreeing with round_bf16, and by staying within bf16 error of vit_forward.
//   generator - the mt19937_64 10000th-output value fixed by the C++ standard,
//     committed first-values fixtures, distribution moments.
//   round_bf16 - exhaustive properties on special values and ties.
//   preprocess - bit-exact against the reference's src/runtime/image.cpp
//     compiled into oracle/_ref; closed forms that fix it without the
//     reference: identity geometry (a size x size image with crop fraction 1
//     reproduces the normalised pixels), exact 2x2 box averages at a 2x
//     downscale, transposing the image transposes the tensor, and the
//     reference's own image_test cases (uniform grey, planar channels, centre
//     crop, rejected settings).
#include "oracle.h"

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <random>
#include <string>
#include <vector>

namespace {

/// @p value rounded to the nearest bf16 (ties to even), widened back to float;
/// a NaN stays NaN. The same rounding as oracle_round_bf16.
float round_to_bf16_value(float value) {
    std::uint32_t bits = 0;
    std::memcpy(&bits, &value, sizeof(bits));
    if ((bits & 0x7F800000U) == 0x7F800000U && (bits & 0x007FFFFFU) != 0) {
        bits |= 0x00400000U;
    } else {
        bits += 0x7FFFU + ((bits >> 16) & 1U);
    }
    bits &= 0xFFFF0000U;
    float out = 0.0F;
    std::memcpy(&out, &bits, sizeof(out));
    return out;
}

float gelu_value(float value) {
    // tests/reference/linear_algebra.hpp:120-123 (erf form).
    return 0.5F * value * (1.0F + std::erf(value * 0.7071067811865475F));
}

} // namespace

extern "C" {

// tests/reference/linear_algebra.hpp:70-96: double mean and biased variance,
// then float((x - mean) * inv) * gamma + beta in float.
void oracle_layer_norm(const float* input, const float* gamma, const float* beta, float* output,
                       int rows, int columns, float epsilon) {
    for (int r = 0; r < rows; ++r) {
        const float* x = input + static_cast<std::int64_t>(r) * columns;
        float* y = output + static_cast<std::int64_t>(r) * columns;
        double total = 0.0;
        for (int c = 0; c < columns; ++c) {
            total += x[c];
        }
        const double mean = total / columns;
        double spread = 0.0;
        for (int c = 0; c < columns; ++c) {
            const double centred = x[c] - mean;
            spread += centred * centred;
        }
        spread /= columns;
        const double inverse = 1.0 / std::sqrt(spread + epsilon);
        for (int c = 0; c < columns; ++c) {
            y[c] = static_cast<float>((x[c] - mean) * inverse) * gamma[c] + beta[c];
        }
    }
}

// tests/reference/linear_algebra.hpp:98-118: float max, double exp and sum,
// the exponential stored as float and divided by the double sum.
void oracle_softmax(const float* input, float* output, int rows, int columns) {
    for (int r = 0; r < rows; ++r) {
        const float* x = input + static_cast<std::int64_t>(r) * columns;
        float* y = output + static_cast<std::int64_t>(r) * columns;
        float peak = x[0];
        for (int c = 1; c < columns; ++c) {
            peak = std::max(peak, x[c]);
        }
        double total = 0.0;
        for (int c = 0; c < columns; ++c) {
            const double e = std::exp(static_cast<double>(x[c]) - peak);
            y[c] = static_cast<float>(e);
            total += e;
        }
        for (int c = 0; c < columns; ++c) {
            y[c] = static_cast<float>(y[c] / total);
        }
    }
}

float oracle_gelu_scalar(float value) { return gelu_value(value); }

// tests/reference/linear_algebra.hpp:125-129.
void oracle_gelu(const float* input, float* output, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        output[i] = gelu_value(input[i]);
    }
}

// tests/reference/linear_algebra.hpp:17-31: sequential float k-loop, then
// alpha * sum + bias.
void oracle_gemm(const float* a, const float* b, const float* bias, float* c, int m, int n, int k,
                 float alpha) {
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float sum = 0.0F;
            for (int p = 0; p < k; ++p) {
                sum += a[static_cast<std::int64_t>(i) * k + p] * b[static_cast<std::int64_t>(p) * n + j];
            }
            c[static_cast<std::int64_t>(i) * n + j] = alpha * sum + (bias != nullptr ? bias[j] : 0.0F);
        }
    }
}

// tests/reference/linear_algebra.hpp:33-48: B stored [N, K].
void oracle_gemm_transposed(const float* a, const float* b, const float* bias, float* c, int m,
                            int n, int k, float alpha) {
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float sum = 0.0F;
            for (int p = 0; p < k; ++p) {
                sum += a[static_cast<std::int64_t>(i) * k + p] * b[static_cast<std::int64_t>(j) * k + p];
            }
            c[static_cast<std::int64_t>(i) * n + j] = alpha * sum + (bias != nullptr ? bias[j] : 0.0F);
        }
    }
}

// tests/reference/linear_algebra.hpp:52-68: sum of |a * b| per output, times |alpha|.
void oracle_gemm_term_magnitudes(const float* a, const float* b, float* scale, int m, int n, int k,
                                 int transposed, float alpha) {
    for (int i = 0; i < m; ++i) {
        for (int j = 0; j < n; ++j) {
            float total = 0.0F;
            for (int p = 0; p < k; ++p) {
                const float left = a[static_cast<std::int64_t>(i) * k + p];
                const float right = transposed != 0 ? b[static_cast<std::int64_t>(j) * k + p]
                                                    : b[static_cast<std::int64_t>(p) * n + j];
                total += std::abs(left * right);
            }
            scale[static_cast<std::int64_t>(i) * n + j] = std::abs(alpha) * total;
        }
    }
}

// The launch_gemm contract in plain loops: batch addressing
// (src/kernels/gemm.cu:58-72), leading-dimension defaults (gemm.cu:225-228),
// and the epilogue alpha -> bias -> GELU -> store or accumulate
// (gemm.cu:153-162, include/cuvit/kernels.hpp:61-73).
void oracle_gemm_problem_run(const float* a, const float* b, const float* bias, float* c,
                             const oracle_gemm_problem* p) {
    const bool transposed = p->layout == 1;
    const int lda = p->lda != 0 ? p->lda : p->k;
    const int ldb = p->ldb != 0 ? p->ldb : (transposed ? p->k : p->n);
    const int ldc = p->ldc != 0 ? p->ldc : p->n;
    const bool split = p->inner > 0 && p->inner < p->count;
    for (int entry = 0; entry < p->count; ++entry) {
        std::int64_t oa = 0;
        std::int64_t ob = 0;
        std::int64_t oc = 0;
        if (split) {
            const std::int64_t outer = entry / p->inner;
            const std::int64_t index = entry % p->inner;
            oa = outer * p->outer_stride_a + index * p->stride_a;
            ob = outer * p->outer_stride_b + index * p->stride_b;
            oc = outer * p->outer_stride_c + index * p->stride_c;
        } else {
            oa = entry * p->stride_a;
            ob = entry * p->stride_b;
            oc = entry * p->stride_c;
        }
        for (int i = 0; i < p->m; ++i) {
            for (int j = 0; j < p->n; ++j) {
                float sum = 0.0F;
                for (int q = 0; q < p->k; ++q) {
                    const float left = a[oa + static_cast<std::int64_t>(i) * lda + q];
                    const float right = transposed ? b[ob + static_cast<std::int64_t>(j) * ldb + q]
                                                   : b[ob + static_cast<std::int64_t>(q) * ldb + j];
                    sum += left * right;
                }
                float value = p->alpha * sum;
                if (bias != nullptr) {
                    value += bias[j];
                }
                if (p->gelu != 0) {
                    value = gelu_value(value);
                }
                float& out = c[oc + static_cast<std::int64_t>(i) * ldc + j];
                out = p->accumulate != 0 ? out + value : value;
            }
        }
    }
}

// tests/reference/vit.hpp:65-87 (one image) with the batch laid out image-major
// as src/kernels/normalization.cu:168-191 does.
void oracle_extract_patches(const float* images, float* patches, int batch, int channels,
                            int height, int width, int patch) {
    const int across = width / patch;
    const int down = height / patch;
    const std::int64_t row_length = static_cast<std::int64_t>(channels) * patch * patch;
    const std::int64_t plane = static_cast<std::int64_t>(channels) * height * width;
    for (int image = 0; image < batch; ++image) {
        for (int index = 0; index < down * across; ++index) {
            const int patch_row = index / across;
            const int patch_column = index % across;
            const std::int64_t row = static_cast<std::int64_t>(image) * down * across + index;
            for (int channel = 0; channel < channels; ++channel) {
                for (int y = 0; y < patch; ++y) {
                    for (int x = 0; x < patch; ++x) {
                        patches[row * row_length + (static_cast<std::int64_t>(channel) * patch + y) * patch + x] =
                            images[image * plane +
                                   (static_cast<std::int64_t>(channel) * height + patch_row * patch + y) * width +
                                   patch_column * patch + x];
                    }
                }
            }
        }
    }
}

// src/kernels/normalization.cu:148-154; tests/reference/elementwise.hpp:14-18.
void oracle_add(float* accumulator, const float* addend, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        accumulator[i] += addend[i];
    }
}

// src/kernels/normalization.cu:194-201; CPU form tests/reference/vit.hpp:96-98.
void oracle_add_broadcast(float* accumulator, const float* addend, int64_t count, int batch) {
    for (int s = 0; s < batch; ++s) {
        for (int64_t i = 0; i < count; ++i) {
            accumulator[s * count + i] += addend[i];
        }
    }
}

// src/kernels/normalization.cu:203-212; CPU form tests/reference/vit.hpp:89-92.
void oracle_broadcast(float* destination, const float* source, int64_t count,
                      int64_t destination_stride, int batch) {
    for (int s = 0; s < batch; ++s) {
        for (int64_t i = 0; i < count; ++i) {
            destination[s * destination_stride + i] = source[i];
        }
    }
}

// tests/reference/vit.hpp:57-112 (forward) and 134-206 (run_block): one image,
// one named buffer per step, per-head attention in plain loops.
//
// With reduced set, the same steps with every stored value rounded to bf16 at
// the point where the bf16 model stores it (the extension has no reference;
// this is its definition): the image, the GEMM weight matrices, every token
// row after the embedding and after each residual accumulate, each LayerNorm
// output, q/k/v, the attention logits (after the 1/sqrt(head_dim) scale), the
// attention weights, the context, the MLP hidden (after GELU) and the logits.
// Biases, gamma, beta, cls and pos stay fp32; an accumulate rounds
// x + (sum + bias) once. With reduced clear nothing is rounded and this is
// the fp32 forward above.
static void vit_forward(const oracle_vit_config* cfg, const float* const* tensors,
                        const float* image_in, float* logits, bool reduced) {
    const int embed = cfg->embed_dim;
    const int across = cfg->image_size / cfg->patch_size;
    const int patch_count = across * across;
    const int tokens = patch_count + 1;
    const int patch_elements = cfg->channels * cfg->patch_size * cfg->patch_size;
    const int heads = cfg->heads;
    const int head_dim = embed / heads;
    const int hidden = cfg->mlp_hidden;
    const float eps = cfg->layer_norm_epsilon;

    auto round = [reduced](std::vector<float>& v) {
        if (reduced) {
            for (float& x : v) {
                x = round_to_bf16_value(x);
            }
        }
    };
    // A GEMM weight matrix as the model stores it.
    auto matrix = [&](const float* w, std::size_t count) {
        std::vector<float> m(w, w + count);
        round(m);
        return m;
    };

    const float* cls = tensors[0];
    const float* pos = tensors[1];
    const std::vector<float> patch_weight =
        matrix(tensors[2], static_cast<std::size_t>(embed) * patch_elements);
    const float* patch_bias = tensors[3];

    std::vector<float> image(image_in, image_in + static_cast<std::size_t>(cfg->channels) *
                                                      cfg->image_size * cfg->image_size);
    round(image);
    std::vector<float> patches(static_cast<std::size_t>(patch_count) * patch_elements);
    oracle_extract_patches(image.data(), patches.data(), 1, cfg->channels, cfg->image_size,
                           cfg->image_size, cfg->patch_size);

    std::vector<float> x(static_cast<std::size_t>(tokens) * embed);
    for (int i = 0; i < embed; ++i) {
        x[static_cast<std::size_t>(i)] = cls[i];
    }
    oracle_gemm_transposed(patches.data(), patch_weight.data(), patch_bias, x.data() + embed,
                           patch_count, embed, patch_elements, 1.0F);
    for (std::size_t i = 0; i < x.size(); ++i) {
        x[i] += pos[i];
    }
    round(x);

    std::vector<float> normalized(x.size());
    std::vector<float> qkv(static_cast<std::size_t>(tokens) * 3 * embed);
    std::vector<float> context(x.size());
    std::vector<float> logits_tt(static_cast<std::size_t>(tokens) * tokens);
    std::vector<float> weights_tt(logits_tt.size());
    std::vector<float> projected(x.size());
    std::vector<float> mlp(static_cast<std::size_t>(tokens) * hidden);
    const float scale = 1.0F / std::sqrt(static_cast<float>(head_dim));
    const int row = 3 * embed;

    for (int block = 0; block < cfg->depth; ++block) {
        const float* const* t = tensors + 4 + 12 * block;
        // t: norm1 w/b, qkv w/b, proj w/b, norm2 w/b, fc1 w/b, fc2 w/b
        const std::vector<float> qkv_weight = matrix(t[2], static_cast<std::size_t>(row) * embed);
        const std::vector<float> proj_weight = matrix(t[4], static_cast<std::size_t>(embed) * embed);
        const std::vector<float> fc1_weight = matrix(t[8], static_cast<std::size_t>(hidden) * embed);
        const std::vector<float> fc2_weight = matrix(t[10], static_cast<std::size_t>(embed) * hidden);

        oracle_layer_norm(x.data(), t[0], t[1], normalized.data(), tokens, embed, eps);
        round(normalized);
        oracle_gemm_transposed(normalized.data(), qkv_weight.data(), t[3], qkv.data(), tokens, row,
                               embed, 1.0F);
        round(qkv);
        for (int h = 0; h < heads; ++h) {
            for (int q = 0; q < tokens; ++q) {
                for (int kk = 0; kk < tokens; ++kk) {
                    float sum = 0.0F;
                    for (int d = 0; d < head_dim; ++d) {
                        sum += qkv[static_cast<std::size_t>(q) * row + h * head_dim + d] *
                               qkv[static_cast<std::size_t>(kk) * row + embed + h * head_dim + d];
                    }
                    logits_tt[static_cast<std::size_t>(q) * tokens + kk] = sum * scale;
                }
            }
            round(logits_tt);
            oracle_softmax(logits_tt.data(), weights_tt.data(), tokens, tokens);
            round(weights_tt);
            for (int q = 0; q < tokens; ++q) {
                for (int d = 0; d < head_dim; ++d) {
                    float sum = 0.0F;
                    for (int kk = 0; kk < tokens; ++kk) {
                        sum += weights_tt[static_cast<std::size_t>(q) * tokens + kk] *
                               qkv[static_cast<std::size_t>(kk) * row + 2 * embed + h * head_dim + d];
                    }
                    context[static_cast<std::size_t>(q) * embed + h * head_dim + d] = sum;
                }
            }
        }
        round(context);
        oracle_gemm_transposed(context.data(), proj_weight.data(), t[5], projected.data(), tokens,
                               embed, embed, 1.0F);
        for (std::size_t i = 0; i < x.size(); ++i) {
            x[i] += projected[i];
        }
        round(x);
        oracle_layer_norm(x.data(), t[6], t[7], normalized.data(), tokens, embed, eps);
        round(normalized);
        oracle_gemm_transposed(normalized.data(), fc1_weight.data(), t[9], mlp.data(), tokens,
                               hidden, embed, 1.0F);
        oracle_gelu(mlp.data(), mlp.data(), static_cast<int64_t>(mlp.size()));
        round(mlp);
        oracle_gemm_transposed(mlp.data(), fc2_weight.data(), t[11], projected.data(), tokens, embed,
                               hidden, 1.0F);
        for (std::size_t i = 0; i < x.size(); ++i) {
            x[i] += projected[i];
        }
        round(x);
    }

    const float* const* tail = tensors + 4 + 12 * cfg->depth;
    const std::vector<float> head_weight =
        matrix(tail[2], static_cast<std::size_t>(cfg->classes) * embed);
    oracle_layer_norm(x.data(), tail[0], tail[1], normalized.data(), tokens, embed, eps);
    round(normalized);
    std::vector<float> out(static_cast<std::size_t>(cfg->classes));
    oracle_gemm_transposed(normalized.data(), head_weight.data(), tail[3], out.data(), 1,
                           cfg->classes, embed, 1.0F);
    round(out);
    std::copy(out.begin(), out.end(), logits);
}

void oracle_vit_forward(const oracle_vit_config* cfg, const float* const* tensors,
                        const float* image, float* logits) {
    vit_forward(cfg, tensors, image, logits, false);
}

void oracle_vit_forward_bf16(const oracle_vit_config* cfg, const float* const* tensors,
                             const float* image, float* logits) {
    vit_forward(cfg, tensors, image, logits, true);
}

void oracle_round_bf16(const float* input, uint16_t* output, int64_t count) {
    for (int64_t i = 0; i < count; ++i) {
        std::uint32_t bits = 0;
        std::memcpy(&bits, input + i, sizeof(bits));
        if ((bits & 0x7F800000U) == 0x7F800000U && (bits & 0x007FFFFFU) != 0) {
            output[i] = static_cast<uint16_t>((bits >> 16) | 0x0040U);
            continue;
        }
        const std::uint32_t lsb = (bits >> 16) & 1U;
        output[i] = static_cast<uint16_t>((bits + 0x7FFFU + lsb) >> 16);
    }
}

int oracle_preprocess(const uint8_t* pixels, int width, int height, int size, float crop_fraction,
                      const float* mean, const float* stddev, float* tensor) {
    // src/runtime/image.cpp:95-135, with the bilinear sample of 37-55 inline.
    if (width <= 0 || height <= 0) {
        return 1;
    }
    if (size <= 0) {
        return 2;
    }
    if (!(crop_fraction > 0.0F) || crop_fraction > 1.0F) {
        return 3;
    }
    for (int c = 0; c < 3; ++c) {
        if (stddev[c] == 0.0F) {
            return 4;
        }
    }
    const float side = static_cast<float>(size);
    const float target = std::round(side / crop_fraction);
    const float scale = static_cast<float>(std::min(width, height)) / target;
    const float window = side * scale;
    const float x_origin = (static_cast<float>(width) - window) * 0.5F;
    const float y_origin = (static_cast<float>(height) - window) * 0.5F;
    const float step = window / side;

    auto at = [&](int x, int y, int c) -> float {
        const int cx = x < 0 ? 0 : (x >= width ? width - 1 : x);
        const int cy = y < 0 ? 0 : (y >= height ? height - 1 : y);
        return static_cast<float>(
            pixels[(static_cast<std::size_t>(cy) * static_cast<std::size_t>(width) +
                    static_cast<std::size_t>(cx)) * 3 + static_cast<std::size_t>(c)]);
    };
    const std::size_t plane = static_cast<std::size_t>(size) * static_cast<std::size_t>(size);
    for (int c = 0; c < 3; ++c) {
        for (int r = 0; r < size; ++r) {
            const float y = y_origin + (static_cast<float>(r) + 0.5F) * step - 0.5F;
            const int y0 = static_cast<int>(std::floor(y));
            const float fy = y - static_cast<float>(y0);
            for (int q = 0; q < size; ++q) {
                const float x = x_origin + (static_cast<float>(q) + 0.5F) * step - 0.5F;
                const int x0 = static_cast<int>(std::floor(x));
                const float fx = x - static_cast<float>(x0);
                const float upper = at(x0, y0, c) * (1.0F - fx) + at(x0 + 1, y0, c) * fx;
                const float lower = at(x0, y0 + 1, c) * (1.0F - fx) + at(x0 + 1, y0 + 1, c) * fx;
                const float sample = upper * (1.0F - fy) + lower * fy;
                tensor[static_cast<std::size_t>(c) * plane +
                       static_cast<std::size_t>(r) * static_cast<std::size_t>(size) +
                       static_cast<std::size_t>(q)] = (sample / 255.0F - mean[c]) / stddev[c];
            }
        }
    }
    return 0;
}

} // extern "C"

// tests/test_utils.hpp:233-263: DataGenerator. A fresh distribution object per
// fill call, so libstdc++'s normal_distribution drops its cached second value
// between calls exactly as the reference's does.
struct oracle_generator {
    std::mt19937_64 engine;
};

extern "C" {

oracle_generator* oracle_generator_create(uint64_t seed) {
    auto* g = new oracle_generator();
    g->engine.seed(seed);
    return g;
}

void oracle_generator_uniform(oracle_generator* g, float* data, int64_t count, float low,
                              float high) {
    std::uniform_real_distribution<float> distribution(low, high);
    for (int64_t i = 0; i < count; ++i) {
        data[i] = distribution(g->engine);
    }
}

void oracle_generator_normal(oracle_generator* g, float* data, int64_t count, float mean,
                             float stddev) {
    std::normal_distribution<float> distribution(mean, stddev);
    for (int64_t i = 0; i < count; ++i) {
        data[i] = distribution(g->engine);
    }
}

void oracle_generator_integers(oracle_generator* g, int64_t* data, int64_t count, int64_t low,
                               int64_t high) {
    std::uniform_int_distribution<int64_t> distribution(low, high);
    for (int64_t i = 0; i < count; ++i) {
        data[i] = distribution(g->engine);
    }
}

uint64_t oracle_generator_raw(oracle_generator* g) { return g->engine(); }

void oracle_generator_destroy(oracle_generator* g) { delete g; }

} // extern "C"
