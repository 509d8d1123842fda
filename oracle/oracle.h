/*
 * CPU oracle for the layer-kernel path. TEST INFRASTRUCTURE ONLY: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline compare the HIP library
 * against it. It is never linked into, or called by, the product.
 *
 * Every function restates the reference's CPU path in plain loops
 * (tests/reference/linear_algebra.hpp, tests/reference/vit.hpp,
 * tests/test_utils.hpp), or, where the reference defines a behaviour only on
 * the GPU side (batched GEMM addressing, the epilogue order, the batched patch
 * gather), the plain-loop form of that behaviour. Each definition in oracle.cpp
 * cites the reference lines it follows and names what pins it.
 *
 * Built with -O2 -ffp-contract=off and no fast-math, so float expressions round
 * exactly as written, like the reference's own loops.
 */
#ifndef CUVIT_ORACLE_H
#define CUVIT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same layout as cuvit_gemm_problem in include/cuvit/capi.h. */
typedef struct oracle_gemm_problem {
    int m, n, k;
    int32_t layout; /* 0 = B is [K, N], 1 = B is [N, K] */
    float alpha;
    int lda, ldb, ldc;
    int count;
    int64_t stride_a, stride_b, stride_c;
    int inner;
    int64_t outer_stride_a, outer_stride_b, outer_stride_c;
    uint8_t accumulate, gelu;
} oracle_gemm_problem;

typedef struct oracle_vit_config {
    int image_size, patch_size, channels, embed_dim, depth, heads, mlp_hidden, classes;
    float layer_norm_epsilon;
} oracle_vit_config;

void oracle_layer_norm(const float* input, const float* gamma, const float* beta, float* output,
                       int rows, int columns, float epsilon);
void oracle_softmax(const float* input, float* output, int rows, int columns);
float oracle_gelu_scalar(float value);
void oracle_gelu(const float* input, float* output, int64_t count);
void oracle_gemm(const float* a, const float* b, const float* bias, float* c, int m, int n, int k,
                 float alpha);
void oracle_gemm_transposed(const float* a, const float* b, const float* bias, float* c, int m,
                            int n, int k, float alpha);
void oracle_gemm_term_magnitudes(const float* a, const float* b, float* scale, int m, int n, int k,
                                 int transposed, float alpha);
/* Full GemmProblem semantics: batch addressing, leading dimensions, epilogue. */
void oracle_gemm_problem_run(const float* a, const float* b, const float* bias, float* c,
                             const oracle_gemm_problem* problem);
void oracle_extract_patches(const float* images, float* patches, int batch, int channels,
                            int height, int width, int patch);
void oracle_add(float* accumulator, const float* addend, int64_t count);
void oracle_add_broadcast(float* accumulator, const float* addend, int64_t count, int batch);
void oracle_broadcast(float* destination, const float* source, int64_t count,
                      int64_t destination_stride, int batch);
/* Whole single-image forward pass. @p tensors are host pointers in the order of
 * VisionTransformer::expected_tensor_names. */
void oracle_vit_forward(const oracle_vit_config* config, const float* const* tensors,
                        const float* image, float* logits);
/* The bf16 model's forward (an extension): oracle_vit_forward with every
 * stored activation and each GEMM weight matrix rounded to bf16 where the
 * model stores it; logits are the rounded values widened to float. */
void oracle_vit_forward_bf16(const oracle_vit_config* config, const float* const* tensors,
                             const float* image, float* logits);
/* Round to bfloat16 bits, nearest-even (NaN kept quiet). */
void oracle_round_bf16(const float* input, uint16_t* output, int64_t count);

/* preprocess(image, settings) of src/runtime/image.cpp:95-135 for one
 * interleaved RGB image: the [3, size, size] tensor. Returns 0, or the first
 * failed check in the reference's order: 1 empty image, 2 size, 3 crop
 * fraction, 4 zero stddev (then @p tensor is untouched). */
int oracle_preprocess(const uint8_t* pixels, int width, int height, int size, float crop_fraction,
                      const float* mean, const float* stddev, float* tensor);

/* The reference tests' seeded DataGenerator (std::mt19937_64 with libstdc++'s
 * distributions, a fresh distribution object per fill call). */
typedef struct oracle_generator oracle_generator;
oracle_generator* oracle_generator_create(uint64_t seed);
void oracle_generator_uniform(oracle_generator* g, float* data, int64_t count, float low,
                              float high);
void oracle_generator_normal(oracle_generator* g, float* data, int64_t count, float mean,
                             float stddev);
void oracle_generator_integers(oracle_generator* g, int64_t* data, int64_t count, int64_t low,
                               int64_t high);
uint64_t oracle_generator_raw(oracle_generator* g);
void oracle_generator_destroy(oracle_generator* g);

#ifdef __cplusplus
}
#endif

#endif /* CUVIT_ORACLE_H */
