/*
 * C ABI of the MI355X (gfx950) layer-kernel library, libcuvit_amd.so.
 *
 * Every entry point is `extern "C"`, takes plain device pointers and sizes, and
 * returns a cuvit_status. None of them throws, synchronizes or allocates device
 * memory (the model entry points excepted, as noted). The C++ launchers in
 * cuvit/kernels.hpp sit on top of these and turn a status back into the
 * exception the reference's launcher throws.
 *
 * Validation order is the reference's (src/kernels/normalization.cu:224-350,
 * src/kernels/gemm.cu:199-231):
 *   1. a zero extent returns CUVIT_OK before anything else, null pointers included;
 *   2. a negative extent            -> CUVIT_ERROR_INVALID_ARGUMENT;
 *   3. a null operand               -> CUVIT_ERROR_INVALID_ARGUMENT;
 *   4. shape-specific checks        -> CUVIT_ERROR_INVALID_ARGUMENT;
 *   5. a grid beyond 2^31-1 blocks  -> CUVIT_ERROR_LENGTH;
 *   6. a failed launch              -> CUVIT_ERROR_HIP (cuvit_last_hip_error()).
 * Steps 1-5 run before any HIP call, so they behave the same without a GPU.
 *
 * The message of the last failure on the calling thread is cuvit_last_error().
 */
#ifndef CUVIT_CAPI_H
#define CUVIT_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The same type as hipStream_t; NULL is the default stream. */
typedef struct ihipStream_t* cuvit_stream_t;

/* bfloat16 storage: the upper 16 bits of an IEEE float, round-to-nearest-even. */
typedef uint16_t cuvit_bf16;

typedef enum cuvit_status {
    CUVIT_OK = 0,
    CUVIT_ERROR_INVALID_ARGUMENT = 1, /* std::invalid_argument in the reference */
    CUVIT_ERROR_LENGTH = 2,           /* std::length_error */
    CUVIT_ERROR_HIP = 3,              /* CudaError (cuda_check.hpp:11-31) */
    CUVIT_ERROR_RUNTIME = 4,          /* std::runtime_error (weight files, arena) */
    CUVIT_ERROR_OUT_OF_RANGE = 5      /* std::out_of_range */
} cuvit_status;

/* Message describing the last failure on this thread ("" when none). */
const char* cuvit_last_error(void);
/* hipError_t of the last CUVIT_ERROR_HIP on this thread (0 when none). */
int cuvit_last_hip_error(void);
/* Library version, major * 10000 + minor * 100 + patch. */
int cuvit_version(void);

/* ---------------------------------------------------------------------------
 * GEMM problem description. Field for field the layout of cuvit::GemmProblem
 * (include/cuvit/kernels.hpp:30-85 of the reference); the C++ side
 * static_asserts that the two agree.
 * ------------------------------------------------------------------------- */
typedef enum cuvit_gemm_layout {
    CUVIT_GEMM_NO_TRANSPOSE = 0, /* B is [K, N] */
    CUVIT_GEMM_TRANSPOSED = 1    /* B is [N, K] */
} cuvit_gemm_layout;

typedef struct cuvit_gemm_batch {
    int count;
    int64_t stride_a;
    int64_t stride_b;
    int64_t stride_c;
    int inner;
    int64_t outer_stride_a;
    int64_t outer_stride_b;
    int64_t outer_stride_c;
} cuvit_gemm_batch;

typedef struct cuvit_gemm_epilogue {
    uint8_t accumulate; /* C += value instead of C = value */
    uint8_t gelu;       /* erf GELU after the bias */
} cuvit_gemm_epilogue;

typedef struct cuvit_gemm_problem {
    int m;
    int n;
    int k;
    int32_t layout; /* cuvit_gemm_layout */
    float alpha;
    int lda;
    int ldb;
    int ldc;
    cuvit_gemm_batch batch;
    cuvit_gemm_epilogue epilogue;
} cuvit_gemm_problem;

/* Fills *problem like the reference's gemm_problem() (kernels.hpp:89-96):
 * one un-batched problem, packed operands, alpha 1, no epilogue. */
void cuvit_gemm_problem_init(cuvit_gemm_problem* problem, int m, int n, int k, int layout);

/* ---------------------------------------------------------------------------
 * fp32 launchers: one per launcher of the reference's kernels.hpp.
 * ------------------------------------------------------------------------- */

/* Replaces cuvit::launch_gemm (kernels.hpp:98-99; gemm.cu:199-242).
 * C[i][m][n] = epilogue(alpha * sum_k A[i][m][k] * B_layout[i][k][n] + bias[n]).
 * The epilogue order is alpha, then bias, then GELU, then accumulate. */
int cuvit_gemm_f32(const float* a, const float* b, const float* bias, float* c,
                   const cuvit_gemm_problem* problem, cuvit_stream_t stream);

/* Replaces cuvit::launch_layer_norm (kernels.hpp:107-109; normalization.cu:224-239). */
int cuvit_layer_norm_f32(const float* input, const float* gamma, const float* beta, float* output,
                         int rows, int columns, float epsilon, cuvit_stream_t stream);

/* Replaces cuvit::launch_gelu (kernels.hpp:117-118; normalization.cu:257-271). */
int cuvit_gelu_f32(const float* input, float* output, int64_t count, cuvit_stream_t stream);

/* Replaces cuvit::launch_softmax (kernels.hpp:122-123; normalization.cu:241-255).
 * input == output (in place) is allowed, as the model uses it (vit.cu:225). */
int cuvit_softmax_f32(const float* input, float* output, int rows, int columns,
                      cuvit_stream_t stream);

/* Replaces cuvit::launch_extract_patches (kernels.hpp:137-138; normalization.cu:273-298). */
int cuvit_extract_patches_f32(const float* images, float* patches, int batch, int channels,
                              int height, int width, int patch, cuvit_stream_t stream);

/* Replaces cuvit::launch_add (kernels.hpp:141-142; normalization.cu:300-314). */
int cuvit_add_f32(float* accumulator, const float* addend, int64_t count, cuvit_stream_t stream);

/* Replaces cuvit::launch_add_broadcast (kernels.hpp:147-148; normalization.cu:316-332). */
int cuvit_add_broadcast_f32(float* accumulator, const float* addend, int64_t count, int batch,
                            cuvit_stream_t stream);

/* Replaces cuvit::launch_broadcast (kernels.hpp:153-154; normalization.cu:334-350). */
int cuvit_broadcast_f32(float* destination, const float* source, int64_t count,
                        int64_t destination_stride, int batch, cuvit_stream_t stream);

/* Fused attention. An extension with no single reference counterpart: it
 * replaces the three launches of the reference's attention (vit.cu:205-245:
 * the Q.K^T GEMM with alpha 1/sqrt(head_dim), launch_softmax in place, the
 * weights.V GEMM) and returns bitwise the same context as that sequence run
 * through this library, without writing the [images, heads, tokens, tokens]
 * logits. qkv is [images, tokens, 3, heads, head_dim] (the QKV projection),
 * context is [images, tokens, heads, head_dim]; both 16-byte aligned.
 * Supports head_dim 64 and up to 256 tokens; other shapes are
 * CUVIT_ERROR_INVALID_ARGUMENT (cuvit_attention_supported tells first).
 * More than 65535 (image, head) pairs, or one image's qkv rows past
 * 0x7FFFFFF0 bytes (the kernels' 32-bit offsets), are CUVIT_ERROR_LENGTH. */
int cuvit_attention_supported(int tokens, int head_dim);
int cuvit_attention_f32(const float* qkv, float* context, int images, int heads, int tokens,
                        int head_dim, cuvit_stream_t stream);
/* The bf16 twin: the same three launches through the bf16 twins (logits and
 * probabilities rounded to bf16 where those launches store them), bitwise. */
int cuvit_attention_bf16(const cuvit_bf16* qkv, cuvit_bf16* context, int images, int heads,
                         int tokens, int head_dim, cuvit_stream_t stream);

/* ---------------------------------------------------------------------------
 * bfloat16 I/O twins. An extension: the reference has no reduced-precision
 * path (README.md:472-473). Storage is bf16, every reduction and every
 * intermediate is fp32, gamma/beta/bias stay fp32, and each result is rounded
 * to bf16 once, to nearest-even. Validation is the fp32 twin's.
 * ------------------------------------------------------------------------- */
int cuvit_layer_norm_bf16(const cuvit_bf16* input, const float* gamma, const float* beta,
                          cuvit_bf16* output, int rows, int columns, float epsilon,
                          cuvit_stream_t stream);
int cuvit_softmax_bf16(const cuvit_bf16* input, cuvit_bf16* output, int rows, int columns,
                       cuvit_stream_t stream);
int cuvit_gelu_bf16(const cuvit_bf16* input, cuvit_bf16* output, int64_t count,
                    cuvit_stream_t stream);
int cuvit_extract_patches_bf16(const cuvit_bf16* images, cuvit_bf16* patches, int batch,
                               int channels, int height, int width, int patch,
                               cuvit_stream_t stream);
/* bf16 A and B, fp32 bias and accumulation, bf16 C. With accumulate, the
 * existing bf16 C is widened, added in fp32 and rounded once. */
int cuvit_gemm_bf16(const cuvit_bf16* a, const cuvit_bf16* b, const float* bias, cuvit_bf16* c,
                    const cuvit_gemm_problem* problem, cuvit_stream_t stream);
/* broadcast's bf16 twin: a bit copy of count values into batch slots. */
int cuvit_broadcast_bf16(cuvit_bf16* destination, const cuvit_bf16* source, int64_t count,
                         int64_t destination_stride, int batch, cuvit_stream_t stream);
/* Storage conversion, no counterpart in the reference: fp32 -> bf16 rounds to
 * nearest-even (NaN stays NaN), bf16 -> fp32 is exact. in == out is not
 * allowed. Validation is gelu's. */
int cuvit_convert_f32_to_bf16(const float* input, cuvit_bf16* output, int64_t count,
                              cuvit_stream_t stream);
int cuvit_convert_bf16_to_f32(const cuvit_bf16* input, float* output, int64_t count,
                              cuvit_stream_t stream);
/* fp32 images gathered into bf16 patch rows in one pass, no counterpart in the
 * reference: bitwise cuvit_convert_f32_to_bf16 of the images followed by
 * cuvit_extract_patches_bf16, without the bf16 image copy in between (the
 * bf16 model's image intake). Any alignment and geometry; validation is
 * extract_patches'. */
int cuvit_extract_patches_f32_to_bf16(const float* images, cuvit_bf16* patches, int batch,
                                      int channels, int height, int width, int patch,
                                      cuvit_stream_t stream);

/* ---------------------------------------------------------------------------
 * Weight files: the reference's .cvw v1 format (weights.hpp:16-92,
 * weights.cpp:13-23), little-endian: header {magic "CVIT", version 1, count,
 * reserved}; entries {name_len u32, name, type u32 (1 = float32), rank u32,
 * extents i64[rank], offset u64, bytes u64}; payloads 64-byte aligned.
 * Version 2 (an extension) is the same layout plus type 2 = bfloat16; the
 * writer emits it only for a file holding a bf16 tensor.
 * ------------------------------------------------------------------------- */
typedef struct cuvit_weight_writer cuvit_weight_writer;
typedef struct cuvit_weight_file cuvit_weight_file;

/* WeightFileWriter (weights.hpp:78-92). */
int cuvit_weight_writer_create(cuvit_weight_writer** writer);
int cuvit_weight_writer_add(cuvit_weight_writer* writer, const char* name, int rank,
                            const int64_t* extents, const float* data);
/* A bfloat16 tensor (bit patterns); the file becomes version 2. Extension. */
int cuvit_weight_writer_add_bf16(cuvit_weight_writer* writer, const char* name, int rank,
                                 const int64_t* extents, const cuvit_bf16* data);
int cuvit_weight_writer_write(const cuvit_weight_writer* writer, const char* path);
void cuvit_weight_writer_destroy(cuvit_weight_writer* writer);

/* WeightFile (weights.hpp:45-74). */
int cuvit_weight_file_load(const char* path, cuvit_weight_file** file);
int64_t cuvit_weight_file_size(const cuvit_weight_file* file);
int cuvit_weight_file_contains(const cuvit_weight_file* file, const char* name);
/* Host pointer to a float32 payload after checking its shape, as float_data(). */
int cuvit_weight_file_float_data(const cuvit_weight_file* file, const char* name, int rank,
                                 const int64_t* extents, const float** data);
/* Host pointer to a bfloat16 payload after checking its type and shape. Extension. */
int cuvit_weight_file_bf16_data(const cuvit_weight_file* file, const char* name, int rank,
                                const int64_t* extents, const cuvit_bf16** data);
/* The file's format version (1 or 2), 0 for a null file. */
int cuvit_weight_file_version(const cuvit_weight_file* file);
/* Data type of tensor @p name (1 float32, 2 bfloat16), 0 when absent. */
int cuvit_weight_file_type(const cuvit_weight_file* file, const char* name);
/* Name of entry @p index; NULL when out of range. Valid while the file lives. */
const char* cuvit_weight_file_entry_name(const cuvit_weight_file* file, int64_t index);
uint64_t cuvit_weight_file_payload_bytes(const cuvit_weight_file* file);
void cuvit_weight_file_destroy(cuvit_weight_file* file);

/* ---------------------------------------------------------------------------
 * The model driver: VisionTransformer (vit.hpp:15-120, vit.cu:36-344).
 * Creation allocates device memory (weights and activations, sized for
 * max_batch); a forward pass allocates nothing.
 * ------------------------------------------------------------------------- */
typedef struct cuvit_vit_config {
    int image_size;
    int patch_size;
    int channels;
    int embed_dim;
    int depth;
    int heads;
    int mlp_hidden;
    int classes;
    float layer_norm_epsilon;
} cuvit_vit_config;

typedef struct cuvit_vit cuvit_vit;

/* ViT-Tiny/16 at 224x224, the defaults of VitConfig (vit.hpp:15-24). */
void cuvit_vit_config_default(cuvit_vit_config* config);
/* VitConfig::validate (vit.cu:36-47). */
int cuvit_vit_config_validate(const cuvit_vit_config* config);
/* VisionTransformer(config, file, max_batch) (vit.cu:69-171). */
int cuvit_vit_create(const cuvit_vit_config* config, const cuvit_weight_file* file, int max_batch,
                     cuvit_vit** model);
/* Storage precision of a model (an extension; the reference is fp32 only). */
typedef enum cuvit_precision {
    CUVIT_PRECISION_F32 = 0,
    /* bf16 GEMM weights and activations; LayerNorm gamma/beta, biases and the
     * positional embedding stay fp32; fp32 reductions; images and logits fp32. */
    CUVIT_PRECISION_BF16 = 1
} cuvit_precision;
/* cuvit_vit_create with a storage precision (a cuvit_precision value). */
int cuvit_vit_create_ex(const cuvit_vit_config* config, const cuvit_weight_file* file,
                        int max_batch, int precision, cuvit_vit** model);
/* The model's cuvit_precision, or -1 for a null model. */
int cuvit_vit_precision(const cuvit_vit* model);
/* VisionTransformer::forward(images, logits, batch, stream) (vit.cu:263-317). */
int cuvit_vit_forward(cuvit_vit* model, const float* images, float* logits, int batch,
                      cuvit_stream_t stream);
uint64_t cuvit_vit_weight_bytes(const cuvit_vit* model);
uint64_t cuvit_vit_activation_bytes(const cuvit_vit* model);
void cuvit_vit_destroy(cuvit_vit* model);

/* ---------------------------------------------------------------------------
 * Images (include/cuvit/image.hpp:10-52, src/runtime/image.cpp:57-135): binary
 * PPM loading on the host and preprocessing on the device.
 * ------------------------------------------------------------------------- */
typedef struct cuvit_image cuvit_image;

/* load_ppm(path) (image.cpp:57-93): a P6 file with maximum 255. Failures are
 * CUVIT_ERROR_RUNTIME with the reference's messages. */
int cuvit_image_load_ppm(const char* path, cuvit_image** image);
/* Extents of a loaded image (0 for a null image). */
int cuvit_image_width(const cuvit_image* image);
int cuvit_image_height(const cuvit_image* image);
/* width * height * 3 interleaved RGB bytes; valid while the image lives. */
const uint8_t* cuvit_image_pixels(const cuvit_image* image);
void cuvit_image_destroy(cuvit_image* image);

/* Preprocessing (image.hpp:30-38). */
typedef struct cuvit_preprocessing {
    int size;
    float crop_fraction;
    float mean[3];
    float stddev[3];
} cuvit_preprocessing;

/* Preprocessing{}: size 224, crop fraction 0.9, mean and stddev 0.5. */
void cuvit_preprocessing_default(cuvit_preprocessing* settings);

/* preprocess(image, settings) (image.cpp:95-135) on the device for @p batch
 * images of one size: pixels [batch, height, width, 3] uint8, tensor
 * [batch, 3, size, size] float, bit-identical to the reference's host loop.
 * Validation: batch 0 returns at once; then a negative batch, a null settings
 * pointer, the reference's four checks in its order (empty image, size,
 * crop fraction, zero stddev), null operands (all CUVIT_ERROR_INVALID_ARGUMENT),
 * a size above 32768 and images whose bytes overflow int64 (CUVIT_ERROR_LENGTH).
 * The batch is an extension. */
int cuvit_preprocess_u8(const uint8_t* pixels, int batch, int width, int height,
                        const cuvit_preprocessing* settings, float* tensor,
                        cuvit_stream_t stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* CUVIT_CAPI_H */
