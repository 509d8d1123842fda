// VisionTransformer: the launch sequence of the reference's forward pass
// (src/model/vit.cu:173-317) over arena-carved activations.
//
// Per block (run_block, vit.cu:173-261): LN1 -> QKV GEMM -> attention -> proj
// GEMM accumulating into the residual stream -> LN2 -> FC1 GEMM with the GELU
// epilogue -> FC2 GEMM accumulating into the residual stream. Attention is
// the reference's Q.K^T GEMM (alpha 1/sqrt(head_dim), split batch over
// (image, head)) -> softmax in place -> attention.V GEMM written straight into
// [tokens, heads * head_dim]; where the shape allows it runs as one fused
// launch with bitwise the same result and no logits buffer.
// Around the blocks (forward, vit.cu:263-317): patch gather -> embedding GEMM
// into rows 1.. of each image -> class token into row 0 -> positional add ->
// blocks -> final LN -> head GEMM on the class rows only. Here the positional
// add rides in the embedding GEMM's epilogue and row 0 is one broadcast of
// cls + pos[0], with the same bits as the separate launches. The model's
// LayerNorms store their rows with plain (cached) stores, since a GEMM reads
// them next; the C ABI's LayerNorm stores non-temporally. Same values.
#include "cuvit/vit.hpp"

#include "cuvit/capi.h"
#include "cuvit/device_arena.hpp"
#include "cuvit/hip_check.hpp"
#include "cuvit/host_buffer.hpp"
#include "cuvit/kernels.hpp"
#include "cuvit/stream.hpp"

#include "../capi/status.hpp"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <iterator>
#include <string>
#include <type_traits>
#include <utility>

namespace cuvit {
namespace {

std::string block_prefix(int index) { return "blocks." + std::to_string(index) + '.'; }

Extent element_count(const std::vector<Extent>& extents) {
    Extent count = 1;
    for (const Extent e : extents) {
        count *= e;
    }
    return count;
}

/// bf16 bits of @p value, rounded to nearest with ties to even; a NaN stays a
/// quiet NaN. The rounding of the kernels' stores (v_cvt_pk_bf16_f32).
std::uint16_t round_to_bf16(float value) {
    std::uint32_t bits = 0;
    std::memcpy(&bits, &value, sizeof(bits));
    if ((bits & 0x7F800000U) == 0x7F800000U && (bits & 0x007FFFFFU) != 0) {
        return static_cast<std::uint16_t>((bits >> 16) | 0x0040U);
    }
    bits += 0x7FFFU + ((bits >> 16) & 1U);
    return static_cast<std::uint16_t>(bits >> 16);
}

/// Weights on their way to the device: each tensor is carved from the device
/// arena and copied (shape-checked) into a pinned host mirror of the arena,
/// and one asynchronous copy then moves the whole arena. The reference issues
/// one synchronous cudaMemcpy per tensor (vit.cu:29-30).
class Staging {
  public:
    Staging(DeviceArena& arena, std::size_t bytes) : arena_(arena), host_(bytes) {}

    /// Carves @p count elements; returns the device pointer and the host mirror.
    template <typename T> std::pair<T*, T*> carve(std::size_t count) {
        T* const device = arena_.allocate_raw<T>(count);
        const auto offset = reinterpret_cast<const std::byte*>(device) - arena_.data();
        return {device, reinterpret_cast<T*>(host_.data() + offset)};
    }

    /// Stages tensor @p name (float32 or, from a version 2 file, bfloat16)
    /// in storage type T: copied when the types match, else widened exactly
    /// to fp32 or rounded to bf16 bits.
    template <typename T>
    const T* upload(const WeightFile& file, const std::string& name,
                    const std::vector<Extent>& extents) {
        const bool stored_bf16 = file.entry(name).type == DataType::kBFloat16;
        const auto count = static_cast<std::size_t>(element_count(extents));
        const auto [device, mirror] = carve<T>(count);
        if constexpr (std::is_same_v<T, float>) {
            if (stored_bf16) {
                const std::uint16_t* const source = file.bf16_data(name, extents);
                for (std::size_t i = 0; i < count; ++i) {
                    const std::uint32_t widened = static_cast<std::uint32_t>(source[i]) << 16;
                    std::memcpy(mirror + i, &widened, sizeof(float));
                }
            } else {
                std::memcpy(mirror, file.float_data(name, extents), count * sizeof(float));
            }
        } else {
            if (stored_bf16) {
                std::memcpy(mirror, file.bf16_data(name, extents), count * sizeof(std::uint16_t));
            } else {
                const float* const source = file.float_data(name, extents);
                for (std::size_t i = 0; i < count; ++i) {
                    mirror[i] = round_to_bf16(source[i]);
                }
            }
        }
        return device;
    }

    /// Copies everything carved so far to the device and waits for it.
    void finish() {
        Stream stream;
        CUVIT_HIP_CHECK(hipMemcpyAsync(const_cast<std::byte*>(arena_.data()), host_.data(), arena_.used(),
                                       hipMemcpyHostToDevice, stream.get()));
        stream.synchronize();
    }

  private:
    DeviceArena& arena_;
    HostBuffer<std::byte> host_;
};

// Launch overloads by storage type. fp32 and bf16 share the launchers of
// cuvit/kernels.hpp; the rest go through the C ABI.
void gemm_with_addend(const float* a, const float* b, const float* bias, const float* addend,
                      int ld_addend, float* c, const GemmProblem& problem, hipStream_t stream) {
    throw_on_error(capi::gemm_f32_with_addend(a, b, bias, addend, ld_addend, c,
                                              reinterpret_cast<const cuvit_gemm_problem*>(&problem),
                                              stream));
}

void gemm_with_addend(const std::uint16_t* a, const std::uint16_t* b, const float* bias,
                      const float* addend, int ld_addend, std::uint16_t* c,
                      const GemmProblem& problem, hipStream_t stream) {
    throw_on_error(capi::gemm_bf16_with_addend(a, b, bias, addend, ld_addend, c,
                                               reinterpret_cast<const cuvit_gemm_problem*>(&problem),
                                               stream));
}

cuvit_stream_t as_c(hipStream_t stream) { return reinterpret_cast<cuvit_stream_t>(stream); }

} // namespace

void VitConfig::validate() const {
    if (image_size <= 0 || patch_size <= 0 || channels <= 0 || embed_dim <= 0 || depth <= 0 ||
        heads <= 0 || mlp_hidden <= 0 || classes <= 0) {
        throw std::invalid_argument("Every ViT dimension must be positive");
    }
    if (image_size % patch_size != 0) {
        throw std::invalid_argument("The image size must divide into whole patches");
    }
    if (embed_dim % heads != 0) {
        throw std::invalid_argument("The embedding dimension must divide across the heads");
    }
}

std::vector<std::string> VisionTransformer::expected_tensor_names(const VitConfig& config) {
    std::vector<std::string> names = {"cls_token", "pos_embed", "patch_embed.proj.weight",
                                      "patch_embed.proj.bias"};
    static const char* const kBlockTensors[] = {
        "norm1.weight",     "norm1.bias",     "attn.qkv.weight", "attn.qkv.bias",
        "attn.proj.weight", "attn.proj.bias", "norm2.weight",    "norm2.bias",
        "mlp.fc1.weight",   "mlp.fc1.bias",   "mlp.fc2.weight",  "mlp.fc2.bias"};
    for (int block = 0; block < config.depth; ++block) {
        for (const char* suffix : kBlockTensors) {
            names.push_back(block_prefix(block) + suffix);
        }
    }
    for (const char* name : {"norm.weight", "norm.bias", "head.weight", "head.bias"}) {
        names.emplace_back(name);
    }
    return names;
}

std::size_t VisionTransformer::image_elements() const noexcept {
    return static_cast<std::size_t>(config_.channels) * config_.image_size * config_.image_size;
}

VisionTransformer::VisionTransformer(const VitConfig& config, const WeightFile& file, int max_batch,
                                     Precision precision)
    : config_(config), max_batch_(max_batch), precision_(precision) {
    config_.validate();
    if (max_batch_ < 1) {
        throw std::invalid_argument("The maximum batch size must be at least one");
    }
    if (precision_ != Precision::kFloat32 && precision_ != Precision::kBFloat16) {
        throw std::invalid_argument("Unknown model precision");
    }
    if (precision_ == Precision::kFloat32) {
        load(file, f32_);
        reserve_activations(f32_);
    } else {
        load(file, bf16_);
        reserve_activations(bf16_);
    }
}

template <typename T> void VisionTransformer::load(const WeightFile& file, Stored<T>& stored) {
    constexpr bool kFloat = std::is_same_v<T, float>;
    const Extent embed = config_.embed_dim;
    const Extent tokens = config_.token_count();
    const Extent hidden = config_.mlp_hidden;
    const Extent patch_elements = config_.patch_elements();
    const Extent classes = config_.classes;

    // The weight arena is sized from the configuration, not from the file, so
    // extra tensors in a file cost nothing. Vectors are fp32; the GEMM
    // matrices and the class row are in storage type T.
    std::size_t weight_bytes = 0;
    auto vector = [&](Extent count) {
        weight_bytes += DeviceArena::reserved_bytes<float>(static_cast<std::size_t>(count));
    };
    auto matrix = [&](Extent count) {
        weight_bytes += DeviceArena::reserved_bytes<T>(static_cast<std::size_t>(count));
    };
    vector(embed);          // cls
    vector(tokens * embed); // pos
    matrix(embed * patch_elements);
    vector(embed);
    for (int block = 0; block < config_.depth; ++block) {
        vector(embed);
        vector(embed);
        matrix(3 * embed * embed);
        vector(3 * embed);
        matrix(embed * embed);
        vector(embed);
        vector(embed);
        vector(embed);
        matrix(hidden * embed);
        vector(hidden);
        matrix(embed * hidden);
        vector(embed);
    }
    vector(embed);
    vector(embed);
    matrix(classes * embed);
    vector(classes);
    matrix(embed); // cls + pos[0]
    weights_.reserve(weight_bytes);

    Staging staging(weights_, weight_bytes);
    auto upload = [&](const std::string& name, const std::vector<Extent>& extents) {
        return staging.upload<float>(file, name, extents);
    };
    auto upload_matrix = [&](const std::string& name, const std::vector<Extent>& extents) {
        return staging.upload<T>(file, name, extents);
    };

    class_token_ = upload("cls_token", {1, 1, embed});
    position_embedding_ = upload("pos_embed", {1, tokens, embed});
    // The Conv2d weight [embed, C, P, P] is already the [embed, C*P*P] matrix
    // the embedding GEMM wants.
    stored.patch_weight = upload_matrix(
        "patch_embed.proj.weight", {embed, config_.channels, config_.patch_size, config_.patch_size});
    patch_bias_ = upload("patch_embed.proj.bias", {embed});

    blocks_.assign(static_cast<std::size_t>(config_.depth), BlockWeights{});
    stored.blocks.assign(static_cast<std::size_t>(config_.depth), typename Stored<T>::Matrices{});
    for (int index = 0; index < config_.depth; ++index) {
        const std::string p = block_prefix(index);
        BlockWeights& b = blocks_[static_cast<std::size_t>(index)];
        typename Stored<T>::Matrices& m = stored.blocks[static_cast<std::size_t>(index)];
        b.norm1_gamma = upload(p + "norm1.weight", {embed});
        b.norm1_beta = upload(p + "norm1.bias", {embed});
        m.qkv = upload_matrix(p + "attn.qkv.weight", {3 * embed, embed});
        b.qkv_bias = upload(p + "attn.qkv.bias", {3 * embed});
        m.proj = upload_matrix(p + "attn.proj.weight", {embed, embed});
        b.proj_bias = upload(p + "attn.proj.bias", {embed});
        b.norm2_gamma = upload(p + "norm2.weight", {embed});
        b.norm2_beta = upload(p + "norm2.bias", {embed});
        m.fc1 = upload_matrix(p + "mlp.fc1.weight", {hidden, embed});
        b.fc1_bias = upload(p + "mlp.fc1.bias", {hidden});
        m.fc2 = upload_matrix(p + "mlp.fc2.weight", {embed, hidden});
        b.fc2_bias = upload(p + "mlp.fc2.bias", {embed});
        if constexpr (kFloat) {
            b.qkv_weight = m.qkv;
            b.proj_weight = m.proj;
            b.fc1_weight = m.fc1;
            b.fc2_weight = m.fc2;
        }
    }

    final_gamma_ = upload("norm.weight", {embed});
    final_beta_ = upload("norm.bias", {embed});
    stored.head_weight = upload_matrix("head.weight", {classes, embed});
    head_bias_ = upload("head.bias", {classes});
    if constexpr (kFloat) {
        patch_weight_ = stored.patch_weight;
        head_weight_ = stored.head_weight;
    }

    // Token row 0 of every image is cls + pos[0]: one fp32 add per element,
    // the same rounding as the reference's broadcast-then-add (vit.cu:295-300),
    // then (bf16) one rounding to storage, as every other stored token.
    {
        const std::vector<float> cls = file.values("cls_token", {1, 1, embed});
        const std::vector<float> pos = file.values("pos_embed", {1, tokens, embed});
        const auto [device, mirror] = staging.carve<T>(static_cast<std::size_t>(embed));
        for (Extent i = 0; i < embed; ++i) {
            const float sum = cls[static_cast<std::size_t>(i)] + pos[static_cast<std::size_t>(i)];
            if constexpr (kFloat) {
                mirror[i] = sum;
            } else {
                mirror[i] = round_to_bf16(sum);
            }
        }
        stored.class_position = device;
    }
    staging.finish();
}

template <typename T> void VisionTransformer::reserve_activations(Stored<T>& stored) {
    constexpr bool kFloat = std::is_same_v<T, float>;
    // Attention runs fused (no logits buffer) whenever the shape allows: the
    // C ABI's limits on it (pairs, an image's bytes of the QKV projection).
    fused_attention_ = cuvit_attention_supported(config_.token_count(), config_.head_dim()) != 0 &&
                       static_cast<std::int64_t>(max_batch_) * config_.heads <= 65535 &&
                       static_cast<std::int64_t>(config_.token_count()) * 3 * config_.embed_dim *
                               static_cast<std::int64_t>(sizeof(T)) <= 0x7FFFFFF0;

    const Extent images = max_batch_;
    const Extent embed = config_.embed_dim;
    const Extent tokens = config_.token_count();
    const Extent hidden = config_.mlp_hidden;
    // Activation scratch for max_batch images, shared by every block.
    const Extent counts[] = {
        kFloat ? 0 : images * static_cast<Extent>(image_elements()),          // input in bf16
        images * config_.patch_count() * config_.patch_elements(),           // patch matrix
        images * tokens * embed,                                              // residual stream
        images * tokens * embed,                                              // normalized
        images * tokens * 3 * embed,                                          // packed q, k, v
        fused_attention_ ? 0 : images * config_.heads * tokens * tokens,      // attention logits
        images * tokens * embed,                                              // attention context
        images * tokens * hidden,                                             // MLP hidden
        kFloat ? 0 : images * config_.classes,                                // logits in bf16
    };
    std::size_t bytes = 0;
    for (const Extent count : counts) {
        bytes += DeviceArena::reserved_bytes<T>(static_cast<std::size_t>(count));
    }
    activations_.reserve(bytes);
    T** const slots[] = {&stored.images, &stored.patches,   &stored.tokens,
                         &stored.normalized, &stored.qkv,   &stored.attention,
                         &stored.context,    &stored.hidden, &stored.logits};
    static_assert(std::size(slots) == std::size(counts));
    for (std::size_t i = 0; i < std::size(slots); ++i) {
        *slots[i] = counts[i] == 0 ? nullptr
                                   : activations_.allocate_raw<T>(static_cast<std::size_t>(counts[i]));
    }
}

template <typename T>
void VisionTransformer::attention_unfused(Stored<T>& stored, int batch, hipStream_t stream) {
    const int token_count = config_.token_count();
    const int embed = config_.embed_dim;
    const int heads = config_.heads;
    const int head_dim = config_.head_dim();
    const std::int64_t tokens_per_image = static_cast<std::int64_t>(token_count) * embed;
    const std::int64_t qkv_per_image = tokens_per_image * 3;
    const std::int64_t logits_per_head = static_cast<std::int64_t>(token_count) * token_count;
    const int qkv_row = 3 * embed;

    // Q.K^T per (image, head), read in place from the packed projection.
    GemmProblem logits = gemm_problem(token_count, token_count, head_dim, GemmLayout::kTransposed);
    logits.alpha = 1.0F / std::sqrt(static_cast<float>(head_dim));
    logits.lda = qkv_row;
    logits.ldb = qkv_row;
    logits.ldc = token_count;
    logits.batch.count = batch * heads;
    logits.batch.inner = heads;
    logits.batch.stride_a = head_dim;
    logits.batch.stride_b = head_dim;
    logits.batch.stride_c = logits_per_head;
    logits.batch.outer_stride_a = qkv_per_image;
    logits.batch.outer_stride_b = qkv_per_image;
    logits.batch.outer_stride_c = heads * logits_per_head;
    launch_gemm(stored.qkv, stored.qkv + embed, nullptr, stored.attention, logits, stream);

    launch_softmax(stored.attention, stored.attention, batch * heads * token_count, token_count,
                   stream);

    // weights.V straight into the [tokens, heads * head_dim] context layout.
    GemmProblem context = gemm_problem(token_count, head_dim, token_count, GemmLayout::kNoTranspose);
    context.lda = token_count;
    context.ldb = qkv_row;
    context.ldc = embed;
    context.batch.count = batch * heads;
    context.batch.inner = heads;
    context.batch.stride_a = logits_per_head;
    context.batch.stride_b = head_dim;
    context.batch.stride_c = head_dim;
    context.batch.outer_stride_a = heads * logits_per_head;
    context.batch.outer_stride_b = qkv_per_image;
    context.batch.outer_stride_c = tokens_per_image;
    launch_gemm(stored.attention, stored.qkv + 2 * embed, nullptr, stored.context, context, stream);
}

template <typename T>
void VisionTransformer::run_block(const BlockWeights& block,
                                  const typename Stored<T>::Matrices& matrices, Stored<T>& stored,
                                  int batch, hipStream_t stream) {
    const int token_count = config_.token_count();
    const int embed = config_.embed_dim;
    const int heads = config_.heads;
    const int head_dim = config_.head_dim();
    const int hidden = config_.mlp_hidden;
    const int rows = batch * token_count;
    const int qkv_row = 3 * embed;
    T* const tokens = stored.tokens;

    throw_on_error(capi::layer_norm_cached(tokens, block.norm1_gamma, block.norm1_beta,
                                           stored.normalized, rows, embed,
                                           config_.layer_norm_epsilon, stream));

    // [tokens, 3, heads, head_dim] in one projection.
    launch_gemm(stored.normalized, matrices.qkv, block.qkv_bias, stored.qkv,
                gemm_problem(rows, qkv_row, embed, GemmLayout::kTransposed), stream);

    // softmax(Q.K^T / sqrt(head_dim)).V per (image, head) in one fused launch
    // when the shape allows; it is bitwise equal to the three launches.
    if (fused_attention_) {
        if constexpr (std::is_same_v<T, float>) {
            throw_on_error(cuvit_attention_f32(stored.qkv, stored.context, batch, heads, token_count,
                                               head_dim, as_c(stream)));
        } else {
            throw_on_error(cuvit_attention_bf16(stored.qkv, stored.context, batch, heads,
                                                token_count, head_dim, as_c(stream)));
        }
    } else {
        attention_unfused(stored, batch, stream);
    }

    GemmProblem projection = gemm_problem(rows, embed, embed, GemmLayout::kTransposed);
    projection.epilogue.accumulate = true;
    launch_gemm(stored.context, matrices.proj, block.proj_bias, tokens, projection, stream);

    throw_on_error(capi::layer_norm_cached(tokens, block.norm2_gamma, block.norm2_beta,
                                           stored.normalized, rows, embed,
                                           config_.layer_norm_epsilon, stream));

    GemmProblem fc1 = gemm_problem(rows, hidden, embed, GemmLayout::kTransposed);
    fc1.epilogue.gelu = true;
    launch_gemm(stored.normalized, matrices.fc1, block.fc1_bias, stored.hidden, fc1, stream);

    GemmProblem fc2 = gemm_problem(rows, embed, hidden, GemmLayout::kTransposed);
    fc2.epilogue.accumulate = true;
    launch_gemm(stored.hidden, matrices.fc2, block.fc2_bias, tokens, fc2, stream);
}

void VisionTransformer::check_batch(long long batch) const {
    if (batch < 0 || batch > max_batch_) {
        throw std::invalid_argument("This model was built for at most " + std::to_string(max_batch_) +
                                    " images, but " + std::to_string(batch) + " were given");
    }
}

void VisionTransformer::forward(const float* images, float* logits, int batch, hipStream_t stream) {
    if (batch == 0) {
        return;
    }
    check_batch(batch);
    if (images == nullptr || logits == nullptr) {
        throw std::invalid_argument("Forward pass operands cannot be null");
    }
    if (precision_ == Precision::kFloat32) {
        forward_stored(f32_, images, logits, batch, stream);
    } else {
        forward_stored(bf16_, images, logits, batch, stream);
    }
}

template <typename T>
void VisionTransformer::forward_stored(Stored<T>& stored, const float* images, float* logits,
                                       int batch, hipStream_t stream) {
    constexpr bool kFloat = std::is_same_v<T, float>;
    const int token_count = config_.token_count();
    const int patch_count = config_.patch_count();
    const int embed = config_.embed_dim;
    const std::int64_t tokens_per_image = static_cast<std::int64_t>(token_count) * embed;

    if constexpr (kFloat) {
        launch_extract_patches(images, stored.patches, batch, config_.channels, config_.image_size,
                               config_.image_size, config_.patch_size, stream);
    } else {
        // The conversion to bf16 and the gather in one pass where the layout
        // allows (the same bits: rounding does not depend on the position);
        // else the images are converted, then gathered.
        bool fused = false;
        throw_on_error(capi::extract_patches_f32_to_bf16(
            images, stored.patches, batch, config_.channels, config_.image_size,
            config_.image_size, config_.patch_size, stream, &fused));
        if (!fused) {
            throw_on_error(cuvit_convert_f32_to_bf16(images, stored.images,
                                                     static_cast<std::int64_t>(batch) * image_elements(),
                                                     as_c(stream)));
            launch_extract_patches(stored.images, stored.patches, batch, config_.channels,
                                   config_.image_size, config_.image_size, config_.patch_size,
                                   stream);
        }
    }

    // Patch embeddings land in rows 1.. of each image, with the positional
    // embedding of those rows added in the GEMM's epilogue after the bias:
    // (sum + bias) + pos, the order of the reference's embedding GEMM followed
    // by its positional add, so the same bits. Row 0 gets cls + pos[0].
    GemmProblem embedding =
        gemm_problem(patch_count, embed, config_.patch_elements(), GemmLayout::kTransposed);
    embedding.batch.count = batch;
    embedding.batch.stride_a = static_cast<std::int64_t>(patch_count) * config_.patch_elements();
    embedding.batch.stride_c = tokens_per_image;
    gemm_with_addend(stored.patches, stored.patch_weight, patch_bias_, position_embedding_ + embed,
                     embed, stored.tokens + embed, embedding, stream);
    launch_broadcast(stored.tokens, stored.class_position, embed, tokens_per_image, batch, stream);

    for (std::size_t index = 0; index < blocks_.size(); ++index) {
        run_block<T>(blocks_[index], stored.blocks[index], stored, batch, stream);
    }

    // Class-token pooling: only row 0 of each image feeds the head, so the
    // final LayerNorm normalizes those rows alone (tokens_per_image apart, into
    // [batch, embed]) and the head is one [batch, embed] x [classes, embed]^T
    // product. Each row is computed by the same operations as in the
    // reference's LayerNorm over every token followed by its batch of
    // one-row head GEMMs (vit.cu:305-316), so the logits are the same bits.
    throw_on_error(capi::layer_norm_cached(stored.tokens, final_gamma_, final_beta_,
                                           stored.normalized, batch, embed,
                                           config_.layer_norm_epsilon, stream, tokens_per_image));
    GemmProblem head = gemm_problem(batch, config_.classes, embed, GemmLayout::kTransposed);
    if constexpr (kFloat) {
        launch_gemm(stored.normalized, stored.head_weight, head_bias_, logits, head, stream);
    } else {
        launch_gemm(stored.normalized, stored.head_weight, head_bias_, stored.logits, head, stream);
        throw_on_error(cuvit_convert_bf16_to_f32(
            stored.logits, logits, static_cast<std::int64_t>(batch) * config_.classes, as_c(stream)));
    }
}

std::vector<float> VisionTransformer::forward(const std::vector<float>& images) {
    // Contract (vit.hpp:78-80 of the reference): host images in, host logits
    // out, synchronized; the batch is the number of whole images given.
    const std::size_t per_image = image_elements();
    if (per_image == 0 || images.size() % per_image != 0) {
        throw std::invalid_argument("The input holds " + std::to_string(images.size()) +
                                    " elements, which is not a whole number of " +
                                    std::to_string(per_image) + "-element images");
    }
    const auto batch = static_cast<long long>(images.size() / per_image);
    check_batch(batch);
    const std::size_t logit_count = static_cast<std::size_t>(batch) * config_.classes;
    std::vector<float> logits(logit_count);
    if (batch == 0) {
        return logits;
    }

    // Images and logits share one device block, each on its own 256-byte
    // granule; it is released when the call returns, after the stream drains.
    DeviceArena io(DeviceArena::reserved_bytes<float>(images.size()) +
                   DeviceArena::reserved_bytes<float>(logit_count));
    float* device_images = io.allocate_raw<float>(images.size());
    float* device_logits = io.allocate_raw<float>(logit_count);
    Stream stream;
    CUVIT_HIP_CHECK(hipMemcpyAsync(device_images, images.data(), images.size() * sizeof(float),
                                   hipMemcpyHostToDevice, stream.get()));
    forward(device_images, device_logits, static_cast<int>(batch), stream.get());
    CUVIT_HIP_CHECK(hipMemcpyAsync(logits.data(), device_logits, logit_count * sizeof(float),
                                   hipMemcpyDeviceToHost, stream.get()));
    stream.synchronize();
    return logits;
}

} // namespace cuvit
