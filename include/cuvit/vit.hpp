#pragma once

// The model driver: the counterpart of the reference's include/cuvit/vit.hpp
// (VitConfig 15-35, BlockWeights 38-51, VisionTransformer 53-120) and
// src/model/vit.cu. It sequences the layer kernels of cuvit/kernels.hpp over
// activations carved once from a DeviceArena, so a forward pass allocates
// nothing and queues every launch on one stream.

#include "cuvit/device_arena.hpp"
#include "cuvit/device_buffer.hpp"
#include "cuvit/stream.hpp"
#include "cuvit/tensor.hpp"
#include "cuvit/weights.hpp"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <string>
#include <vector>

namespace cuvit {

/// Storage precision of a model. kBFloat16 is an extension (the reference is
/// fp32 only, README.md:472-473): the GEMM weight matrices and every
/// activation are bf16, while LayerNorm's gamma and beta, the biases and the
/// positional embedding stay fp32, every reduction and epilogue runs in fp32,
/// and each stored value is rounded once, to nearest-even. Images in and
/// logits out stay fp32 either way.
enum class Precision { kFloat32, kBFloat16 };

/// Shape of a Vision Transformer; the defaults are ViT-Tiny/16 at 224x224.
struct VitConfig {
    int image_size = 224;
    int patch_size = 16;
    int channels = 3;
    int embed_dim = 192;
    int depth = 12;
    int heads = 3;
    int mlp_hidden = 768;
    int classes = 1000;
    float layer_norm_epsilon = 1.0e-6F;

    [[nodiscard]] int patches_per_side() const { return image_size / patch_size; }
    [[nodiscard]] int patch_count() const { return patches_per_side() * patches_per_side(); }
    /// Patches plus the class token.
    [[nodiscard]] int token_count() const { return patch_count() + 1; }
    [[nodiscard]] int head_dim() const { return embed_dim / heads; }
    [[nodiscard]] int patch_elements() const { return channels * patch_size * patch_size; }

    /// Throws std::invalid_argument when the shape cannot describe a model.
    void validate() const;
};

struct BlockWeights {
    const float* norm1_gamma = nullptr;
    const float* norm1_beta = nullptr;
    const float* qkv_weight = nullptr;
    const float* qkv_bias = nullptr;
    const float* proj_weight = nullptr;
    const float* proj_bias = nullptr;
    const float* norm2_gamma = nullptr;
    const float* norm2_beta = nullptr;
    const float* fc1_weight = nullptr;
    const float* fc1_bias = nullptr;
    const float* fc2_weight = nullptr;
    const float* fc2_bias = nullptr;
};

class VisionTransformer final {
  public:
    /// Uploads @p file (shape-checked against @p config, timm names) and
    /// reserves activations for @p max_batch images. With kBFloat16 the GEMM
    /// weights are rounded to bf16 as they are staged.
    VisionTransformer(const VitConfig& config, const WeightFile& file, int max_batch = 1,
                      Precision precision = Precision::kFloat32);

    /// @p batch planar images in device memory -> batch x classes logits in
    /// device memory, queued on @p stream.
    void forward(const float* images, float* logits, int batch, hipStream_t stream = nullptr);

    /// Host-memory convenience form; synchronizes before returning.
    [[nodiscard]] std::vector<float> forward(const std::vector<float>& images);

    [[nodiscard]] const VitConfig& config() const noexcept { return config_; }
    [[nodiscard]] int max_batch() const noexcept { return max_batch_; }
    [[nodiscard]] Precision precision() const noexcept { return precision_; }
    [[nodiscard]] std::size_t image_elements() const noexcept;
    [[nodiscard]] std::size_t weight_bytes() const noexcept { return weights_.used(); }
    [[nodiscard]] std::size_t activation_bytes() const noexcept { return activations_.used(); }

    /// The timm tensor names this configuration expects, in load order.
    [[nodiscard]] static std::vector<std::string> expected_tensor_names(const VitConfig& config);

  private:
    /// What depends on the storage type T (float or bf16 bits): the GEMM
    /// weight matrices, the class row cls + pos[0] and the activations.
    template <typename T> struct Stored {
        struct Matrices {
            const T* qkv = nullptr;
            const T* proj = nullptr;
            const T* fc1 = nullptr;
            const T* fc2 = nullptr;
        };
        const T* patch_weight = nullptr;
        const T* head_weight = nullptr;
        const T* class_position = nullptr; // cls + pos[0]
        std::vector<Matrices> blocks;

        T* images = nullptr; // the input in storage precision (bf16 only)
        T* patches = nullptr;
        T* tokens = nullptr;
        T* normalized = nullptr;
        T* qkv = nullptr;
        T* attention = nullptr;
        T* context = nullptr;
        T* hidden = nullptr;
        T* logits = nullptr; // the head's output before widening (bf16 only)
    };

    /// Throws std::invalid_argument unless 0 <= @p batch <= max_batch().
    void check_batch(long long batch) const;
    template <typename T> void load(const WeightFile& file, Stored<T>& stored);
    template <typename T> void reserve_activations(Stored<T>& stored);
    template <typename T>
    void forward_stored(Stored<T>& stored, const float* images, float* logits, int batch,
                        hipStream_t stream);
    template <typename T>
    void run_block(const BlockWeights& block, const typename Stored<T>::Matrices& matrices,
                   Stored<T>& stored, int batch, hipStream_t stream);
    /// The reference's three attention launches (vit.cu:205-245), used when
    /// the fused kernel does not cover the shape or the precision.
    template <typename T> void attention_unfused(Stored<T>& stored, int batch, hipStream_t stream);

    VitConfig config_;
    int max_batch_ = 1;
    Precision precision_ = Precision::kFloat32;
    bool fused_attention_ = false;

    DeviceArena weights_;
    DeviceArena activations_;

    const float* class_token_ = nullptr;
    const float* position_embedding_ = nullptr;
    const float* patch_weight_ = nullptr; // fp32 models only
    const float* patch_bias_ = nullptr;
    const float* final_gamma_ = nullptr;
    const float* final_beta_ = nullptr;
    const float* head_weight_ = nullptr; // fp32 models only
    const float* head_bias_ = nullptr;
    /// fp32 parameters of each block; the GEMM matrices are set for fp32
    /// models only (bf16 models keep theirs in bf16_.blocks).
    std::vector<BlockWeights> blocks_;

    Stored<float> f32_;
    Stored<std::uint16_t> bf16_;
};

} // namespace cuvit
