// C ABI of the host-side classes: weight files (cuvit/weights.hpp), the
// model driver (cuvit/vit.hpp) and PPM images (cuvit/image.hpp). Exceptions
// become status codes here.
#include "cuvit/capi.h"
#include "cuvit/image.hpp"
#include "cuvit/vit.hpp"
#include "cuvit/weights.hpp"
#include "status.hpp"

#include <memory>
#include <string>
#include <vector>

struct cuvit_weight_writer {
    cuvit::WeightFileWriter writer;
};

struct cuvit_weight_file {
    cuvit::WeightFile file;
};

struct cuvit_image {
    cuvit::RgbImage image;
};

struct cuvit_vit {
    std::unique_ptr<cuvit::VisionTransformer> model;
};

namespace {

using cuvit::capi::fail;
using cuvit::capi::guarded;

std::vector<cuvit::Extent> extents_of(int rank, const int64_t* extents) {
    if (rank < 0 || (rank > 0 && extents == nullptr)) {
        throw std::invalid_argument("Tensor extents are missing");
    }
    return std::vector<cuvit::Extent>(extents, extents + rank);
}

cuvit::VitConfig to_config(const cuvit_vit_config& c) {
    cuvit::VitConfig config;
    config.image_size = c.image_size;
    config.patch_size = c.patch_size;
    config.channels = c.channels;
    config.embed_dim = c.embed_dim;
    config.depth = c.depth;
    config.heads = c.heads;
    config.mlp_hidden = c.mlp_hidden;
    config.classes = c.classes;
    config.layer_norm_epsilon = c.layer_norm_epsilon;
    return config;
}

} // namespace

extern "C" {

int cuvit_weight_writer_create(cuvit_weight_writer** writer) {
    return guarded([&]() -> int {
        if (writer == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "writer out-pointer cannot be null");
        }
        *writer = new cuvit_weight_writer();
        return CUVIT_OK;
    });
}

int cuvit_weight_writer_add(cuvit_weight_writer* writer, const char* name, int rank,
                            const int64_t* extents, const float* data) {
    return guarded([&]() -> int {
        if (writer == nullptr || name == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "writer and name cannot be null");
        }
        writer->writer.add(name, extents_of(rank, extents), data);
        return CUVIT_OK;
    });
}

int cuvit_weight_writer_add_bf16(cuvit_weight_writer* writer, const char* name, int rank,
                                 const int64_t* extents, const cuvit_bf16* data) {
    return guarded([&]() -> int {
        if (writer == nullptr || name == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "writer and name cannot be null");
        }
        writer->writer.add_bf16(name, extents_of(rank, extents), data);
        return CUVIT_OK;
    });
}

int cuvit_weight_writer_write(const cuvit_weight_writer* writer, const char* path) {
    return guarded([&]() -> int {
        if (writer == nullptr || path == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "writer and path cannot be null");
        }
        writer->writer.write(path);
        return CUVIT_OK;
    });
}

void cuvit_weight_writer_destroy(cuvit_weight_writer* writer) { delete writer; }

int cuvit_weight_file_load(const char* path, cuvit_weight_file** file) {
    return guarded([&]() -> int {
        if (path == nullptr || file == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "path and out-pointer cannot be null");
        }
        auto loaded = std::make_unique<cuvit_weight_file>();
        loaded->file = cuvit::WeightFile::load(path);
        *file = loaded.release();
        return CUVIT_OK;
    });
}

int64_t cuvit_weight_file_size(const cuvit_weight_file* file) {
    return file == nullptr ? 0 : static_cast<int64_t>(file->file.size());
}

int cuvit_weight_file_contains(const cuvit_weight_file* file, const char* name) {
    return file != nullptr && name != nullptr && file->file.contains(name) ? 1 : 0;
}

int cuvit_weight_file_float_data(const cuvit_weight_file* file, const char* name, int rank,
                                 const int64_t* extents, const float** data) {
    return guarded([&]() -> int {
        if (file == nullptr || name == nullptr || data == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "file, name and out-pointer cannot be null");
        }
        *data = file->file.float_data(name, extents_of(rank, extents));
        return CUVIT_OK;
    });
}

int cuvit_weight_file_bf16_data(const cuvit_weight_file* file, const char* name, int rank,
                                const int64_t* extents, const cuvit_bf16** data) {
    return guarded([&]() -> int {
        if (file == nullptr || name == nullptr || data == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "file, name and out-pointer cannot be null");
        }
        *data = file->file.bf16_data(name, extents_of(rank, extents));
        return CUVIT_OK;
    });
}

int cuvit_weight_file_version(const cuvit_weight_file* file) {
    return file == nullptr ? 0 : static_cast<int>(file->file.version());
}

int cuvit_weight_file_type(const cuvit_weight_file* file, const char* name) {
    if (file == nullptr || name == nullptr || !file->file.contains(name)) {
        return 0;
    }
    return static_cast<int>(file->file.entry(name).type);
}

const char* cuvit_weight_file_entry_name(const cuvit_weight_file* file, int64_t index) {
    if (file == nullptr || index < 0 || index >= static_cast<int64_t>(file->file.size())) {
        return nullptr;
    }
    return file->file.entries()[static_cast<std::size_t>(index)].name.c_str();
}

uint64_t cuvit_weight_file_payload_bytes(const cuvit_weight_file* file) {
    return file == nullptr ? 0 : file->file.payload_bytes();
}

void cuvit_weight_file_destroy(cuvit_weight_file* file) { delete file; }

void cuvit_vit_config_default(cuvit_vit_config* config) {
    if (config == nullptr) {
        return;
    }
    const cuvit::VitConfig d;
    *config = cuvit_vit_config{d.image_size, d.patch_size, d.channels, d.embed_dim, d.depth,
                               d.heads,      d.mlp_hidden, d.classes,  d.layer_norm_epsilon};
}

int cuvit_vit_config_validate(const cuvit_vit_config* config) {
    return guarded([&]() -> int {
        if (config == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "config cannot be null");
        }
        to_config(*config).validate();
        return CUVIT_OK;
    });
}

int cuvit_vit_create(const cuvit_vit_config* config, const cuvit_weight_file* file, int max_batch,
                     cuvit_vit** model) {
    return cuvit_vit_create_ex(config, file, max_batch, CUVIT_PRECISION_F32, model);
}

int cuvit_vit_create_ex(const cuvit_vit_config* config, const cuvit_weight_file* file,
                        int max_batch, int precision, cuvit_vit** model) {
    return guarded([&]() -> int {
        if (config == nullptr || file == nullptr || model == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "config, file and out-pointer cannot be null");
        }
        if (precision != CUVIT_PRECISION_F32 && precision != CUVIT_PRECISION_BF16) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "precision is not a cuvit_precision value");
        }
        auto created = std::make_unique<cuvit_vit>();
        created->model = std::make_unique<cuvit::VisionTransformer>(
            to_config(*config), file->file, max_batch,
            precision == CUVIT_PRECISION_BF16 ? cuvit::Precision::kBFloat16
                                              : cuvit::Precision::kFloat32);
        *model = created.release();
        return CUVIT_OK;
    });
}

int cuvit_vit_precision(const cuvit_vit* model) {
    if (model == nullptr) {
        return -1;
    }
    return model->model->precision() == cuvit::Precision::kBFloat16 ? CUVIT_PRECISION_BF16
                                                                    : CUVIT_PRECISION_F32;
}

int cuvit_vit_forward(cuvit_vit* model, const float* images, float* logits, int batch,
                      cuvit_stream_t stream) {
    return guarded([&]() -> int {
        if (model == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "model cannot be null");
        }
        model->model->forward(images, logits, batch, reinterpret_cast<hipStream_t>(stream));
        return CUVIT_OK;
    });
}

uint64_t cuvit_vit_weight_bytes(const cuvit_vit* model) {
    return model == nullptr ? 0 : model->model->weight_bytes();
}

uint64_t cuvit_vit_activation_bytes(const cuvit_vit* model) {
    return model == nullptr ? 0 : model->model->activation_bytes();
}

void cuvit_vit_destroy(cuvit_vit* model) { delete model; }

int cuvit_image_load_ppm(const char* path, cuvit_image** image) {
    return guarded([&]() -> int {
        if (path == nullptr || image == nullptr) {
            return fail(CUVIT_ERROR_INVALID_ARGUMENT, "path and out-pointer cannot be null");
        }
        auto loaded = std::make_unique<cuvit_image>();
        loaded->image = cuvit::load_ppm(path);
        *image = loaded.release();
        return CUVIT_OK;
    });
}

int cuvit_image_width(const cuvit_image* image) { return image == nullptr ? 0 : image->image.width; }

int cuvit_image_height(const cuvit_image* image) {
    return image == nullptr ? 0 : image->image.height;
}

const uint8_t* cuvit_image_pixels(const cuvit_image* image) {
    return image == nullptr ? nullptr : image->image.pixels.data();
}

void cuvit_image_destroy(cuvit_image* image) { delete image; }

} // extern "C"
