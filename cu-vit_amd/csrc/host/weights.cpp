// .cvw reader and writer (format: include/cuvit/weights.hpp). Byte layout,
// validation and error conditions follow the reference's
// src/runtime/weights.cpp:13-296 so version 1 files move between the two
// unchanged; version 2 adds the bf16 type and nothing else.
#include "cuvit/weights.hpp"

#include <cstring>
#include <fstream>
#include <ios>
#include <limits>
#include <stdexcept>
#include <type_traits>
#include <utility>

namespace cuvit {
namespace {

constexpr std::uint64_t kPayloadAlignment = 64;

std::uint64_t next_payload_offset(std::uint64_t position) {
    return (position + kPayloadAlignment - 1) & ~(kPayloadAlignment - 1);
}

/// Bounds-checked little-endian reader over the file image.
class Cursor {
  public:
    explicit Cursor(const std::vector<std::byte>& bytes) : bytes_(bytes) {}

    template <typename T> T scalar() {
        static_assert(std::is_trivially_copyable<T>::value, "plain values only");
        if (sizeof(T) > bytes_.size() - position_) {
            throw std::runtime_error("Weight file ends inside a header field");
        }
        T value{};
        std::memcpy(&value, bytes_.data() + position_, sizeof(T));
        position_ += sizeof(T);
        return value;
    }

    std::string text(std::uint32_t length) {
        if (length > bytes_.size() - position_) {
            throw std::runtime_error("Weight file ends inside a tensor name");
        }
        std::string value(reinterpret_cast<const char*>(bytes_.data() + position_), length);
        position_ += length;
        return value;
    }

  private:
    const std::vector<std::byte>& bytes_;
    std::size_t position_ = 0;
};

template <typename T> void put(std::ostream& out, T value) {
    out.write(reinterpret_cast<const char*>(&value), sizeof(T));
}

std::string shape_text(const std::vector<Extent>& extents) {
    std::string text = "[";
    for (std::size_t i = 0; i < extents.size(); ++i) {
        text += (i == 0 ? "" : ", ") + std::to_string(extents[i]);
    }
    return text + ']';
}

} // namespace

const char* data_type_name(DataType type) {
    switch (type) {
    case DataType::kFloat32: return "float32";
    case DataType::kBFloat16: return "bfloat16";
    }
    return "unknown";
}

std::size_t data_type_size(DataType type) {
    switch (type) {
    case DataType::kFloat32: return sizeof(float);
    case DataType::kBFloat16: return sizeof(std::uint16_t);
    }
    throw std::runtime_error("Weight file names an unsupported data type");
}

Extent WeightEntry::element_count() const {
    Extent count = 1;
    for (const Extent e : extents) {
        count *= e;
    }
    return count;
}

std::string WeightEntry::shape_string() const { return shape_text(extents); }

WeightFile WeightFile::load(const std::string& path) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) {
        throw std::runtime_error("Cannot open weight file: " + path);
    }
    const std::streamoff length = in.tellg();
    if (length < 0) {
        throw std::runtime_error("Cannot determine the size of weight file: " + path);
    }
    in.seekg(0, std::ios::beg);

    WeightFile file;
    file.blob_.resize(static_cast<std::size_t>(length));
    if (length > 0 && !in.read(reinterpret_cast<char*>(file.blob_.data()), length)) {
        throw std::runtime_error("Cannot read weight file: " + path);
    }

    Cursor cursor(file.blob_);
    if (cursor.scalar<std::uint32_t>() != kMagic) {
        throw std::runtime_error("Not a Cu-Vit weight file: " + path);
    }
    const auto version = cursor.scalar<std::uint32_t>();
    if (version != kVersion && version != kBFloat16Version) {
        throw std::runtime_error("Weight file " + path + " has version " + std::to_string(version) +
                                 ", but this reader takes versions " + std::to_string(kVersion) +
                                 " and " + std::to_string(kBFloat16Version));
    }
    file.version_ = version;
    const auto count = cursor.scalar<std::uint32_t>();
    static_cast<void>(cursor.scalar<std::uint32_t>()); // reserved

    const std::uint64_t size = file.blob_.size();
    file.entries_.reserve(count);
    for (std::uint32_t i = 0; i < count; ++i) {
        WeightEntry entry;
        entry.name = cursor.text(cursor.scalar<std::uint32_t>());

        const auto type = cursor.scalar<std::uint32_t>();
        const bool known = type == static_cast<std::uint32_t>(DataType::kFloat32) ||
                           (version == kBFloat16Version &&
                            type == static_cast<std::uint32_t>(DataType::kBFloat16));
        if (!known) {
            throw std::runtime_error("Tensor '" + entry.name + "' has unsupported data type " +
                                     std::to_string(type));
        }
        entry.type = static_cast<DataType>(type);

        const auto rank = cursor.scalar<std::uint32_t>();
        if (rank == 0 || rank > static_cast<std::uint32_t>(kMaxTensorRank)) {
            throw std::runtime_error("Tensor '" + entry.name + "' has rank " + std::to_string(rank) +
                                     ", outside 1.." + std::to_string(kMaxTensorRank));
        }
        for (std::uint32_t axis = 0; axis < rank; ++axis) {
            const auto extent = cursor.scalar<std::int64_t>();
            if (extent < 0) {
                throw std::runtime_error("Tensor '" + entry.name + "' has a negative extent");
            }
            entry.extents.push_back(extent);
        }
        entry.offset = cursor.scalar<std::uint64_t>();
        entry.bytes = cursor.scalar<std::uint64_t>();

        const std::uint64_t needed =
            static_cast<std::uint64_t>(entry.element_count()) * data_type_size(entry.type);
        if (entry.bytes != needed) {
            throw std::runtime_error("Tensor '" + entry.name + "' declares " +
                                     std::to_string(entry.bytes) + " bytes but its shape " +
                                     entry.shape_string() + " needs " + std::to_string(needed));
        }
        if (entry.offset > size || entry.bytes > size - entry.offset) {
            throw std::runtime_error("Tensor '" + entry.name + "' lies outside the file");
        }
        if (!file.index_.emplace(entry.name, file.entries_.size()).second) {
            throw std::runtime_error("Weight file contains two tensors named '" + entry.name + "'");
        }
        file.entries_.push_back(std::move(entry));
    }
    return file;
}

bool WeightFile::contains(const std::string& name) const { return index_.count(name) != 0; }

const WeightEntry& WeightFile::entry(const std::string& name) const {
    const auto found = index_.find(name);
    if (found == index_.end()) {
        throw std::runtime_error("Weight file has no tensor named '" + name + "'");
    }
    return entries_[found->second];
}

const WeightEntry& WeightFile::checked(const std::string& name,
                                       const std::vector<Extent>& expected_extents,
                                       DataType type) const {
    const WeightEntry& found = entry(name);
    if (found.type != type) {
        throw std::runtime_error("Tensor '" + name + "' is " + data_type_name(found.type) +
                                 ", not " + data_type_name(type));
    }
    if (found.extents != expected_extents) {
        throw std::runtime_error("Tensor '" + name + "' has shape " + found.shape_string() +
                                 ", but " + shape_text(expected_extents) + " was expected");
    }
    return found;
}

const float* WeightFile::float_data(const std::string& name,
                                    const std::vector<Extent>& expected_extents) const {
    const WeightEntry& found = checked(name, expected_extents, DataType::kFloat32);
    return reinterpret_cast<const float*>(blob_.data() + found.offset);
}

const std::uint16_t* WeightFile::bf16_data(const std::string& name,
                                           const std::vector<Extent>& expected_extents) const {
    const WeightEntry& found = checked(name, expected_extents, DataType::kBFloat16);
    return reinterpret_cast<const std::uint16_t*>(blob_.data() + found.offset);
}

std::vector<float> WeightFile::values(const std::string& name,
                                      const std::vector<Extent>& expected_extents) const {
    const WeightEntry& found = entry(name);
    const auto count = static_cast<std::size_t>(found.element_count());
    std::vector<float> out(count);
    if (found.type == DataType::kBFloat16) {
        const std::uint16_t* const bits = bf16_data(name, expected_extents);
        for (std::size_t i = 0; i < count; ++i) {
            const std::uint32_t widened = static_cast<std::uint32_t>(bits[i]) << 16;
            std::memcpy(&out[i], &widened, sizeof(float));
        }
    } else if (count > 0) {
        std::memcpy(out.data(), float_data(name, expected_extents), count * sizeof(float));
    } else {
        static_cast<void>(float_data(name, expected_extents)); // shape and type check
    }
    return out;
}

std::uint64_t WeightFile::payload_bytes() const noexcept {
    std::uint64_t total = 0;
    for (const WeightEntry& e : entries_) {
        total += e.bytes;
    }
    return total;
}

Extent WeightFileWriter::check_new(const std::string& name, const std::vector<Extent>& extents,
                                   const void* data) const {
    if (name.empty()) {
        throw std::invalid_argument("A weight tensor needs a name");
    }
    if (extents.empty() || extents.size() > static_cast<std::size_t>(kMaxTensorRank)) {
        throw std::invalid_argument("Tensor '" + name + "' has an unsupported rank");
    }
    Extent count = 1;
    for (const Extent e : extents) {
        if (e < 0) {
            throw std::invalid_argument("Tensor '" + name + "' has a negative extent");
        }
        count *= e;
    }
    for (const Pending& existing : entries_) {
        if (existing.name == name) {
            throw std::invalid_argument("Tensor '" + name + "' was added twice");
        }
    }
    if (count > 0 && data == nullptr) {
        throw std::invalid_argument("Tensor '" + name + "' has no data");
    }
    return count;
}

void WeightFileWriter::add(const std::string& name, const std::vector<Extent>& extents,
                           const float* data) {
    const auto count = static_cast<std::size_t>(check_new(name, extents, data));
    const auto* const bytes = reinterpret_cast<const std::byte*>(data);
    entries_.push_back(Pending{name, DataType::kFloat32, extents,
                               std::vector<std::byte>(bytes, bytes + count * sizeof(float))});
}

void WeightFileWriter::add_bf16(const std::string& name, const std::vector<Extent>& extents,
                                const std::uint16_t* data) {
    const auto count = static_cast<std::size_t>(check_new(name, extents, data));
    const auto* const bytes = reinterpret_cast<const std::byte*>(data);
    entries_.push_back(Pending{name, DataType::kBFloat16, extents,
                               std::vector<std::byte>(bytes, bytes + count * sizeof(std::uint16_t))});
}

void WeightFileWriter::write(const std::string& path) const {
    if (entries_.size() > std::numeric_limits<std::uint32_t>::max()) {
        throw std::runtime_error("Too many tensors for one weight file");
    }

    // The table's size is known up front, so every payload offset is too.
    std::uint64_t table = 4 * sizeof(std::uint32_t);
    for (const Pending& e : entries_) {
        table += sizeof(std::uint32_t) + e.name.size() + 2 * sizeof(std::uint32_t) +
                 e.extents.size() * sizeof(std::int64_t) + 2 * sizeof(std::uint64_t);
    }
    std::vector<std::uint64_t> offsets;
    offsets.reserve(entries_.size());
    std::uint64_t position = next_payload_offset(table);
    bool reduced = false;
    for (const Pending& e : entries_) {
        offsets.push_back(position);
        position = next_payload_offset(position + e.data.size());
        reduced = reduced || e.type != DataType::kFloat32;
    }

    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    if (!out) {
        throw std::runtime_error("Cannot create weight file: " + path);
    }
    put(out, WeightFile::kMagic);
    put(out, reduced ? WeightFile::kBFloat16Version : WeightFile::kVersion);
    put(out, static_cast<std::uint32_t>(entries_.size()));
    put(out, std::uint32_t{0});
    for (std::size_t i = 0; i < entries_.size(); ++i) {
        const Pending& e = entries_[i];
        put(out, static_cast<std::uint32_t>(e.name.size()));
        out.write(e.name.data(), static_cast<std::streamsize>(e.name.size()));
        put(out, static_cast<std::uint32_t>(e.type));
        put(out, static_cast<std::uint32_t>(e.extents.size()));
        for (const Extent extent : e.extents) {
            put(out, static_cast<std::int64_t>(extent));
        }
        put(out, offsets[i]);
        put(out, static_cast<std::uint64_t>(e.data.size()));
    }
    for (std::size_t i = 0; i < entries_.size(); ++i) {
        const auto at = static_cast<std::uint64_t>(out.tellp());
        if (at > offsets[i]) {
            throw std::runtime_error("Weight file layout overran a payload offset");
        }
        const std::vector<char> zeros(offsets[i] - at, '\0');
        out.write(zeros.data(), static_cast<std::streamsize>(zeros.size()));
        out.write(reinterpret_cast<const char*>(entries_[i].data.data()),
                  static_cast<std::streamsize>(entries_[i].data.size()));
    }
    if (!out) {
        throw std::runtime_error("Failed while writing weight file: " + path);
    }
}

} // namespace cuvit
