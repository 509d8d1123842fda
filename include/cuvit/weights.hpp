#pragma once

// The .cvw v1 weight format, the counterpart of the reference's
// include/cuvit/weights.hpp:16-92 with the byte layout of
// src/runtime/weights.cpp:13-23, little-endian:
//
//   magic u32 ("CVIT" = 0x54495643), version u32 (1), entry_count u32, reserved u32
//   entry_count x { name_length u32, name, type u32, rank u32, extents i64[rank],
//                   offset u64 (absolute), bytes u64 }
//   payloads, each starting on a 64-byte boundary
//
// Loading validates the header, every table field and that each payload lies
// inside the file; lookups check type and shape.

#include "cuvit/tensor.hpp"

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace cuvit {

enum class DataType : std::uint32_t {
    kFloat32 = 1,
};

[[nodiscard]] const char* data_type_name(DataType type);
[[nodiscard]] std::size_t data_type_size(DataType type);

struct WeightEntry {
    std::string name;
    DataType type = DataType::kFloat32;
    std::vector<Extent> extents;
    std::uint64_t offset = 0; // from the start of the file
    std::uint64_t bytes = 0;

    [[nodiscard]] Extent element_count() const;
    [[nodiscard]] std::string shape_string() const;
};

class WeightFile final {
  public:
    static constexpr std::uint32_t kMagic = 0x54495643U; // "CVIT"
    static constexpr std::uint32_t kVersion = 1;

    static WeightFile load(const std::string& path);

    [[nodiscard]] bool contains(const std::string& name) const;
    [[nodiscard]] const WeightEntry& entry(const std::string& name) const;
    /// Host pointer to a float32 payload whose shape must equal @p expected_extents.
    [[nodiscard]] const float* float_data(const std::string& name,
                                          const std::vector<Extent>& expected_extents) const;

    [[nodiscard]] const std::vector<WeightEntry>& entries() const noexcept { return entries_; }
    [[nodiscard]] std::size_t size() const noexcept { return entries_.size(); }
    [[nodiscard]] std::uint64_t payload_bytes() const noexcept;

  private:
    std::vector<WeightEntry> entries_;
    std::unordered_map<std::string, std::size_t> index_;
    std::vector<std::byte> blob_;
};

class WeightFileWriter final {
  public:
    void add(const std::string& name, const std::vector<Extent>& extents, const float* data);
    void write(const std::string& path) const;
    [[nodiscard]] std::size_t size() const noexcept { return entries_.size(); }

  private:
    struct Pending {
        std::string name;
        std::vector<Extent> extents;
        std::vector<float> data;
    };
    std::vector<Pending> entries_;
};

} // namespace cuvit
