#pragma once

// The .cvw weight format, the counterpart of the reference's
// include/cuvit/weights.hpp:16-92 with the byte layout of
// src/runtime/weights.cpp:13-23, little-endian:
//
//   magic u32 ("CVIT" = 0x54495643), version u32, entry_count u32, reserved u32
//   entry_count x { name_length u32, name, type u32, rank u32, extents i64[rank],
//                   offset u64 (absolute), bytes u64 }
//   payloads, each starting on a 64-byte boundary
//
// Version 1 is the reference's: every tensor is float32 (type 1). Version 2
// (an extension) has the same layout and adds type 2, bfloat16 (the upper 16
// bits of an IEEE float, carried as uint16). The writer emits version 1
// whenever every tensor is float32, byte for byte what the reference writes,
// and version 2 only for a file holding a bf16 tensor, which the reference's
// reader then refuses by its version check. Loading accepts both, validates
// the header, every table field and that each payload lies inside the file;
// lookups check type and shape.

#include "cuvit/tensor.hpp"

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace cuvit {

enum class DataType : std::uint32_t {
    kFloat32 = 1,
    kBFloat16 = 2, // version 2 files only
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
    static constexpr std::uint32_t kVersion = 1;         // float32 only, the reference's
    static constexpr std::uint32_t kBFloat16Version = 2; // adds DataType::kBFloat16

    static WeightFile load(const std::string& path);

    [[nodiscard]] bool contains(const std::string& name) const;
    [[nodiscard]] const WeightEntry& entry(const std::string& name) const;
    /// Host pointer to a float32 payload whose shape must equal @p expected_extents.
    [[nodiscard]] const float* float_data(const std::string& name,
                                          const std::vector<Extent>& expected_extents) const;
    /// Host pointer to a bfloat16 payload (bit patterns) of the expected shape.
    [[nodiscard]] const std::uint16_t* bf16_data(const std::string& name,
                                                 const std::vector<Extent>& expected_extents) const;
    /// The payload of either type, shape-checked, as float: widened exactly
    /// from bf16 or copied.
    [[nodiscard]] std::vector<float> values(const std::string& name,
                                            const std::vector<Extent>& expected_extents) const;
    [[nodiscard]] std::uint32_t version() const noexcept { return version_; }

    [[nodiscard]] const std::vector<WeightEntry>& entries() const noexcept { return entries_; }
    [[nodiscard]] std::size_t size() const noexcept { return entries_.size(); }
    [[nodiscard]] std::uint64_t payload_bytes() const noexcept;

  private:
    /// The entry @p name, checked to have @p type and @p expected_extents.
    const WeightEntry& checked(const std::string& name, const std::vector<Extent>& expected_extents,
                               DataType type) const;

    std::vector<WeightEntry> entries_;
    std::unordered_map<std::string, std::size_t> index_;
    std::vector<std::byte> blob_;
    std::uint32_t version_ = kVersion;
};

class WeightFileWriter final {
  public:
    void add(const std::string& name, const std::vector<Extent>& extents, const float* data);
    /// A bfloat16 tensor (bit patterns); the file becomes version 2.
    void add_bf16(const std::string& name, const std::vector<Extent>& extents,
                  const std::uint16_t* data);
    void write(const std::string& path) const;
    [[nodiscard]] std::size_t size() const noexcept { return entries_.size(); }

  private:
    struct Pending {
        std::string name;
        DataType type;
        std::vector<Extent> extents;
        std::vector<std::byte> data;
    };
    /// Validates name and extents; returns the element count.
    Extent check_new(const std::string& name, const std::vector<Extent>& extents,
                     const void* data) const;
    std::vector<Pending> entries_;
};

} // namespace cuvit
