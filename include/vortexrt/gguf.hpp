// GGUF v2/v3 reader (include/vortexrt/gguf.hpp:14-128 of Vortex-RT): same public API, host only;
// the private part is this reader's own (a read-only memory map of the file).
#pragma once

#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <memory>
#include <optional>
#include <string>
#include <variant>
#include <vector>

namespace vortexrt {

enum class GgufValueType : std::uint32_t {
    UInt8 = 0,
    Int8 = 1,
    UInt16 = 2,
    Int16 = 3,
    UInt32 = 4,
    Int32 = 5,
    Float32 = 6,
    Bool = 7,
    String = 8,
    Array = 9,
    UInt64 = 10,
    Int64 = 11,
    Float64 = 12,
};

using GgufScalar = std::variant<std::monostate, std::uint64_t, std::int64_t, double, bool, std::string>;

struct GgufValue {
    GgufValueType type = GgufValueType::UInt8;
    GgufScalar scalar{};
    GgufValueType array_element_type = GgufValueType::UInt8;
    std::vector<GgufValue> array{};

    [[nodiscard]] bool is_array() const noexcept { return type == GgufValueType::Array; }

    [[nodiscard]] std::optional<std::string> as_string() const;
    [[nodiscard]] std::optional<std::uint64_t> as_u64() const;
    [[nodiscard]] std::optional<std::int64_t> as_i64() const;
    [[nodiscard]] std::optional<double> as_f64() const;
    [[nodiscard]] std::optional<bool> as_bool() const;
};

struct GgufMetadata {
    std::string key;
    GgufValue value;
};

struct GgufTensorInfo {
    std::string name;
    std::vector<std::uint64_t> dimensions;
    std::uint32_t type = 0;
    std::uint64_t offset = 0;   // relative to data_offset()
};

class GgufFile {
public:
    explicit GgufFile(const std::filesystem::path& path);
    ~GgufFile();
    GgufFile(GgufFile&&) noexcept;
    GgufFile& operator=(GgufFile&&) noexcept;
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    [[nodiscard]] std::uint32_t version() const noexcept;
    [[nodiscard]] std::uint64_t file_size() const noexcept;
    [[nodiscard]] std::uint64_t data_offset() const noexcept;
    [[nodiscard]] std::uint32_t alignment() const noexcept;

    [[nodiscard]] const std::vector<GgufMetadata>& metadata() const noexcept;
    [[nodiscard]] const std::vector<GgufTensorInfo>& tensors() const noexcept;

    [[nodiscard]] const GgufValue* find_metadata(const std::string& key) const noexcept;
    [[nodiscard]] const GgufTensorInfo* find_tensor(const std::string& name) const noexcept;

    [[nodiscard]] std::optional<std::string> metadata_string(const std::string& key) const;
    [[nodiscard]] std::optional<std::uint64_t> metadata_u64(const std::string& key) const;

    [[nodiscard]] std::optional<std::uint64_t> tensor_byte_size(const GgufTensorInfo& tensor) const;
    [[nodiscard]] std::vector<std::byte> read_tensor_bytes(const GgufTensorInfo& tensor) const;
    [[nodiscard]] std::vector<float> read_f32_tensor(const GgufTensorInfo& tensor) const;
    [[nodiscard]] std::vector<float> read_q8_0_row(const GgufTensorInfo& tensor, std::uint64_t row) const;

    // Every tensor's byte range lies inside the file, past data_offset, at an aligned offset.
    void validate() const;

    // Reads `bytes` of the tensor-data section starting at data_offset() + offset.
    void read_data(std::uint64_t offset, void* destination, std::size_t bytes) const;

private:
    // The file mapped read-only into memory and the header parsed from the mapping (gguf.cpp).
    // Every read is a bounds-checked copy out of the mapping, so one GgufFile serves concurrent
    // readers without a lock.
    struct Image;
    std::unique_ptr<const Image> image_;
};

[[nodiscard]] const char* gguf_value_type_name(GgufValueType type) noexcept;
[[nodiscard]] const char* ggml_type_name(std::uint32_t type) noexcept;

// IEEE binary16 -> binary32, exact (subnormals, infinities and NaN included).
[[nodiscard]] float f16_to_f32(std::uint16_t bits) noexcept;

}  // namespace vortexrt
