// GGUF v2/v3 reader behind include/vortexrt/gguf.hpp. The container format (magic, header
// counts, typed key/value pairs, tensor directory, aligned tensor-data section) is the public
// GGUF specification; the checks and messages follow the reference reader
// (src/gguf.cpp:312-403, :525-664) so that callers see the same failures.
#include "vortexrt/gguf.hpp"

#include <bit>
#include <cstring>
#include <limits>
#include <stdexcept>

namespace vortexrt {
namespace {

constexpr std::uint32_t kMagic = 0x46554747u;   // "GGUF" little-endian
constexpr std::uint64_t kMaxString = 1ull << 30;
constexpr std::uint64_t kMaxArray = 1ull << 31;
constexpr std::uint64_t kMaxCount = 1ull << 24;
constexpr std::uint32_t kMaxDims = 4;
constexpr int kMaxNesting = 8;

struct Layout {
    std::uint64_t elems;   // elements per block
    std::uint64_t bytes;   // bytes per block
};

// ggml tensor types this reader sizes (F32, F16, Q8_0, I8..I64, F64, BF16).
std::optional<Layout> layout_of(std::uint32_t type) {
    switch (type) {
        case 0: return Layout{1, 4};
        case 1: return Layout{1, 2};
        case 8: return Layout{32, 34};
        case 24: return Layout{1, 1};
        case 25: return Layout{1, 2};
        case 26: return Layout{1, 4};
        case 27: return Layout{1, 8};
        case 28: return Layout{1, 8};
        case 30: return Layout{1, 2};
        default: return std::nullopt;
    }
}

// Sequential little-endian reader over the header part of the file.
class Cursor {
public:
    Cursor(std::ifstream& in, std::uint64_t size) : in_(in), size_(size) {}

    void read(void* dst, std::size_t n) {
        if (n > size_ || pos_ > size_ - n) throw std::runtime_error("Unexpected end of GGUF file");
        in_.read(static_cast<char*>(dst), static_cast<std::streamsize>(n));
        if (!in_) throw std::runtime_error("Failed while reading GGUF file");
        pos_ += n;
    }
    template <typename T>
    T get() {
        T v;
        read(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const auto n = get<std::uint64_t>();
        if (n > kMaxString) throw std::runtime_error("GGUF string length exceeds safety limit");
        std::string s(static_cast<std::size_t>(n), '\0');
        if (n) read(s.data(), static_cast<std::size_t>(n));
        return s;
    }
    [[nodiscard]] std::uint64_t pos() const noexcept { return pos_; }

private:
    std::ifstream& in_;
    std::uint64_t size_;
    std::uint64_t pos_ = 0;
};

bool valid_type(std::uint32_t t) { return t <= static_cast<std::uint32_t>(GgufValueType::Float64); }

GgufValue read_value(Cursor& c, GgufValueType type, int depth) {
    GgufValue v;
    v.type = type;
    switch (type) {
        case GgufValueType::UInt8: v.scalar = static_cast<std::uint64_t>(c.get<std::uint8_t>()); break;
        case GgufValueType::UInt16: v.scalar = static_cast<std::uint64_t>(c.get<std::uint16_t>()); break;
        case GgufValueType::UInt32: v.scalar = static_cast<std::uint64_t>(c.get<std::uint32_t>()); break;
        case GgufValueType::UInt64: v.scalar = c.get<std::uint64_t>(); break;
        case GgufValueType::Int8: v.scalar = static_cast<std::int64_t>(c.get<std::int8_t>()); break;
        case GgufValueType::Int16: v.scalar = static_cast<std::int64_t>(c.get<std::int16_t>()); break;
        case GgufValueType::Int32: v.scalar = static_cast<std::int64_t>(c.get<std::int32_t>()); break;
        case GgufValueType::Int64: v.scalar = c.get<std::int64_t>(); break;
        case GgufValueType::Float32: v.scalar = static_cast<double>(c.get<float>()); break;
        case GgufValueType::Float64: v.scalar = c.get<double>(); break;
        case GgufValueType::Bool: {
            const auto b = c.get<std::uint8_t>();
            if (b > 1) throw std::runtime_error("GGUF boolean value is not 0/1");
            v.scalar = b != 0;
            break;
        }
        case GgufValueType::String: v.scalar = c.str(); break;
        case GgufValueType::Array: {
            if (depth >= kMaxNesting) throw std::runtime_error("GGUF array nesting is too deep");
            const auto et = c.get<std::uint32_t>();
            if (!valid_type(et)) throw std::runtime_error("GGUF array has invalid element type");
            const auto n = c.get<std::uint64_t>();
            if (n > kMaxArray) throw std::runtime_error("GGUF array length exceeds safety limit");
            v.array_element_type = static_cast<GgufValueType>(et);
            v.array.reserve(static_cast<std::size_t>(n));
            for (std::uint64_t i = 0; i < n; ++i) v.array.push_back(read_value(c, v.array_element_type, depth + 1));
            break;
        }
    }
    return v;
}

}  // namespace

// ---- GgufValue accessors ------------------------------------------------------------------

std::optional<std::string> GgufValue::as_string() const {
    if (const auto* s = std::get_if<std::string>(&scalar)) return *s;
    return std::nullopt;
}
std::optional<std::uint64_t> GgufValue::as_u64() const {
    if (const auto* u = std::get_if<std::uint64_t>(&scalar)) return *u;
    if (const auto* i = std::get_if<std::int64_t>(&scalar); i && *i >= 0) return static_cast<std::uint64_t>(*i);
    return std::nullopt;
}
std::optional<std::int64_t> GgufValue::as_i64() const {
    if (const auto* i = std::get_if<std::int64_t>(&scalar)) return *i;
    if (const auto* u = std::get_if<std::uint64_t>(&scalar);
        u && *u <= static_cast<std::uint64_t>(std::numeric_limits<std::int64_t>::max()))
        return static_cast<std::int64_t>(*u);
    return std::nullopt;
}
std::optional<double> GgufValue::as_f64() const {
    if (const auto* d = std::get_if<double>(&scalar)) return *d;
    if (const auto* u = std::get_if<std::uint64_t>(&scalar)) return static_cast<double>(*u);
    if (const auto* i = std::get_if<std::int64_t>(&scalar)) return static_cast<double>(*i);
    return std::nullopt;
}
std::optional<bool> GgufValue::as_bool() const {
    if (const auto* b = std::get_if<bool>(&scalar)) return *b;
    return std::nullopt;
}

// ---- GgufFile ------------------------------------------------------------------------------

GgufFile::GgufFile(const std::filesystem::path& path) : path_(path) {
    static_assert(std::endian::native == std::endian::little, "GGUF reader requires a little-endian host");
    std::ifstream in(path, std::ios::binary);
    if (!in) throw std::runtime_error("Failed to open GGUF file: " + path.string());
    std::error_code ec;
    file_size_ = std::filesystem::file_size(path, ec);
    if (ec) throw std::runtime_error("Failed to determine GGUF file size");

    Cursor c(in, file_size_);
    if (c.get<std::uint32_t>() != kMagic) throw std::runtime_error("Invalid GGUF magic");
    version_ = c.get<std::uint32_t>();
    if (version_ != 2 && version_ != 3) throw std::runtime_error("Unsupported GGUF version: " + std::to_string(version_));
    const auto n_tensors = c.get<std::uint64_t>();
    const auto n_meta = c.get<std::uint64_t>();
    if (n_tensors > kMaxCount || n_meta > kMaxCount) throw std::runtime_error("GGUF header counts exceed safety limits");

    metadata_.reserve(static_cast<std::size_t>(n_meta));
    for (std::uint64_t i = 0; i < n_meta; ++i) {
        GgufMetadata m;
        m.key = c.str();
        const auto t = c.get<std::uint32_t>();
        if (!valid_type(t)) throw std::runtime_error("GGUF metadata has invalid value type");
        m.value = read_value(c, static_cast<GgufValueType>(t), 0);
        metadata_index_[m.key] = metadata_.size();
        metadata_.push_back(std::move(m));
    }
    if (const auto* a = find_metadata("general.alignment")) {
        const auto v = a->as_u64();
        if (!v || *v > std::numeric_limits<std::uint32_t>::max()) throw std::runtime_error("Invalid general.alignment metadata");
        alignment_ = static_cast<std::uint32_t>(*v);
    }
    if (alignment_ == 0) throw std::runtime_error("GGUF alignment must be non-zero");
    if ((alignment_ & (alignment_ - 1u)) != 0) throw std::runtime_error("GGUF alignment must be a power of two");

    tensors_.reserve(static_cast<std::size_t>(n_tensors));
    for (std::uint64_t i = 0; i < n_tensors; ++i) {
        GgufTensorInfo t;
        t.name = c.str();
        const auto nd = c.get<std::uint32_t>();
        if (nd == 0 || nd > kMaxDims) throw std::runtime_error("GGUF tensor has invalid dimension count");
        t.dimensions.resize(nd);
        for (auto& d : t.dimensions) d = c.get<std::uint64_t>();
        t.type = c.get<std::uint32_t>();
        t.offset = c.get<std::uint64_t>();
        tensor_index_[t.name] = tensors_.size();
        tensors_.push_back(std::move(t));
    }
    const std::uint64_t a = alignment_;
    data_offset_ = (c.pos() + a - 1u) / a * a;
    if (data_offset_ > file_size_) throw std::runtime_error("GGUF tensor data offset lies beyond end of file");

    payload_stream_.open(path, std::ios::binary);
    if (!payload_stream_) throw std::runtime_error("Failed to open GGUF file: " + path.string());
}

const GgufValue* GgufFile::find_metadata(const std::string& key) const noexcept {
    const auto it = metadata_index_.find(key);
    return it == metadata_index_.end() ? nullptr : &metadata_[it->second].value;
}

const GgufTensorInfo* GgufFile::find_tensor(const std::string& name) const noexcept {
    const auto it = tensor_index_.find(name);
    return it == tensor_index_.end() ? nullptr : &tensors_[it->second];
}

std::optional<std::string> GgufFile::metadata_string(const std::string& key) const {
    const auto* v = find_metadata(key);
    return v ? v->as_string() : std::nullopt;
}

std::optional<std::uint64_t> GgufFile::metadata_u64(const std::string& key) const {
    const auto* v = find_metadata(key);
    return v ? v->as_u64() : std::nullopt;
}

std::optional<std::uint64_t> GgufFile::tensor_byte_size(const GgufTensorInfo& tensor) const {
    const auto lay = layout_of(tensor.type);
    if (!lay) return std::nullopt;
    std::uint64_t n = 1;
    for (const auto d : tensor.dimensions) {
        if (d != 0 && n > std::numeric_limits<std::uint64_t>::max() / d) throw std::runtime_error("GGUF tensor element count overflow");
        n *= d;
    }
    if (n % lay->elems != 0) throw std::runtime_error("GGUF tensor element count is not divisible by quant block size");
    const std::uint64_t blocks = n / lay->elems;
    if (blocks > std::numeric_limits<std::uint64_t>::max() / lay->bytes) throw std::runtime_error("GGUF tensor byte size overflow");
    return blocks * lay->bytes;
}

void GgufFile::read_bytes_at(std::uint64_t absolute_offset, void* destination, std::size_t bytes) const {
    if (bytes > file_size_ || absolute_offset > file_size_ - bytes) throw std::runtime_error("GGUF read lies beyond end of file");
    std::lock_guard<std::mutex> lock(payload_stream_mutex_);
    payload_stream_.clear();
    payload_stream_.seekg(static_cast<std::streamoff>(absolute_offset));
    payload_stream_.read(static_cast<char*>(destination), static_cast<std::streamsize>(bytes));
    if (!payload_stream_) throw std::runtime_error("Failed while reading GGUF file");
}

void GgufFile::read_data(std::uint64_t offset, void* destination, std::size_t bytes) const {
    if (offset > file_size_ - data_offset_) throw std::runtime_error("GGUF read lies beyond end of file");
    read_bytes_at(data_offset_ + offset, destination, bytes);
}

std::vector<std::byte> GgufFile::read_tensor_bytes(const GgufTensorInfo& tensor) const {
    const auto n = tensor_byte_size(tensor);
    if (!n) throw std::runtime_error("Unsupported GGUF tensor type for " + tensor.name);
    std::vector<std::byte> out(static_cast<std::size_t>(*n));
    read_data(tensor.offset, out.data(), out.size());
    return out;
}

std::vector<float> GgufFile::read_f32_tensor(const GgufTensorInfo& tensor) const {
    if (tensor.type != 0) throw std::runtime_error("GGUF tensor is not F32: " + tensor.name);
    const auto bytes = read_tensor_bytes(tensor);
    std::vector<float> out(bytes.size() / 4u);
    std::memcpy(out.data(), bytes.data(), out.size() * 4u);
    return out;
}

std::vector<float> GgufFile::read_q8_0_row(const GgufTensorInfo& tensor, std::uint64_t row) const {
    if (tensor.type != 8) throw std::runtime_error("GGUF tensor is not Q8_0: " + tensor.name);
    if (tensor.dimensions.size() < 2) throw std::runtime_error("GGUF Q8_0 row read requires a matrix: " + tensor.name);
    const std::uint64_t k = tensor.dimensions[0];
    std::uint64_t rows = 1;
    for (std::size_t i = 1; i < tensor.dimensions.size(); ++i) rows *= tensor.dimensions[i];
    if (k % 32u != 0) throw std::runtime_error("GGUF Q8_0 row width is not a multiple of 32: " + tensor.name);
    if (row >= rows) throw std::runtime_error("GGUF Q8_0 row index out of range: " + tensor.name);
    const std::uint64_t nb = k / 32u;
    std::vector<unsigned char> raw(static_cast<std::size_t>(nb * 34u));
    read_data(tensor.offset + row * nb * 34u, raw.data(), raw.size());
    std::vector<float> out(static_cast<std::size_t>(k));
    for (std::uint64_t b = 0; b < nb; ++b) {
        const unsigned char* blk = raw.data() + b * 34u;
        const float s = f16_to_f32(static_cast<std::uint16_t>(blk[0] | (blk[1] << 8)));
        for (int j = 0; j < 32; ++j) out[b * 32u + j] = s * static_cast<float>(static_cast<std::int8_t>(blk[2 + j]));
    }
    return out;
}

void GgufFile::validate() const {
    for (const auto& t : tensors_) {
        const auto n = tensor_byte_size(t);
        if (!n) throw std::runtime_error("Unsupported GGUF tensor type for " + t.name);
        if (t.offset % alignment_ != 0) throw std::runtime_error("GGUF tensor offset is not aligned: " + t.name);
        const std::uint64_t room = file_size_ - data_offset_;
        if (t.offset > room || *n > room - t.offset) throw std::runtime_error("GGUF tensor data lies beyond end of file: " + t.name);
    }
}

const char* gguf_value_type_name(GgufValueType type) noexcept {
    switch (type) {
        case GgufValueType::UInt8: return "u8";
        case GgufValueType::Int8: return "i8";
        case GgufValueType::UInt16: return "u16";
        case GgufValueType::Int16: return "i16";
        case GgufValueType::UInt32: return "u32";
        case GgufValueType::Int32: return "i32";
        case GgufValueType::Float32: return "f32";
        case GgufValueType::Bool: return "bool";
        case GgufValueType::String: return "string";
        case GgufValueType::Array: return "array";
        case GgufValueType::UInt64: return "u64";
        case GgufValueType::Int64: return "i64";
        case GgufValueType::Float64: return "f64";
    }
    return "unknown";
}

const char* ggml_type_name(std::uint32_t type) noexcept {
    switch (type) {
        case 0: return "F32";
        case 1: return "F16";
        case 8: return "Q8_0";
        case 24: return "I8";
        case 25: return "I16";
        case 26: return "I32";
        case 27: return "I64";
        case 28: return "F64";
        case 30: return "BF16";
        default: return "unknown";
    }
}

// binary16: sign 1, exponent 5 (bias 15), mantissa 10.
float f16_to_f32(std::uint16_t h) noexcept {
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const std::uint32_t exp = (h >> 10) & 0x1fu;
    std::uint32_t man = h & 0x3ffu;
    std::uint32_t bits;
    if (exp == 0x1fu) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {   // subnormal: normalise
        std::uint32_t e = 113u;
        while ((man & 0x400u) == 0) {
            man <<= 1;
            --e;
        }
        bits = sign | (e << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

}  // namespace vortexrt
