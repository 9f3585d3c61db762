// GGUF v2/v3 reader behind include/vortexrt/gguf.hpp. The container format (magic, header
// counts, typed key/value pairs, tensor directory, aligned tensor-data section) is the public
// GGUF specification; the checks and messages follow the reference reader
// (src/gguf.cpp:312-403, :525-664) so that callers see the same failures.
#include "vortexrt/gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <bit>
#include <cstring>
#include <limits>
#include <stdexcept>
#include <unordered_map>

namespace vortexrt {
namespace {

constexpr std::uint32_t kMagic = 0x46554747u;   // "GGUF" little-endian
constexpr std::uint64_t kMaxString = 1ull << 30;
constexpr std::uint64_t kMaxArray = 1ull << 28;       // src/gguf.cpp:16
constexpr std::uint64_t kMaxCount = 1000000ull;       // src/gguf.cpp:334
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

// Sequential little-endian reader over the mapped header bytes.
class Cursor {
public:
    Cursor(const unsigned char* base, std::uint64_t size) : base_(base), size_(size) {}

    void read(void* dst, std::size_t n) {
        if (n > size_ || pos_ > size_ - n) throw std::runtime_error("Unexpected end of GGUF file");
        if (n) std::memcpy(dst, base_ + pos_, n);
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
    [[nodiscard]] std::uint64_t remaining() const noexcept { return size_ - pos_; }

private:
    const unsigned char* base_;
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
            // every element takes at least one byte of the file, so a count the file cannot hold
            // fails at its end instead of reserving memory for it
            v.array.reserve(static_cast<std::size_t>(std::min(n, c.remaining())));
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

// The whole file mapped read-only (PROT_READ, MAP_PRIVATE) plus the parsed header. A zero-length
// file is not mapped; its header read fails like any truncated file's.
struct GgufFile::Image {
    const unsigned char* bytes = nullptr;
    std::uint64_t size = 0;
    std::uint32_t version = 0;
    std::uint64_t data_offset = 0;
    std::uint32_t alignment = 32;
    std::vector<GgufMetadata> metadata;
    std::vector<GgufTensorInfo> tensors;
    std::unordered_map<std::string, std::size_t> metadata_at;
    std::unordered_map<std::string, std::size_t> tensor_at;

    explicit Image(const std::filesystem::path& path) {
        const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
        if (fd < 0) throw std::runtime_error("Failed to open GGUF file: " + path.string());
        struct stat st {};
        if (::fstat(fd, &st) != 0 || st.st_size < 0) {
            ::close(fd);
            throw std::runtime_error("Failed to determine GGUF file size");
        }
        size = static_cast<std::uint64_t>(st.st_size);
        if (size) {
            void* m = ::mmap(nullptr, static_cast<std::size_t>(size), PROT_READ, MAP_PRIVATE, fd, 0);
            if (m == MAP_FAILED) {
                ::close(fd);
                throw std::runtime_error("Failed to open GGUF file: " + path.string());
            }
            bytes = static_cast<const unsigned char*>(m);
        }
        ::close(fd);   // the mapping keeps the file
    }
    ~Image() {
        if (bytes) ::munmap(const_cast<unsigned char*>(bytes), static_cast<std::size_t>(size));
    }
    Image(const Image&) = delete;
    Image& operator=(const Image&) = delete;

    void parse() {
        Cursor c(bytes, size);
        if (c.get<std::uint32_t>() != kMagic) throw std::runtime_error("Invalid GGUF magic");
        version = c.get<std::uint32_t>();
        if (version != 2 && version != 3) throw std::runtime_error("Unsupported GGUF version: " + std::to_string(version));
        const auto n_tensors = c.get<std::uint64_t>();
        const auto n_meta = c.get<std::uint64_t>();
        if (n_tensors > kMaxCount || n_meta > kMaxCount) throw std::runtime_error("GGUF header counts exceed safety limits");

        metadata.reserve(static_cast<std::size_t>(n_meta));
        for (std::uint64_t i = 0; i < n_meta; ++i) {
            GgufMetadata m;
            m.key = c.str();
            const auto t = c.get<std::uint32_t>();
            if (!valid_type(t)) throw std::runtime_error("GGUF metadata has invalid value type");
            m.value = read_value(c, static_cast<GgufValueType>(t), 0);
            metadata_at[m.key] = metadata.size();
            metadata.push_back(std::move(m));
        }
        if (const auto it = metadata_at.find("general.alignment"); it != metadata_at.end()) {
            const auto v = metadata[it->second].value.as_u64();
            if (!v || *v > std::numeric_limits<std::uint32_t>::max()) throw std::runtime_error("Invalid general.alignment metadata");
            alignment = static_cast<std::uint32_t>(*v);
        }
        if (alignment == 0) throw std::runtime_error("GGUF alignment must be non-zero");
        if ((alignment & (alignment - 1u)) != 0) throw std::runtime_error("GGUF alignment must be a power of two");

        tensors.reserve(static_cast<std::size_t>(n_tensors));
        for (std::uint64_t i = 0; i < n_tensors; ++i) {
            GgufTensorInfo t;
            t.name = c.str();
            const auto nd = c.get<std::uint32_t>();
            if (nd == 0 || nd > kMaxDims) throw std::runtime_error("GGUF tensor has invalid dimension count");
            t.dimensions.resize(nd);
            for (auto& d : t.dimensions) d = c.get<std::uint64_t>();
            t.type = c.get<std::uint32_t>();
            t.offset = c.get<std::uint64_t>();
            tensor_at[t.name] = tensors.size();
            tensors.push_back(std::move(t));
        }
        const std::uint64_t a = alignment;
        data_offset = (c.pos() + a - 1u) / a * a;
        if (data_offset > size) throw std::runtime_error("GGUF tensor data offset lies beyond end of file");
    }

    // Copies bytes [absolute, absolute + n) of the file.
    void copy(std::uint64_t absolute, void* destination, std::size_t n) const {
        if (n > size || absolute > size - n) throw std::runtime_error("GGUF read lies beyond end of file");
        if (n) std::memcpy(destination, bytes + absolute, n);
    }
};

GgufFile::GgufFile(const std::filesystem::path& path) {
    static_assert(std::endian::native == std::endian::little, "GGUF reader requires a little-endian host");
    auto image = std::make_unique<Image>(path);
    image->parse();
    image_ = std::move(image);
}

GgufFile::~GgufFile() = default;
GgufFile::GgufFile(GgufFile&&) noexcept = default;
GgufFile& GgufFile::operator=(GgufFile&&) noexcept = default;

std::uint32_t GgufFile::version() const noexcept { return image_->version; }
std::uint64_t GgufFile::file_size() const noexcept { return image_->size; }
std::uint64_t GgufFile::data_offset() const noexcept { return image_->data_offset; }
std::uint32_t GgufFile::alignment() const noexcept { return image_->alignment; }
const std::vector<GgufMetadata>& GgufFile::metadata() const noexcept { return image_->metadata; }
const std::vector<GgufTensorInfo>& GgufFile::tensors() const noexcept { return image_->tensors; }

const GgufValue* GgufFile::find_metadata(const std::string& key) const noexcept {
    const auto it = image_->metadata_at.find(key);
    return it == image_->metadata_at.end() ? nullptr : &image_->metadata[it->second].value;
}

const GgufTensorInfo* GgufFile::find_tensor(const std::string& name) const noexcept {
    const auto it = image_->tensor_at.find(name);
    return it == image_->tensor_at.end() ? nullptr : &image_->tensors[it->second];
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

void GgufFile::read_data(std::uint64_t offset, void* destination, std::size_t bytes) const {
    const Image& im = *image_;
    if (offset > im.size - im.data_offset) throw std::runtime_error("GGUF read lies beyond end of file");
    im.copy(im.data_offset + offset, destination, bytes);
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
    const Image& im = *image_;
    for (const auto& t : im.tensors) {
        const auto n = tensor_byte_size(t);
        if (!n) throw std::runtime_error("Unsupported GGUF tensor type for " + t.name);
        if (t.offset % im.alignment != 0) throw std::runtime_error("GGUF tensor offset is not aligned: " + t.name);
        const std::uint64_t room = im.size - im.data_offset;
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
