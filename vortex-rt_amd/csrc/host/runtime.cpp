// DeviceContext, Buffer, Q8MatVecPipeline and ArgmaxPipeline over the C ABI of libvrt_hip.so.
// Argument checks and messages follow the reference (src/buffer.cpp:20-160,
// src/q8_matvec.cpp:801-1016, :1360-1520, :2007-2110); every run* call is synchronous.
#include "vortexrt/argmax.hpp"
#include "vortexrt/buffer.hpp"
#include "vortexrt/q8_matvec.hpp"
#include "vortexrt/vulkan_context.hpp"

#include "vrt_hip.h"

#include <limits>
#include <stdexcept>

namespace vortexrt {

void check_vrt(int rc) {
    if (rc != VRT_OK) {
        const char* msg = vrt_last_error();
        throw std::runtime_error(msg && *msg ? msg : "libvrt_hip call failed");
    }
}

// ---- DeviceContext --------------------------------------------------------------------------

DeviceContext::DeviceContext(std::string device_selector) {
    check_vrt(vrt_ctx_create(device_selector.c_str(), &ctx_));
    vrt_device_info info{};
    if (int rc = vrt_ctx_info(ctx_, &info)) {
        vrt_ctx_destroy(ctx_);
        check_vrt(rc);
    }
    caps_.name = info.name;
    caps_.arch = info.arch;
    caps_.device_index = info.device_index;
    caps_.vendor_id = info.vendor_id;
    caps_.device_id = info.device_id;
    caps_.subgroup_size = info.subgroup_size;
    caps_.compute_units = info.compute_units;
    caps_.fp16 = info.fp16 != 0;
    caps_.int8 = info.int8 != 0;
    caps_.storage8 = info.storage8 != 0;
    caps_.storage16 = info.storage16 != 0;
    caps_.device_local_bytes = info.device_local_bytes;
    caps_.l2_bytes = info.l2_bytes;
}

DeviceContext::~DeviceContext() {
    if (ctx_) vrt_ctx_destroy(ctx_);
}

void* DeviceContext::stream() const {
    void* s = nullptr;
    check_vrt(vrt_stream(ctx_, &s));
    return s;
}

void DeviceContext::synchronize() { check_vrt(vrt_sync(ctx_)); }

// ---- Buffer ---------------------------------------------------------------------------------

Buffer::Buffer(DeviceContext& context, std::uint64_t size, BufferUsageFlags, MemoryPropertyFlags memory_properties)
    : context_(context), size_(size), props_(memory_properties) {
    if (size == 0) throw std::runtime_error("Buffer size must be non-zero");
    const std::uint32_t kind = (memory_properties & kMemoryHostVisible) ? VRT_MEM_HOST : VRT_MEM_DEVICE;
    check_vrt(vrt_alloc(context.handle(), size, kind, &ptr_));
}

Buffer::~Buffer() {
    if (ptr_) vrt_free(context_.handle(), ptr_);
}

void Buffer::upload(const void* data, std::size_t bytes, std::uint64_t offset) {
    if (data == nullptr) throw std::runtime_error("Buffer::upload received null data");
    if (offset > size_ || bytes > size_ - offset) throw std::runtime_error("Buffer::upload out of range");
    if (bytes) check_vrt(vrt_memcpy(context_.handle(), static_cast<char*>(ptr_) + offset, data, bytes));
}

void Buffer::download(void* data, std::size_t bytes, std::uint64_t offset) const {
    if (data == nullptr) throw std::runtime_error("Buffer::download received null data");
    if (offset > size_ || bytes > size_ - offset) throw std::runtime_error("Buffer::download out of range");
    if (bytes) check_vrt(vrt_memcpy(context_.handle(), data, static_cast<const char*>(ptr_) + offset, bytes));
}

// ---- Q8MatVecPipeline -----------------------------------------------------------------------

namespace {

constexpr std::uint64_t kBlockBytes = 34;

std::uint64_t matrix_bytes(std::uint32_t input_dim, std::uint32_t rows) {
    return static_cast<std::uint64_t>(rows) * (input_dim / 32u) * kBlockBytes;
}

void check_dims(std::uint32_t input_dim, std::uint32_t output_dim, std::uint32_t offset) {
    if (input_dim == 0 || output_dim == 0) throw std::runtime_error("Q8MatVecPipeline dimensions must be non-zero");
    if (input_dim % 32u != 0) throw std::runtime_error("Q8MatVecPipeline input_dim must be divisible by 32");
    if ((offset & 3u) != 0) throw std::runtime_error("Q8MatVecPipeline weight byte offset must be 4-byte aligned");
}

}  // namespace

Q8MatVecPipeline::Q8MatVecPipeline(DeviceContext& context, const std::string&, const std::string&, const std::string&)
    : context_(context) {}

void Q8MatVecPipeline::run(Buffer& weights, Buffer& input, Buffer& output, std::uint32_t weight_byte_offset,
                           std::uint32_t input_dim, std::uint32_t output_dim) {
    check_dims(input_dim, output_dim, weight_byte_offset);
    if (weight_byte_offset + matrix_bytes(input_dim, output_dim) > weights.size())
        throw std::runtime_error("Q8MatVecPipeline weight buffer is too small");
    if (static_cast<std::uint64_t>(input_dim) * 4u > input.size()) throw std::runtime_error("Q8MatVecPipeline input buffer is too small");
    if (static_cast<std::uint64_t>(output_dim) * 4u > output.size())
        throw std::runtime_error("Q8MatVecPipeline output buffer is too small");
    check_vrt(vrt_q8_matvec(context_.handle(), weights.handle(), weights.size(), weight_byte_offset,
                            static_cast<const float*>(input.handle()), static_cast<float*>(output.handle()), input_dim,
                            output_dim));
    context_.synchronize();
}

void Q8MatVecPipeline::run_staged(Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input,
                                  Buffer& staging_output, const void* host_input, std::size_t host_input_bytes,
                                  void* host_output, std::size_t host_output_bytes, std::uint32_t weight_byte_offset,
                                  std::uint32_t input_dim, std::uint32_t output_dim) {
    if (host_input == nullptr) throw std::runtime_error("Q8MatVecPipeline::run_staged received null host input");
    check_dims(input_dim, output_dim, weight_byte_offset);
    const std::uint64_t in_bytes = static_cast<std::uint64_t>(input_dim) * 4u;
    const std::uint64_t out_bytes = static_cast<std::uint64_t>(output_dim) * 4u;
    const bool readback = host_output != nullptr;
    if (weight_byte_offset + matrix_bytes(input_dim, output_dim) > weights.size() || in_bytes > input.size() ||
        out_bytes > output.size())
        throw std::runtime_error("Q8MatVecPipeline device buffer is too small");
    if (in_bytes > staging_input.size() || (readback && out_bytes > staging_output.size()))
        throw std::runtime_error("Q8MatVecPipeline staging buffer is too small");
    if (host_input_bytes < in_bytes || (readback && host_output_bytes < out_bytes))
        throw std::runtime_error("Q8MatVecPipeline host buffer is too small");
    input.upload(host_input, in_bytes);
    check_vrt(vrt_q8_matvec(context_.handle(), weights.handle(), weights.size(), weight_byte_offset,
                            static_cast<const float*>(input.handle()), static_cast<float*>(output.handle()), input_dim,
                            output_dim));
    if (readback) output.download(host_output, out_bytes);
    context_.synchronize();
}

void Q8MatVecPipeline::run_staged_ffn(Buffer& weights, Buffer& input, Buffer& workspace, Buffer& staging_input,
                                      Buffer& staging_output, const void* host_input, std::size_t host_input_bytes,
                                      void* host_output, std::size_t host_output_bytes,
                                      std::uint32_t gate_weight_byte_offset, std::uint32_t up_weight_byte_offset,
                                      std::uint32_t down_weight_byte_offset, std::uint32_t input_dim,
                                      std::uint32_t ffn_dim, std::uint32_t output_dim) {
    if (host_input == nullptr || host_output == nullptr)
        throw std::runtime_error("Q8MatVecPipeline::run_staged_ffn received null host buffer");
    if (input_dim == 0 || ffn_dim == 0 || output_dim == 0 || input_dim % 32u != 0 || ffn_dim % 32u != 0)
        throw std::runtime_error("Q8 fused FFN dimensions must be non-zero and Q8 aligned");
    if ((gate_weight_byte_offset & 3u) || (up_weight_byte_offset & 3u) || (down_weight_byte_offset & 3u))
        throw std::runtime_error("Q8 fused FFN weight offsets must be 4-byte aligned");
    if (gate_weight_byte_offset + matrix_bytes(input_dim, ffn_dim) > weights.size() ||
        up_weight_byte_offset + matrix_bytes(input_dim, ffn_dim) > weights.size() ||
        down_weight_byte_offset + matrix_bytes(ffn_dim, output_dim) > weights.size())
        throw std::runtime_error("Q8 fused FFN weight buffer is too small");
    const std::uint64_t in_bytes = static_cast<std::uint64_t>(input_dim) * 4u;
    const std::uint64_t ws_bytes = 2ull * ffn_dim * 4u;
    const std::uint64_t out_bytes = static_cast<std::uint64_t>(output_dim) * 4u;
    if (in_bytes > input.size() || in_bytes > staging_input.size() || host_input_bytes < in_bytes ||
        ws_bytes + out_bytes > workspace.size() || out_bytes > staging_output.size() || host_output_bytes < out_bytes)
        throw std::runtime_error("Q8 fused FFN activation/staging buffer is too small");
    input.upload(host_input, in_bytes);
    float* ws = static_cast<float*>(workspace.handle());
    check_vrt(vrt_q8_ffn(context_.handle(), weights.handle(), weights.size(), gate_weight_byte_offset,
                         up_weight_byte_offset, down_weight_byte_offset, input_dim, ffn_dim, output_dim,
                         static_cast<const float*>(input.handle()), ws, ws_bytes, ws + 2ull * ffn_dim));
    workspace.download(host_output, out_bytes, ws_bytes);
    context_.synchronize();
}

template <std::size_t N>
void Q8MatVecPipeline::run_multi(const char* what, Buffer& weights, Buffer& input, Buffer& output,
                                 Buffer& staging_input, Buffer& staging_output, const void* host_input,
                                 std::size_t host_input_bytes, void* host_output, std::size_t host_output_bytes,
                                 const std::array<std::uint32_t, N>& offsets, std::uint32_t input_dim,
                                 const std::array<std::uint32_t, N>& output_dims) {
    const std::string w(what);
    if (host_input == nullptr || host_output == nullptr)
        throw std::runtime_error("Q8MatVecPipeline::run_staged_" + w + " received null host buffer");
    if (input_dim == 0 || input_dim % 32u != 0)
        throw std::runtime_error("Q8MatVecPipeline " + w + " input_dim must be non-zero and divisible by 32");
    const std::uint64_t in_bytes = static_cast<std::uint64_t>(input_dim) * 4u;
    if (in_bytes > input.size() || in_bytes > staging_input.size() || host_input_bytes < in_bytes)
        throw std::runtime_error("Q8 " + w + " input buffer is too small");
    std::uint64_t total = 0;
    for (std::size_t i = 0; i < N; ++i) {
        if (output_dims[i] == 0) throw std::runtime_error("Q8 " + w + " output dimensions must be non-zero");
        if ((offsets[i] & 3u) != 0) throw std::runtime_error("Q8 " + w + " weight offsets must be 4-byte aligned");
        if (offsets[i] + matrix_bytes(input_dim, output_dims[i]) > weights.size())
            throw std::runtime_error("Q8 " + w + " weight buffer is too small");
        total += static_cast<std::uint64_t>(output_dims[i]) * 4u;
    }
    if (total > output.size() || total > staging_output.size() || host_output_bytes < total)
        throw std::runtime_error("Q8 " + w + " output buffer is too small");
    input.upload(host_input, in_bytes);
    check_vrt(vrt_q8_matvec_multi(context_.handle(), weights.handle(), weights.size(), static_cast<std::uint32_t>(N),
                                  offsets.data(), output_dims.data(), input_dim,
                                  static_cast<const float*>(input.handle()), static_cast<float*>(output.handle())));
    output.download(host_output, total);
    context_.synchronize();
}

void Q8MatVecPipeline::run_staged_pair(Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input,
                                       Buffer& staging_output, const void* host_input, std::size_t host_input_bytes,
                                       void* host_output, std::size_t host_output_bytes,
                                       const std::array<std::uint32_t, 2>& weight_byte_offsets,
                                       std::uint32_t input_dim, const std::array<std::uint32_t, 2>& output_dims) {
    run_multi<2>("pair", weights, input, output, staging_input, staging_output, host_input, host_input_bytes,
                 host_output, host_output_bytes, weight_byte_offsets, input_dim, output_dims);
}

void Q8MatVecPipeline::run_staged_triplet(Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input,
                                          Buffer& staging_output, const void* host_input,
                                          std::size_t host_input_bytes, void* host_output,
                                          std::size_t host_output_bytes,
                                          const std::array<std::uint32_t, 3>& weight_byte_offsets,
                                          std::uint32_t input_dim, const std::array<std::uint32_t, 3>& output_dims) {
    run_multi<3>("triplet", weights, input, output, staging_input, staging_output, host_input, host_input_bytes,
                 host_output, host_output_bytes, weight_byte_offsets, input_dim, output_dims);
}

// ---- ArgmaxPipeline -------------------------------------------------------------------------

ArgmaxPipeline::ArgmaxPipeline(DeviceContext& context, const std::string&) : context_(context) {}

void ArgmaxPipeline::run(Buffer& input, Buffer& output, std::uint32_t element_count) {
    if (element_count == 0) throw std::runtime_error("ArgmaxPipeline element count must be non-zero");
    if (static_cast<std::uint64_t>(element_count) * 4u > input.size())
        throw std::runtime_error("ArgmaxPipeline input buffer is too small");
    if (output.size() < sizeof(ArgmaxResult)) throw std::runtime_error("ArgmaxPipeline output buffer is too small");
    check_vrt(vrt_argmax(context_.handle(), static_cast<const float*>(input.handle()), element_count,
                         static_cast<vrt_argmax_result*>(output.handle())));
    context_.synchronize();
}

}  // namespace vortexrt
