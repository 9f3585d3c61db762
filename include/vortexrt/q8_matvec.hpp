// Q8_0 matrix-vector products (include/vortexrt/q8_matvec.hpp:15-100 of Vortex-RT).
// Weights are GGUF Q8_0 rows: input_dim/32 blocks of 34 bytes {f16 scale, int8[32]}.
#pragma once

#include "vortexrt/buffer.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>

namespace vortexrt {

class Q8MatVecPipeline {
public:
    // The shader paths are accepted for signature compatibility; the kernels are built in
    // (wave64 gfx950 code, one variant per row width).
    Q8MatVecPipeline(DeviceContext& context, const std::string& spirv_path = {}, const std::string& u8_spirv_path = {},
                     const std::string& gelu_mul_spirv_path = {});
    ~Q8MatVecPipeline() = default;

    Q8MatVecPipeline(const Q8MatVecPipeline&) = delete;
    Q8MatVecPipeline& operator=(const Q8MatVecPipeline&) = delete;

    // Byte loads are native on gfx950, and the fused FFN is always available.
    [[nodiscard]] bool using_native_u8() const noexcept { return true; }
    [[nodiscard]] bool ffn_available() const noexcept { return true; }

    // output[0..output_dim) = W x with W at weight_byte_offset of weights. Synchronous.
    void run(Buffer& weights, Buffer& input, Buffer& output, std::uint32_t weight_byte_offset, std::uint32_t input_dim,
             std::uint32_t output_dim);

    // host_input -> input, run, output -> host_output (skipped when host_output is null).
    // The staging buffers are checked for size as the reference does; the copies go
    // directly between host memory and the device buffers.
    void run_staged(Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input, Buffer& staging_output,
                    const void* host_input, std::size_t host_input_bytes, void* host_output,
                    std::size_t host_output_bytes, std::uint32_t weight_byte_offset, std::uint32_t input_dim,
                    std::uint32_t output_dim);

    // gate = Wg x, up = Wu x, h = gelu_tanh(gate) * up, out = Wd h. workspace holds
    // [gate | up | out] (2 * ffn_dim + output_dim floats); out is copied to host_output.
    void run_staged_ffn(Buffer& weights, Buffer& input, Buffer& workspace, Buffer& staging_input,
                        Buffer& staging_output, const void* host_input, std::size_t host_input_bytes,
                        void* host_output, std::size_t host_output_bytes, std::uint32_t gate_weight_byte_offset,
                        std::uint32_t up_weight_byte_offset, std::uint32_t down_weight_byte_offset,
                        std::uint32_t input_dim, std::uint32_t ffn_dim, std::uint32_t output_dim);

    // Two / three matrices sharing x; outputs packed contiguously in call order.
    void run_staged_pair(Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input,
                         Buffer& staging_output, const void* host_input, std::size_t host_input_bytes,
                         void* host_output, std::size_t host_output_bytes,
                         const std::array<std::uint32_t, 2>& weight_byte_offsets, std::uint32_t input_dim,
                         const std::array<std::uint32_t, 2>& output_dims);

    void run_staged_triplet(Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input,
                            Buffer& staging_output, const void* host_input, std::size_t host_input_bytes,
                            void* host_output, std::size_t host_output_bytes,
                            const std::array<std::uint32_t, 3>& weight_byte_offsets, std::uint32_t input_dim,
                            const std::array<std::uint32_t, 3>& output_dims);

private:
    template <std::size_t N>
    void run_multi(const char* what, Buffer& weights, Buffer& input, Buffer& output, Buffer& staging_input,
                   Buffer& staging_output, const void* host_input, std::size_t host_input_bytes, void* host_output,
                   std::size_t host_output_bytes, const std::array<std::uint32_t, N>& offsets,
                   std::uint32_t input_dim, const std::array<std::uint32_t, N>& output_dims);

    DeviceContext& context_;
};

}  // namespace vortexrt
