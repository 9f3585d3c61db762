// Gemma 3 executor (include/vortexrt/gemma3.hpp:17-117 of Vortex-RT): the same public surface,
// running the MI355X decode path of libvrt_hip.so.
#pragma once

#include "vortexrt/argmax.hpp"
#include "vortexrt/gguf.hpp"
#include "vortexrt/q8_matvec.hpp"
#include "vortexrt/tokenizer.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

struct vrt_g3;

namespace vortexrt {

struct Gemma3Config {
    std::uint32_t context_length = 0;
    std::uint32_t embedding_length = 0;
    std::uint32_t block_count = 0;
    std::uint32_t feed_forward_length = 0;
    std::uint32_t head_count = 0;
    std::uint32_t head_count_kv = 0;
    std::uint32_t head_dim = 0;
    std::uint32_t value_dim = 0;
    std::uint32_t vocab_size = 0;
    std::uint32_t sliding_window = 0;
    float rms_epsilon = 1.0e-6f;
    float global_rope_base = 1.0e6f;
    float local_rope_base = 1.0e4f;
};

struct Gemma3TopToken {
    std::uint32_t token_id = 0;
    float logit = 0.0f;
    std::string piece;
};

struct Gemma3SingleTokenResult {
    std::vector<float> hidden;
    std::vector<Gemma3TopToken> top_tokens;
};

struct Gemma3GenerationResult {
    std::vector<std::uint32_t> token_ids;
    std::string text;
};

class Gemma3Model {
public:
    // The shader paths are accepted for signature compatibility (the kernels are built in);
    // q8_lane_override must be 0, 8, 16, 32 or 64 (see narrow_q8_lane_count()).
    Gemma3Model(const std::string& gguf_path, DeviceContext& context, const std::string& q8_matvec_spirv = {},
                const std::string& q8_matvec_u8_spirv = {}, const std::string& argmax_spirv = {},
                const std::string& q8_matvec_32_spirv = {}, const std::string& q8_matvec_u8_32_spirv = {},
                const std::string& gelu_mul_spirv = {}, const std::string& q8_matvec_16_spirv = {},
                const std::string& q8_matvec_u8_16_spirv = {}, const std::string& q8_matvec_8_spirv = {},
                const std::string& q8_matvec_u8_8_spirv = {}, std::uint32_t q8_lane_override = 0);
    ~Gemma3Model();

    Gemma3Model(const Gemma3Model&) = delete;
    Gemma3Model& operator=(const Gemma3Model&) = delete;

    [[nodiscard]] const Gemma3Config& config() const noexcept { return config_; }

    // Lane and fusion policy (src/gemma3.cpp:94-172, :656-671). Fusion is on by default (the
    // reference's rule for GPU devices); off, every step runs the unfused sequence: q, k, v, gate
    // and up as separate matvec launches and the GELU product as its own launch
    // (:1529-1541, :1783-1847). A q8_lane_override of 8, 16, 32 or 64 runs the projections'
    // rows in slots of that many lanes (a 2048-input row needs at least 16); 0 sizes the slots
    // per matrix. narrow_q8_lane_count() reports the lanes per row the embedding-width
    // projections run with. Neither setting changes results beyond the parity tolerances.
    [[nodiscard]] bool projection_fusion_enabled() const noexcept;
    void set_projection_fusion_enabled(bool enabled) noexcept;
    [[nodiscard]] std::uint32_t narrow_q8_lane_count() const noexcept;
    [[nodiscard]] bool fused_ffn_enabled() const noexcept { return projection_fusion_enabled(); }

    // reset_cache(); decode_token(token_id, 0, top_k); reset_cache() (src/gemma3.cpp:1884-1893).
    [[nodiscard]] Gemma3SingleTokenResult run_single_token(std::uint32_t token_id, std::size_t top_k = 8);

    void reset_cache();

    // One step at `position` (positions must be contiguous from 0). top_k = 0 skips the LM
    // head; 1 is the fused device argmax; > 1 sorts the logits on the host. On error the
    // cache is reset and std::runtime_error is thrown.
    [[nodiscard]] Gemma3SingleTokenResult decode_token(std::uint32_t token_id, std::uint32_t position,
                                                       std::size_t top_k = 1);

    // Whitespace-normalised highest-scoring segmentation into vocabulary pieces, BOS first
    // when add_bos (src/gemma3.cpp:1920-2062); see Gemma3Tokenizer.
    [[nodiscard]] std::vector<std::uint32_t> tokenize(const std::string& text, bool add_bos = true) const;
    [[nodiscard]] Gemma3GenerationResult generate_greedy(const std::string& prompt, std::size_t max_new_tokens);

    // The whole loop runs on the device (src/gemma3.cpp:2080-2149 semantics: n + N - 1 steps,
    // EOS appended then generation stops); text holds the decoded pieces before EOS.
    [[nodiscard]] Gemma3GenerationResult generate_greedy_tokens(const std::vector<std::uint32_t>& prompt_tokens,
                                                                std::size_t max_new_tokens);
    [[nodiscard]] Gemma3GenerationResult generate_greedy_from_bos(std::size_t max_new_tokens);

    // The executor handle of the C ABI (vrt_hip.h), for options and diagnostics.
    [[nodiscard]] vrt_g3* handle() const noexcept { return g3_; }

private:
    [[nodiscard]] std::string token_piece(std::uint32_t token_id) const;
    [[nodiscard]] std::string decode_piece(std::uint32_t token_id) const;

    GgufFile gguf_;
    DeviceContext& context_;
    Gemma3Config config_{};
    std::unique_ptr<Buffer> weights_arena_;
    vrt_g3* g3_ = nullptr;
    std::unique_ptr<Gemma3Tokenizer> tokenizer_;
    std::uint32_t tokenizer_bos_id_ = 2;
    std::uint32_t tokenizer_eos_id_ = 1;
};

}  // namespace vortexrt
