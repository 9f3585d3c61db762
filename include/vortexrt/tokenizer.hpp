// Gemma 3 text tokenizer of the HIP build, host only. Vortex-RT keeps this inside
// Gemma3Model (index: src/gemma3.cpp:289-454; tokenize: :1920-2062; pieces: :1237-1299);
// here it is its own class, owned by Gemma3Model, so it can run without a device.
#pragma once

#include "vortexrt/gguf.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace vortexrt {

class Gemma3Tokenizer {
public:
    // Builds the piece index from tokenizer.ggml.{tokens, scores, token_type} (each exactly
    // vocab_size entries, else std::runtime_error "Gemma 3 tokenizer metadata is incomplete"),
    // the byte pieces <0xHH> (type 6), add_space_prefix, and the unknown / BOS / EOS ids
    // (defaults 3 / 2 / 1; a BOS id outside the vocabulary throws). The GgufFile must outlive
    // the tokenizer: the index points into its metadata strings.
    Gemma3Tokenizer(const GgufFile& gguf, std::uint32_t vocab_size);

    // Whitespace runs become one U+2581 marker (plus a leading marker when add_space_prefix
    // is set), then the highest-scoring segmentation into pieces (a byte piece, or the
    // unknown id, scores -100 where no piece starts), with BOS first when add_bos is set.
    [[nodiscard]] std::vector<std::uint32_t> tokenize(const std::string& text, bool add_bos) const;

    // The vocabulary string of an id ("" past the vocabulary).
    [[nodiscard]] std::string token_piece(std::uint32_t token_id) const;
    // Printable text of an id: control ids 0..3 print nothing, <0xHH> prints its byte and the
    // U+2581 marker prints as a space.
    [[nodiscard]] std::string decode_piece(std::uint32_t token_id) const;

    [[nodiscard]] std::uint32_t bos_id() const noexcept { return bos_id_; }
    [[nodiscard]] std::uint32_t eos_id() const noexcept { return eos_id_; }
    [[nodiscard]] std::uint32_t unknown_id() const noexcept { return unk_id_; }
    [[nodiscard]] bool add_space_prefix() const noexcept { return add_space_prefix_; }
    [[nodiscard]] std::size_t piece_count() const noexcept { return pieces_.size(); }

private:
    struct Entry {
        std::uint32_t id;
        float score;
    };
    const GgufValue* tokens_ = nullptr;
    std::unordered_map<std::string_view, Entry> pieces_;
    std::array<std::uint32_t, 256> byte_tokens_{};
    std::size_t max_piece_bytes_ = 0;
    bool add_space_prefix_ = false;
    std::uint32_t unk_id_ = 3;
    std::uint32_t bos_id_ = 2;
    std::uint32_t eos_id_ = 1;
};

}  // namespace vortexrt
