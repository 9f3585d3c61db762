// Gemma3Tokenizer: the piece index and the Viterbi segmentation of Gemma3Model's tokenizer
// (src/gemma3.cpp:289-454, :1920-2062), the piece printing of :1237-1299.
#include "vortexrt/tokenizer.hpp"

#include <algorithm>
#include <cmath>
#include <limits>
#include <stdexcept>

namespace vortexrt {
namespace {

constexpr std::string_view kMarker = "\xE2\x96\x81";   // U+2581, the SentencePiece space
constexpr std::uint32_t kNone = std::numeric_limits<std::uint32_t>::max();

int hex_digit(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

// The byte of a "<0xHH>" piece, or -1.
int byte_piece(const std::string& p) {
    if (p.size() != 6 || p[0] != '<' || p[1] != '0' || p[2] != 'x' || p[5] != '>') return -1;
    const int hi = hex_digit(p[3]), lo = hex_digit(p[4]);
    return hi < 0 || lo < 0 ? -1 : (hi << 4) | lo;
}

}  // namespace

Gemma3Tokenizer::Gemma3Tokenizer(const GgufFile& gguf, std::uint32_t vocab_size) {
    const GgufValue* tokens = gguf.find_metadata("tokenizer.ggml.tokens");
    const GgufValue* scores = gguf.find_metadata("tokenizer.ggml.scores");
    const GgufValue* types = gguf.find_metadata("tokenizer.ggml.token_type");
    if (tokens == nullptr || scores == nullptr || types == nullptr || !tokens->is_array() || !scores->is_array() ||
        !types->is_array() || tokens->array.size() != vocab_size || scores->array.size() != vocab_size ||
        types->array.size() != vocab_size)
        throw std::runtime_error("Gemma 3 tokenizer metadata is incomplete");
    tokens_ = tokens;
    byte_tokens_.fill(kNone);
    pieces_.reserve(vocab_size);
    for (std::uint32_t id = 0; id < vocab_size; ++id) {
        const auto* piece = std::get_if<std::string>(&tokens->array[id].scalar);
        const auto score = scores->array[id].as_f64();
        const auto type = types->array[id].as_i64();
        if (piece == nullptr || !score || !type) continue;
        if (*type == 6) {   // byte piece: the last id of a byte wins
            if (const int b = byte_piece(*piece); b >= 0) {
                byte_tokens_[static_cast<std::size_t>(b)] = id;
                continue;
            }
        }
        if (*type != 1 && *type != 4) continue;   // normal and user-defined pieces only
        const float s = static_cast<float>(*score);
        const std::string_view key(*piece);
        const auto it = pieces_.find(key);
        if (it == pieces_.end() || s > it->second.score) pieces_[key] = Entry{id, s};   // ties: lowest id
        max_piece_bytes_ = std::max(max_piece_bytes_, piece->size());
    }
    if (const auto* v = gguf.find_metadata("tokenizer.ggml.add_space_prefix")) add_space_prefix_ = v->as_bool().value_or(false);
    const auto unk = gguf.metadata_u64("tokenizer.ggml.unknown_token_id").value_or(3);
    unk_id_ = static_cast<std::uint32_t>(std::min<std::uint64_t>(unk, vocab_size - 1u));
    const auto bos = gguf.metadata_u64("tokenizer.ggml.bos_token_id").value_or(2);
    if (bos >= vocab_size) throw std::runtime_error("Gemma 3 BOS token id is out of range");
    bos_id_ = static_cast<std::uint32_t>(bos);
    const auto eos = gguf.metadata_u64("tokenizer.ggml.eos_token_id").value_or(1);
    eos_id_ = static_cast<std::uint32_t>(std::min<std::uint64_t>(eos, kNone));
}

std::vector<std::uint32_t> Gemma3Tokenizer::tokenize(const std::string& text, bool add_bos) const {
    if (tokens_ == nullptr || pieces_.empty()) throw std::runtime_error("Gemma 3 tokenizer index is unavailable");
    // whitespace runs -> one marker
    std::string s;
    s.reserve(text.size() + kMarker.size());
    bool in_space = false;
    for (const char c : text) {
        if (c == ' ' || c == '\t' || c == '\r' || c == '\n') {
            if (!in_space) s += kMarker;
            in_space = true;
        } else {
            s += c;
            in_space = false;
        }
    }
    if (add_space_prefix_ && !s.empty() && s.compare(0, kMarker.size(), kMarker) != 0) s.insert(0, kMarker);

    // best[i]: the highest fp32 score of a segmentation of s[0, i); a later candidate replaces
    // an earlier one only when strictly better
    const std::size_t n = s.size();
    std::vector<float> best(n + 1, -std::numeric_limits<float>::infinity());
    std::vector<std::size_t> from(n + 1, std::numeric_limits<std::size_t>::max());
    std::vector<std::uint32_t> via(n + 1, kNone);
    best[0] = 0.0f;
    const std::string_view sv(s);
    for (std::size_t i = 0; i < n; ++i) {
        if (!std::isfinite(best[i])) continue;
        bool any = false;
        const std::size_t longest = std::min(max_piece_bytes_, n - i);
        for (std::size_t len = 1; len <= longest; ++len) {
            const auto it = pieces_.find(sv.substr(i, len));
            if (it == pieces_.end()) continue;
            any = true;
            const float cand = best[i] + it->second.score;
            if (cand > best[i + len]) {
                best[i + len] = cand;
                from[i + len] = i;
                via[i + len] = it->second.id;
            }
        }
        if (!any) {   // no piece starts here: the byte's piece, or the unknown id
            std::uint32_t id = byte_tokens_[static_cast<unsigned char>(s[i])];
            if (id == kNone) id = unk_id_;
            const float cand = best[i] - 100.0f;
            if (cand > best[i + 1]) {
                best[i + 1] = cand;
                from[i + 1] = i;
                via[i + 1] = id;
            }
        }
    }
    if (n != 0 && !std::isfinite(best[n])) throw std::runtime_error("Gemma 3 tokenizer could not segment prompt");
    std::vector<std::uint32_t> out;
    for (std::size_t at = n; at != 0; at = from[at]) {
        if (from[at] == std::numeric_limits<std::size_t>::max() || via[at] == kNone)
            throw std::runtime_error("Gemma 3 tokenizer backtracking failed");
        out.push_back(via[at]);
    }
    if (add_bos) out.push_back(bos_id_);
    std::reverse(out.begin(), out.end());
    return out;
}

std::string Gemma3Tokenizer::token_piece(std::uint32_t token_id) const {
    if (tokens_ == nullptr || token_id >= tokens_->array.size()) return {};
    return tokens_->array[token_id].as_string().value_or(std::string{});
}

std::string Gemma3Tokenizer::decode_piece(std::uint32_t token_id) const {
    if (token_id <= 3u) return {};
    const std::string piece = token_piece(token_id);
    if (const int b = byte_piece(piece); b >= 0) return std::string(1, static_cast<char>(b));
    std::string out;
    out.reserve(piece.size());
    for (std::size_t i = 0; i < piece.size();) {
        if (piece.compare(i, kMarker.size(), kMarker) == 0) {
            out += ' ';
            i += kMarker.size();
        } else {
            out += piece[i++];
        }
    }
    return out;
}

}  // namespace vortexrt
