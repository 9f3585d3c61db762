// Gemma3Model over libvrt_hip.so: the host half of the constructor (GGUF metadata and tensor
// directory, src/gemma3.cpp:174-505), the arena upload, and the public methods
// (src/gemma3.cpp:1138-1300, :1454-1893, :2064-2166), each a call into the device executor.
#include "vortexrt/gemma3.hpp"

#include "vrt_hip.h"

#include <algorithm>
#include <cmath>
#include <limits>
#include <numeric>
#include <stdexcept>

namespace vortexrt {
namespace {

std::uint32_t require_u32(const GgufFile& f, const std::string& key) {
    const auto v = f.metadata_u64(key);
    if (!v || *v > std::numeric_limits<std::uint32_t>::max())
        throw std::runtime_error("Missing/invalid Gemma 3 metadata: " + key);
    return static_cast<std::uint32_t>(*v);
}

float require_f32(const GgufFile& f, const std::string& key) {
    const auto* v = f.find_metadata(key);
    if (v == nullptr) throw std::runtime_error("Missing Gemma 3 metadata: " + key);
    const auto x = v->as_f64();
    if (!x || !std::isfinite(*x)) throw std::runtime_error("Invalid Gemma 3 floating metadata: " + key);
    return static_cast<float>(*x);
}

const GgufTensorInfo& require_tensor(const GgufFile& f, const std::string& name, std::uint32_t type) {
    const auto* t = f.find_tensor(name);
    if (t == nullptr) throw std::runtime_error("Missing Gemma 3 tensor: " + name);
    if (t->type != type) throw std::runtime_error("Unsupported Gemma 3 tensor type: " + name);
    return *t;
}

}  // namespace

Gemma3Model::Gemma3Model(const std::string& gguf_path, DeviceContext& context, const std::string&, const std::string&,
                         const std::string&, const std::string&, const std::string&, const std::string&,
                         const std::string&, const std::string&, const std::string&, const std::string&,
                         std::uint32_t q8_lane_override)
    : gguf_(gguf_path), context_(context) {
    if (q8_lane_override != 0u && q8_lane_override != 8u && q8_lane_override != 16u && q8_lane_override != 32u &&
        q8_lane_override != 64u)
        throw std::runtime_error("Q8 lane override must be 0, 8, 16, 32, or 64");   // src/gemma3.cpp:163-166
    gguf_.validate();
    if (gguf_.metadata_string("general.architecture").value_or("") != "gemma3")
        throw std::runtime_error("Gemma3Model requires general.architecture=gemma3");
    config_.context_length = require_u32(gguf_, "gemma3.context_length");
    config_.embedding_length = require_u32(gguf_, "gemma3.embedding_length");
    config_.block_count = require_u32(gguf_, "gemma3.block_count");
    config_.feed_forward_length = require_u32(gguf_, "gemma3.feed_forward_length");
    config_.head_count = require_u32(gguf_, "gemma3.attention.head_count");
    config_.head_count_kv = require_u32(gguf_, "gemma3.attention.head_count_kv");
    config_.head_dim = require_u32(gguf_, "gemma3.attention.key_length");
    config_.value_dim = require_u32(gguf_, "gemma3.attention.value_length");
    config_.rms_epsilon = require_f32(gguf_, "gemma3.attention.layer_norm_rms_epsilon");
    if (const auto sw = gguf_.metadata_u64("gemma3.attention.sliding_window");
        sw && *sw <= std::numeric_limits<std::uint32_t>::max())
        config_.sliding_window = static_cast<std::uint32_t>(*sw);
    if (const auto* rope = gguf_.find_metadata("gemma3.rope.freq_base")) {
        if (const auto x = rope->as_f64(); x && std::isfinite(*x) && *x > 0.0)
            config_.global_rope_base = static_cast<float>(*x);
    }
    const auto& emb = require_tensor(gguf_, "token_embd.weight", 8);
    if (emb.dimensions.size() != 2 || emb.dimensions[0] != config_.embedding_length ||
        emb.dimensions[1] > std::numeric_limits<std::uint32_t>::max())
        throw std::runtime_error("Unsupported token_embd.weight layout");
    config_.vocab_size = static_cast<std::uint32_t>(emb.dimensions[1]);
    // the tokenizer index (src/gemma3.cpp:289-454): incomplete metadata fails the load
    tokenizer_ = std::make_unique<Gemma3Tokenizer>(gguf_, config_.vocab_size);
    tokenizer_bos_id_ = tokenizer_->bos_id();
    tokenizer_eos_id_ = tokenizer_->eos_id();

    // arena: the whole tensor-data section, uploaded in chunks
    const std::uint64_t arena_bytes = gguf_.file_size() - gguf_.data_offset();
    if (arena_bytes == 0) throw std::runtime_error("Gemma 3 GGUF has no tensor data");
    weights_arena_ = std::make_unique<Buffer>(context_, arena_bytes, kBufferUsageStorage, kMemoryDeviceLocal);
    {
        constexpr std::uint64_t kChunk = 64ull << 20;
        std::vector<unsigned char> chunk(static_cast<std::size_t>(std::min(kChunk, arena_bytes)));
        for (std::uint64_t o = 0; o < arena_bytes; o += kChunk) {
            const auto n = static_cast<std::size_t>(std::min(kChunk, arena_bytes - o));
            gguf_.read_data(o, chunk.data(), n);
            weights_arena_->upload(chunk.data(), n, o);
        }
    }

    // executor description: Q8_0 offsets into the arena, F32 norm weights on the host
    std::vector<std::vector<float>> keep;
    auto f32 = [&](const std::string& name) {
        keep.push_back(gguf_.read_f32_tensor(require_tensor(gguf_, name, 0)));
        return keep.back().data();
    };
    std::vector<vrt_g3_layer> layers(config_.block_count);
    keep.reserve(6u * config_.block_count + 1u);
    for (std::uint32_t l = 0; l < config_.block_count; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        vrt_g3_layer& L = layers[l];
        L.attn_q = require_tensor(gguf_, p + "attn_q.weight", 8).offset;
        L.attn_k = require_tensor(gguf_, p + "attn_k.weight", 8).offset;
        L.attn_v = require_tensor(gguf_, p + "attn_v.weight", 8).offset;
        L.attn_output = require_tensor(gguf_, p + "attn_output.weight", 8).offset;
        L.ffn_gate = require_tensor(gguf_, p + "ffn_gate.weight", 8).offset;
        L.ffn_up = require_tensor(gguf_, p + "ffn_up.weight", 8).offset;
        L.ffn_down = require_tensor(gguf_, p + "ffn_down.weight", 8).offset;
        L.attn_norm = f32(p + "attn_norm.weight");
        L.attn_q_norm = f32(p + "attn_q_norm.weight");
        L.attn_k_norm = f32(p + "attn_k_norm.weight");
        L.post_attention_norm = f32(p + "post_attention_norm.weight");
        L.ffn_norm = f32(p + "ffn_norm.weight");
        L.post_ffw_norm = f32(p + "post_ffw_norm.weight");
    }
    vrt_g3_desc d{};
    d.config.context_length = config_.context_length;
    d.config.embedding_length = config_.embedding_length;
    d.config.block_count = config_.block_count;
    d.config.feed_forward_length = config_.feed_forward_length;
    d.config.head_count = config_.head_count;
    d.config.head_count_kv = config_.head_count_kv;
    d.config.head_dim = config_.head_dim;
    d.config.value_dim = config_.value_dim;
    d.config.vocab_size = config_.vocab_size;
    d.config.sliding_window = config_.sliding_window;
    d.config.rms_epsilon = config_.rms_epsilon;
    d.config.global_rope_base = config_.global_rope_base;
    d.config.local_rope_base = config_.local_rope_base;
    d.arena = weights_arena_->handle();
    d.arena_bytes = arena_bytes;
    d.token_embd = emb.offset;
    d.output_norm = f32("output_norm.weight");
    d.layers = layers.data();
    d.eos_token_id = tokenizer_eos_id_;
    check_vrt(vrt_g3_create(context_.handle(), &d, &g3_));
    if (q8_lane_override != 0u && vrt_g3_set_option(g3_, VRT_G3_OPT_Q8_LANES, q8_lane_override) != VRT_OK) {
        const std::string msg = vrt_last_error();   // the destructor does not run for a throwing constructor
        vrt_g3_destroy(g3_);
        g3_ = nullptr;
        throw std::runtime_error(msg);
    }
}

Gemma3Model::~Gemma3Model() {
    if (g3_) vrt_g3_destroy(g3_);
}

bool Gemma3Model::projection_fusion_enabled() const noexcept {
    std::uint32_t v = 1;
    return vrt_g3_get_option(g3_, VRT_G3_OPT_FUSION, &v) != VRT_OK || v != 0u;
}

void Gemma3Model::set_projection_fusion_enabled(bool enabled) noexcept {
    (void)vrt_g3_set_option(g3_, VRT_G3_OPT_FUSION, enabled ? 1u : 0u);
}

std::uint32_t Gemma3Model::narrow_q8_lane_count() const noexcept {
    std::uint32_t v = 0;
    return vrt_g3_get_option(g3_, VRT_G3_OPT_QUERY_Q8_LANES, &v) == VRT_OK ? v : 0u;
}

void Gemma3Model::reset_cache() { check_vrt(vrt_g3_reset(g3_)); }

Gemma3SingleTokenResult Gemma3Model::decode_token(std::uint32_t token_id, std::uint32_t position, std::size_t top_k) {
    Gemma3SingleTokenResult r;
    r.hidden.resize(config_.embedding_length);
    vrt_argmax_result best{};
    const auto k = static_cast<std::uint32_t>(std::min<std::size_t>(top_k, config_.vocab_size));
    check_vrt(vrt_g3_decode(g3_, token_id, position, k, &best, r.hidden.data()));
    if (k == 1) {
        r.top_tokens.push_back(Gemma3TopToken{best.index, best.value, token_piece(best.index)});
    } else if (k > 1) {   // src/gemma3.cpp:1187-1234: host partial sort of the logits
        std::vector<float> logits(config_.vocab_size);
        check_vrt(vrt_g3_logits(g3_, logits.data(), config_.vocab_size));
        std::vector<std::uint32_t> ids(logits.size());
        std::iota(ids.begin(), ids.end(), 0u);
        std::partial_sort(ids.begin(), ids.begin() + k, ids.end(),
                          [&](std::uint32_t a, std::uint32_t b) { return logits[a] > logits[b]; });
        r.top_tokens.reserve(k);
        for (std::uint32_t i = 0; i < k; ++i) {
            const auto id = ids[i];
            if (!std::isfinite(logits[id])) {
                reset_cache();
                throw std::runtime_error("Non-finite Gemma 3 logit");
            }
            r.top_tokens.push_back(Gemma3TopToken{id, logits[id], token_piece(id)});
        }
    }
    return r;
}

Gemma3SingleTokenResult Gemma3Model::run_single_token(std::uint32_t token_id, std::size_t top_k) {
    reset_cache();
    auto r = decode_token(token_id, 0, top_k);
    reset_cache();
    return r;
}

std::vector<std::uint32_t> Gemma3Model::tokenize(const std::string& text, bool add_bos) const {
    return tokenizer_->tokenize(text, add_bos);
}

Gemma3GenerationResult Gemma3Model::generate_greedy(const std::string& prompt, std::size_t max_new_tokens) {
    if (max_new_tokens == 0) {
        reset_cache();
        return {};
    }
    return generate_greedy_tokens(tokenize(prompt, true), max_new_tokens);
}

Gemma3GenerationResult Gemma3Model::generate_greedy_tokens(const std::vector<std::uint32_t>& prompt_tokens,
                                                           std::size_t max_new_tokens) {
    Gemma3GenerationResult out;
    if (max_new_tokens == 0) {
        reset_cache();
        return out;
    }
    if (prompt_tokens.empty()) {
        reset_cache();
        throw std::runtime_error("Gemma 3 prompt produced no input tokens");
    }
    if (max_new_tokens > std::numeric_limits<std::uint32_t>::max() ||
        prompt_tokens.size() > std::numeric_limits<std::uint32_t>::max())
        throw std::runtime_error("Gemma 3 context length exceeded");
    out.token_ids.resize(max_new_tokens);
    std::uint32_t n = 0;
    check_vrt(vrt_g3_generate(g3_, prompt_tokens.data(), static_cast<std::uint32_t>(prompt_tokens.size()),
                              static_cast<std::uint32_t>(max_new_tokens), out.token_ids.data(), &n));
    out.token_ids.resize(n);
    for (const auto id : out.token_ids)
        if (id != tokenizer_eos_id_) out.text += decode_piece(id);
    return out;
}

Gemma3GenerationResult Gemma3Model::generate_greedy_from_bos(std::size_t max_new_tokens) {
    if (max_new_tokens == 0) {
        reset_cache();
        return {};
    }
    return generate_greedy_tokens(std::vector<std::uint32_t>{tokenizer_bos_id_}, max_new_tokens);
}

std::string Gemma3Model::token_piece(std::uint32_t token_id) const { return tokenizer_->token_piece(token_id); }

// Control ids 0..3 print nothing, <0xNN> byte pieces print their byte, and the SentencePiece
// space marker U+2581 prints as a space (src/gemma3.cpp:1251-1299).
std::string Gemma3Model::decode_piece(std::uint32_t token_id) const { return tokenizer_->decode_piece(token_id); }

}  // namespace vortexrt
