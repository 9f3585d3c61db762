// vortexrt-gemma: the command line of Vortex-RT's Gemma 3 runtime (src/gemma_main.cpp) on the
// HIP build. Same options and the same report lines, so scripts that grep the reference's
// output ("Layers:", "Final hidden checksum:", "Top logits:", "Prompt token ids:",
// "Generated token ids:", "TEXT_BEGIN", "TEXT_END", "Validation: OK") run unchanged.
//
//   vortexrt-gemma model.gguf [--token-id N] [--top-k N] [--prompt TEXT] [--generate N]
//                  [--projection-fusion auto|on|off] [--q8-lanes auto|8|16|32|64]
//                  [--device <index|name>]
//
// Without --generate: one forward pass of --token-id at position 0 (default 2, BOS) with the
// final hidden state's RMS, max |x| and checksum sum_i x_i * (i + 1), and the top-k logits
// (k = 0 skips the LM head). With --generate N (at most 128): --prompt is tokenized with BOS
// (an empty prompt is BOS alone) and N tokens are generated greedily with the KV cache.
#include "vortexrt/build_config.hpp"
#include "vortexrt/gemma3.hpp"
#include "vortexrt/vulkan_context.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <exception>
#include <iomanip>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>

namespace {

struct Options {
    std::string model_path;
    std::string device;
    std::string prompt;
    std::uint32_t token_id = 2;
    std::size_t top_k = 8;
    std::size_t generate_tokens = 0;
    std::string projection_fusion = "auto";
    std::uint32_t q8_lanes = 0;
};

constexpr const char* kUsage =
    "usage: vortexrt-gemma <model.gguf> [options]\n"
    "  --token-id N          input token id (default: 2/BOS)\n"
    "  --top-k N             display top logits; 0 skips LM head\n"
    "  --prompt TEXT         tokenize/prefill a text prompt before generation\n"
    "  --generate N          greedy-generate N tokens with KV cache\n"
    "  --projection-fusion auto|on|off\n"
    "                        override QKV/FFN projection fusion policy\n"
    "  --q8-lanes auto|8|16|32|64\n"
    "                        override narrow Q8 workgroup width\n"
    "  --device <index|name> GPU selector (index or name substring)\n";

unsigned long long parse_unsigned(const std::string& text, const char* option, unsigned long long max,
                                  const char* what) {
    std::size_t used = 0;
    unsigned long long v = 0;
    try {
        v = std::stoull(text, &used, 10);
    } catch (const std::exception&) {
        used = 0;
    }
    if (text.empty() || used != text.size() || text[0] == '-' || v > max)
        throw std::runtime_error(std::string(option) + what);
    return v;
}

Options parse_options(int argc, char** argv) {
    if (argc < 2)
        throw std::runtime_error(
            "usage: vortexrt-gemma <model.gguf> [--token-id N] [--top-k N] [--generate N] "
            "[--projection-fusion auto|on|off] [--q8-lanes auto|8|16|32|64] [--device <index|name>]");
    Options o{};
    o.model_path = argv[1];
    for (int i = 2; i < argc; ++i) {
        const std::string arg = argv[i];
        auto value = [&](const char* name) -> std::string {
            if (i + 1 >= argc) throw std::runtime_error(std::string(name) + " requires a value");
            return argv[++i];
        };
        if (arg == "--token-id") {
            o.token_id = static_cast<std::uint32_t>(
                parse_unsigned(value("--token-id"), "--token-id", std::numeric_limits<std::uint32_t>::max(), " must be a uint32"));
        } else if (arg == "--top-k") {
            o.top_k = parse_unsigned(value("--top-k"), "--top-k", std::numeric_limits<std::size_t>::max(), " is out of range");
        } else if (arg == "--prompt") {
            o.prompt = value("--prompt");
        } else if (arg == "--generate") {
            o.generate_tokens =
                parse_unsigned(value("--generate"), "--generate", std::numeric_limits<std::size_t>::max(), " is out of range");
            if (o.generate_tokens > 128) throw std::runtime_error("--generate is capped at 128 during bring-up");
        } else if (arg == "--projection-fusion") {
            o.projection_fusion = value("--projection-fusion");
            if (o.projection_fusion != "auto" && o.projection_fusion != "on" && o.projection_fusion != "off")
                throw std::runtime_error("--projection-fusion must be auto, on, or off");
        } else if (arg == "--q8-lanes") {
            const std::string lanes = value("--q8-lanes");
            if (lanes == "auto") {
                o.q8_lanes = 0;
            } else {
                o.q8_lanes = static_cast<std::uint32_t>(
                    parse_unsigned(lanes, "--q8-lanes", std::numeric_limits<std::uint32_t>::max(), " must be a uint32"));
                if (o.q8_lanes != 8u && o.q8_lanes != 16u && o.q8_lanes != 32u && o.q8_lanes != 64u)
                    throw std::runtime_error("--q8-lanes must be auto, 8, 16, 32, or 64");
            }
        } else if (arg == "--device") {
            o.device = value("--device");
        } else if (arg == "--help" || arg == "-h") {
            std::cout << kUsage;
            std::exit(0);
        } else {
            throw std::runtime_error("unknown argument: " + arg);
        }
    }
    return o;
}

// Printable form of a piece: \n, \r, \t and bytes outside [0x20, 0x7e] escaped.
std::string escape_piece(const std::string& piece) {
    std::ostringstream out;
    for (const unsigned char c : piece) {
        if (c == '\n') {
            out << "\\n";
        } else if (c == '\r') {
            out << "\\r";
        } else if (c == '\t') {
            out << "\\t";
        } else if (c >= 0x20 && c < 0x7f) {
            out << static_cast<char>(c);
        } else {
            out << "\\x" << std::hex << std::setw(2) << std::setfill('0') << static_cast<unsigned>(c) << std::dec
                << std::setfill(' ');
        }
    }
    return out.str();
}

double ms_since(std::chrono::steady_clock::time_point t0, std::chrono::steady_clock::time_point t1) {
    return std::chrono::duration<double, std::milli>(t1 - t0).count();
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const Options opt = parse_options(argc, argv);
        const auto t_runtime = std::chrono::steady_clock::now();
        vortexrt::VulkanContext context(opt.device);
        const auto t_model = std::chrono::steady_clock::now();
        namespace bc = vortexrt::build_config;
        vortexrt::Gemma3Model model(opt.model_path, context, bc::q8_matvec_spv, bc::q8_matvec_u8_spv, bc::argmax_spv,
                                    bc::q8_matvec_32_spv, bc::q8_matvec_u8_32_spv, bc::gelu_mul_spv, bc::q8_matvec_16_spv,
                                    bc::q8_matvec_u8_16_spv, bc::q8_matvec_8_spv, bc::q8_matvec_u8_8_spv, opt.q8_lanes);
        if (opt.projection_fusion == "on") model.set_projection_fusion_enabled(true);
        if (opt.projection_fusion == "off") model.set_projection_fusion_enabled(false);
        const auto t_ready = std::chrono::steady_clock::now();
        const auto& c = model.config();
        std::cout << "Vortex-RT Gemma 3 runtime\n"
                  << "  GPU: " << context.capabilities().name << "\n"
                  << "  Layers: " << c.block_count << "\n"
                  << "  Hidden: " << c.embedding_length << "\n"
                  << "  FFN: " << c.feed_forward_length << "\n"
                  << "  Heads: " << c.head_count << " / KV " << c.head_count_kv << "\n"
                  << "  Head dim: " << c.head_dim << "\n"
                  << "  Sliding window: " << c.sliding_window << "\n"
                  << "  Vocab: " << c.vocab_size << "\n"
                  << "  Narrow Q8 kernel: " << model.narrow_q8_lane_count() << " lanes\n"
                  << "  Projection fusion: " << (model.projection_fusion_enabled() ? "enabled" : "disabled") << "\n"
                  << "  Fused FFN: " << (model.fused_ffn_enabled() ? "enabled" : "disabled") << "\n"
                  << "  Model load: " << ms_since(t_model, t_ready) << " ms\n"
                  << "  Runtime setup: " << ms_since(t_runtime, t_ready) << " ms\n";

        if (opt.generate_tokens != 0) {
            std::cout << "  Greedy generation from BOS: " << opt.generate_tokens << " token(s)\n";
            const auto prompt = model.tokenize(opt.prompt, true);
            std::cout << "  Prompt token ids:";
            for (const auto id : prompt) std::cout << " " << id;
            std::cout << "\n";
            const auto t0 = std::chrono::steady_clock::now();
            const auto gen = model.generate_greedy_tokens(prompt, opt.generate_tokens);
            const double ms = ms_since(t0, std::chrono::steady_clock::now());
            std::cout << "  Generated token ids:";
            for (const auto id : gen.token_ids) std::cout << " " << id;
            std::cout << "\n"
                      << "  Generation time: " << ms << " ms\n"
                      << "  Throughput: " << (ms > 0.0 ? static_cast<double>(gen.token_ids.size()) * 1000.0 / ms : 0.0)
                      << " tok/s\n"
                      << "  Generated text: \"" << escape_piece(gen.text) << "\"\n"
                      << "TEXT_BEGIN\n"
                      << gen.text << "\nTEXT_END\n"
                      << "  Validation: OK\n";
            return 0;
        }

        std::cout << "  Token: " << opt.token_id << "\n";
        const auto t0 = std::chrono::steady_clock::now();
        const auto r = model.run_single_token(opt.token_id, opt.top_k);
        const double ms = ms_since(t0, std::chrono::steady_clock::now());
        double checksum = 0.0, sum_sq = 0.0;
        float max_abs = 0.0f;
        for (std::size_t i = 0; i < r.hidden.size(); ++i) {
            const float v = r.hidden[i];
            if (!std::isfinite(v)) throw std::runtime_error("final hidden state is non-finite");
            checksum += static_cast<double>(v) * static_cast<double>(i + 1);
            sum_sq += static_cast<double>(v) * static_cast<double>(v);
            max_abs = std::max(max_abs, std::fabs(v));
        }
        std::cout << "  Forward time: " << ms << " ms\n"
                  << "  Final hidden RMS: " << std::sqrt(sum_sq / static_cast<double>(r.hidden.size())) << "\n"
                  << "  Final hidden max abs: " << max_abs << "\n"
                  << "  Final hidden checksum: " << std::setprecision(12) << checksum << "\n";
        if (!r.top_tokens.empty()) {
            std::cout << "  Top logits:\n";
            for (std::size_t i = 0; i < r.top_tokens.size(); ++i)
                std::cout << "    " << i + 1 << ": id=" << r.top_tokens[i].token_id << " logit=" << r.top_tokens[i].logit
                          << " piece=\"" << escape_piece(r.top_tokens[i].piece) << "\"\n";
        }
        std::cout << "  Validation: OK\n";
        return 0;
    } catch (const std::exception& e) {
        std::cerr << "vortexrt-gemma: " << e.what() << "\n";
        return 1;
    }
}
