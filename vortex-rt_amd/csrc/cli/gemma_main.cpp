// vortexrt-gemma: the Gemma 3 command line over the vortexrt:: API (libvortexrt.so, HIP).
//
// Interface kept from src/gemma_main.cpp, because scripts drive and grep it
// (.github/workflows/build.yml:81-123): the option spellings (--token-id, --top-k, --prompt,
// --generate, --projection-fusion, --q8-lanes, --device), the report labels ("Layers:",
// "Final hidden checksum:", "Top logits:", "Prompt token ids:", "Generated token ids:",
// "TEXT_BEGIN" / "TEXT_END", "Fused FFN:", "Validation: OK"), the definitions of the reported
// figures (checksum sum_i x_i * (i + 1), RMS, max |x|) and the error texts of rejected options.
//
// Two modes. Forward (no --generate): one token at position 0 through every block, the final
// hidden state summarised and, unless --top-k 0, the top logits. Generate (--generate N, N <= 128):
// the prompt is tokenized with BOS and N tokens follow greedily on the KV cache.
#include "vortexrt/build_config.hpp"
#include "vortexrt/gemma3.hpp"
#include "vortexrt/vulkan_context.hpp"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <exception>
#include <iostream>
#include <limits>
#include <sstream>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace {

using Clock = std::chrono::steady_clock;

// ---- settings and the option table ----------------------------------------------------------

struct Settings {
    std::string model;
    std::string device;          // "" = VORTEXRT_DEVICE or device 0
    std::string prompt;
    std::uint32_t token = 2;     // BOS
    std::size_t top_k = 8;
    std::size_t generate = 0;    // 0: forward mode
    int fusion = -1;             // -1 auto, 0 off, 1 on
    std::uint32_t lanes = 0;     // 0 = auto
};

constexpr std::size_t kMaxGenerate = 128;

std::uint64_t to_uint(const std::string& text, std::uint64_t max, const std::string& error) {
    const bool digits = !text.empty() && std::all_of(text.begin(), text.end(), [](char c) { return c >= '0' && c <= '9'; });
    if (!digits) throw std::runtime_error(error);
    errno = 0;
    char* end = nullptr;
    const unsigned long long v = std::strtoull(text.c_str(), &end, 10);
    if (errno == ERANGE || *end != '\0' || v > max) throw std::runtime_error(error);
    return v;
}

struct OptionSpec {
    const char* name;
    const char* arg;
    const char* help;
    void (*apply)(Settings&, const std::string&);
};

const OptionSpec kOptions[] = {
    {"--token-id", "N", "token fed at position 0 in forward mode (default 2, BOS)",
     [](Settings& s, const std::string& v) {
         s.token = static_cast<std::uint32_t>(to_uint(v, std::numeric_limits<std::uint32_t>::max(), "--token-id must be a uint32"));
     }},
    {"--top-k", "N", "logits listed in forward mode (default 8; 0 stops before the LM head)",
     [](Settings& s, const std::string& v) {
         s.top_k = static_cast<std::size_t>(to_uint(v, std::numeric_limits<std::size_t>::max(), "--top-k is out of range"));
     }},
    {"--prompt", "TEXT", "text tokenized (with BOS) ahead of generation", [](Settings& s, const std::string& v) { s.prompt = v; }},
    {"--generate", "N", "greedy tokens to generate on the KV cache (at most 128)",
     [](Settings& s, const std::string& v) {
         s.generate = static_cast<std::size_t>(to_uint(v, std::numeric_limits<std::size_t>::max(), "--generate is out of range"));
         if (s.generate > kMaxGenerate) throw std::runtime_error("--generate is capped at 128 during bring-up");
     }},
    {"--projection-fusion", "auto|on|off", "projection fusion policy",
     [](Settings& s, const std::string& v) {
         if (v == "auto") s.fusion = -1;
         else if (v == "on") s.fusion = 1;
         else if (v == "off") s.fusion = 0;
         else throw std::runtime_error("--projection-fusion must be auto, on, or off");
     }},
    {"--q8-lanes", "auto|8|16|32|64", "Q8 row-slot width request",
     [](Settings& s, const std::string& v) {
         const std::string err = "--q8-lanes must be auto, 8, 16, 32, or 64";
         if (v == "auto") { s.lanes = 0; return; }
         const auto n = to_uint(v, 64, err);
         if (n != 8 && n != 16 && n != 32 && n != 64) throw std::runtime_error(err);
         s.lanes = static_cast<std::uint32_t>(n);
     }},
    {"--device", "INDEX|NAME", "GPU by index or by a substring of its name", [](Settings& s, const std::string& v) { s.device = v; }},
};

std::string usage() {
    std::ostringstream u;
    u << "vortexrt-gemma MODEL.gguf [option VALUE]...\n";
    for (const auto& o : kOptions) {
        std::string head = std::string(o.name) + " " + o.arg;
        if (head.size() < 32) head.resize(32, ' ');
        u << "  " << head << " " << o.help << "\n";
    }
    return u.str();
}

Settings parse(int argc, char** argv) {
    const std::vector<std::string> args(argv + 1, argv + argc);
    if (args.empty()) throw std::runtime_error("usage: " + usage());
    if (args[0] == "--help" || args[0] == "-h") {
        std::cout << usage();
        std::exit(0);
    }
    Settings s;
    s.model = args[0];
    for (std::size_t i = 1; i < args.size(); ++i) {
        const std::string& a = args[i];
        if (a == "--help" || a == "-h") {
            std::cout << usage();
            std::exit(0);
        }
        const auto* spec = std::find_if(std::begin(kOptions), std::end(kOptions), [&](const OptionSpec& o) { return a == o.name; });
        if (spec == std::end(kOptions)) throw std::runtime_error("unknown argument: " + a);
        if (i + 1 >= args.size()) throw std::runtime_error(std::string(spec->name) + " requires a value");
        spec->apply(s, args[++i]);
    }
    return s;
}

// ---- report ----------------------------------------------------------------------------------

// "  Label: value" lines under the title, the layout the reference's report uses.
class Report {
public:
    explicit Report(std::ostream& os) : os_(os) { os_ << "Vortex-RT Gemma 3 runtime\n"; }
    template <typename T>
    Report& line(std::string_view label, const T& value) {
        os_ << "  " << label << ": " << value << "\n";
        return *this;
    }
    Report& ids(std::string_view label, const std::vector<std::uint32_t>& v) {
        os_ << "  " << label << ":";
        for (const auto id : v) os_ << ' ' << id;
        os_ << "\n";
        return *this;
    }
    std::ostream& raw() { return os_; }
    void ok() { os_ << "  Validation: OK\n"; }

private:
    std::ostream& os_;
};

// Bytes as printable ASCII: \n \r \t and anything outside 0x20..0x7e escaped.
std::string printable(std::string_view bytes) {
    static const char kHex[] = "0123456789abcdef";
    std::string out;
    out.reserve(bytes.size());
    for (const unsigned char c : bytes) {
        switch (c) {
        case '\n': out += "\\n"; break;
        case '\r': out += "\\r"; break;
        case '\t': out += "\\t"; break;
        default:
            if (c < 0x20 || c > 0x7e) {
                out += "\\x";
                out += kHex[c >> 4];
                out += kHex[c & 15];
            } else {
                out += static_cast<char>(c);
            }
        }
    }
    return out;
}

double elapsed_ms(Clock::time_point since) {
    return std::chrono::duration<double, std::milli>(Clock::now() - since).count();
}

// The final hidden state's summary figures.
struct HiddenSummary {
    double rms = 0.0;
    float max_abs = 0.0f;
    double checksum = 0.0;   // sum_i x_i * (i + 1)
};

HiddenSummary summarize(const std::vector<float>& h) {
    HiddenSummary s;
    double sum_sq = 0.0;
    std::size_t i = 0;
    for (const float v : h) {
        ++i;
        if (!std::isfinite(v)) throw std::runtime_error("final hidden state is non-finite");
        sum_sq += static_cast<double>(v) * v;
        s.checksum += static_cast<double>(v) * static_cast<double>(i);
        s.max_abs = std::max(s.max_abs, std::fabs(v));
    }
    s.rms = h.empty() ? 0.0 : std::sqrt(sum_sq / static_cast<double>(h.size()));
    return s;
}

// ---- the two modes -----------------------------------------------------------------------------

int run_generate(vortexrt::Gemma3Model& model, const Settings& s, Report& r) {
    r.line("Greedy generation from BOS", std::to_string(s.generate) + " token(s)");
    const std::vector<std::uint32_t> prompt = model.tokenize(s.prompt, true);
    r.ids("Prompt token ids", prompt);
    const auto t0 = Clock::now();
    const auto result = model.generate_greedy_tokens(prompt, s.generate);
    const double ms = elapsed_ms(t0);
    r.ids("Generated token ids", result.token_ids);
    r.line("Generation time", std::to_string(ms) + " ms");
    const double rate = ms > 0.0 ? 1000.0 * static_cast<double>(result.token_ids.size()) / ms : 0.0;
    r.line("Throughput", std::to_string(rate) + " tok/s");
    r.line("Generated text", "\"" + printable(result.text) + "\"");
    r.raw() << "TEXT_BEGIN\n" << result.text << "\nTEXT_END\n";
    r.ok();
    return 0;
}

int run_forward(vortexrt::Gemma3Model& model, const Settings& s, Report& r) {
    r.line("Token", s.token);
    const auto t0 = Clock::now();
    const auto result = model.run_single_token(s.token, s.top_k);
    const double ms = elapsed_ms(t0);
    const HiddenSummary h = summarize(result.hidden);
    r.line("Forward time", std::to_string(ms) + " ms");
    r.line("Final hidden RMS", h.rms);
    r.line("Final hidden max abs", h.max_abs);
    std::ostringstream cs;
    cs.precision(12);
    cs << h.checksum;
    r.line("Final hidden checksum", cs.str());
    if (!result.top_tokens.empty()) {
        r.raw() << "  Top logits:\n";
        std::size_t rank = 0;
        for (const auto& t : result.top_tokens)
            r.raw() << "    " << ++rank << ": id=" << t.token_id << " logit=" << t.logit << " piece=\"" << printable(t.piece)
                    << "\"\n";
    }
    r.ok();
    return 0;
}

int run(const Settings& s) {
    const auto t_start = Clock::now();
    vortexrt::VulkanContext device(s.device);
    const auto t_load = Clock::now();
    namespace bc = vortexrt::build_config;
    // the kernel paths are the reference constructor's (ignored: the HIP kernels are built in)
    vortexrt::Gemma3Model model(s.model, device, bc::q8_matvec_spv, bc::q8_matvec_u8_spv, bc::argmax_spv, bc::q8_matvec_32_spv,
                                bc::q8_matvec_u8_32_spv, bc::gelu_mul_spv, bc::q8_matvec_16_spv, bc::q8_matvec_u8_16_spv,
                                bc::q8_matvec_8_spv, bc::q8_matvec_u8_8_spv, s.lanes);
    if (s.fusion >= 0) model.set_projection_fusion_enabled(s.fusion == 1);
    const double load_ms = elapsed_ms(t_load), setup_ms = elapsed_ms(t_start);

    const auto& c = model.config();
    Report r(std::cout);
    r.line("GPU", device.capabilities().name)
        .line("Layers", c.block_count)
        .line("Hidden", c.embedding_length)
        .line("FFN", c.feed_forward_length)
        .line("Heads", std::to_string(c.head_count) + " / KV " + std::to_string(c.head_count_kv))
        .line("Head dim", c.head_dim)
        .line("Sliding window", c.sliding_window)
        .line("Vocab", c.vocab_size)
        .line("Narrow Q8 kernel", std::to_string(model.narrow_q8_lane_count()) + " lanes")
        .line("Projection fusion", model.projection_fusion_enabled() ? "enabled" : "disabled")
        .line("Fused FFN", model.fused_ffn_enabled() ? "enabled" : "disabled")
        .line("Model load", std::to_string(load_ms) + " ms")
        .line("Runtime setup", std::to_string(setup_ms) + " ms");
    return s.generate ? run_generate(model, s, r) : run_forward(model, s, r);
}

}  // namespace

int main(int argc, char** argv) {
    try {
        return run(parse(argc, argv));
    } catch (const std::exception& e) {
        std::cerr << "vortexrt-gemma: " << e.what() << "\n";
        return 1;
    }
}
