// Gemma3Tokenizer (vortexrt:: host tokenizer) on a GGUF file's tokenizer metadata: tokenizes
// the texts given as hex-encoded UTF-8 arguments and prints one JSON object with the ids (with
// and without BOS) and the decoded piece of every id, as hex. No GPU.
// Usage: tokenizer_test file.gguf vocab_size hex_text...
#include "vortexrt/gguf.hpp"
#include "vortexrt/tokenizer.hpp"

#include <cstdio>
#include <exception>
#include <string>
#include <vector>

namespace {

std::string unhex(const std::string& h) {
    std::string out;
    for (std::size_t i = 0; i + 1 < h.size(); i += 2) out += static_cast<char>(std::stoi(h.substr(i, 2), nullptr, 16));
    return out;
}

void print_ids(const std::vector<std::uint32_t>& ids) {
    std::printf("[");
    for (std::size_t i = 0; i < ids.size(); ++i) std::printf("%s%u", i ? ", " : "", ids[i]);
    std::printf("]");
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) return 2;
    try {
        vortexrt::GgufFile f(argv[1]);
        const auto vocab = static_cast<std::uint32_t>(std::stoul(argv[2]));
        vortexrt::Gemma3Tokenizer tok(f, vocab);
        std::printf("{\"bos\": %u, \"eos\": %u, \"unk\": %u, \"prefix\": %d, \"pieces\": %zu, \"ids\": [", tok.bos_id(),
                    tok.eos_id(), tok.unknown_id(), tok.add_space_prefix() ? 1 : 0, tok.piece_count());
        for (int i = 3; i < argc; ++i) {
            std::printf("%s", i > 3 ? ", " : "");
            print_ids(tok.tokenize(unhex(argv[i]), true));
        }
        std::printf("], \"ids_nobos\": [");
        for (int i = 3; i < argc; ++i) {
            std::printf("%s", i > 3 ? ", " : "");
            print_ids(tok.tokenize(unhex(argv[i]), false));
        }
        std::printf("], \"decoded\": [");
        for (std::uint32_t id = 0; id < vocab; ++id) {
            std::printf("%s\"", id ? ", " : "");
            for (const unsigned char c : tok.decode_piece(id)) std::printf("%02x", c);
            std::printf("\"");
        }
        std::printf("]}\n");
    } catch (const std::exception& e) {
        std::printf("{\"error\": \"%s\"}\n", e.what());
        return 1;
    }
    return 0;
}
