// Gemma3Model (vortexrt:: surface over libvrt_hip.so) on a GGUF file: prints one JSON object
// that the Python test compares with the oracle. Usage: gemma3_test model.gguf max_new id...
#include "common.hpp"

#include "vortexrt/gemma3.hpp"

#include <cstdio>
#include <iostream>
#include <string>

int main(int argc, char** argv) {
    if (argc < 4) {
        std::fprintf(stderr, "usage: %s model.gguf max_new prompt_id...\n", argv[0]);
        return 2;
    }
    vt::DeviceContext ctx;
    vt::Gemma3Model model(argv[1], ctx);
    const auto max_new = static_cast<std::size_t>(std::stoul(argv[2]));
    std::vector<std::uint32_t> prompt;
    for (int i = 3; i < argc; ++i) prompt.push_back(static_cast<std::uint32_t>(std::stoul(argv[i])));
    const auto& c = model.config();

    const auto gen = model.generate_greedy_tokens(prompt, max_new);

    // the same prompt step by step: top-4 at the last prompt position
    model.reset_cache();
    vt::Gemma3SingleTokenResult last;
    for (std::size_t i = 0; i < prompt.size(); ++i)
        last = model.decode_token(prompt[i], static_cast<std::uint32_t>(i), i + 1 == prompt.size() ? 4 : 0);
    const auto single = model.run_single_token(prompt[0], 1);

    // errors (src/gemma3.cpp:1467-1474, :1878-1881): a non-contiguous position is rejected
    // and leaves the cache as it was; a token out of range fails the step and resets it
    model.reset_cache();
    (void)model.decode_token(prompt[0], 0, 0);
    const bool err_pos = throws([&] { (void)model.decode_token(prompt[0], 5, 0); });
    const bool err_vocab = throws([&] { (void)model.decode_token(c.vocab_size, 1, 0); });
    const bool restart = !throws([&] { (void)model.decode_token(prompt[0], 0, 0); });
    const bool err_empty = throws([&] { (void)model.generate_greedy_tokens({}, 3); });

    std::printf("{\"config\": [%u, %u, %u, %u, %u, %u, %u], \"generate\": [", c.block_count, c.embedding_length,
                c.head_count, c.head_dim, c.feed_forward_length, c.vocab_size, c.sliding_window);
    for (std::size_t i = 0; i < gen.token_ids.size(); ++i) std::printf("%s%u", i ? ", " : "", gen.token_ids[i]);
    std::printf("], \"top4\": [");
    for (std::size_t i = 0; i < last.top_tokens.size(); ++i)
        std::printf("%s[%u, %.9g]", i ? ", " : "", last.top_tokens[i].token_id, last.top_tokens[i].logit);
    std::printf("], \"hidden\": [");
    for (std::size_t i = 0; i < last.hidden.size(); ++i) std::printf("%s%.9g", i ? ", " : "", last.hidden[i]);
    std::printf("], \"single\": [%u, %.9g], \"errors\": [%d, %d, %d, %d]}\n", single.top_tokens.at(0).token_id,
                single.top_tokens.at(0).logit, err_pos, err_vocab, restart, err_empty);
    return 0;
}
