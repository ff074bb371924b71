// runner_driver.cpp -- test infrastructure: drives LiteMind's DeepSeekRunner
// (include/DeepSeekRunner.hpp:67-118) through its public API and prints, as bit
// patterns, everything two builds must agree on.  `make ref-tests` builds it
// twice: over LiteMind's own sources (_ref/runner_cpu, the reference) and with
// this repository's drop-in sources in place of Gemm, MoeRouter, ExpertCache,
// Attention, KvCache and Rope (_ref/runner_gpu, the GPU build), every other
// source of LiteMind (DeepSeekRunner.cpp included) compiled unchanged.
//
//   runner_driver <model_dir> <context> <expert_budget_bytes> <max_new> <token>...
//
// For every prefix of the prompt, generate() (which starts with reset(), i.e.
// KvCache::clear on every layer) with max_new_tokens 0 for the shorter
// prefixes and <max_new> for the whole prompt, greedy sampling, and top_logits
// = the vocabulary: prints every logit after the prefix (rank order, id and
// bits), then the generated tokens and the stop reason of the last run.
#include "DeepSeekRunner.hpp"

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

int main(int argc, char** argv) {
    if (argc < 6) {
        std::fprintf(stderr, "usage: runner_driver <model_dir> <context> <expert_budget_bytes> <max_new> <token>...\n");
        return 2;
    }
    litemind::RunnerOptions options;
    options.threads = 1;
    options.context_length = std::strtoull(argv[2], nullptr, 10);
    options.expert_budget_bytes = std::strtoull(argv[3], nullptr, 10);
    options.verbose = false;
    const std::size_t max_new = std::strtoull(argv[4], nullptr, 10);
    std::vector<std::uint32_t> prompt;
    for (int i = 5; i < argc; ++i) {
        prompt.push_back(static_cast<std::uint32_t>(std::strtoul(argv[i], nullptr, 10)));
    }
    litemind::DeepSeekRunner runner;
    std::string error;
    if (!runner.load(argv[1], options, error)) {
        std::fprintf(stderr, "load: %s\n", error.c_str());
        return 1;
    }
    for (std::size_t k = 1; k <= prompt.size(); ++k) {
        litemind::GenerationOptions gen;
        gen.max_new_tokens = k == prompt.size() ? max_new : 0U;
        gen.show_progress = false;
        gen.top_logits = runner.config().vocab_size;
        litemind::GenerationResult result;
        const std::vector<std::uint32_t> prefix(prompt.begin(), prompt.begin() + static_cast<std::ptrdiff_t>(k));
        if (!runner.generate(prefix, gen, result, error)) {
            std::fprintf(stderr, "generate: %s\n", error.c_str());
            return 1;
        }
        std::printf("prefix %zu:", k);
        for (const auto& [token, logit] : result.prompt_top_logits) {
            std::uint32_t bits = 0;
            std::memcpy(&bits, &logit, sizeof bits);
            std::printf(" %u:%08x", token, bits);
        }
        std::printf("\n");
        if (k == prompt.size()) {
            std::printf("tokens:");
            for (const std::uint32_t t : result.tokens) {
                std::printf(" %u", t);
            }
            std::printf("\nstop: %s\n", result.stop_reason.c_str());
        }
    }
    return 0;
}
