// Drives the drop-in classes the way LiteMind's runner does.
//
//   dropin_demo moe <case_dir>
//       Reads one MoE layer and T tokens from <case_dir> (raw little-endian
//       arrays named below, shapes in case.txt) and writes
//         y_token / index_token / weight_token: the MoE block of
//           DeepSeekRunner::Impl::forward (src/DeepSeekRunner.cpp:273-290) run
//           token by token through gemm::, MoeRouter and ExpertCache, exactly
//           as LiteMind composes them;
//         y_batch / index_batch / weight_batch: the same tokens through
//           gpu::MoeBlockGpu (one batched lm_moe_forward);
//         cache.txt: the ExpertCache counters after the per-token run.
//   dropin_demo moe-timeout <case_dir>
//       The same layer through gpu::MoeBlockGpu with the single-token kernel's
//       hand-off waits made to give up at once (lm_decode_wait_test): forward
//       must throw with the library's LM_EKERNEL message, and a second forward
//       with normal waits must succeed.  Exit status 0 when both hold.
//   dropin_demo cache-trace <budget> <block_bytes> <layer expert>...
//       Replays touches on an ExpertCache with byte-less views and prints its
//       counters after each touch and after clear(): resident_bytes,
//       resident_experts, loads, hits, evictions, bytes_streamed, enabled.
//       Uses no GPU.
//
// case.txt: hidden inter experts top_k shared_inter tokens norm_topk_prob
//           routed_scaling_factor cache_budget_experts
// Inputs: router.f32 [E,H], gate.bf16 / up.bf16 [E,I,H], down.bf16 [E,H,I],
//         shared_{gate,up}.bf16 [S,H], shared_down.bf16 [H,S] (when S > 0),
//         x.f32 [T,H].
#include "ExpertCache.hpp"
#include "Gemm.hpp"
#include "MoeRouter.hpp"
#include "Threading.hpp"
#include "litemind_gpu.hpp"
#include "litemind_moe.h"

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

using namespace litemind;

namespace {

template <typename T>
std::vector<T> read_array(const std::string& path, std::size_t count) {
    std::vector<T> out(count);
    std::ifstream in(path, std::ios::binary);
    if (!in.read(reinterpret_cast<char*>(out.data()), static_cast<std::streamsize>(count * sizeof(T)))) {
        throw std::runtime_error("cannot read " + std::to_string(count) + " elements from " + path);
    }
    return out;
}

template <typename T>
void write_array(const std::string& path, const std::vector<T>& data) {
    std::ofstream out(path, std::ios::binary);
    out.write(reinterpret_cast<const char*>(data.data()), static_cast<std::streamsize>(data.size() * sizeof(T)));
    if (!out) {
        throw std::runtime_error("cannot write " + path);
    }
}

WeightView view_of(const std::vector<std::uint16_t>& data, std::size_t offset, std::size_t elements) {
    WeightView v;
    v.bytes = reinterpret_cast<const std::byte*>(data.data() + offset);
    v.size = elements * sizeof(std::uint16_t);
    return v;
}

struct Ffn {
    WeightView gate, up, down;
    std::size_t inter{};
};

// DeepSeekRunner::Impl::feed_forward (src/DeepSeekRunner.cpp:228-240) over the
// drop-in gemm::.
void feed_forward(ThreadPool& pool, const Ffn& w, const float* input, float* output, float scale,
                  std::size_t hidden, std::vector<float>& gate, std::vector<float>& up, std::vector<float>& act) {
    gemm::matvec_bf16(pool, w.gate.as_bf16(), input, gate.data(), w.inter, hidden);
    gemm::matvec_bf16(pool, w.up.as_bf16(), input, up.data(), w.inter, hidden);
    gemm::silu_multiply(gate.data(), up.data(), act.data(), w.inter);
    gemm::matvec_bf16_accumulate(pool, w.down.as_bf16(), act.data(), output, hidden, w.inter, scale);
}

int run_moe(const std::string& dir) {
    std::ifstream cfg(dir + "/case.txt");
    std::size_t H = 0, I = 0, E = 0, K = 0, S = 0, T = 0, budget_experts = 0;
    int norm = 0;
    float scale = 1.0F;
    if (!(cfg >> H >> I >> E >> K >> S >> T >> norm >> scale >> budget_experts)) {
        throw std::runtime_error("bad case.txt");
    }
    Config config;
    config.hidden_size = H;
    config.moe_intermediate_size = I;
    config.n_routed_experts = E;
    config.num_experts_per_tok = K;
    config.n_shared_experts = I != 0U ? S / I : 0U;
    config.intermediate_size = 0U;
    config.norm_topk_prob = norm != 0;
    config.routed_scaling_factor = scale;

    const auto router = read_array<float>(dir + "/router.f32", E * H);
    const auto gate = read_array<std::uint16_t>(dir + "/gate.bf16", E * I * H);
    const auto up = read_array<std::uint16_t>(dir + "/up.bf16", E * I * H);
    const auto down = read_array<std::uint16_t>(dir + "/down.bf16", E * H * I);
    std::vector<std::uint16_t> sg, su, sd;
    if (S > 0U) {
        sg = read_array<std::uint16_t>(dir + "/shared_gate.bf16", S * H);
        su = read_array<std::uint16_t>(dir + "/shared_up.bf16", S * H);
        sd = read_array<std::uint16_t>(dir + "/shared_down.bf16", H * S);
    }
    const auto x = read_array<float>(dir + "/x.f32", T * H);

    std::vector<Ffn> experts(E);
    for (std::size_t e = 0; e < E; ++e) {
        experts[e] = Ffn{view_of(gate, e * I * H, I * H), view_of(up, e * I * H, I * H),
                         view_of(down, e * H * I, H * I), I};
    }
    const Ffn shared{S > 0U ? view_of(sg, 0, S * H) : WeightView{}, S > 0U ? view_of(su, 0, S * H) : WeightView{},
                     S > 0U ? view_of(sd, 0, H * S) : WeightView{}, S};

    // ---- per-token drop-in path ----
    ThreadPool pool;
    MoeRouter moe_router(config);
    ExpertCache cache;
    cache.configure(budget_experts * 3U * I * H * sizeof(std::uint16_t));
    const std::size_t widest = std::max(I, S);
    std::vector<float> gate_buf(widest), up_buf(widest), act_buf(widest), logits(E);
    std::vector<float> y_token(T * H, 0.0F), w_token(T * K, 0.0F);
    std::vector<std::int32_t> i_token(T * K, -1);
    std::vector<ExpertSelection> selection;
    const std::size_t layer = 1;
    for (std::size_t t = 0; t < T; ++t) {
        const float* xt = x.data() + t * H;
        float* yt = y_token.data() + t * H;
        gemm::matvec_f32(router.data(), xt, logits.data(), E, H);
        moe_router.select(logits, selection);
        for (std::size_t r = 0; r < selection.size(); ++r) {
            const ExpertSelection& choice = selection[r];
            const Ffn& ex = experts[choice.expert_index];
            cache.touch(ExpertCache::make_key(layer, choice.expert_index), ExpertCache::Block{ex.gate, ex.up, ex.down});
            feed_forward(pool, ex, xt, yt, choice.weight, H, gate_buf, up_buf, act_buf);
            i_token[t * K + r] = static_cast<std::int32_t>(choice.expert_index);
            w_token[t * K + r] = choice.weight;
        }
        if (S > 0U) {
            feed_forward(pool, shared, xt, yt, 1.0F, H, gate_buf, up_buf, act_buf);
        }
    }
    write_array(dir + "/y_token.f32", y_token);
    write_array(dir + "/index_token.i32", i_token);
    write_array(dir + "/weight_token.f32", w_token);
    {
        std::ofstream out(dir + "/cache.txt");
        out << cache.resident_bytes() << ' ' << cache.resident_experts() << ' ' << cache.loads() << ' '
            << cache.hits() << ' ' << cache.evictions() << ' ' << cache.bytes_streamed() << ' '
            << (cache.enabled() ? 1 : 0) << '\n';
    }
    cache.clear();

    // ---- batched path ----
    gpu::MoeBlockGpu block(config, 1);
    std::vector<WeightView> gv(E), uv(E), dv(E);
    for (std::size_t e = 0; e < E; ++e) {
        gv[e] = experts[e].gate;
        uv[e] = experts[e].up;
        dv[e] = experts[e].down;
    }
    block.upload_layer(0, router, gv, uv, dv, S > 0U ? &shared.gate : nullptr, S > 0U ? &shared.up : nullptr,
                       S > 0U ? &shared.down : nullptr);
    std::vector<float> y_batch(T * H), w_batch(T * K);
    std::vector<std::int32_t> i_batch(T * K);
    block.forward(0, x, T, y_batch, i_batch, w_batch);
    write_array(dir + "/y_batch.f32", y_batch);
    write_array(dir + "/index_batch.i32", i_batch);
    write_array(dir + "/weight_batch.f32", w_batch);
    std::printf("moe case %s: H=%zu I=%zu E=%zu k=%zu S=%zu T=%zu done (%s)\n", dir.c_str(), H, I, E, K, S, T,
                gemm::kernel_description().c_str());
    return 0;
}
int run_moe_timeout(const std::string& dir) {
    std::ifstream cfg(dir + "/case.txt");
    std::size_t H = 0, I = 0, E = 0, K = 0, S = 0, T = 0, budget_experts = 0;
    int norm = 0;
    float scale = 1.0F;
    if (!(cfg >> H >> I >> E >> K >> S >> T >> norm >> scale >> budget_experts) || S == 0U) {
        throw std::runtime_error("bad case.txt (the single-token kernel needs a shared expert)");
    }
    Config config;
    config.hidden_size = H;
    config.moe_intermediate_size = I;
    config.n_routed_experts = E;
    config.num_experts_per_tok = K;
    config.n_shared_experts = S / I;
    config.intermediate_size = 0U;
    config.norm_topk_prob = norm != 0;
    config.routed_scaling_factor = scale;
    const auto router = read_array<float>(dir + "/router.f32", E * H);
    const auto gate = read_array<std::uint16_t>(dir + "/gate.bf16", E * I * H);
    const auto up = read_array<std::uint16_t>(dir + "/up.bf16", E * I * H);
    const auto down = read_array<std::uint16_t>(dir + "/down.bf16", E * H * I);
    const auto sg = read_array<std::uint16_t>(dir + "/shared_gate.bf16", S * H);
    const auto su = read_array<std::uint16_t>(dir + "/shared_up.bf16", S * H);
    const auto sd = read_array<std::uint16_t>(dir + "/shared_down.bf16", H * S);
    const auto x = read_array<float>(dir + "/x.f32", T * H);
    std::vector<WeightView> gv(E), uv(E), dv(E);
    for (std::size_t e = 0; e < E; ++e) {
        gv[e] = view_of(gate, e * I * H, I * H);
        uv[e] = view_of(up, e * I * H, I * H);
        dv[e] = view_of(down, e * H * I, H * I);
    }
    const WeightView sgv = view_of(sg, 0, S * H), suv = view_of(su, 0, S * H), sdv = view_of(sd, 0, H * S);
    gpu::MoeBlockGpu block(config, 1);
    block.upload_layer(0, router, gv, uv, dv, &sgv, &suv, &sdv);
    std::vector<float> y(H);
    gpu::check(lm_decode_wait_test(block.context(), 1), "lm_decode_wait_test");
    bool reported = false;
    try {
        block.forward(0, std::span<const float>(x.data(), H), 1, y);
    } catch (const std::runtime_error& error) {
        reported = std::string(error.what()).find("timed out") != std::string::npos;
        std::printf("forward with waits that give up: %s\n", error.what());
    }
    gpu::check(lm_decode_wait_test(block.context(), 0), "lm_decode_wait_test");
    if (!reported) {
        std::fprintf(stderr, "dropin_demo: a wait that gave up was not reported\n");
        return 3;
    }
    block.forward(0, std::span<const float>(x.data(), H), 1, y);  // normal waits: must succeed
    std::printf("moe-timeout case %s: LM_EKERNEL reported, next forward ok\n", dir.c_str());
    return 0;
}

int run_cache_trace(int argc, char** argv) {
    if (argc < 4 || (argc - 4) % 2 != 0) {
        throw std::runtime_error("usage: cache-trace <budget> <block_bytes> <layer expert>...");
    }
    const std::uint64_t budget = std::strtoull(argv[2], nullptr, 10);
    const std::uint64_t block_bytes = std::strtoull(argv[3], nullptr, 10);
    ExpertCache cache;
    cache.configure(budget);
    auto print = [&] {
        std::printf("%llu %llu %llu %llu %llu %llu %d\n", static_cast<unsigned long long>(cache.resident_bytes()),
                    static_cast<unsigned long long>(cache.resident_experts()),
                    static_cast<unsigned long long>(cache.loads()), static_cast<unsigned long long>(cache.hits()),
                    static_cast<unsigned long long>(cache.evictions()),
                    static_cast<unsigned long long>(cache.bytes_streamed()), cache.enabled() ? 1 : 0);
    };
    // Views without bytes: only their sizes matter to the bookkeeping, and each
    // of gate, up and down is a third of the block.
    WeightView third;
    third.size = block_bytes / 3U;
    for (int i = 4; i + 1 < argc; i += 2) {
        const std::size_t layer = std::strtoull(argv[i], nullptr, 10);
        const std::size_t expert = std::strtoull(argv[i + 1], nullptr, 10);
        cache.touch(ExpertCache::make_key(layer, expert), ExpertCache::Block{third, third, third});
        print();
    }
    cache.clear();
    print();
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc >= 3 && std::strcmp(argv[1], "moe") == 0) {
            return run_moe(argv[2]);
        }
        if (argc >= 3 && std::strcmp(argv[1], "moe-timeout") == 0) {
            return run_moe_timeout(argv[2]);
        }
        if (argc >= 2 && std::strcmp(argv[1], "cache-trace") == 0) {
            return run_cache_trace(argc, argv);
        }
        std::fprintf(stderr, "usage: dropin_demo moe|moe-timeout <case_dir> | cache-trace <budget> <block_bytes> <l e>...\n");
        return 2;
    } catch (const std::exception& error) {
        std::fprintf(stderr, "dropin_demo: %s\n", error.what());
        return 1;
    }
}
