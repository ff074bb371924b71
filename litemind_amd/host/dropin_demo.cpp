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
//   dropin_demo attention <case_dir>
//       Drives one Attention (configured as DeepSeekRunner does, with a
//       RotaryEmbedding and one KvCache per cache id) through the commands of
//       script.txt, one per line:
//         fwd <cache> <weights> <position> <x_row>   Attention::forward of row
//             x_row of x.f32; appends the output row to out.f32 and 1 / 0 (the
//             return value; a refused call leaves its row NaN) to results.txt
//         clear <cache>                                KvCache::clear
//         copy <dst> <src>                             dst.clear(), then src's
//             entries written into dst through KvCache's writable accessors
//             and appended, as a caller filling a cache by hand does
//         dump <cache>                                 the entries in KvCache's
//             layout to cache<c>_{kn,kr,v}.f32 and the count to cache<c>.txt
//       case.txt: hidden heads q_lora_rank kv_lora_rank qk_nope qk_rope v_head
//                 layers capacity rms_norm_eps rope_theta yarn factor
//                 beta_fast beta_slow mscale mscale_all_dim original_max
//                 weight_sets caches rows
//       Weights of set i: w<i>_q.bf16 (q_lora_rank 0) or w<i>_qa.bf16,
//       w<i>_qan.f32, w<i>_qb.bf16; w<i>_kva.bf16, w<i>_kvan.f32, w<i>_kvb.bf16,
//       w<i>_o.bf16.  The rotary table has `capacity` positions.
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
#include "Attention.hpp"
#include "ExpertCache.hpp"
#include "Gemm.hpp"
#include "KvCache.hpp"
#include "Rope.hpp"
#include "MoeRouter.hpp"
#include "Threading.hpp"
#include "litemind_gpu.hpp"
#include "litemind_moe.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <exception>
#include <fstream>
#include <iostream>
#include <limits>
#include <sstream>
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

int run_attention(const std::string& dir) {
    std::ifstream cfg(dir + "/case.txt");
    std::size_t H = 0, heads = 0, ql = 0, rank = 0, nope = 0, rope_dim = 0, vh = 0, layers = 0, cap = 0;
    std::size_t sets = 0, caches = 0, rows = 0, original_max = 0;
    int yarn = 0;
    float eps = 0.0F, theta = 0.0F;
    double factor = 0, beta_fast = 0, beta_slow = 0, mscale = 0, mscale_all = 0;
    if (!(cfg >> H >> heads >> ql >> rank >> nope >> rope_dim >> vh >> layers >> cap >> eps >> theta >> yarn >>
          factor >> beta_fast >> beta_slow >> mscale >> mscale_all >> original_max >> sets >> caches >> rows)) {
        throw std::runtime_error("bad case.txt");
    }
    Config config;
    config.hidden_size = H;
    config.num_hidden_layers = layers;
    config.num_attention_heads = heads;
    config.q_lora_rank = ql;
    config.kv_lora_rank = rank;
    config.qk_nope_head_dim = nope;
    config.qk_rope_head_dim = rope_dim;
    config.v_head_dim = vh;
    config.rms_norm_eps = eps;
    config.rope_theta = theta;
    config.rope_scaling.enabled = yarn != 0;
    config.rope_scaling.factor = factor;
    config.rope_scaling.beta_fast = beta_fast;
    config.rope_scaling.beta_slow = beta_slow;
    config.rope_scaling.mscale = mscale;
    config.rope_scaling.mscale_all_dim = mscale_all;
    config.rope_scaling.original_max_position_embeddings = original_max;

    // weights, held for the whole run (the views borrow them)
    const std::size_t qk = nope + rope_dim;
    std::vector<std::vector<std::uint16_t>> bf16;
    std::vector<AttentionWeights> weights(sets);
    auto load_view = [&](const std::string& name, std::size_t count) {
        bf16.push_back(read_array<std::uint16_t>(dir + "/" + name, count));
        return view_of(bf16.back(), 0, count);
    };
    bf16.reserve(sets * 6);
    for (std::size_t i = 0; i < sets; ++i) {
        const std::string w = "w" + std::to_string(i) + "_";
        AttentionWeights& aw = weights[i];
        if (ql == 0U) {
            aw.q_proj = load_view(w + "q.bf16", heads * qk * H);
        } else {
            aw.q_a_proj = load_view(w + "qa.bf16", ql * H);
            aw.q_a_layernorm = read_array<float>(dir + "/" + w + "qan.f32", ql);
            aw.q_b_proj = load_view(w + "qb.bf16", heads * qk * ql);
        }
        aw.kv_a_proj = load_view(w + "kva.bf16", (rank + rope_dim) * H);
        aw.kv_a_layernorm = read_array<float>(dir + "/" + w + "kvan.f32", rank);
        aw.kv_b_proj = load_view(w + "kvb.bf16", heads * (nope + vh) * rank);
        aw.o_proj = load_view(w + "o.bf16", H * heads * vh);
    }
    const auto x = read_array<float>(dir + "/x.f32", rows * H);

    // src/DeepSeekRunner.cpp:358-360 and :416-420
    ThreadPool pool(1);
    RotaryEmbedding rope;
    rope.build(config, cap);
    Attention attention;
    attention.configure(config, pool, rope);
    std::vector<KvCache> cache(caches);
    for (KvCache& c : cache) {
        c.configure(heads, nope, rope_dim, vh, cap);
    }

    std::ifstream script(dir + "/script.txt");
    std::ofstream out(dir + "/out.f32", std::ios::binary);
    std::ofstream results(dir + "/results.txt");
    std::vector<float> y(H);
    std::string line;
    while (std::getline(script, line)) {
        std::istringstream cmd(line);
        std::string op;
        if (!(cmd >> op)) {
            continue;
        }
        if (op == "fwd") {
            std::size_t c = 0, w = 0, pos = 0, row = 0;
            cmd >> c >> w >> pos >> row;
            std::fill(y.begin(), y.end(), std::numeric_limits<float>::quiet_NaN());
            const bool ok = attention.forward(x.data() + row * H, weights.at(w), cache.at(c), pos, y.data());
            out.write(reinterpret_cast<const char*>(y.data()), static_cast<std::streamsize>(H * sizeof(float)));
            results << (ok ? 1 : 0) << "\n";
        } else if (op == "clear") {
            std::size_t c = 0;
            cmd >> c;
            cache.at(c).clear();
        } else if (op == "copy") {
            std::size_t dst = 0, src = 0;
            cmd >> dst >> src;
            KvCache& d = cache.at(dst);
            const KvCache& s = cache.at(src);
            d.clear();
            for (std::size_t t = 0; t < s.token_count(); ++t) {
                const std::size_t slot = d.append();
                for (std::size_t h = 0; h < heads; ++h) {
                    std::copy_n(s.key_nope(t, h), nope, d.key_nope(slot) + h * nope);
                    std::copy_n(s.value(t, h), vh, d.value(slot) + h * vh);
                }
                std::copy_n(s.key_rope(t), rope_dim, d.key_rope(slot));
            }
        } else if (op == "dump") {
            std::size_t c = 0;
            cmd >> c;
            const KvCache& k = cache.at(c);
            const std::size_t n = k.token_count();
            std::vector<float> kn(n * heads * nope), kr(n * rope_dim), v(n * heads * vh);
            for (std::size_t t = 0; t < n; ++t) {
                for (std::size_t h = 0; h < heads; ++h) {
                    std::copy_n(k.key_nope(t, h), nope, kn.data() + (t * heads + h) * nope);
                    std::copy_n(k.value(t, h), vh, v.data() + (t * heads + h) * vh);
                }
                std::copy_n(k.key_rope(t), rope_dim, kr.data() + t * rope_dim);
            }
            const std::string base = dir + "/cache" + std::to_string(c);
            write_array(base + "_kn.f32", kn);
            write_array(base + "_kr.f32", kr);
            write_array(base + "_v.f32", v);
            std::ofstream(base + ".txt") << n << "\n";
        } else {
            throw std::runtime_error("unknown script command: " + line);
        }
    }
    std::printf("attention case %s: %s\n", dir.c_str(), rope.summary().c_str());
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
        if (argc >= 3 && std::strcmp(argv[1], "attention") == 0) {
            return run_attention(argv[2]);
        }
        if (argc >= 2 && std::strcmp(argv[1], "cache-trace") == 0) {
            return run_cache_trace(argc, argv);
        }
        std::fprintf(stderr, "usage: dropin_demo moe|moe-timeout|attention <case_dir> | cache-trace <budget> "
                             "<block_bytes> <l e>...\n");
        return 2;
    } catch (const std::exception& error) {
        std::fprintf(stderr, "dropin_demo: %s\n", error.what());
        return 1;
    }
}
