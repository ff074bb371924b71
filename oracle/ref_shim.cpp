// ref_shim.cpp -- extern "C" bindings over LiteMind's own C++ sources.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's src/Gemm.cpp, src/MoeRouter.cpp, src/Threading.cpp,
// src/ExpertCache.cpp and their few dependencies, straight from the LiteMind
// source tree, into oracle/_ref/libref.so.  Nothing from the reference is copied
// here: this file only calls the reference's public functions so Python tests
// (ctypes) can cross-check the oracle restatement and time LiteMind's CPU path.
//
// ref_mla_sequence() runs the reference's Attention::forward (src/Attention.cpp)
// with its RotaryEmbedding and KvCache over a sequence of tokens;
// ref_rope_tables() reads RotaryEmbedding's private tables back through its
// public apply() on unit channel pairs, which returns (cos, sin) exactly.
//
// ref_moe_layer() composes the reference's kernels in the order of
// DeepSeekRunner::Impl::feed_forward (src/DeepSeekRunner.cpp:228-240) and the
// MoE block of DeepSeekRunner::Impl::forward (:264-290), because those two are
// private members of a class that also needs a tokenizer, attention and a
// checkpoint on disk.
#include "Attention.hpp"
#include "ExpertCache.hpp"
#include "Gemm.hpp"
#include "KvCache.hpp"
#include "Rope.hpp"
#include "MoeRouter.hpp"
#include "Threading.hpp"

#include <algorithm>
#include <bit>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <random>
#include <stdexcept>
#include <vector>

using namespace litemind;

namespace {

ThreadPool& pool_for(std::size_t workers) {
    static std::mutex guard;
    static std::map<std::size_t, std::unique_ptr<ThreadPool>> pools;
    std::scoped_lock lock(guard);
    auto& slot = pools[workers];
    if (!slot) {
        slot = std::make_unique<ThreadPool>(workers);
    }
    return *slot;
}

Config routing_config(std::int32_t experts, std::int32_t top_k, std::int32_t n_group, std::int32_t topk_group,
                      std::int32_t group_limited, std::int32_t normalize, float scale) {
    Config config;
    config.n_routed_experts = static_cast<std::size_t>(experts);
    config.num_experts_per_tok = static_cast<std::size_t>(top_k);
    config.n_group = static_cast<std::size_t>(n_group);
    config.topk_group = static_cast<std::size_t>(topk_group);
    config.topk_method = group_limited != 0 ? "group_limited_greedy" : "greedy";
    config.norm_topk_prob = normalize != 0;
    config.routed_scaling_factor = scale;
    return config;
}

Config mla_config(std::int32_t hidden, std::int32_t heads, std::int32_t q_lora_rank, std::int32_t kv_lora_rank,
                  std::int32_t qk_nope, std::int32_t qk_rope, std::int32_t v_head, float eps, double theta,
                  std::int32_t yarn, double factor, double beta_fast, double beta_slow, double mscale,
                  double mscale_all_dim, std::int64_t original_max) {
    Config c;
    c.hidden_size = static_cast<std::size_t>(hidden);
    c.num_attention_heads = static_cast<std::size_t>(heads);
    c.q_lora_rank = static_cast<std::size_t>(q_lora_rank);
    c.kv_lora_rank = static_cast<std::size_t>(kv_lora_rank);
    c.qk_nope_head_dim = static_cast<std::size_t>(qk_nope);
    c.qk_rope_head_dim = static_cast<std::size_t>(qk_rope);
    c.v_head_dim = static_cast<std::size_t>(v_head);
    c.rms_norm_eps = eps;
    c.rope_theta = static_cast<float>(theta);
    c.rope_scaling.enabled = yarn != 0;
    c.rope_scaling.factor = factor;
    c.rope_scaling.beta_fast = beta_fast;
    c.rope_scaling.beta_slow = beta_slow;
    c.rope_scaling.mscale = mscale;
    c.rope_scaling.mscale_all_dim = mscale_all_dim;
    c.rope_scaling.original_max_position_embeddings = static_cast<std::size_t>(original_max);
    return c;
}

WeightView view_of(const std::uint16_t* p) {
    WeightView v;
    v.bytes = reinterpret_cast<const std::byte*>(p);
    return v;
}

}  // namespace

extern "C" {

// Config::softmax_scale (src/Config.cpp:114-121) for the given rope scaling.
float ref_softmax_scale(std::int32_t qk_nope, std::int32_t qk_rope, std::int32_t yarn, double factor,
                        double mscale_all_dim) {
    Config c;
    c.qk_nope_head_dim = static_cast<std::size_t>(qk_nope);
    c.qk_rope_head_dim = static_cast<std::size_t>(qk_rope);
    c.rope_scaling.enabled = yarn != 0;
    c.rope_scaling.factor = factor;
    c.rope_scaling.mscale_all_dim = mscale_all_dim;
    return c.softmax_scale();
}

// RotaryEmbedding::build's tables [positions, dim / 2], read back through apply().
int ref_rope_tables(std::int32_t dim, std::int32_t positions, double theta, std::int32_t yarn, double factor,
                    double beta_fast, double beta_slow, double mscale, double mscale_all_dim,
                    std::int64_t original_max, float* cos_out, float* sin_out) {
    Config c = mla_config(16, 1, 0, 16, 16, dim, 16, 1e-6F, theta, yarn, factor, beta_fast, beta_slow, mscale,
                          mscale_all_dim, original_max);
    RotaryEmbedding rope;
    rope.build(c, static_cast<std::size_t>(positions));
    const std::size_t half = static_cast<std::size_t>(dim) / 2U;
    std::vector<float> v(static_cast<std::size_t>(dim));
    for (std::size_t p = 0; p < static_cast<std::size_t>(positions); ++p) {
        for (std::size_t i = 0; i < half; ++i) {
            v[2 * i] = 1.0F;
            v[2 * i + 1] = 0.0F;
        }
        rope.apply(v.data(), p);
        for (std::size_t i = 0; i < half; ++i) {
            cos_out[p * half + i] = v[i];
            sin_out[p * half + i] = v[i + half];
        }
    }
    return 0;
}

// RotaryEmbedding::apply on `values` (dim channels) at `position`.
int ref_rope_apply(std::int32_t dim, std::int32_t positions, double theta, std::int32_t yarn, double factor,
                   double beta_fast, double beta_slow, double mscale, double mscale_all_dim, std::int64_t original_max,
                   float* values, std::int64_t position) {
    Config c = mla_config(16, 1, 0, 16, 16, dim, 16, 1e-6F, theta, yarn, factor, beta_fast, beta_slow, mscale,
                          mscale_all_dim, original_max);
    RotaryEmbedding rope;
    rope.build(c, static_cast<std::size_t>(positions));
    rope.apply(values, static_cast<std::size_t>(position));
    return 0;
}

// Attention::forward for tokens [0, T) at positions position0 + t, one cache of
// `capacity` positions, then the cache contents.  Returns the number of tokens
// processed before the cache was full.
std::int64_t ref_mla_sequence(std::int32_t hidden, std::int32_t heads, std::int32_t q_lora_rank,
                              std::int32_t kv_lora_rank, std::int32_t qk_nope, std::int32_t qk_rope,
                              std::int32_t v_head, float eps, double theta, std::int32_t yarn, double factor,
                              double beta_fast, double beta_slow, double mscale, double mscale_all_dim,
                              std::int64_t original_max, std::int64_t capacity, const std::uint16_t* q_proj,
                              const std::uint16_t* q_a_proj, const float* q_a_layernorm, const std::uint16_t* q_b_proj,
                              const std::uint16_t* kv_a_proj, const float* kv_a_layernorm,
                              const std::uint16_t* kv_b_proj, const std::uint16_t* o_proj, const float* x,
                              std::int64_t tokens, std::int64_t position0, float* out, float* key_nope,
                              float* key_rope, float* value) {
    const Config c = mla_config(hidden, heads, q_lora_rank, kv_lora_rank, qk_nope, qk_rope, v_head, eps, theta, yarn,
                                factor, beta_fast, beta_slow, mscale, mscale_all_dim, original_max);
    RotaryEmbedding rope;
    rope.build(c, static_cast<std::size_t>(capacity));
    ThreadPool& pool = pool_for(0);
    Attention attention;
    attention.configure(c, pool, rope);
    AttentionWeights w;
    if (q_lora_rank == 0) {
        w.q_proj = view_of(q_proj);
    } else {
        w.q_a_proj = view_of(q_a_proj);
        w.q_a_layernorm.assign(q_a_layernorm, q_a_layernorm + q_lora_rank);
        w.q_b_proj = view_of(q_b_proj);
    }
    w.kv_a_proj = view_of(kv_a_proj);
    w.kv_a_layernorm.assign(kv_a_layernorm, kv_a_layernorm + kv_lora_rank);
    w.kv_b_proj = view_of(kv_b_proj);
    w.o_proj = view_of(o_proj);
    KvCache cache;
    cache.configure(static_cast<std::size_t>(heads), static_cast<std::size_t>(qk_nope),
                    static_cast<std::size_t>(qk_rope), static_cast<std::size_t>(v_head),
                    static_cast<std::size_t>(capacity));
    std::int64_t done = 0;
    for (std::int64_t t = 0; t < tokens; ++t) {
        if (!attention.forward(x + t * hidden, w, cache, static_cast<std::size_t>(position0 + t), out + t * hidden)) {
            break;
        }
        ++done;
    }
    const std::size_t n = cache.token_count();
    for (std::size_t slot = 0; slot < n; ++slot) {
        std::memcpy(key_nope + slot * heads * qk_nope, cache.key_nope(slot), sizeof(float) * heads * qk_nope);
        std::memcpy(key_rope + slot * qk_rope, cache.key_rope(slot), sizeof(float) * qk_rope);
        std::memcpy(value + slot * heads * v_head, cache.value(slot), sizeof(float) * heads * v_head);
    }
    return done;
}

int ref_kernel_description(char* buffer, std::size_t size) {
    const std::string text = gemm::kernel_description();
    if (size == 0) {
        return -1;
    }
    std::strncpy(buffer, text.c_str(), size - 1);
    buffer[size - 1] = '\0';
    return 0;
}

std::size_t ref_hardware_threads() { return ThreadPool::hardware_threads(); }

void ref_matvec_bf16(std::size_t workers, const std::uint16_t* w, const float* x, float* out, std::size_t out_dim,
                     std::size_t in_dim) {
    gemm::matvec_bf16(pool_for(workers), w, x, out, out_dim, in_dim);
}

void ref_matvec_bf16_serial(const std::uint16_t* w, const float* x, float* out, std::size_t out_dim,
                            std::size_t in_dim) {
    gemm::matvec_bf16_serial(w, x, out, out_dim, in_dim);
}

void ref_matvec_bf16_accumulate(std::size_t workers, const std::uint16_t* w, const float* x, float* out,
                                std::size_t out_dim, std::size_t in_dim, float scale) {
    gemm::matvec_bf16_accumulate(pool_for(workers), w, x, out, out_dim, in_dim, scale);
}

void ref_matvec_f32(const float* w, const float* x, float* out, std::size_t out_dim, std::size_t in_dim) {
    gemm::matvec_f32(w, x, out, out_dim, in_dim);
}

float ref_dot(const float* a, const float* b, std::size_t n) { return gemm::dot(a, b, n); }
void ref_axpy(float scale, const float* src, float* dst, std::size_t n) { gemm::axpy(scale, src, dst, n); }
void ref_rms_norm(float* v, const float* w, std::size_t n, float eps) { gemm::rms_norm(v, w, n, eps); }
void ref_softmax(float* v, std::size_t n) { gemm::softmax(v, n); }
void ref_silu_multiply(const float* g, const float* u, float* out, std::size_t n) {
    gemm::silu_multiply(g, u, out, n);
}
void ref_widen_bf16(const std::uint16_t* src, float* dst, std::size_t n) { gemm::widen_bf16(src, dst, n); }

// MoeRouter::select for one token; returns the number of selections.
int ref_router_select(std::int32_t experts, std::int32_t top_k, std::int32_t n_group, std::int32_t topk_group,
                      std::int32_t group_limited, std::int32_t normalize, float scale, const float* logits,
                      std::int32_t logit_count, std::int32_t* out_index, float* out_weight) {
    const MoeRouter router(routing_config(experts, top_k, n_group, topk_group, group_limited, normalize, scale));
    const auto selection = router.select(std::span<const float>(logits, static_cast<std::size_t>(logit_count)));
    for (std::size_t i = 0; i < selection.size(); ++i) {
        out_index[i] = static_cast<std::int32_t>(selection[i].expert_index);
        out_weight[i] = selection[i].weight;
    }
    return static_cast<int>(selection.size());
}

// MoeRouter::select_top_k; returns -1 when the reference throws.
int ref_router_select_top_k(const float* logits, std::int32_t logit_count, std::int32_t experts, std::int32_t top_k,
                            std::int32_t normalize, std::int32_t* out_index, float* out_weight) {
    try {
        const auto selection = MoeRouter::select_top_k(
            std::span<const float>(logits, static_cast<std::size_t>(logit_count)), static_cast<std::size_t>(experts),
            static_cast<std::size_t>(top_k), normalize != 0);
        for (std::size_t i = 0; i < selection.size(); ++i) {
            out_index[i] = static_cast<std::int32_t>(selection[i].expert_index);
            out_weight[i] = selection[i].weight;
        }
        return static_cast<int>(selection.size());
    } catch (const std::invalid_argument&) {
        return -1;
    }
}

// The inputs of LiteMind's matvec test (tests/KernelTest.cpp:28-48): mt19937(12345),
// uniform(-1, 1) floats, weights rounded to BF16 with round-to-nearest-even,
// drawn in the same order (all weights, then the input vector).
void ref_kerneltest_inputs(std::uint16_t* weights_bf16, float* input, std::size_t out_dim, std::size_t in_dim) {
    std::mt19937 generator(12345U);
    std::uniform_real_distribution<float> distribution(-1.0F, 1.0F);
    for (std::size_t i = 0; i < out_dim * in_dim; ++i) {
        const std::uint32_t bits = std::bit_cast<std::uint32_t>(distribution(generator));
        weights_bf16[i] = static_cast<std::uint16_t>((bits + 0x7fffU + ((bits >> 16U) & 1U)) >> 16U);
    }
    for (std::size_t i = 0; i < in_dim; ++i) {
        input[i] = distribution(generator);
    }
}

// ThreadPool::parallel_for visiting every index (tests/KernelTest.cpp:112-121).
void ref_parallel_for_visit(std::size_t workers, std::size_t count, std::int32_t* visits) {
    ThreadPool pool(workers);
    pool.parallel_for(count, [visits](std::size_t index) { visits[index] += 1; });
}

// ---- ExpertCache: LRU bookkeeping over synthetic blocks of a given byte size ----
struct RefCache {
    ExpertCache cache;
    std::vector<std::unique_ptr<Tensor>> metas;
};

void* ref_cache_create(std::uint64_t budget) {
    auto* c = new RefCache();
    c->cache.configure(budget);
    return c;
}
void ref_cache_destroy(void* handle) { delete static_cast<RefCache*>(handle); }
void ref_cache_configure(void* handle, std::uint64_t budget) { static_cast<RefCache*>(handle)->cache.configure(budget); }
void ref_cache_clear(void* handle) { static_cast<RefCache*>(handle)->cache.clear(); }
std::uint64_t ref_cache_make_key(std::size_t layer, std::size_t expert) { return ExpertCache::make_key(layer, expert); }

// Touches one expert whose gate, up and down matrices are [rows, cols], [rows, cols], [cols, rows] BF16.
void ref_cache_touch(void* handle, std::uint64_t key, std::size_t rows, std::size_t cols) {
    auto* c = static_cast<RefCache*>(handle);
    c->metas.push_back(std::make_unique<Tensor>("gate", std::vector<std::size_t>{rows, cols}, DataType::BFloat16, 0U));
    const Tensor* gate = c->metas.back().get();
    c->metas.push_back(std::make_unique<Tensor>("up", std::vector<std::size_t>{rows, cols}, DataType::BFloat16, 0U));
    const Tensor* up = c->metas.back().get();
    c->metas.push_back(std::make_unique<Tensor>("down", std::vector<std::size_t>{cols, rows}, DataType::BFloat16, 0U));
    const Tensor* down = c->metas.back().get();
    static const std::byte dummy{};
    ExpertCache::Block block{WeightView{nullptr, gate, &dummy}, WeightView{nullptr, up, &dummy},
                             WeightView{nullptr, down, &dummy}};
    c->cache.touch(key, block);
}

// counters: resident_bytes, resident_experts, loads, hits, evictions, bytes_streamed, enabled
void ref_cache_counters(void* handle, std::uint64_t* out7) {
    const ExpertCache& cache = static_cast<RefCache*>(handle)->cache;
    out7[0] = cache.resident_bytes();
    out7[1] = cache.resident_experts();
    out7[2] = cache.loads();
    out7[3] = cache.hits();
    out7[4] = cache.evictions();
    out7[5] = cache.bytes_streamed();
    out7[6] = cache.enabled() ? 1U : 0U;
}

// ---- The per-token MoE block, composed from the reference's kernels ----
//
// router: [E, H] fp32; gate/up: E pointers to [I, H]; down: E pointers to [H, I];
// shared_*: [S, H], [S, H], [H, S] or null; x, y: [T, H].
int ref_moe_layer(std::int32_t hidden, std::int32_t inter, std::int32_t experts, std::int32_t top_k,
                  std::int32_t shared_inter, std::int32_t normalize, float scale, std::int32_t n_group,
                  std::int32_t topk_group, std::int32_t group_limited, const float* router,
                  const std::uint16_t* const* gate, const std::uint16_t* const* up, const std::uint16_t* const* down,
                  const std::uint16_t* shared_gate, const std::uint16_t* shared_up, const std::uint16_t* shared_down,
                  const float* x, std::int64_t tokens, const float* logit_bias, float* y, std::int32_t* out_index,
                  float* out_weight, std::size_t workers) {
    ThreadPool& pool = pool_for(workers);
    const MoeRouter moe_router(routing_config(experts, top_k, n_group, topk_group, group_limited, normalize, scale));
    const std::size_t H = static_cast<std::size_t>(hidden);
    const std::size_t widest = static_cast<std::size_t>(std::max(inter, shared_inter));
    std::vector<float> normalised(H), ffn(H), gate_buffer(widest), up_buffer(widest), act(widest),
        router_logits(static_cast<std::size_t>(experts));
    std::vector<ExpertSelection> selection;

    auto feed_forward = [&](const std::uint16_t* g, const std::uint16_t* u, const std::uint16_t* d, std::size_t I,
                            float weight) {
        gemm::matvec_bf16(pool, g, normalised.data(), gate_buffer.data(), I, H);
        gemm::matvec_bf16(pool, u, normalised.data(), up_buffer.data(), I, H);
        gemm::silu_multiply(gate_buffer.data(), up_buffer.data(), act.data(), I);
        gemm::matvec_bf16_accumulate(pool, d, act.data(), ffn.data(), H, I, weight);
    };

    for (std::int64_t t = 0; t < tokens; ++t) {
        std::copy(x + t * hidden, x + (t + 1) * hidden, normalised.begin());
        std::fill(ffn.begin(), ffn.end(), 0.0F);
        gemm::matvec_f32(router, normalised.data(), router_logits.data(), static_cast<std::size_t>(experts), H);
        if (logit_bias != nullptr) {
            for (std::int32_t e = 0; e < experts; ++e) {
                router_logits[static_cast<std::size_t>(e)] += logit_bias[e];
            }
        }
        moe_router.select(router_logits, selection);
        if (static_cast<std::int32_t>(selection.size()) != top_k) {
            return -1;
        }
        for (std::size_t r = 0; r < selection.size(); ++r) {
            const std::size_t e = selection[r].expert_index;
            if (out_index != nullptr) {
                out_index[t * top_k + static_cast<std::int64_t>(r)] = static_cast<std::int32_t>(e);
                out_weight[t * top_k + static_cast<std::int64_t>(r)] = selection[r].weight;
            }
            feed_forward(gate[e], up[e], down[e], static_cast<std::size_t>(inter), selection[r].weight);
        }
        if (shared_gate != nullptr && shared_inter > 0) {
            feed_forward(shared_gate, shared_up, shared_down, static_cast<std::size_t>(shared_inter), 1.0F);
        }
        std::copy(ffn.begin(), ffn.end(), y + t * hidden);
    }
    return 0;
}

}  // extern "C"
