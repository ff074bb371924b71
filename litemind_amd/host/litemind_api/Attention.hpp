#pragma once
// litemind::Attention's interface and AttentionWeights (include/Attention.hpp:
// 14-73).  Inside LiteMind its own header takes this file's place; the drop-in's
// Attention.cpp uses only the members declared here, under the same names.

#include "Config.hpp"
#include "KvCache.hpp"
#include "Rope.hpp"
#include "Threading.hpp"
#include "WeightStore.hpp"

#include <cstddef>
#include <vector>

namespace litemind {

struct AttentionWeights final {
    WeightView q_proj;                 // q_lora_rank == 0: [heads * qk_head_dim, hidden]
    WeightView q_a_proj;               // q_lora_rank > 0: [q_lora_rank, hidden]
    std::vector<float> q_a_layernorm;  // [q_lora_rank]
    WeightView q_b_proj;               // [heads * qk_head_dim, q_lora_rank]
    WeightView kv_a_proj;              // [kv_lora_rank + qk_rope_head_dim, hidden]
    std::vector<float> kv_a_layernorm; // [kv_lora_rank]
    WeightView kv_b_proj;              // [heads * (qk_nope_head_dim + v_head_dim), kv_lora_rank]
    WeightView o_proj;                 // [hidden, heads * v_head_dim]
};

class Attention final {
public:
    Attention() = default;

    void configure(const Config& config, ThreadPool& pool, const RotaryEmbedding& rope);
    [[nodiscard]] bool forward(const float* input, const AttentionWeights& weights, KvCache& cache,
                               std::size_t position, float* output);

private:
    const Config* config_{nullptr};
    ThreadPool* pool_{nullptr};
    const RotaryEmbedding* rope_{nullptr};
};

}  // namespace litemind
