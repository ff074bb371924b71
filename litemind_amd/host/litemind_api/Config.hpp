#pragma once
// The fields of litemind::Config (include/Config.hpp:31-115) that the MoE
// feed-forward path and the attention drop-in read, with DeepSeek-V2-Lite's
// defaults.  Dropped into LiteMind, its own Config.hpp takes the place of this
// file: the drop-in sources read only the members declared here, under the same
// names and types.

#include <cstddef>
#include <string>

namespace litemind {

// include/Config.hpp:14-27
struct RopeScaling final {
    bool enabled{false};
    std::string type{"yarn"};
    double factor{1.0};
    double beta_fast{32.0};
    double beta_slow{1.0};
    double mscale{1.0};
    double mscale_all_dim{0.0};
    std::size_t original_max_position_embeddings{4096U};
};

class Config final {
public:
    std::size_t hidden_size{2048U};
    std::size_t num_hidden_layers{27U};
    std::size_t num_attention_heads{16U};
    float rms_norm_eps{1e-6F};

    std::size_t kv_lora_rank{512U};
    std::size_t q_lora_rank{0U};
    std::size_t qk_nope_head_dim{128U};
    std::size_t qk_rope_head_dim{64U};
    std::size_t v_head_dim{128U};
    float rope_theta{10000.0F};
    RopeScaling rope_scaling{};

    std::size_t intermediate_size{10944U};
    std::size_t moe_intermediate_size{1408U};
    std::size_t n_routed_experts{64U};
    std::size_t n_shared_experts{2U};
    std::size_t num_experts_per_tok{6U};
    std::size_t first_k_dense_replace{1U};
    bool norm_topk_prob{false};
    float routed_scaling_factor{1.0F};
    std::string topk_method{"greedy"};
    std::size_t n_group{1U};
    std::size_t topk_group{1U};

    [[nodiscard]] std::size_t qk_head_dim() const noexcept { return qk_nope_head_dim + qk_rope_head_dim; }

    [[nodiscard]] std::size_t shared_expert_intermediate_size() const noexcept {
        return moe_intermediate_size * n_shared_experts;
    }
};

}  // namespace litemind
