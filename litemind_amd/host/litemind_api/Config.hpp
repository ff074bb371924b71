#pragma once
// The fields of litemind::Config (include/Config.hpp:31-115) that the MoE
// feed-forward path reads, with DeepSeek-V2-Lite's defaults.  Dropped into
// LiteMind, its own Config.hpp takes the place of this file: the drop-in sources
// read only the members declared here, under the same names and types.

#include <cstddef>
#include <string>

namespace litemind {

class Config final {
public:
    std::size_t hidden_size{2048U};
    std::size_t num_hidden_layers{27U};
    float rms_norm_eps{1e-6F};

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

    [[nodiscard]] std::size_t shared_expert_intermediate_size() const noexcept {
        return moe_intermediate_size * n_shared_experts;
    }
};

}  // namespace litemind
