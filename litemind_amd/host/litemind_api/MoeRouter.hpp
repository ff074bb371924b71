#pragma once
// litemind::MoeRouter and ExpertSelection with LiteMind's signatures
// (include/MoeRouter.hpp:12-55).  select() runs the selection on the GPU
// (softmax over all experts, top-k with LiteMind's comparator, normalise XOR
// scale, optional group mask) and returns exactly what LiteMind's router returns.

#include "Config.hpp"

#include <cstddef>
#include <span>
#include <vector>

namespace litemind {

struct ExpertSelection final {
    std::size_t expert_index{};
    float weight{};
};

class MoeRouter final {
public:
    MoeRouter() = default;
    explicit MoeRouter(const Config& config);

    void select(std::span<const float> gate_logits, std::vector<ExpertSelection>& selection) const;

    [[nodiscard]] std::vector<ExpertSelection> select(std::span<const float> gate_logits) const;

    [[nodiscard]] static std::vector<ExpertSelection> select_top_k(std::span<const float> gate_logits,
                                                                   std::size_t expert_count, std::size_t top_k,
                                                                   bool normalize_selected_weights);

private:
    std::size_t expert_count_{64U};
    std::size_t top_k_{6U};
    std::size_t n_group_{1U};
    std::size_t topk_group_{1U};
    bool group_limited_{false};
    bool normalize_{false};
    float routed_scaling_factor_{1.0F};
};

}  // namespace litemind
