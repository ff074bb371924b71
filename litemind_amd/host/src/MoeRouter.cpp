// litemind::MoeRouter on the GPU (behaviour of src/MoeRouter.cpp:38-130).
#include "MoeRouter.hpp"

#include "litemind_gpu.hpp"
#include "litemind_moe.h"

#include <algorithm>
#include <mutex>
#include <stdexcept>

namespace litemind {
namespace {

// Device staging for one token's logits and selection, per router context.
struct Staging {
    float* logits = nullptr;
    std::int32_t* index = nullptr;
    float* weight = nullptr;
};

Staging& staging_for(lm_context* ctx, std::size_t experts, std::size_t top_k) {
    static std::mutex mutex;
    static auto* table = new std::vector<std::pair<lm_context*, Staging>>();
    std::lock_guard<std::mutex> lock(mutex);
    for (auto& entry : *table) {
        if (entry.first == ctx) {
            return entry.second;
        }
    }
    Staging s;
    void* p = nullptr;
    gpu::check(lm_alloc(ctx, experts * sizeof(float), &p), "lm_alloc");
    s.logits = static_cast<float*>(p);
    gpu::check(lm_alloc(ctx, top_k * sizeof(std::int32_t), &p), "lm_alloc");
    s.index = static_cast<std::int32_t*>(p);
    gpu::check(lm_alloc(ctx, top_k * sizeof(float), &p), "lm_alloc");
    s.weight = static_cast<float*>(p);
    table->emplace_back(ctx, s);
    return table->back().second;
}

}  // namespace

MoeRouter::MoeRouter(const Config& config)
    : expert_count_(config.n_routed_experts),
      top_k_(config.num_experts_per_tok),
      n_group_(std::max<std::size_t>(config.n_group, 1U)),
      topk_group_(std::max<std::size_t>(config.topk_group, 1U)),
      group_limited_(config.topk_method == "group_limited_greedy"),
      normalize_(config.norm_topk_prob),
      routed_scaling_factor_(config.routed_scaling_factor) {
    if (expert_count_ % n_group_ != 0U) {
        group_limited_ = false;  // groups that do not divide the experts: plain greedy
        n_group_ = 1U;
    }
}

void MoeRouter::select(std::span<const float> gate_logits, std::vector<ExpertSelection>& selection) const {
    selection.clear();
    if (gate_logits.size() != expert_count_ || top_k_ == 0U || expert_count_ == 0U) {
        return;  // LiteMind returns an empty selection on a size mismatch
    }
    const std::size_t k = std::min(top_k_, expert_count_);
    lm_moe_config c{};
    c.n_routed_experts = static_cast<int32_t>(expert_count_);
    c.num_experts_per_tok = static_cast<int32_t>(k);
    c.norm_topk_prob = normalize_ ? 1 : 0;
    c.routed_scaling_factor = routed_scaling_factor_;
    c.group_limited = group_limited_ && n_group_ > 1U ? 1 : 0;
    c.n_group = static_cast<int32_t>(n_group_);
    c.topk_group = static_cast<int32_t>(std::min(topk_group_, n_group_));
    lm_context* ctx = gpu::router_session(c);
    Staging& s = staging_for(ctx, expert_count_, k);
    gpu::check(lm_copy_h2d(ctx, s.logits, gate_logits.data(), expert_count_ * sizeof(float)), "lm_copy_h2d");
    gpu::check(lm_router_select(ctx, s.logits, 1, s.index, s.weight), "lm_router_select");
    std::vector<std::int32_t> index(k);
    std::vector<float> weight(k);
    gpu::check(lm_copy_d2h(ctx, index.data(), s.index, k * sizeof(std::int32_t)), "lm_copy_d2h");
    gpu::check(lm_copy_d2h(ctx, weight.data(), s.weight, k * sizeof(float)), "lm_copy_d2h");
    selection.reserve(k);
    for (std::size_t r = 0; r < k; ++r) {
        selection.push_back(ExpertSelection{static_cast<std::size_t>(index[r]), weight[r]});
    }
}

std::vector<ExpertSelection> MoeRouter::select(std::span<const float> gate_logits) const {
    std::vector<ExpertSelection> selection;
    select(gate_logits, selection);
    return selection;
}

std::vector<ExpertSelection> MoeRouter::select_top_k(std::span<const float> gate_logits, std::size_t expert_count,
                                                     std::size_t top_k, bool normalize_selected_weights) {
    if (expert_count == 0U || top_k == 0U || top_k > expert_count || gate_logits.size() != expert_count) {
        throw std::invalid_argument("MoE routing requires one logit per expert and a valid top-k value.");
    }
    Config config;
    config.n_routed_experts = expert_count;
    config.num_experts_per_tok = top_k;
    config.norm_topk_prob = normalize_selected_weights;
    config.routed_scaling_factor = 1.0F;
    config.topk_method = "greedy";
    config.n_group = 1U;
    config.topk_group = 1U;
    return MoeRouter(config).select(gate_logits);
}

}  // namespace litemind
