// GPU session management and the batched MoE block for the drop-in layer.
#include "litemind_gpu.hpp"

#include "litemind_attention.h"
#include "litemind_moe.h"

#include <cstdlib>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <tuple>

namespace litemind::gpu {
namespace {

int device_from_env() {
    const char* value = std::getenv("LITEMIND_DEVICE");
    return value != nullptr ? std::atoi(value) : 0;
}

// Contexts live until the process ends: LiteMind's callers hold no handle to
// release them, and destroying device state during static destruction races
// the HIP runtime's own teardown.
struct Sessions {
    std::mutex mutex;
    lm_context* main = nullptr;
    std::map<std::tuple<int, int, int, float, int, int, int>, lm_context*> routers;
};

Sessions& sessions() {
    static Sessions* instance = new Sessions();
    return *instance;
}

lm_moe_config minimal_config() {
    lm_moe_config c{};
    c.hidden_size = 16;
    c.moe_intermediate_size = 16;
    c.n_routed_experts = 1;
    c.num_experts_per_tok = 1;
    c.n_shared_experts = 0;
    c.intermediate_size = 0;
    c.norm_topk_prob = 0;
    c.routed_scaling_factor = 1.0F;
    c.group_limited = 0;
    c.n_group = 1;
    c.topk_group = 1;
    c.rms_norm_eps = 1e-6F;
    c.num_layers = 1;
    return c;
}

}  // namespace

void check(int status, const char* what) {
    if (status != LM_OK) {
        throw std::runtime_error(std::string(what) + ": " + lm_last_error());
    }
}

int device() { return device_from_env(); }

lm_context* create_context(std::size_t hidden, int num_layers) {
    lm_moe_config c = minimal_config();
    c.hidden_size = static_cast<int32_t>(hidden);
    c.num_layers = num_layers > 0 ? num_layers : 1;
    lm_context* ctx = nullptr;
    check(lm_context_create(device_from_env(), &c, &ctx), "lm_context_create");
    return ctx;
}

lm_context* session() {
    Sessions& s = sessions();
    std::lock_guard<std::mutex> lock(s.mutex);
    if (s.main == nullptr) {
        const lm_moe_config c = minimal_config();
        check(lm_context_create(device_from_env(), &c, &s.main), "lm_context_create");
    }
    return s.main;
}

lm_context* router_session(const lm_moe_config& config) {
    Sessions& s = sessions();
    std::lock_guard<std::mutex> lock(s.mutex);
    const auto key = std::make_tuple(config.n_routed_experts, config.num_experts_per_tok, config.norm_topk_prob,
                                     config.routed_scaling_factor, config.group_limited, config.n_group,
                                     config.topk_group);
    auto it = s.routers.find(key);
    if (it != s.routers.end()) {
        return it->second;
    }
    lm_moe_config c = minimal_config();
    c.n_routed_experts = config.n_routed_experts;
    c.num_experts_per_tok = config.num_experts_per_tok;
    c.norm_topk_prob = config.norm_topk_prob;
    c.routed_scaling_factor = config.routed_scaling_factor;
    c.group_limited = config.group_limited;
    c.n_group = config.n_group;
    c.topk_group = config.topk_group;
    lm_context* ctx = nullptr;
    check(lm_context_create(device_from_env(), &c, &ctx), "lm_context_create");
    s.routers.emplace(key, ctx);
    return ctx;
}

lm_moe_config moe_config(const Config& config, int num_layers) {
    lm_moe_config c{};
    c.hidden_size = static_cast<int32_t>(config.hidden_size);
    c.moe_intermediate_size = static_cast<int32_t>(config.moe_intermediate_size);
    c.n_routed_experts = static_cast<int32_t>(config.n_routed_experts);
    c.num_experts_per_tok = static_cast<int32_t>(config.num_experts_per_tok);
    c.n_shared_experts = static_cast<int32_t>(config.n_shared_experts);
    c.intermediate_size = static_cast<int32_t>(config.intermediate_size);
    c.norm_topk_prob = config.norm_topk_prob ? 1 : 0;
    c.routed_scaling_factor = config.routed_scaling_factor;
    const std::size_t groups = config.n_group > 1U ? config.n_group : 1U;
    // MoeRouter's constructor (src/MoeRouter.cpp:38-52): the group mask applies
    // only for group_limited_greedy, and falls back to greedy when the groups do
    // not divide the experts.
    const bool grouped = config.topk_method == "group_limited_greedy" && config.n_routed_experts % groups == 0U;
    c.group_limited = grouped ? 1 : 0;
    c.n_group = grouped ? static_cast<int32_t>(groups) : 1;
    c.topk_group = grouped ? static_cast<int32_t>(config.topk_group > 1U ? config.topk_group : 1U) : 1;
    c.rms_norm_eps = config.rms_norm_eps;
    c.num_layers = num_layers;
    return c;
}

lm_mla_config mla_config(const Config& config, std::int64_t positions) {
    lm_mla_config c{};
    c.hidden_size = static_cast<int32_t>(config.hidden_size);
    c.num_heads = static_cast<int32_t>(config.num_attention_heads);
    c.q_lora_rank = static_cast<int32_t>(config.q_lora_rank);
    c.kv_lora_rank = static_cast<int32_t>(config.kv_lora_rank);
    c.qk_nope_head_dim = static_cast<int32_t>(config.qk_nope_head_dim);
    c.qk_rope_head_dim = static_cast<int32_t>(config.qk_rope_head_dim);
    c.v_head_dim = static_cast<int32_t>(config.v_head_dim);
    c.rms_norm_eps = config.rms_norm_eps;
    c.rope_theta = static_cast<double>(config.rope_theta);
    c.yarn = config.rope_scaling.enabled ? 1 : 0;
    c.factor = config.rope_scaling.factor;
    c.beta_fast = config.rope_scaling.beta_fast;
    c.beta_slow = config.rope_scaling.beta_slow;
    c.mscale = config.rope_scaling.mscale;
    c.mscale_all_dim = config.rope_scaling.mscale_all_dim;
    c.original_max_positions = static_cast<int64_t>(config.rope_scaling.original_max_position_embeddings);
    c.context_length = positions;
    return c;
}

MoeBlockGpu::MoeBlockGpu(const Config& config, int num_layers, int device)
    : hidden_(config.hidden_size), top_k_(config.num_experts_per_tok) {
    const lm_moe_config c = moe_config(config, num_layers);
    check(lm_context_create(device, &c, &ctx_), "lm_context_create");
}

MoeBlockGpu::~MoeBlockGpu() {
    if (ctx_ != nullptr) {
        (void)lm_context_destroy(ctx_);  // frees the context's buffers and weights
    }
}

void MoeBlockGpu::upload_layer(int layer, std::span<const float> router, std::span<const WeightView> gate,
                               std::span<const WeightView> up, std::span<const WeightView> down,
                               const WeightView* shared_gate, const WeightView* shared_up,
                               const WeightView* shared_down) {
    if (gate.size() != up.size() || gate.size() != down.size()) {
        throw std::invalid_argument("gate, up and down need one view per routed expert");
    }
    check(lm_upload_router(ctx_, layer, router.data()), "lm_upload_router");
    for (std::size_t e = 0; e < gate.size(); ++e) {
        check(lm_upload_expert(ctx_, layer, static_cast<int32_t>(e), gate[e].as_bf16(), up[e].as_bf16(),
                               down[e].as_bf16()),
              "lm_upload_expert");
    }
    if (shared_gate != nullptr && shared_up != nullptr && shared_down != nullptr) {
        check(lm_upload_shared(ctx_, layer, shared_gate->as_bf16(), shared_up->as_bf16(), shared_down->as_bf16()),
              "lm_upload_shared");
    }
    check(lm_finalize_layer(ctx_, layer), "lm_finalize_layer");
}

void MoeBlockGpu::reserve(std::size_t tokens) {
    if (tokens <= capacity_) {
        return;
    }
    for (void* p : {x_dev_, y_dev_, idx_dev_, w_dev_}) {
        if (p != nullptr) {
            check(lm_free(ctx_, p), "lm_free");
        }
    }
    x_dev_ = y_dev_ = idx_dev_ = w_dev_ = nullptr;
    capacity_ = 0;
    check(lm_alloc(ctx_, tokens * hidden_ * sizeof(float), &x_dev_), "lm_alloc");
    check(lm_alloc(ctx_, tokens * hidden_ * sizeof(float), &y_dev_), "lm_alloc");
    check(lm_alloc(ctx_, tokens * top_k_ * sizeof(std::int32_t), &idx_dev_), "lm_alloc");
    check(lm_alloc(ctx_, tokens * top_k_ * sizeof(float), &w_dev_), "lm_alloc");
    capacity_ = tokens;
}

void MoeBlockGpu::forward(int layer, std::span<const float> x, std::size_t tokens, std::span<float> y,
                          std::span<std::int32_t> index, std::span<float> weight) {
    if (x.size() < tokens * hidden_ || y.size() < tokens * hidden_) {
        throw std::invalid_argument("x and y need tokens * hidden_size floats");
    }
    if ((!index.empty() && index.size() < tokens * top_k_) || (!weight.empty() && weight.size() < tokens * top_k_)) {
        throw std::invalid_argument("index and weight need tokens * num_experts_per_tok entries");
    }
    if (tokens == 0) {
        return;
    }
    reserve(tokens);
    check(lm_copy_h2d(ctx_, x_dev_, x.data(), tokens * hidden_ * sizeof(float)), "lm_copy_h2d");
    check(lm_moe_forward(ctx_, layer, static_cast<const float*>(x_dev_), static_cast<int64_t>(tokens),
                         static_cast<float*>(y_dev_), nullptr, static_cast<int32_t*>(idx_dev_),
                         static_cast<float*>(w_dev_), nullptr, LM_PATH_AUTO),
          "lm_moe_forward");
    // Kernel-side failures (a single-token hand-off wait that gave up) are
    // reported when the stream drains, not by the enqueueing call.
    check(lm_synchronize(ctx_), "lm_synchronize");
    check(lm_copy_d2h(ctx_, y.data(), y_dev_, tokens * hidden_ * sizeof(float)), "lm_copy_d2h");
    if (!index.empty()) {
        check(lm_copy_d2h(ctx_, index.data(), idx_dev_, tokens * top_k_ * sizeof(std::int32_t)), "lm_copy_d2h");
    }
    if (!weight.empty()) {
        check(lm_copy_d2h(ctx_, weight.data(), w_dev_, tokens * top_k_ * sizeof(float)), "lm_copy_d2h");
    }
}

}  // namespace litemind::gpu
