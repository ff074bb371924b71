#pragma once
// Process-wide GPU session behind the drop-in classes, and the batched MoE block.
//
// LiteMind's gemm:: functions and ExpertCache take no device argument, so the
// drop-in binds them to one lm_context per process (device 0, or the device named
// by LITEMIND_DEVICE).  Status codes from the C ABI become std::runtime_error
// carrying lm_last_error(), except in the noexcept functions LiteMind declares
// (ExpertCache::configure), which never call the GPU.

#include "Config.hpp"
#include "WeightStore.hpp"

#include <cstddef>
#include <cstdint>
#include <span>
#include <vector>

struct lm_context;
struct lm_moe_config;
struct lm_mla_config;

namespace litemind::gpu {

/** Throws std::runtime_error with lm_last_error() when status is not LM_OK. */
void check(int status, const char* what);

/** The process-wide context used by gemm:: and ExpertCache (created on first use). */
lm_context* session();

/** The device the drop-in uses: 0, or the one LITEMIND_DEVICE names. */
int device();

/** A new context of `num_layers` layers of width `hidden` for callers that use
 * only its non-MoE services (attention); the caller destroys it. */
lm_context* create_context(std::size_t hidden, int num_layers);

/** A context whose routing policy matches `config` (cached per policy). */
lm_context* router_session(const lm_moe_config& config);

/** lm_moe_config for a LiteMind Config (its MoE subset). */
lm_moe_config moe_config(const Config& config, int num_layers);

/** lm_mla_config for a LiteMind Config (its attention subset), with `positions`
 * rotary table rows and KV cache capacity per layer. */
lm_mla_config mla_config(const Config& config, std::int64_t positions);

/**
 * The MoE block of DeepSeekRunner::Impl::forward (src/DeepSeekRunner.cpp:273-290)
 * for T tokens at once: router, selection, six routed SwiGLU experts in rank
 * order, the shared expert, all resident in HBM.  This is the throughput path a
 * runner uses in place of the per-token loop over gemm:: calls.
 */
class MoeBlockGpu final {
public:
    MoeBlockGpu(const Config& config, int num_layers, int device = 0);
    ~MoeBlockGpu();
    MoeBlockGpu(const MoeBlockGpu&) = delete;
    MoeBlockGpu& operator=(const MoeBlockGpu&) = delete;

    /** Uploads one MoE layer: router [E, H] fp32, per-expert gate/up/down, shared (optional). */
    void upload_layer(int layer, std::span<const float> router, std::span<const WeightView> gate,
                      std::span<const WeightView> up, std::span<const WeightView> down,
                      const WeightView* shared_gate, const WeightView* shared_up, const WeightView* shared_down);

    /**
     * y[T, H] = MoE(x[T, H]) from host buffers (copied in and out; the device work
     * is the batched path).  index / weight receive the selection [T, k] in rank
     * order when non-empty.
     */
    void forward(int layer, std::span<const float> x, std::size_t tokens, std::span<float> y,
                 std::span<std::int32_t> index = {}, std::span<float> weight = {});

    [[nodiscard]] lm_context* context() const noexcept { return ctx_; }

private:
    void reserve(std::size_t tokens);

    lm_context* ctx_{nullptr};
    std::size_t hidden_{};
    std::size_t top_k_{};
    std::size_t capacity_{};
    void* x_dev_{nullptr};
    void* y_dev_{nullptr};
    void* idx_dev_{nullptr};
    void* w_dev_{nullptr};
};

}  // namespace litemind::gpu
