// Attention::configure / forward (include/Attention.hpp:45-60) on the GPU.  The
// whole of forward for one token (projections, rotary steps, cache append,
// causal attention over the cache, output projection; src/Attention.cpp:22-103)
// is lm_attention_forward over weights and a KV cache resident in HBM, bit for
// bit LiteMind's result.
//
// Each configured Attention owns a device context with one attention layer per
// KvCache it is given (up to Config::num_hidden_layers, as DeepSeekRunner keeps
// one cache per layer), whose rotary tables and cache capacity are the
// RotaryEmbedding's max_positions(): positions past the table skip the rotation
// as RotaryEmbedding::apply does, so the host KvCache's capacity must not exceed
// it (DeepSeekRunner sizes both from the context length).  A layer's weights are
// uploaded when the layer first sees them and again whenever a call passes
// other weights; LiteMind's weights are read-only views of the mapped
// checkpoint, so their host addresses identify them.
//
// The host KvCache stays LiteMind's (its accessors are inline).  Before each
// call the device cache is brought to the host's token_count(): entries past it
// are dropped (KvCache::clear cannot reach the GPU) and entries the device
// lacks are uploaded from the host (written through KvCache's accessors).  The
// entry a call appends is written back into the host cache.  Host entries
// overwritten in place after the device has them are not uploaded again.
#include "Attention.hpp"

#include "litemind_attention.h"
#include "litemind_gpu.hpp"
#include "litemind_moe.h"

#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace litemind {
namespace {

// The host addresses of one layer's weights.
struct WeightsId {
    const std::byte* q = nullptr;
    const std::byte* q_a = nullptr;
    const float* q_a_norm = nullptr;
    const std::byte* q_b = nullptr;
    const std::byte* kv_a = nullptr;
    const float* kv_a_norm = nullptr;
    const std::byte* kv_b = nullptr;
    const std::byte* o = nullptr;
    bool operator==(const WeightsId&) const = default;
};

struct DeviceAttention {
    lm_context* ctx = nullptr;
    std::size_t hidden = 0;
    std::size_t positions = 0;
    int layers = 0;
    std::map<const KvCache*, int> layer_of;
    std::vector<WeightsId> held;  // per layer
    void* x = nullptr;            // one token's input and output, device
    void* y = nullptr;

    DeviceAttention(const Config& config, std::size_t rope_positions)
        : hidden(config.hidden_size), positions(rope_positions),
          layers(config.num_hidden_layers > 0 ? static_cast<int>(config.num_hidden_layers) : 1) {
        ctx = gpu::create_context(hidden, layers);
        try {
            const lm_mla_config c = gpu::mla_config(config, static_cast<std::int64_t>(positions));
            gpu::check(lm_attention_configure(ctx, &c), "lm_attention_configure");
            gpu::check(lm_alloc(ctx, hidden * sizeof(float), &x), "lm_alloc");
            gpu::check(lm_alloc(ctx, hidden * sizeof(float), &y), "lm_alloc");
        } catch (...) {
            (void)lm_context_destroy(ctx);
            throw;
        }
        held.resize(static_cast<std::size_t>(layers));
    }
    ~DeviceAttention() { (void)lm_context_destroy(ctx); }  // frees x, y, weights and caches
    DeviceAttention(const DeviceAttention&) = delete;
    DeviceAttention& operator=(const DeviceAttention&) = delete;

    int layer(const KvCache* cache) {
        const auto it = layer_of.find(cache);
        if (it != layer_of.end()) {
            return it->second;
        }
        const int next = static_cast<int>(layer_of.size());
        if (next >= layers) {
            throw std::runtime_error("Attention::forward: more KvCache objects than Config::num_hidden_layers (" +
                                     std::to_string(layers) + ")");
        }
        layer_of.emplace(cache, next);
        return next;
    }
};

// Device state per Attention object.  Never destroyed as a whole: a context
// outlives its Attention until the object is configured again (LiteMind's
// Attention has no destructor to hook), and tearing contexts down during static
// destruction would race the HIP runtime's own teardown.
struct Registry {
    std::mutex mutex;
    std::map<const Attention*, std::unique_ptr<DeviceAttention>> by_owner;
};

Registry& registry() {
    static Registry* instance = new Registry();
    return *instance;
}

}  // namespace

void Attention::configure(const Config& config, ThreadPool& pool, const RotaryEmbedding& rope) {
    config_ = &config;
    pool_ = &pool;
    rope_ = &rope;
    // the device context is made on the first forward, when the rotary table
    // it mirrors has been built
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mutex);
    r.by_owner.erase(this);
}

bool Attention::forward(const float* input, const AttentionWeights& weights, KvCache& cache, std::size_t position,
                        float* output) {
    if (cache.full()) {
        return false;  // KvCache::append refuses; LiteMind's forward returns false without output
    }
    const Config& config = *config_;
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mutex);
    std::unique_ptr<DeviceAttention>& owned = r.by_owner[this];
    if (owned == nullptr || owned->positions != rope_->max_positions()) {
        owned = std::make_unique<DeviceAttention>(config, rope_->max_positions());
    }
    DeviceAttention& d = *owned;
    if (cache.capacity() > d.positions) {
        throw std::runtime_error("Attention::forward: a KvCache of " + std::to_string(cache.capacity()) +
                                 " positions exceeds the rotary table's " + std::to_string(d.positions));
    }
    const int layer = d.layer(&cache);
    const bool lora = config.q_lora_rank != 0U;
    const WeightsId id{lora ? nullptr : weights.q_proj.bytes,   lora ? weights.q_a_proj.bytes : nullptr,
                       lora ? weights.q_a_layernorm.data() : nullptr, lora ? weights.q_b_proj.bytes : nullptr,
                       weights.kv_a_proj.bytes,                 weights.kv_a_layernorm.data(),
                       weights.kv_b_proj.bytes,                 weights.o_proj.bytes};
    WeightsId& held = d.held[static_cast<std::size_t>(layer)];
    if (!(held == id)) {
        held = WeightsId{};
        gpu::check(lm_upload_attention(d.ctx, layer, lora ? nullptr : weights.q_proj.as_bf16(),
                                       lora ? weights.q_a_proj.as_bf16() : nullptr, id.q_a_norm,
                                       lora ? weights.q_b_proj.as_bf16() : nullptr, weights.kv_a_proj.as_bf16(),
                                       id.kv_a_norm, weights.kv_b_proj.as_bf16(), weights.o_proj.as_bf16()),
                   "lm_upload_attention");
        held = id;
    }
    // the device cache to the host's count, then this token at slot `slot`
    const std::size_t slot = cache.token_count();
    std::int64_t have = 0;
    gpu::check(lm_kv_cache_tokens(d.ctx, layer, &have), "lm_kv_cache_tokens");
    const auto want = static_cast<std::int64_t>(slot);
    if (have > want) {
        gpu::check(lm_kv_cache_truncate(d.ctx, layer, want), "lm_kv_cache_truncate");
    } else if (have < want) {
        const auto from = static_cast<std::size_t>(have);
        gpu::check(lm_kv_cache_write(d.ctx, layer, have, want - have, cache.key_nope(from), cache.key_rope(from),
                                     cache.value(from)),
                   "lm_kv_cache_write");
    }
    const std::size_t bytes = d.hidden * sizeof(float);
    gpu::check(lm_copy_h2d(d.ctx, d.x, input, bytes), "lm_copy_h2d");
    gpu::check(lm_attention_forward(d.ctx, layer, static_cast<const float*>(d.x), 1,
                                    static_cast<std::int64_t>(position), static_cast<float*>(d.y), 0),
               "lm_attention_forward");
    gpu::check(lm_copy_d2h(d.ctx, output, d.y, bytes), "lm_copy_d2h");
    gpu::check(lm_kv_cache_read_range(d.ctx, layer, want, 1, cache.key_nope(slot), cache.key_rope(slot),
                                      cache.value(slot)),
               "lm_kv_cache_read_range");
    (void)cache.append();  // == slot
    return true;
}

}  // namespace litemind
