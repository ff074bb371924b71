#pragma once
// litemind::KvCache's interface (include/KvCache.hpp:23-84): host storage in
// KvCache's layout, which LiteMind's inline accessors address directly.
// Inside LiteMind its own header takes this file's place; the drop-in's
// KvCache.cpp and Attention.cpp use only the members declared here, under the
// same names.  The device copy of a cache lives in the attention context and is
// kept in step by Attention::forward.

#include <cstddef>
#include <cstdint>
#include <vector>

namespace litemind {

class KvCache final {
public:
    KvCache() = default;

    void configure(std::size_t num_heads, std::size_t qk_nope_head_dim, std::size_t qk_rope_head_dim,
                   std::size_t v_head_dim, std::size_t max_tokens);
    void clear() noexcept { token_count_ = 0U; }
    [[nodiscard]] std::size_t append() noexcept;

    [[nodiscard]] std::size_t token_count() const noexcept { return token_count_; }
    [[nodiscard]] std::size_t capacity() const noexcept { return capacity_; }
    [[nodiscard]] bool full() const noexcept { return token_count_ >= capacity_; }
    [[nodiscard]] std::uint64_t reserved_bytes() const noexcept;

    // entry `token`: [heads, qk_nope] keys, [qk_rope] rotary key, [heads, v_head] values
    [[nodiscard]] float* key_nope(std::size_t token) noexcept {
        return key_nope_.data() + token * num_heads_ * qk_nope_head_dim_;
    }
    [[nodiscard]] float* key_rope(std::size_t token) noexcept { return key_rope_.data() + token * qk_rope_head_dim_; }
    [[nodiscard]] float* value(std::size_t token) noexcept { return value_.data() + token * num_heads_ * v_head_dim_; }
    [[nodiscard]] const float* key_nope(std::size_t token, std::size_t head) const noexcept {
        return key_nope_.data() + (token * num_heads_ + head) * qk_nope_head_dim_;
    }
    [[nodiscard]] const float* key_rope(std::size_t token) const noexcept {
        return key_rope_.data() + token * qk_rope_head_dim_;
    }
    [[nodiscard]] const float* value(std::size_t token, std::size_t head) const noexcept {
        return value_.data() + (token * num_heads_ + head) * v_head_dim_;
    }

private:
    std::size_t num_heads_{};
    std::size_t qk_nope_head_dim_{};
    std::size_t qk_rope_head_dim_{};
    std::size_t v_head_dim_{};
    std::size_t capacity_{};
    std::size_t token_count_{};
    std::vector<float> key_nope_;
    std::vector<float> key_rope_;
    std::vector<float> value_;
};

}  // namespace litemind
