// KvCache (include/KvCache.hpp, src/KvCache.cpp): the host copy LiteMind's
// inline accessors address.  The attention drop-in (Attention.cpp) keeps a
// device copy of each cache it is given in step with this one: it truncates
// the device entries past token_count() (KvCache::clear is inline and cannot
// reach the GPU), uploads entries written here that the device lacks, and
// writes each entry it appends back here.
#include "KvCache.hpp"

namespace litemind {

void KvCache::configure(std::size_t num_heads, std::size_t qk_nope_head_dim, std::size_t qk_rope_head_dim,
                        std::size_t v_head_dim, std::size_t max_tokens) {
    num_heads_ = num_heads;
    qk_nope_head_dim_ = qk_nope_head_dim;
    qk_rope_head_dim_ = qk_rope_head_dim;
    v_head_dim_ = v_head_dim;
    capacity_ = max_tokens;
    token_count_ = 0U;
    // zero-filled storage for every position, as LiteMind reserves it
    key_nope_.assign(max_tokens * num_heads * qk_nope_head_dim, 0.0F);
    key_rope_.assign(max_tokens * qk_rope_head_dim, 0.0F);
    value_.assign(max_tokens * num_heads * v_head_dim, 0.0F);
}

std::size_t KvCache::append() noexcept {
    // the next free position, or capacity() once every position is taken
    return token_count_ < capacity_ ? token_count_++ : capacity_;
}

std::uint64_t KvCache::reserved_bytes() const noexcept {
    return sizeof(float) * (static_cast<std::uint64_t>(key_nope_.size()) + key_rope_.size() + value_.size());
}

}  // namespace litemind
