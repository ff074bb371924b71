// litemind::ExpertCache with HBM residency (bookkeeping of src/ExpertCache.cpp:5-76).
#include "ExpertCache.hpp"

#include "litemind_gpu.hpp"
#include "litemind_moe.h"

namespace litemind {
namespace {

// A view with no bytes (bookkeeping-only callers, such as tests of the LRU
// policy) has nothing to move; LiteMind's WeightView::prefetch is a no-op for it
// too (src/WeightStore.cpp:40-50).
void upload(const WeightView& view) {
    if (view.bytes != nullptr && view.byte_size() != 0U) {
        gpu::check(lm_weight_prefetch(gpu::session(), view.bytes, view.byte_size()), "lm_weight_prefetch");
    }
}

void drop(const WeightView& view) {
    if (view.bytes != nullptr && view.byte_size() != 0U) {
        gpu::check(lm_weight_release(gpu::session(), view.bytes), "lm_weight_release");
    }
}

}  // namespace

void ExpertCache::configure(std::uint64_t budget_bytes) noexcept { budget_bytes_ = budget_bytes; }

void ExpertCache::touch(std::uint64_t key, const Block& block) {
    if (!enabled()) {
        return;
    }
    if (auto found = entries_.find(key); found != entries_.end()) {
        recency_.splice(recency_.begin(), recency_, found->second.position);
        found->second.position = recency_.begin();
        ++hits_;
        return;
    }
    const std::uint64_t bytes = block.byte_size();
    while (!recency_.empty() && resident_bytes_ + bytes > budget_bytes_) {
        evict_oldest();  // room first, so the budget is never exceeded transiently
    }
    upload(block.gate);
    upload(block.up);
    upload(block.down);
    recency_.push_front(key);
    entries_.emplace(key, Entry{block, bytes, recency_.begin()});
    resident_bytes_ += bytes;
    bytes_streamed_ += bytes;
    ++loads_;
}

void ExpertCache::evict_oldest() {
    if (recency_.empty()) {
        return;
    }
    const std::uint64_t key = recency_.back();
    recency_.pop_back();
    auto found = entries_.find(key);
    if (found == entries_.end()) {
        return;
    }
    drop(found->second.block.gate);
    drop(found->second.block.up);
    drop(found->second.block.down);
    resident_bytes_ -= found->second.bytes;
    entries_.erase(found);
    ++evictions_;
}

void ExpertCache::clear() {
    while (!recency_.empty()) {
        evict_oldest();
    }
    entries_.clear();
    resident_bytes_ = 0U;
}

}  // namespace litemind
