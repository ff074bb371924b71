#pragma once
// litemind::ExpertCache with LiteMind's interface and bookkeeping
// (include/ExpertCache.hpp:29-89, src/ExpertCache.cpp:5-76): a byte-budgeted LRU
// over expert blocks.  Here "resident" means resident in HBM: a load uploads the
// block's three matrices (lm_weight_prefetch), an eviction frees their device
// copies (lm_weight_release), and gemm:: calls on a resident matrix read it from
// HBM instead of crossing PCIe.  As in LiteMind, residency never changes a result.

#include "WeightStore.hpp"

#include <cstdint>
#include <list>
#include <unordered_map>

namespace litemind {

class ExpertCache final {
public:
    struct Block final {
        WeightView gate;
        WeightView up;
        WeightView down;

        [[nodiscard]] std::uint64_t byte_size() const noexcept {
            return gate.byte_size() + up.byte_size() + down.byte_size();
        }
    };

    ExpertCache() = default;

    void configure(std::uint64_t budget_bytes) noexcept;
    void touch(std::uint64_t key, const Block& block);
    void clear();

    [[nodiscard]] bool enabled() const noexcept { return budget_bytes_ != 0U; }
    [[nodiscard]] std::uint64_t budget_bytes() const noexcept { return budget_bytes_; }
    [[nodiscard]] std::uint64_t resident_bytes() const noexcept { return resident_bytes_; }
    [[nodiscard]] std::size_t resident_experts() const noexcept { return entries_.size(); }

    [[nodiscard]] std::uint64_t loads() const noexcept { return loads_; }
    [[nodiscard]] std::uint64_t hits() const noexcept { return hits_; }
    [[nodiscard]] std::uint64_t evictions() const noexcept { return evictions_; }
    [[nodiscard]] std::uint64_t bytes_streamed() const noexcept { return bytes_streamed_; }

    [[nodiscard]] static std::uint64_t make_key(std::size_t layer, std::size_t expert) noexcept {
        return (static_cast<std::uint64_t>(layer) << 32U) | static_cast<std::uint32_t>(expert);
    }

private:
    struct Entry final {
        Block block;
        std::uint64_t bytes{};
        std::list<std::uint64_t>::iterator position;
    };

    void evict_oldest();

    std::uint64_t budget_bytes_{};
    std::uint64_t resident_bytes_{};
    std::list<std::uint64_t> recency_;  // most recently used first
    std::unordered_map<std::uint64_t, Entry> entries_;

    std::uint64_t loads_{};
    std::uint64_t hits_{};
    std::uint64_t evictions_{};
    std::uint64_t bytes_streamed_{};
};

}  // namespace litemind
