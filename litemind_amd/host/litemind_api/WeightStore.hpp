#pragma once
// The part of litemind::WeightView (include/WeightStore.hpp:22-48) that the MoE
// path uses: a borrowed pointer to a weight's bytes and its size.  Inside
// LiteMind the real WeightView (which also carries the shard and tensor
// metadata) takes this file's place; the drop-in sources use only `bytes`,
// byte_size() and as_bf16().

#include <cstddef>
#include <cstdint>

namespace litemind {

struct WeightView final {
    const std::byte* bytes{nullptr};
    std::uint64_t size{0U};

    [[nodiscard]] bool valid() const noexcept { return bytes != nullptr; }
    [[nodiscard]] std::uint64_t byte_size() const noexcept { return size; }
    [[nodiscard]] const std::uint16_t* as_bf16() const noexcept {
        return reinterpret_cast<const std::uint16_t*>(bytes);
    }
};

}  // namespace litemind
