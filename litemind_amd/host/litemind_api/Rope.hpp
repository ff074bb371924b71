#pragma once
// litemind::RotaryEmbedding's interface (include/Rope.hpp:28-52).  Inside
// LiteMind its own header takes this file's place; the drop-in's Rope.cpp uses
// only the members declared here, under the same names.

#include "Config.hpp"

#include <cstddef>
#include <string>
#include <vector>

namespace litemind {

class RotaryEmbedding final {
public:
    RotaryEmbedding() = default;

    void build(const Config& config, std::size_t max_positions);
    void apply(float* values, std::size_t position) const noexcept;

    [[nodiscard]] std::size_t dimension() const noexcept { return dimension_; }
    [[nodiscard]] std::size_t max_positions() const noexcept { return max_positions_; }
    [[nodiscard]] std::string summary() const;

private:
    std::size_t dimension_{};
    std::size_t half_{};
    std::size_t max_positions_{};
    double magnitude_scale_{1.0};
    bool yarn_{false};
    std::vector<float> cosine_;  // [max_positions_, half_]
    std::vector<float> sine_;
    std::vector<double> inverse_frequency_;
};

}  // namespace litemind
