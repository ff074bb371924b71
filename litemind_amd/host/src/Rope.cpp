// RotaryEmbedding (include/Rope.hpp, src/Rope.cpp) with its tables built by the
// library (lm_rope_tables, the same builder the GPU attention's tables come
// from, bit for bit RotaryEmbedding::build's); apply() rotates on the host.
#include "Rope.hpp"

#include "litemind_attention.h"
#include "litemind_gpu.hpp"

#include <algorithm>
#include <cmath>
#include <sstream>

namespace litemind {

void RotaryEmbedding::build(const Config& config, std::size_t max_positions) {
    dimension_ = config.qk_rope_head_dim;
    half_ = dimension_ / 2U;
    max_positions_ = std::max<std::size_t>(max_positions, 1U);
    yarn_ = config.rope_scaling.enabled;
    // the frequencies stay inside the library; only the tables are kept here
    inverse_frequency_.clear();
    cosine_.assign(max_positions_ * half_, 0.0F);
    sine_.assign(max_positions_ * half_, 0.0F);
    if (half_ > 0U) {
        const lm_mla_config c = gpu::mla_config(config, static_cast<std::int64_t>(max_positions_));
        gpu::check(lm_rope_tables(&c, static_cast<std::int64_t>(max_positions_), cosine_.data(), sine_.data()),
                   "RotaryEmbedding::build");
    }
    // YaRN's amplitude ratio (src/Rope.cpp:82-87), reported by summary()
    magnitude_scale_ = 1.0;
    if (yarn_) {
        const RopeScaling& s = config.rope_scaling;
        const double factor = s.factor <= 0.0 ? 1.0 : s.factor;
        auto mscale = [factor](double m) { return factor <= 1.0 ? 1.0 : 0.1 * m * std::log(factor) + 1.0; };
        magnitude_scale_ = mscale(s.mscale) / mscale(s.mscale_all_dim);
    }
}

void RotaryEmbedding::apply(float* values, std::size_t position) const noexcept {
    if (values == nullptr || half_ == 0U || position >= max_positions_) {
        return;
    }
    const float* const cos_row = cosine_.data() + position * half_;
    const float* const sin_row = sine_.data() + position * half_;
    // pairs (2i, 2i + 1) rotate into channels i and i + half: read from a copy,
    // since the outputs overwrite inputs later pairs still need
    thread_local std::vector<float> in;
    in.assign(values, values + dimension_);
    for (std::size_t i = 0; i < half_; ++i) {
        const float a = in[2U * i];
        const float b = in[2U * i + 1U];
        values[i] = a * cos_row[i] - b * sin_row[i];
        values[i + half_] = b * cos_row[i] + a * sin_row[i];
    }
}

std::string RotaryEmbedding::summary() const {
    std::ostringstream out;
    out << "rope dim=" << dimension_ << " positions=" << max_positions_;
    if (yarn_) {
        out << " yarn (magnitude x" << magnitude_scale_ << ")";
    } else {
        out << " unscaled";
    }
    return out.str();
}

}  // namespace litemind
