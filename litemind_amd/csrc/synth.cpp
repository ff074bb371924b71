// synth.cpp -- seeded synthetic tensors for the MoE workloads (host only).
//
// Every tensor is a pure function of (seed, stream, element index): a
// counter-based SplitMix64 gives two uniforms per element pair and Box-Muller in
// double turns them into normals, which are scaled, rounded to fp32 (RNE) and,
// for weights, to BF16 (RNE, as LiteMind's tests write BF16:
// tests/KernelTest.cpp:15-20).  Tensors are generated on the host and uploaded,
// so the GPU path and the CPU oracle see identical bits.  Generation is split
// across threads by element range; the result does not depend on the split.
#include "lm_math.h"

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

namespace {

inline uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Standard normal for element `index` of stream (seed, stream).
inline double normal_at(uint64_t seed, uint64_t stream, uint64_t index) {
    const uint64_t pair = index >> 1;
    const uint64_t key = splitmix64(seed ^ splitmix64(stream + 0x632be59bd9b4e019ull));
    const uint64_t a = splitmix64(key + 2 * pair);
    const uint64_t b = splitmix64(key + 2 * pair + 1);
    const double u1 = (static_cast<double>(a >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
    const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;          // [0, 1)
    const double radius = std::sqrt(-2.0 * std::log(u1));
    const double angle = 6.283185307179586476925286766559 * u2;
    return (index & 1) ? radius * std::sin(angle) : radius * std::cos(angle);
}

inline uint16_t bf16_rne(float value) {
    const uint32_t bits = lm::float_bits(value);
    return static_cast<uint16_t>((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

template <typename Body>
void split(std::size_t n, int threads, Body body) {
    if (threads <= 0) {
        threads = static_cast<int>(std::thread::hardware_concurrency());
    }
    if (threads <= 1 || n < (1u << 16)) {
        body(0, n);
        return;
    }
    if (threads > 64) {
        threads = 64;
    }
    std::vector<std::thread> pool;
    const std::size_t chunk = (n + static_cast<std::size_t>(threads) - 1) / static_cast<std::size_t>(threads);
    for (int t = 0; t < threads; ++t) {
        const std::size_t first = chunk * static_cast<std::size_t>(t);
        const std::size_t last = first + chunk < n ? first + chunk : n;
        if (first >= last) {
            break;
        }
        pool.emplace_back([=] { body(first, last); });
    }
    for (auto& th : pool) {
        th.join();
    }
}

}  // namespace

extern "C" {

// out[i] = fp32(sigma * N(0,1)) for i in [0, n).
void lms_normal_f32(uint64_t seed, uint64_t stream, float sigma, float* out, std::size_t n, int threads) {
    split(n, threads, [=](std::size_t first, std::size_t last) {
        for (std::size_t i = first; i < last; ++i) {
            out[i] = static_cast<float>(static_cast<double>(sigma) * normal_at(seed, stream, i));
        }
    });
}

// out[i] = bf16(fp32(sigma * N(0,1))).
void lms_normal_bf16(uint64_t seed, uint64_t stream, float sigma, uint16_t* out, std::size_t n, int threads) {
    split(n, threads, [=](std::size_t first, std::size_t last) {
        for (std::size_t i = first; i < last; ++i) {
            out[i] = bf16_rne(static_cast<float>(static_cast<double>(sigma) * normal_at(seed, stream, i)));
        }
    });
}

// Row-wise RMSNorm with unit weight, as the inputs of the MoE block are
// "normalised" activations: x / sqrt(mean(x^2) + eps), sum in double.
void lms_rms_rows(float* x, std::size_t rows, std::size_t cols, float eps, int threads) {
    split(rows, threads, [=](std::size_t first, std::size_t last) {
        for (std::size_t r = first; r < last; ++r) {
            float* row = x + r * cols;
            double sum = 0.0;
            for (std::size_t c = 0; c < cols; ++c) {
                sum += static_cast<double>(row[c]) * static_cast<double>(row[c]);
            }
            const float inv = static_cast<float>(1.0 / std::sqrt(sum / static_cast<double>(cols) + eps));
            for (std::size_t c = 0; c < cols; ++c) {
                row[c] = row[c] * inv;
            }
        }
    });
}

// The kernels' expf, compiled for the host, so tests can compare it with the C library.
void lms_expf_ref(const float* in, float* out, std::size_t n) {
    for (std::size_t i = 0; i < n; ++i) {
        out[i] = lm::expf_ref(in[i]);
    }
}

// Counts, over every float whose bits are k * stride (k = 0, 1, ...) and lie in
// [lo, hi], how often lm::expf_ref differs from the C library's expf.
uint64_t lms_expf_sweep(uint32_t stride, float lo, float hi, uint64_t* checked) {
    uint64_t bad = 0, n = 0;
    const int64_t steps = static_cast<int64_t>((0x100000000ull + stride - 1) / stride);
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : bad, n)
    for (int64_t i = 0; i < steps; ++i) {
        const float x = lm::bits_float(static_cast<uint32_t>(static_cast<uint64_t>(i) * stride));
        if (!(x >= lo && x <= hi)) {
            continue;
        }
        ++n;
        if (lm::float_bits(lm::expf_ref(x)) != lm::float_bits(::expf(x))) {
            ++bad;
        }
    }
    if (checked != nullptr) {
        *checked = n;
    }
    return bad;
}

}  // extern "C"
