#pragma once
// namespace litemind::gemm with LiteMind's signatures (include/Gemm.hpp:23-72),
// executed on the GPU through liblitemind_moe.so.  Every function returns results
// bit-identical to LiteMind's AVX2 build: the kernels restate its association
// order (dot_bf16's four 8-lane accumulators, matvec_f32's left-to-right sum)
// and its expf.  Calls are synchronous; a HIP failure throws std::runtime_error.

#include "Threading.hpp"

#include <cstddef>
#include <cstdint>
#include <string>

namespace litemind {
namespace gemm {

[[nodiscard]] std::string kernel_description();

void matvec_bf16(ThreadPool& pool, const std::uint16_t* weights, const float* input, float* out,
                 std::size_t out_dim, std::size_t in_dim);

void matvec_bf16_accumulate(ThreadPool& pool, const std::uint16_t* weights, const float* input, float* out,
                            std::size_t out_dim, std::size_t in_dim, float scale);

void matvec_bf16_serial(const std::uint16_t* weights, const float* input, float* out, std::size_t out_dim,
                        std::size_t in_dim);

void matvec_f32(const float* weights, const float* input, float* out, std::size_t out_dim, std::size_t in_dim);

void widen_bf16(const std::uint16_t* source, float* destination, std::size_t count);

[[nodiscard]] float dot(const float* left, const float* right, std::size_t count);

void axpy(float scale, const float* source, float* destination, std::size_t count);

void rms_norm(float* values, const float* weight, std::size_t count, float epsilon);

void softmax(float* values, std::size_t count);

void silu_multiply(const float* gate, const float* up, float* destination, std::size_t count);

}  // namespace gemm
}  // namespace litemind
