// namespace litemind::gemm on the GPU (signatures of include/Gemm.hpp:23-72).
#include "Gemm.hpp"

#include "litemind_gpu.hpp"
#include "litemind_moe.h"

#include <string>

namespace litemind::gemm {
namespace {

void vector_op(int op, const void* a, const float* b, float* out, std::size_t count, float scalar,
               const char* what) {
    gpu::check(lm_vector_op(gpu::session(), op, a, b, out, count, scalar), what);
}

}  // namespace

std::string kernel_description() {
    int32_t major = 0;
    int32_t minor = 0;
    (void)lm_version(&major, &minor);
    return "gfx950 HIP (MI355X), liblitemind_moe " + std::to_string(major) + "." + std::to_string(minor) +
           ", LiteMind AVX2+FMA rounding";
}

void matvec_bf16(ThreadPool& /*pool*/, const std::uint16_t* weights, const float* input, float* out,
                 std::size_t out_dim, std::size_t in_dim) {
    gpu::check(lm_gemm_matvec_bf16(gpu::session(), weights, input, out, out_dim, in_dim, 1.0F, 0),
               "gemm::matvec_bf16");
}

void matvec_bf16_accumulate(ThreadPool& /*pool*/, const std::uint16_t* weights, const float* input, float* out,
                            std::size_t out_dim, std::size_t in_dim, float scale) {
    gpu::check(lm_gemm_matvec_bf16(gpu::session(), weights, input, out, out_dim, in_dim, scale, 1),
               "gemm::matvec_bf16_accumulate");
}

void matvec_bf16_serial(const std::uint16_t* weights, const float* input, float* out, std::size_t out_dim,
                        std::size_t in_dim) {
    // LiteMind's serial and threaded products agree bit for bit (the pool only
    // splits rows), and so does the single GPU kernel.
    gpu::check(lm_gemm_matvec_bf16(gpu::session(), weights, input, out, out_dim, in_dim, 1.0F, 0),
               "gemm::matvec_bf16_serial");
}

void matvec_f32(const float* weights, const float* input, float* out, std::size_t out_dim, std::size_t in_dim) {
    gpu::check(lm_gemm_matvec_f32(gpu::session(), weights, input, out, out_dim, in_dim), "gemm::matvec_f32");
}

void widen_bf16(const std::uint16_t* source, float* destination, std::size_t count) {
    vector_op(LM_OP_WIDEN, source, nullptr, destination, count, 0.0F, "gemm::widen_bf16");
}

float dot(const float* left, const float* right, std::size_t count) {
    float result = 0.0F;
    vector_op(LM_OP_DOT, left, right, &result, count, 0.0F, "gemm::dot");
    return result;
}

void axpy(float scale, const float* source, float* destination, std::size_t count) {
    vector_op(LM_OP_AXPY, source, nullptr, destination, count, scale, "gemm::axpy");
}

void rms_norm(float* values, const float* weight, std::size_t count, float epsilon) {
    vector_op(LM_OP_RMS_NORM, values, weight, values, count, epsilon, "gemm::rms_norm");
}

void softmax(float* values, std::size_t count) {
    vector_op(LM_OP_SOFTMAX, values, nullptr, values, count, 0.0F, "gemm::softmax");
}

void silu_multiply(const float* gate, const float* up, float* destination, std::size_t count) {
    vector_op(LM_OP_SILU_MUL, gate, up, destination, count, 0.0F, "gemm::silu_multiply");
}

}  // namespace litemind::gemm
