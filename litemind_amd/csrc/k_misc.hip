// k_misc.hip -- combine/un-permute, residency conversions, RMSNorm, plain GEMV.
#include "lm_internal.h"

namespace lm {
namespace {

// y[t] = sum over ranks r of w[t,r] * down[slot(t,r)], accumulated in rank order
// as out += w * dot (src/DeepSeekRunner.cpp:277-284, src/Gemm.cpp:172, which GCC
// fuses), then + shared (:285-288), optionally + residual (gemm::axpy, :290).
// A gather in a fixed order per token: deterministic, no float atomics.
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int quads = a.hidden / 4;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= a.tokens * quads) {
        return;
    }
    const int64_t t = i / quads;
    const int c = static_cast<int>(i - t * quads) * 4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int r = 0; r < a.top_k; ++r) {
        const int64_t s = a.slot_of[t * a.top_k + r];
        const float w = a.wts[t * a.top_k + r];
        const float4 d = *reinterpret_cast<const float4*>(a.down_out + s * a.hidden + c);
        acc.x = __builtin_fmaf(w, d.x, acc.x);
        acc.y = __builtin_fmaf(w, d.y, acc.y);
        acc.z = __builtin_fmaf(w, d.z, acc.z);
        acc.w = __builtin_fmaf(w, d.w, acc.w);
    }
    if (a.has_shared) {
        const int64_t s = a.tokens * a.top_k + t;
        const float4 d = *reinterpret_cast<const float4*>(a.down_out + s * a.hidden + c);
        acc.x = acc.x + d.x;
        acc.y = acc.y + d.y;
        acc.z = acc.z + d.z;
        acc.w = acc.w + d.w;
    }
    if (a.residual != nullptr) {
        const float4 h = *reinterpret_cast<const float4*>(a.residual + t * a.hidden + c);
        acc.x = h.x + acc.x;
        acc.y = h.y + acc.y;
        acc.z = h.z + acc.z;
        acc.w = h.w + acc.w;
    }
    *reinterpret_cast<float4*>(a.y + t * a.hidden + c) = acc;
}

// BF16 -> fp16 re-encoding of resident weights for the MFMA path.  Exact for
// every BF16 value of magnitude in [2^-17, 65504]; smaller ones round to fp16
// subnormals (absolute error <= 2^-25), larger ones would overflow and are
// counted so the host can refuse the layer.
__global__ __launch_bounds__(256) void bf16_to_f16_kernel(const uint16_t* __restrict__ src, _Float16* __restrict__ dst,
                                                          int64_t n, int* overflow) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int bad = 0;
    for (int64_t k = i; k < n; k += stride) {
        const float v = widen_bf16(src[k]);
        bad += (v > 65504.0f || v < -65504.0f) ? 1 : 0;
        dst[k] = static_cast<_Float16>(v);
    }
    if (bad != 0) {
        atomicAdd(overflow, bad);
    }
}

// gemm::rms_norm per row (src/Gemm.cpp:197-207): sum of squares in double
// (exact squares, tree order), inverse = float(1 / sqrt(mean + eps)), then
// x * inverse * weight with two fp32 roundings.  One workgroup per row.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* in, const float* w, float* out, int32_t cols,
                                                       float eps) {
    __shared__ double part[4];
    const int64_t row = blockIdx.x;
    const float* x = in + row * cols;
    double s = 0.0;
    for (int c = threadIdx.x; c < cols; c += blockDim.x) {
        const double v = static_cast<double>(x[c]);
        s = s + v * v;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        s += __shfl_xor(s, o);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = s;
    }
    __syncthreads();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    const float inverse =
        static_cast<float>(1.0 / __builtin_sqrt(total / static_cast<double>(cols) + static_cast<double>(eps)));
    for (int c = threadIdx.x; c < cols; c += blockDim.x) {
        const float scaled = x[c] * inverse;
        out[row * cols + c] = scaled * w[c];
    }
}

// out[r] = W[r] . x or out[r] += scale * (W[r] . x) for a plain row-major BF16
// matrix (gemm::matvec_bf16 / matvec_bf16_accumulate, src/Gemm.cpp:139-175).
// One wave per row.
__global__ __launch_bounds__(256) void gemv_plain_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                         float* out, int64_t out_dim, int64_t in_dim, float scale,
                                                         int accumulate) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= out_dim) {
        return;
    }
    const uint16_t* wr = w + row * in_dim;
    float acc = 0.0f;
    if ((in_dim & 7) == 0) {
        for (int64_t c = lane * 8; c < in_dim; c += 512) {
            const uint4 q = *reinterpret_cast<const uint4*>(wr + c);
            const float4 x0 = *reinterpret_cast<const float4*>(x + c);
            const float4 x1 = *reinterpret_cast<const float4*>(x + c + 4);
            acc = __builtin_fmaf(bits_float(q.x << 16), x0.x, acc);
            acc = __builtin_fmaf(bits_float(q.x & 0xffff0000u), x0.y, acc);
            acc = __builtin_fmaf(bits_float(q.y << 16), x0.z, acc);
            acc = __builtin_fmaf(bits_float(q.y & 0xffff0000u), x0.w, acc);
            acc = __builtin_fmaf(bits_float(q.z << 16), x1.x, acc);
            acc = __builtin_fmaf(bits_float(q.z & 0xffff0000u), x1.y, acc);
            acc = __builtin_fmaf(bits_float(q.w << 16), x1.z, acc);
            acc = __builtin_fmaf(bits_float(q.w & 0xffff0000u), x1.w, acc);
        }
    } else {
        for (int64_t c = lane; c < in_dim; c += 64) {
            acc = __builtin_fmaf(widen_bf16(wr[c]), x[c], acc);
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        acc += __shfl_xor(acc, o);
    }
    if (lane == 0) {
        out[row] = accumulate ? __builtin_fmaf(scale, acc, out[row]) : acc;
    }
}

// x16[t, c] = fp16(x[t, c]) for c < cols, 0 for cols <= c < cols_p.
__global__ __launch_bounds__(256) void to_f16_rows_kernel(const float* __restrict__ x, _Float16* __restrict__ x16,
                                                          int64_t rows, int32_t cols, int32_t cols_p) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= rows * cols_p) {
        return;
    }
    const int64_t r = i / cols_p;
    const int c = static_cast<int>(i - r * cols_p);
    x16[i] = c < cols ? static_cast<_Float16>(x[r * cols + c]) : static_cast<_Float16>(0.0f);
}

}  // namespace

hipError_t launch_to_f16_rows(const float* x, _Float16* x16, int64_t rows, int32_t cols, int32_t cols_p,
                              hipStream_t s) {
    const int64_t n = rows * cols_p;
    if (n <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(to_f16_rows_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, x, x16,
                       rows, cols, cols_p);
    return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    const int64_t n = a.tokens * (a.hidden / 4);
    hipLaunchKernelGGL(combine_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_bf16_to_f16(const uint16_t* src, _Float16* dst, int64_t n, int* overflow, hipStream_t s) {
    if (n <= 0) {
        return hipSuccess;
    }
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) {
        blocks = 65536;
    }
    hipLaunchKernelGGL(bf16_to_f16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src, dst, n,
                       overflow);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float* in, const float* w, float* out, int64_t rows, int32_t cols, float eps,
                           hipStream_t s) {
    if (rows <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(256), 0, s, in, w, out, cols, eps);
    return hipGetLastError();
}

hipError_t launch_gemv_plain(const uint16_t* w, const float* x, float* out, int64_t out_dim, int64_t in_dim,
                             float scale, int32_t accumulate, hipStream_t s) {
    if (out_dim <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(gemv_plain_kernel, dim3(static_cast<unsigned>((out_dim + 3) / 4)), dim3(256), 0, s, w, x, out,
                       out_dim, in_dim, scale, accumulate);
    return hipGetLastError();
}

}  // namespace lm
