// k_head.hip -- the LM head and the greedy choice of the next token.
//
// Reference: the end of DeepSeekRunner::Impl::forward (src/DeepSeekRunner.cpp:
// 296-300): rms_norm with the final norm weight, then gemm::matvec_bf16 over
// the [V, H] head; and Sampler::select_next's greedy branch
// (src/Sampler.cpp:117-126), std::max_element over the logits.
//
// The logits follow gemm::dot_bf16's association (src/Gemm.cpp:46-82) bit for
// bit, like gemv_plain_kernel: 32 sequential fused chains over the elements
// i = c (mod 32), chains 0..7 continuing over the 8-wide remainder, then
// (a0+a1)+(a2+a3) per lane, lanes j and j+4 added, (h0+h2)+(h1+h3), and a fused
// scalar tail.  A chain's elements lie 64 bytes apart, so instead of each lane
// loading them one by one, a block stages chunks of its 8 rows in LDS with
// 16-byte coalesced loads and the 32 lanes of a row read their chains from
// there.  The head streams 420 MB at V = 102400, H = 2048: the kernel is bound
// by HBM.
#include "lm_internal.h"

namespace lm {
namespace {

constexpr int kRows = 8;                  // head rows per block, 32 lanes each
constexpr int kChunk = 1024;              // row elements staged per step
constexpr int kPitch = kChunk + 32;       // LDS row pitch (elements): the two rows of a wave on different banks
constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void head_logits_kernel(const uint16_t* __restrict__ w,
                                                               const float* __restrict__ x, float* logits,
                                                               int64_t rows, int32_t in_dim, int32_t tokens) {
    __shared__ __align__(16) uint16_t ws[kRows * kPitch];
    __shared__ float part[kRows][33];
    const int tid = threadIdx.x;
    const int c = tid & 31;
    const int slot = tid >> 5;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * kRows;
    const int64_t row = r0 + slot;
    const bool live = row < rows;
    const int n32 = in_dim / 32 * 32;
    const int n8 = n32 + (in_dim - n32) / 8 * 8;
    float acc[kHeadTokens];
#pragma unroll
    for (int t = 0; t < kHeadTokens; ++t) {
        acc[t] = 0.0f;
    }
    for (int k0 = 0; k0 < n32; k0 += kChunk) {
        const int len = n32 - k0 < kChunk ? n32 - k0 : kChunk;  // a multiple of 32
        const int pieces = len / 8;                                // 16-byte pieces per row
        for (int f = tid; f < kRows * pieces; f += kThreads) {
            const int rr = f / pieces;
            const int p = f - rr * pieces;
            const int64_t grow = r0 + rr < rows ? r0 + rr : rows - 1;
            *reinterpret_cast<uint4*>(ws + rr * kPitch + 8 * p) = load_stream16(w + grow * in_dim + k0 + 8 * p);
        }
        __syncthreads();
        if (live) {
            const uint16_t* wr = ws + slot * kPitch + c;
            for (int s = 0; s < len / 32; ++s) {
                const float wv = widen_bf16(wr[32 * s]);
                const int i = k0 + c + 32 * s;
#pragma unroll
                for (int t = 0; t < kHeadTokens; ++t) {
                    if (t < tokens) {
                        acc[t] = __builtin_fmaf(wv, x[static_cast<int64_t>(t) * in_dim + i], acc[t]);
                    }
                }
            }
        }
        __syncthreads();
    }
    const uint16_t* wrow = w + (live ? row : 0) * in_dim;
    if (live && c < 8) {
        for (int i = n32 + c; i < n8; i += 8) {
            const float wv = widen_bf16(wrow[i]);
#pragma unroll
            for (int t = 0; t < kHeadTokens; ++t) {
                if (t < tokens) {
                    acc[t] = __builtin_fmaf(wv, x[static_cast<int64_t>(t) * in_dim + i], acc[t]);
                }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kHeadTokens; ++t) {
        if (t >= tokens) {
            break;
        }
        part[slot][c] = acc[t];
        __syncthreads();
        if (live && c == 0) {
            const float* a = part[slot];
            float lane_sum[8];
            for (int l = 0; l < 8; ++l) {
                const float low = a[l] + a[8 + l];
                const float high = a[16 + l] + a[24 + l];
                lane_sum[l] = low + high;
            }
            const float h0 = lane_sum[0] + lane_sum[4];
            const float h1 = lane_sum[1] + lane_sum[5];
            const float h2 = lane_sum[2] + lane_sum[6];
            const float h3 = lane_sum[3] + lane_sum[7];
            float total = (h0 + h2) + (h1 + h3);
            const float* xt = x + static_cast<int64_t>(t) * in_dim;
            for (int i = n8; i < in_dim; ++i) {
                total = __builtin_fmaf(widen_bf16(wrow[i]), xt[i], total);
            }
            logits[static_cast<int64_t>(t) * rows + row] = total;
        }
        __syncthreads();
    }
}

// (value, index) of the greedy choice so far; `have` false until a non-NaN value.
struct Best {
    float v;
    int32_t i;
    int32_t have;
};

// Combines two candidates: the larger value, the lower index between equal
// values (IEEE equality: -0 equals +0), NaN never chosen.  Associative, so
// the order of the tree does not matter.
__device__ inline Best better(Best a, Best b) {
    if (!b.have) {
        return a;
    }
    if (!a.have || b.v > a.v || (b.v == a.v && b.i < a.i)) {
        return b;
    }
    return a;
}

// Sampler::select_next's greedy branch: std::max_element keeps the first of
// equal values and moves only on a strictly larger one, so a NaN never becomes
// the choice, except at index 0, which nothing after it can replace.  That is
// the first maximum of the non-NaN logits, or 0 when logit 0 is NaN.
__global__ __launch_bounds__(1024) void argmax_first_kernel(const float* __restrict__ logits, int64_t vocab,
                                                            int32_t* out) {
    __shared__ Best wave_best[16];
    const float* l = logits + static_cast<int64_t>(blockIdx.x) * vocab;
    Best b{0.0f, 0, 0};
    for (int64_t i = threadIdx.x; i < vocab; i += 1024) {
        const float v = l[i];
        if (v == v && (!b.have || v > b.v)) {
            b = Best{v, static_cast<int32_t>(i), 1};
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const Best other{__shfl_xor(b.v, o), __shfl_xor(b.i, o), __shfl_xor(b.have, o)};
        b = better(b, other);
    }
    if ((threadIdx.x & 63) == 0) {
        wave_best[threadIdx.x >> 6] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        Best r = wave_best[0];
        for (int k = 1; k < 16; ++k) {
            r = better(r, wave_best[k]);
        }
        const float first = l[0];
        out[blockIdx.x] = (first != first || !r.have) ? 0 : r.i;
    }
}

}  // namespace

hipError_t launch_head_logits(const uint16_t* w, const float* x, float* logits, int64_t rows, int32_t in_dim,
                              int32_t tokens, hipStream_t s) {
    if (rows <= 0 || tokens <= 0) {
        return hipSuccess;
    }
    if (tokens > kHeadTokens || in_dim <= 0 || in_dim % 8 != 0) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(head_logits_kernel, dim3(static_cast<unsigned>((rows + kRows - 1) / kRows)), dim3(kThreads), 0,
                       s, w, x, logits, rows, in_dim, tokens);
    return hipGetLastError();
}

hipError_t launch_argmax_first(const float* logits, int64_t vocab, int64_t tokens, int32_t* out, hipStream_t s) {
    if (tokens <= 0) {
        return hipSuccess;
    }
    if (vocab <= 0 || vocab > INT32_MAX) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(argmax_first_kernel, dim3(static_cast<unsigned>(tokens)), dim3(1024), 0, s, logits, vocab, out);
    return hipGetLastError();
}

}  // namespace lm
