// k_misc.hip -- combine/un-permute, residency conversions, RMSNorm, plain GEMV.
#include "lm_internal.h"

namespace lm {
namespace {

// y[t] = sum over ranks r of w[t,r] * down[slot(t,r)], accumulated in rank order
// as out += w * dot (src/DeepSeekRunner.cpp:277-284, src/Gemm.cpp:172, which GCC
// fuses), then + shared (:285-288), optionally + residual (gemm::axpy, :290).
// A gather in a fixed order per token: deterministic, no float atomics.  With
// K > 0 (the top-k known when compiling) the K rows' loads are all in flight
// before the first addition; K = 0 reads the top-k at run time, one row at a
// time.  The additions are the same either way.
template <int K>
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int quads = a.hidden / 4;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= a.tokens * quads) {
        return;
    }
    const int64_t t = i / quads;
    const int c = static_cast<int>(i - t * quads) * 4;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (K > 0) {
        float4 d[K];
        float w[K];
#pragma unroll
        for (int r = 0; r < K; ++r) {
            const int64_t s = a.slot_of[t * K + r];
            w[r] = a.wts[t * K + r];
            d[r] = *reinterpret_cast<const float4*>(a.down_out + s * a.hidden + c);
        }
#pragma unroll
        for (int r = 0; r < K; ++r) {
            acc.x = __builtin_fmaf(w[r], d[r].x, acc.x);
            acc.y = __builtin_fmaf(w[r], d[r].y, acc.y);
            acc.z = __builtin_fmaf(w[r], d[r].z, acc.z);
            acc.w = __builtin_fmaf(w[r], d[r].w, acc.w);
        }
    } else {
        for (int r = 0; r < a.top_k; ++r) {
            const int64_t s = a.slot_of[t * a.top_k + r];
            const float w = a.wts[t * a.top_k + r];
            const float4 d = *reinterpret_cast<const float4*>(a.down_out + s * a.hidden + c);
            acc.x = __builtin_fmaf(w, d.x, acc.x);
            acc.y = __builtin_fmaf(w, d.y, acc.y);
            acc.z = __builtin_fmaf(w, d.z, acc.z);
            acc.w = __builtin_fmaf(w, d.w, acc.w);
        }
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

// combine_kernel's sum for one token row, then the next layer's RMSNorm of the
// row just written (rms_norm_kernel's arithmetic: thread-strided double sums of
// exact squares, wave butterfly, (w0 + w1) + (w2 + w3), made LiteMind's by
// rms_inverse_exact) and its fp16 panel copy
// (to_f16_rows_kernel's conversion): the next layer's input is the same bits as
// the separate kernels', without reading the hidden state again.  One
// workgroup of 256 threads per token.  The row is formed as combine_kernel
// forms it (16-byte loads, thread t owning columns 4 t .. 4 t + 3 of every
// 1024-column step) and staged in LDS, where thread t then adds the squares of
// columns t, t + 256, ... in rms_norm_kernel's order.  hidden % 4 == 0 and
// hidden <= kCombineNormMax.  With K > 0 (the top-k known when compiling) and
// STEPS * 1024 >= hidden_p, every rank's slot and weight is read first and all
// rows' loads (ranks, shared, residual; clamped to column 0 past the row's
// end) are in flight together before the first addition; K = 0 reads the top-k
// at run time, one rank's loads at a time.  The additions are the same either
// way.
constexpr int kCombineNormMax = 8192;
constexpr int kCombineNormSteps = kCombineNormMax / 1024;

template <int K, int STEPS>
__global__ __launch_bounds__(256) void combine_norm_kernel(CombineArgs a) {
    __shared__ float row[STEPS * 1024];
    __shared__ double part[4];
    const int64_t t = blockIdx.x;
    const int H = a.hidden;
    const int tid = threadIdx.x;
    const float* __restrict__ dout = a.down_out;
    float4 y[STEPS];
#pragma unroll
    for (int k = 0; k < STEPS; ++k) {
        y[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // every load is issued before any store (y may be the residual)
    if constexpr (K > 0) {
        int64_t slot[K];
        float wt[K];
#pragma unroll
        for (int r = 0; r < K; ++r) {
            slot[r] = a.slot_of[t * K + r];
            wt[r] = a.wts[t * K + r];
        }
        const float* shared_row = a.has_shared ? dout + (a.tokens * K + t) * H : dout;
        const float* residual_row = a.residual != nullptr ? a.residual + t * H : dout;
        float4 d[K][STEPS], sh[STEPS], res[STEPS];
#pragma unroll
        for (int k = 0; k < STEPS; ++k) {
            const int c = 1024 * k + 4 * tid;
            const int cc = c < H ? c : 0;
#pragma unroll
            for (int r = 0; r < K; ++r) {
                d[r][k] = *reinterpret_cast<const float4*>(dout + slot[r] * H + cc);
            }
            sh[k] = *reinterpret_cast<const float4*>(shared_row + cc);
            res[k] = *reinterpret_cast<const float4*>(residual_row + cc);
        }
#pragma unroll
        for (int r = 0; r < K; ++r) {
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                y[k].x = __builtin_fmaf(wt[r], d[r][k].x, y[k].x);
                y[k].y = __builtin_fmaf(wt[r], d[r][k].y, y[k].y);
                y[k].z = __builtin_fmaf(wt[r], d[r][k].z, y[k].z);
                y[k].w = __builtin_fmaf(wt[r], d[r][k].w, y[k].w);
            }
        }
#pragma unroll
        for (int k = 0; k < STEPS; ++k) {
            if (a.has_shared) {
                y[k].x = y[k].x + sh[k].x;
                y[k].y = y[k].y + sh[k].y;
                y[k].z = y[k].z + sh[k].z;
                y[k].w = y[k].w + sh[k].w;
            }
            if (a.residual != nullptr) {
                y[k].x = res[k].x + y[k].x;
                y[k].y = res[k].y + y[k].y;
                y[k].z = res[k].z + y[k].z;
                y[k].w = res[k].w + y[k].w;
            }
        }
    } else {
        for (int r = 0; r < a.top_k; ++r) {
            const int64_t slot = a.slot_of[t * a.top_k + r];
            const float w = a.wts[t * a.top_k + r];
#pragma unroll
            for (int k = 0; k < STEPS; ++k) {
                const int c = 1024 * k + 4 * tid;
                if (c < H) {
                    const float4 d = *reinterpret_cast<const float4*>(dout + slot * H + c);
                    y[k].x = __builtin_fmaf(w, d.x, y[k].x);
                    y[k].y = __builtin_fmaf(w, d.y, y[k].y);
                    y[k].z = __builtin_fmaf(w, d.z, y[k].z);
                    y[k].w = __builtin_fmaf(w, d.w, y[k].w);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < STEPS; ++k) {
            const int c = 1024 * k + 4 * tid;
            if (c < H) {
                if (a.has_shared) {
                    const float4 d = *reinterpret_cast<const float4*>(dout + (a.tokens * a.top_k + t) * H + c);
                    y[k].x = y[k].x + d.x;
                    y[k].y = y[k].y + d.y;
                    y[k].z = y[k].z + d.z;
                    y[k].w = y[k].w + d.w;
                }
                if (a.residual != nullptr) {
                    const float4 h = *reinterpret_cast<const float4*>(a.residual + t * H + c);
                    y[k].x = h.x + y[k].x;
                    y[k].y = h.y + y[k].y;
                    y[k].z = h.z + y[k].z;
                    y[k].w = h.w + y[k].w;
                }
            }
        }
    }
#pragma unroll
    for (int k = 0; k < STEPS; ++k) {
        const int c = 1024 * k + 4 * tid;
        if (c < H) {
            *reinterpret_cast<float4*>(a.y + t * H + c) = y[k];
            *reinterpret_cast<float4*>(row + c) = y[k];
        }
    }
    __syncthreads();
    double s = 0.0;
    for (int c = tid; c < H; c += 256) {
        const double v = static_cast<double>(row[c]);
        s = s + v * v;
    }
    for (int o = 32; o >= 1; o >>= 1) {
        s += __shfl_xor(s, o);
    }
    if ((tid & 63) == 0) {
        part[tid >> 6] = s;
    }
    __syncthreads();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    const float inverse =
        rms_inverse_exact(total, H, a.eps, part, row, [] {}, [] { __syncthreads(); });
    typedef _Float16 half4 __attribute__((ext_vector_type(4)));
    const int Hp = a.hidden_p;
    for (int k = 0; 1024 * k < Hp; ++k) {
        const int c = 1024 * k + 4 * tid;
        if (c >= Hp) {
            continue;
        }
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (c < H) {
            float4 yy = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int kk = 0; kk < STEPS; ++kk) {
                if (kk == k) {
                    yy = y[kk];
                }
            }
            const float4 nw = *reinterpret_cast<const float4*>(a.next_norm + c);
            v.x = (yy.x * inverse) * nw.x;
            v.y = (yy.y * inverse) * nw.y;
            v.z = (yy.z * inverse) * nw.z;
            v.w = (yy.w * inverse) * nw.w;
            *reinterpret_cast<float4*>(a.xnorm + t * H + c) = v;
        }
        if (a.x16 != nullptr) {
            // from the rounded fp32 values, as to_f16_rows_kernel converts them:
            // the compiler would otherwise fold the products and the conversions
            // into mixed-precision instructions that round once, to fp16
            asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
            const half4 h = half4{static_cast<_Float16>(v.x), static_cast<_Float16>(v.y), static_cast<_Float16>(v.z),
                                  static_cast<_Float16>(v.w)};
            *reinterpret_cast<half4*>(a.x16 + panel_index(t, c, a.tokens)) = h;
        }
    }
}

// BF16 -> fp16 re-encoding of resident weights for the MFMA path, written in
// panel layout.  Exact for every BF16 value of magnitude in [2^-17, 65504];
// larger ones would overflow and are counted so the host can refuse the
// layer; smaller ones round to fp16 subnormals (absolute error <= 2^-25) and
// are counted into `inexact` (when not null) so the host can report them.
// Thread i produces destination element i (coalesced writes; reads within one
// panel row are contiguous).
__global__ __launch_bounds__(256) void bf16_to_f16_panels_kernel(const uint16_t* __restrict__ src,
                                                                 _Float16* __restrict__ dst, int64_t rows,
                                                                 int64_t cols, int* overflow,
                                                                 unsigned long long* inexact) {
    const int64_t n = rows * cols;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    int bad = 0;
    unsigned lossy = 0;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
        const int64_t panel = i / (rows * kPanel);
        const int64_t rem = i - panel * rows * kPanel;
        const int64_t r = rem / kPanel;
        const int64_t c = panel * kPanel + (rem - r * kPanel);
        const float v = widen_bf16(src[r * cols + c]);
        const bool big = v > 65504.0f || v < -65504.0f;
        const _Float16 h = static_cast<_Float16>(v);
        bad += big ? 1 : 0;
        lossy += (!big && v == v && static_cast<float>(h) != v) ? 1u : 0u;
        dst[i] = h;
    }
    if (bad != 0) {
        atomicAdd(overflow, bad);
    }
    if (inexact != nullptr && lossy != 0) {
        atomicAdd(inexact, static_cast<unsigned long long>(lossy));
    }
}

// gemm::rms_norm per row (src/Gemm.cpp:197-207): sum of squares in double
// (exact squares, tree order, made LiteMind's by rms_inverse_exact), inverse =
// float(1 / sqrt(mean + eps)), then x * inverse * weight with two fp32
// roundings.  One workgroup per row.
__global__ __launch_bounds__(256) void rms_norm_kernel(const float* in, const float* w, float* out, int32_t cols,
                                                       float eps) {
    __shared__ double part[4];
    const int64_t row = blockIdx.x;
    const float* x = in + row * cols;
    const float inverse = rms_inverse_256(x, cols, eps, part);
    // eight elements per thread per pass, loads first (one pass for 2048 columns)
    for (int c0 = static_cast<int>(threadIdx.x); c0 < cols; c0 += 8 * 256) {
        float v[8], wv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + 256 * u;
            const int cc = c < cols ? c : cols - 1;  // unconditional loads
            v[u] = x[cc];
            wv[u] = w[cc];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int c = c0 + 256 * u;
            if (c < cols) {
                const float scaled = v[u] * inverse;
                out[row * cols + c] = scaled * wv[u];
            }
        }
    }
}

// out[r] = W[r] . x or out[r] += scale * (W[r] . x) for a plain row-major BF16
// matrix (gemm::matvec_bf16 / matvec_bf16_accumulate, src/Gemm.cpp:139-175).
// One wave per row.
// out[row] = dot_bf16(w[row], x) in LiteMind's association order, bit for bit
// (src/Gemm.cpp:46-82, AVX2 + FMA branch): 32 fused chains over elements
// i = c (mod 32), chains 0..7 also take the 8-wide remainder, then
// (a0+a1)+(a2+a3) per lane, lanes j and j+4 added, (h0+h2)+(h1+h3), and a fused
// scalar tail.  32 lanes hold one row's chains, so a block takes 8 rows.
// With `accumulate` the row is folded as fma(scale, dot, out[row])
// (src/Gemm.cpp:156-175).
__global__ __launch_bounds__(256) void gemv_plain_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                         float* out, int64_t out_dim, int64_t in_dim, float scale,
                                                         int accumulate) {
    __shared__ float part[8][33];
    const int c = threadIdx.x & 31;
    const int slot = threadIdx.x >> 5;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + slot;
    const bool live = row < out_dim;
    const int64_t n32 = in_dim / 32 * 32;
    const int64_t n8 = n32 + (in_dim - n32) / 8 * 8;
    const uint16_t* wr = w + (live ? row : 0) * in_dim;
    float acc = 0.0f;
    if (live) {
        for (int64_t i = c; i < n32; i += 32) {
            acc = __builtin_fmaf(widen_bf16(wr[i]), x[i], acc);
        }
        if (c < 8) {
            for (int64_t i = n32 + c; i < n8; i += 8) {
                acc = __builtin_fmaf(widen_bf16(wr[i]), x[i], acc);
            }
        }
    }
    part[slot][c] = acc;
    __syncthreads();
    if (!live || c != 0) {
        return;
    }
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
    for (int64_t i = n8; i < in_dim; ++i) {
        total = __builtin_fmaf(widen_bf16(wr[i]), x[i], total);
    }
    out[row] = accumulate ? __builtin_fmaf(scale, total, out[row]) : total;
}

// x16 (panel layout, rows x cols_p) = fp16(x[r, c]) for c < cols, 0 for
// cols <= c < cols_p.  Thread i converts 8 consecutive columns of one row
// (one 16-byte store inside a panel row); consecutive threads walk a row.
__global__ __launch_bounds__(256) void to_f16_rows_kernel(const float* __restrict__ x, _Float16* __restrict__ x16,
                                                          int64_t rows, int32_t cols, int32_t cols_p) {
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int per_row = cols_p / 8;
    if (i >= rows * per_row) {
        return;
    }
    const int64_t r = i / per_row;
    const int c = static_cast<int>(i - r * per_row) * 8;
    const float* src = x + r * cols + c;
    half8 h;
    if (c + 8 <= cols && (cols & 3) == 0) {
        const float4 v0 = *reinterpret_cast<const float4*>(src);
        const float4 v1 = *reinterpret_cast<const float4*>(src + 4);
        h = half8{static_cast<_Float16>(v0.x), static_cast<_Float16>(v0.y), static_cast<_Float16>(v0.z),
                  static_cast<_Float16>(v0.w), static_cast<_Float16>(v1.x), static_cast<_Float16>(v1.y),
                  static_cast<_Float16>(v1.z), static_cast<_Float16>(v1.w)};
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            h[j] = c + j < cols ? static_cast<_Float16>(src[j]) : static_cast<_Float16>(0.0f);
        }
    }
    *reinterpret_cast<half8*>(x16 + panel_index(r, c, rows)) = h;
}

// gemm::matvec_f32 with LiteMind's dot (src/Gemm.cpp:183-189) as its GCC build
// runs it: products rounded and added left to right, the last n % 4 elements
// fused (the scalar epilogue).  One lane per output row.
__device__ inline float dot_ref(const float* a, const float* b, int64_t n, int64_t stride_a) {
    const int64_t unfused = n - n % 4;
    float t = 0.0f;
    int64_t i = 0;
    for (; i < unfused; ++i) {
        const float p = a[i * stride_a] * b[i];
        t = t + p;
    }
    for (; i < n; ++i) {
        t = __builtin_fmaf(a[i * stride_a], b[i], t);
    }
    return t;
}

__global__ __launch_bounds__(64) void matvec_f32_ref_kernel(const float* w, const float* x, float* out,
                                                            int64_t out_dim, int64_t in_dim) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 64 + threadIdx.x;
    if (row < out_dim) {
        out[row] = dot_ref(w + row * in_dim, x, in_dim, 1);
    }
}

// The vector helpers of namespace gemm (src/Gemm.cpp:177-231) with LiteMind's
// rounding: sequential reductions run on one lane, elementwise ops on all.
__global__ __launch_bounds__(256) void vector_op_kernel(int op, const void* a_raw, const float* b, float* out,
                                                        int64_t n, float scalar) {
    const float* a = static_cast<const float*>(a_raw);
    const int tid = threadIdx.x;
    switch (op) {
        case 0:  // dot
            if (tid == 0) {
                out[0] = dot_ref(a, b, n, 1);
            }
            break;
        case 1:  // axpy: out += scalar * a, fused as GCC compiles it
            for (int64_t i = tid; i < n; i += blockDim.x) {
                out[i] = __builtin_fmaf(scalar, a[i], out[i]);
            }
            break;
        case 2:  // softmax
            if (tid == 0 && n > 0) {
                float maximum = a[0];
                for (int64_t i = 1; i < n; ++i) {
                    maximum = maximum < a[i] ? a[i] : maximum;
                }
                float total = 0.0f;
                for (int64_t i = 0; i < n; ++i) {
                    out[i] = expf_ref(a[i] - maximum);
                    total = total + out[i];
                }
                const float inverse = total > 0.0f ? 1.0f / total : 0.0f;
                for (int64_t i = 0; i < n; ++i) {
                    out[i] = out[i] * inverse;
                }
            }
            break;
        case 3:  // silu_multiply
            for (int64_t i = tid; i < n; i += blockDim.x) {
                out[i] = silu_mul_ref(a[i], b[i]);
            }
            break;
        case 4: {  // rms_norm, sum of squares in double left to right
            __shared__ float inverse;
            if (tid == 0) {
                double sum = 0.0;
                for (int64_t i = 0; i < n; ++i) {
                    const double v = static_cast<double>(a[i]);
                    sum = sum + v * v;
                }
                inverse = static_cast<float>(
                    1.0 / __builtin_sqrt(sum / static_cast<double>(n) + static_cast<double>(scalar)));
            }
            __syncthreads();
            for (int64_t i = tid; i < n; i += blockDim.x) {
                const float scaled = a[i] * inverse;
                out[i] = scaled * b[i];
            }
            break;
        }
        case 5:  // widen_bf16
            for (int64_t i = tid; i < n; i += blockDim.x) {
                out[i] = widen_bf16(static_cast<const uint16_t*>(a_raw)[i]);
            }
            break;
        default:
            break;
    }
}

// dst [cols, dst_stride] = transpose of src [rows, src_stride] (16-bit
// elements), through a 64 x 64 LDS tile: reads and writes are row-contiguous.
// dst columns >= rows are left as they are.
__global__ __launch_bounds__(256) void transpose_u16_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                            int64_t rows, int64_t cols, int64_t src_stride,
                                                            int64_t dst_stride) {
    __shared__ uint16_t tile[64][65];
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 64, c0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int i = ty; i < 64; i += 4) {
        const int64_t r = r0 + i, c = c0 + tx;
        tile[i][tx] = r < rows && c < cols ? src[r * src_stride + c] : static_cast<uint16_t>(0);
    }
    __syncthreads();
    for (int i = ty; i < 64; i += 4) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (c < cols && r < rows) {
            dst[c * dst_stride + r] = tile[tx][i];
        }
    }
}

// out[a] = down_out[slot_of[a]] for the T*K routed assignments (assignment
// order), then the T shared rows as they are; float4 per thread, H % 4 == 0.
// The shared rows are zero when the layer has none.
__global__ __launch_bounds__(256) void gather_slots_kernel(const float* __restrict__ down_out,
                                                           const int32_t* __restrict__ slot_of, float* __restrict__ out,
                                                           int64_t assignments, int64_t rows, int32_t hidden,
                                                           int32_t has_shared) {
    const int64_t q = hidden / 4;
    const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i >= rows * q) {
        return;
    }
    const int64_t r = i / q, c = i % q;
    float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (r < assignments) {
        v = reinterpret_cast<const float4*>(down_out + static_cast<int64_t>(slot_of[r]) * hidden)[c];
    } else if (has_shared) {
        v = reinterpret_cast<const float4*>(down_out + r * hidden)[c];
    }
    reinterpret_cast<float4*>(out + r * hidden)[c] = v;
}

// out[i] = out[i] + y[i] (= fma(1, y[i], out[i]): gemm::axpy with scale 1).
__global__ __launch_bounds__(256) void add_rows_kernel(float* __restrict__ out, const float* __restrict__ y, int64_t n) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i < n) {
        out[i] = out[i] + y[i];
    }
}

}  // namespace

hipError_t launch_matvec_f32_ref(const float* w, const float* x, float* out, int64_t out_dim, int64_t in_dim,
                                 hipStream_t s) {
    if (out_dim <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(matvec_f32_ref_kernel, dim3(static_cast<unsigned>((out_dim + 63) / 64)), dim3(64), 0, s, w, x,
                       out, out_dim, in_dim);
    return hipGetLastError();
}

hipError_t launch_vector_op(int op, const void* a, const float* b, float* out, int64_t n, float scalar,
                            hipStream_t s) {
    hipLaunchKernelGGL(vector_op_kernel, dim3(1), dim3(256), 0, s, op, a, b, out, n, scalar);
    return hipGetLastError();
}

hipError_t launch_to_f16_rows(const float* x, _Float16* x16, int64_t rows, int32_t cols, int32_t cols_p,
                              hipStream_t s) {
    const int64_t n = rows * cols_p;
    if (n <= 0) {
        return hipSuccess;
    }
    if (cols_p % kPanel != 0) {
        return hipErrorInvalidValue;
    }
    const int64_t units = n / 8;
    hipLaunchKernelGGL(to_f16_rows_kernel, dim3(static_cast<unsigned>((units + 255) / 256)), dim3(256), 0, s, x, x16,
                       rows, cols, cols_p);
    return hipGetLastError();
}

hipError_t launch_gather_slots(const float* down_out, const int32_t* slot_of, float* out, int64_t assignments,
                               int64_t tokens, int32_t hidden, int32_t has_shared, hipStream_t s) {
    const int64_t rows = assignments + tokens;
    if (rows <= 0) {
        return hipSuccess;
    }
    if (hidden % 4 != 0) {
        return hipErrorInvalidValue;
    }
    const int64_t n = rows * (hidden / 4);
    hipLaunchKernelGGL(gather_slots_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, down_out,
                       slot_of, out, assignments, rows, hidden, has_shared);
    return hipGetLastError();
}

hipError_t launch_add_rows(float* out, const float* y, int64_t n, hipStream_t s) {
    if (n <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(add_rows_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, out, y, n);
    return hipGetLastError();
}

bool combine_norm_supported(int32_t hidden, int32_t hidden_p) {
    return hidden > 0 && hidden % 4 == 0 && hidden_p >= hidden && hidden_p % 4 == 0 && hidden_p <= kCombineNormMax;
}

hipError_t launch_combine(const CombineArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.next_norm != nullptr) {
        if (a.xnorm == nullptr || !combine_norm_supported(a.hidden, a.hidden_p)) {
            return hipErrorInvalidValue;
        }
        if (a.top_k == 6 && a.hidden_p <= 2048) {
            hipLaunchKernelGGL((combine_norm_kernel<6, 2>), dim3(static_cast<unsigned>(a.tokens)), dim3(256), 0, s, a);
        } else {
            hipLaunchKernelGGL((combine_norm_kernel<0, kCombineNormSteps>), dim3(static_cast<unsigned>(a.tokens)),
                               dim3(256), 0, s, a);
        }
        return hipGetLastError();
    }
    const int64_t n = a.tokens * (a.hidden / 4);
    const dim3 grid(static_cast<unsigned>((n + 255) / 256));
    if (a.top_k == 6) {
        hipLaunchKernelGGL(combine_kernel<6>, grid, dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL(combine_kernel<0>, grid, dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_bf16_to_f16_panels(const uint16_t* src, _Float16* dst, int64_t rows, int64_t cols, int* overflow,
                                     unsigned long long* inexact, hipStream_t s) {
    const int64_t n = rows * cols;
    if (n <= 0) {
        return hipSuccess;
    }
    if (cols % kPanel != 0) {
        return hipErrorInvalidValue;
    }
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) {
        blocks = 65536;
    }
    hipLaunchKernelGGL(bf16_to_f16_panels_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, src, dst, rows,
                       cols, overflow, inexact);
    return hipGetLastError();
}

hipError_t launch_transpose_u16(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t cols, int64_t src_stride,
                               int64_t dst_stride, hipStream_t s) {
    if (rows <= 0 || cols <= 0) {
        return hipSuccess;
    }
    if ((rows + 63) / 64 > 65535 || (cols + 63) / 64 > 0x7fffffff) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(transpose_u16_kernel, dim3(static_cast<unsigned>((cols + 63) / 64), static_cast<unsigned>((rows + 63) / 64)),
                       dim3(256), 0, s, src, dst, rows, cols, src_stride, dst_stride);
    return hipGetLastError();
}

// The core clock while other kernels run: one lane of one wave, on its own
// stream, stores (100 MHz real-time counter, core clock counter) pairs every
// `period` real-time ticks until `total` ticks have passed (the exit depends
// on the real-time counter alone, so the kernel always ends).  out:
// [2 * max_pairs] pairs, then the count.
__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t* out, int32_t max_pairs, int64_t period,
                                                         int64_t total) {
    if (threadIdx.x != 0) {
        return;
    }
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    uint64_t next = r0;
    int32_t n = 0;
    for (;;) {
        const uint64_t r = __builtin_amdgcn_s_memrealtime();
        if (r >= next) {
            const uint64_t c = __builtin_amdgcn_s_memtime();
            if (n < max_pairs) {
                out[2 * n] = r;
                out[2 * n + 1] = c;
                ++n;
            }
            next += static_cast<uint64_t>(period);
        }
        if (r - r0 >= static_cast<uint64_t>(total)) {
            break;
        }
        __builtin_amdgcn_s_sleep(2);
    }
    out[2 * max_pairs] = static_cast<uint64_t>(n);
}

hipError_t launch_clock_probe(uint64_t* out, int32_t max_pairs, int64_t period_ticks, int64_t total_ticks,
                              hipStream_t s) {
    hipLaunchKernelGGL(clock_probe_kernel, dim3(1), dim3(64), 0, s, out, max_pairs, period_ticks, total_ticks);
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
    if (matvec_rows_supported(out_dim, in_dim) && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(x) % 16 == 0) {
        // four lanes per row with 16-byte loads (k_head.hip): the same roundings
        return launch_matvec_rows(w, x, out, out_dim, in_dim, scale, accumulate, s);
    }
    hipLaunchKernelGGL(gemv_plain_kernel, dim3(static_cast<unsigned>((out_dim + 7) / 8)), dim3(256), 0, s, w, x, out,
                       out_dim, in_dim, scale, accumulate);
    return hipGetLastError();
}

}  // namespace lm
