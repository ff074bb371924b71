// k_gemv.hip -- grouped SwiGLU for small token counts (weight streaming, fp32 math).
//
// Reference: DeepSeekRunner::Impl::feed_forward (src/DeepSeekRunner.cpp:228-240):
// gate = W_g x, up = W_u x (gemm::matvec_bf16, src/Gemm.cpp:139-154),
// act = silu(gate) * up in fp32 (src/Gemm.cpp:225-231), then
// out += w * (W_d act) (src/Gemm.cpp:156-175).  Activations stay fp32 here, as in
// LiteMind; BF16 weights are widened exactly and accumulated with fp32 FMAs.
//
// At small T every routed expert has a handful of tokens, so the kernels are
// bound by streaming expert weights from HBM.  A work item is a block of weight
// rows of one group (routed expert or the shared expert); each wavefront loads
// its rows once into registers with 16-byte coalesced loads (64 lanes x 16 B =
// 1 KB per instruction), then applies them to every token of the group in
// batches whose activations are staged in LDS.  Per-row sums are finished with
// a transposing butterfly: V values per lane are reduced in log2(V) exchange
// steps instead of 6 * V.
#include "lm_internal.h"

namespace lm {
namespace {

constexpr int kThreads = 256;
constexpr int kGuRows = 16;    // gate rows (and as many up rows) per gate/up item
constexpr int kDownRows = 16;  // output rows per down item

__device__ inline void fma8(float& acc, const uint4 w, const float4 x0, const float4 x1) {
    acc = __builtin_fmaf(bits_float(w.x << 16), x0.x, acc);
    acc = __builtin_fmaf(bits_float(w.x & 0xffff0000u), x0.y, acc);
    acc = __builtin_fmaf(bits_float(w.y << 16), x0.z, acc);
    acc = __builtin_fmaf(bits_float(w.y & 0xffff0000u), x0.w, acc);
    acc = __builtin_fmaf(bits_float(w.z << 16), x1.x, acc);
    acc = __builtin_fmaf(bits_float(w.z & 0xffff0000u), x1.y, acc);
    acc = __builtin_fmaf(bits_float(w.w << 16), x1.z, acc);
    acc = __builtin_fmaf(bits_float(w.w & 0xffff0000u), x1.w, acc);
}

// Reduces V per-lane partial sums (V a power of two, <= 64) across the wave.
// Afterwards every lane holds the full sum of value index lane >> (6 - log2 V).
template <int V>
__device__ inline float transpose_reduce(float (&v)[V], int lane) {
    int off = 32;
#pragma unroll
    for (int half = V / 2; half >= 1; half >>= 1) {
        const bool upper = (lane & off) != 0;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const float keep = upper ? v[i + half] : v[i];
            const float send = upper ? v[i] : v[i + half];
            v[i] = keep + __shfl_xor(send, off);
        }
        off >>= 1;
    }
    float r = v[0];
    for (; off >= 1; off >>= 1) {
        r += __shfl_xor(r, off);
    }
    return r;
}

template <int V>
constexpr int log2c() {
    return V <= 1 ? 0 : 1 + log2c<V / 2>();
}

struct GroupInfo {
    int g;
    int64_t rows;      // tokens in the group
    int64_t slot0;     // first slot of the group
    int width_p;       // padded intermediate width
    float* act_rows;   // activation row of the group's first slot
};

__device__ inline GroupInfo group_info(const ExpertArgs& a, int g) {
    GroupInfo gi;
    gi.g = g;
    if (g < a.experts) {
        gi.rows = a.rb.counts[g];
        gi.slot0 = a.rb.offsets[g];
        gi.width_p = a.inter_p;
        gi.act_rows = a.act + gi.slot0 * a.inter_p;
    } else {
        gi.rows = a.tokens;
        gi.slot0 = a.tokens * a.top_k;
        gi.width_p = a.shared_inter_p;
        gi.act_rows = a.act + a.tokens * a.top_k * static_cast<int64_t>(a.inter_p);
    }
    return gi;
}

__device__ inline int64_t token_of(const ExpertArgs& a, const GroupInfo& gi, int64_t j) {
    return gi.g < a.experts ? a.rb.perm[gi.slot0 + j] / a.top_k : j;
}

// Maps a work-item index onto (group, chunk): chunks of active routed experts in
// expert order, then the shared expert's chunks.  Returns false past the end.
__device__ inline bool decode_item(const ExpertArgs& a, int64_t item, int chunks_routed, int chunks_shared, int& g,
                                   int& chunk) {
    const int n_active = a.rb.active[a.experts];
    const int64_t routed_items = static_cast<int64_t>(n_active) * chunks_routed;
    if (item < routed_items) {
        g = a.rb.active[item / chunks_routed];
        chunk = static_cast<int>(item % chunks_routed);
        return true;
    }
    item -= routed_items;
    if (!a.has_shared || item >= chunks_shared) {
        return false;
    }
    g = a.experts;
    chunk = static_cast<int>(item);
    return true;
}

// ---------------------------------------------------------------------------
// gate/up: each wave owns 4 gate rows and the 4 matching up rows of a 16-row item.
// ITERS = hidden / 512 column steps held in registers (0 = stream, any size).
// ---------------------------------------------------------------------------
template <int ITERS, int NTB>
__global__ __launch_bounds__(kThreads) void gemv_gateup_kernel(ExpertArgs a) {
    extern __shared__ float xs[];  // [NTB][hidden]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int g, chunk;
    if (!decode_item(a, blockIdx.x, a.inter_p / kGuRows, a.shared_inter_p / kGuRows, g, chunk)) {
        return;
    }
    const GroupInfo gi = group_info(a, g);
    const int H = a.hidden;
    const int64_t ldw = a.hidden_p;
    const uint16_t* gu = a.groups.gu[g];

    const uint16_t* wrow[8];
    const int j0 = chunk * kGuRows + wave * 4;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int j = j0 + r;
        const int64_t gate_row = static_cast<int64_t>(j / kGroupRows) * (2 * kGroupRows) + (j % kGroupRows);
        wrow[r] = gu + gate_row * ldw;
        wrow[4 + r] = gu + (gate_row + kGroupRows) * ldw;
    }

    constexpr int CACHED = ITERS > 0 ? ITERS : 1;
    uint4 wreg[8][CACHED];
    if (ITERS > 0) {
#pragma unroll
        for (int it = 0; it < CACHED; ++it) {
            const int c = it * 512 + lane * 8;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                wreg[r][it] = c < H ? *reinterpret_cast<const uint4*>(wrow[r] + c) : make_uint4(0, 0, 0, 0);
            }
        }
    }

    constexpr int V = 8 * NTB;
    constexpr int L = log2c<V>();
    for (int64_t tb = 0; tb < gi.rows; tb += NTB) {
        const int nt = gi.rows - tb < NTB ? static_cast<int>(gi.rows - tb) : NTB;
        __syncthreads();
        for (int idx = tid * 4; idx < NTB * H; idx += kThreads * 4) {
            const int k = idx / H, c = idx - k * H;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < nt) {
                v = *reinterpret_cast<const float4*>(a.x + token_of(a, gi, tb + k) * H + c);
            }
            *reinterpret_cast<float4*>(xs + k * H + c) = v;
        }
        __syncthreads();

        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
            acc[i] = 0.0f;
        }
        if (ITERS > 0) {
#pragma unroll
            for (int it = 0; it < CACHED; ++it) {
                const int c = it * 512 + lane * 8;
                if (c < H) {
#pragma unroll
                    for (int k = 0; k < NTB; ++k) {
                        const float4 x0 = *reinterpret_cast<const float4*>(xs + k * H + c);
                        const float4 x1 = *reinterpret_cast<const float4*>(xs + k * H + c + 4);
#pragma unroll
                        for (int r = 0; r < 8; ++r) {
                            fma8(acc[r + 8 * k], wreg[r][it], x0, x1);
                        }
                    }
                }
            }
        } else {
            for (int c = lane * 8; c < H; c += 512) {
                uint4 w[8];
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    w[r] = *reinterpret_cast<const uint4*>(wrow[r] + c);
                }
#pragma unroll
                for (int k = 0; k < NTB; ++k) {
                    const float4 x0 = *reinterpret_cast<const float4*>(xs + k * H + c);
                    const float4 x1 = *reinterpret_cast<const float4*>(xs + k * H + c + 4);
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        fma8(acc[r + 8 * k], w[r], x0, x1);
                    }
                }
            }
        }
        // Value index vi = r + 8k: r < 4 gate rows, r >= 4 the matching up rows.
        const float sum = transpose_reduce<V>(acc, lane);
        const int vi = lane >> (6 - L);
        const float up = __shfl_xor(sum, 4 << (6 - L));
        const bool writer = (lane & ((1 << (6 - L)) - 1)) == 0 && (vi & 4) == 0;
        const int k = vi >> 3;
        if (writer && k < nt) {
            const int j = j0 + (vi & 3);
            gi.act_rows[(tb + k) * gi.width_p + j] = silu_mul_ref(sum, up);
        }
    }
}

// ---------------------------------------------------------------------------
// down: each wave owns 4 output rows of a 16-row item; activations of a token
// batch are staged in LDS.  ITERS = width / 512 column steps held in registers.
// ---------------------------------------------------------------------------
template <int ITERS, int NTB>
__global__ __launch_bounds__(kThreads) void gemv_down_kernel(ExpertArgs a) {
    extern __shared__ float hs[];  // [NTB][width_p]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int H = a.hidden;
    int g, chunk;
    if (!decode_item(a, blockIdx.x, H / kDownRows, H / kDownRows, g, chunk)) {
        return;
    }
    const GroupInfo gi = group_info(a, g);
    const int W = gi.width_p;
    const uint16_t* down = a.groups.down[g];
    const int h0 = chunk * kDownRows + wave * 4;
    const uint16_t* wrow[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        wrow[r] = down + static_cast<int64_t>(h0 + r) * W;
    }

    constexpr int CACHED = ITERS > 0 ? ITERS : 1;
    uint4 wreg[4][CACHED];
    if (ITERS > 0) {
#pragma unroll
        for (int it = 0; it < CACHED; ++it) {
            const int c = it * 512 + lane * 8;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                wreg[r][it] = c < W ? *reinterpret_cast<const uint4*>(wrow[r] + c) : make_uint4(0, 0, 0, 0);
            }
        }
    }

    constexpr int V = 4 * NTB;
    constexpr int L = log2c<V>();
    for (int64_t tb = 0; tb < gi.rows; tb += NTB) {
        const int nt = gi.rows - tb < NTB ? static_cast<int>(gi.rows - tb) : NTB;
        __syncthreads();
        for (int idx = tid * 4; idx < NTB * W; idx += kThreads * 4) {
            const int k = idx / W, c = idx - k * W;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < nt) {
                v = *reinterpret_cast<const float4*>(gi.act_rows + (tb + k) * W + c);
            }
            *reinterpret_cast<float4*>(hs + k * W + c) = v;
        }
        __syncthreads();

        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
            acc[i] = 0.0f;
        }
        if (ITERS > 0) {
#pragma unroll
            for (int it = 0; it < CACHED; ++it) {
                const int c = it * 512 + lane * 8;
                if (c < W) {
#pragma unroll
                    for (int k = 0; k < NTB; ++k) {
                        const float4 x0 = *reinterpret_cast<const float4*>(hs + k * W + c);
                        const float4 x1 = *reinterpret_cast<const float4*>(hs + k * W + c + 4);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            fma8(acc[r + 4 * k], wreg[r][it], x0, x1);
                        }
                    }
                }
            }
        } else {
            for (int c = lane * 8; c < W; c += 512) {
                uint4 w[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    w[r] = *reinterpret_cast<const uint4*>(wrow[r] + c);
                }
#pragma unroll
                for (int k = 0; k < NTB; ++k) {
                    const float4 x0 = *reinterpret_cast<const float4*>(hs + k * W + c);
                    const float4 x1 = *reinterpret_cast<const float4*>(hs + k * W + c + 4);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        fma8(acc[r + 4 * k], w[r], x0, x1);
                    }
                }
            }
        }
        const float sum = transpose_reduce<V>(acc, lane);
        const int vi = lane >> (6 - L);
        const bool writer = (lane & ((1 << (6 - L)) - 1)) == 0;
        const int k = vi >> 2;
        if (writer && k < nt) {
            a.down_out[(gi.slot0 + tb + k) * H + h0 + (vi & 3)] = sum;
        }
    }
}

template <int NTB>
hipError_t gateup_dispatch(const ExpertArgs& a, int64_t items, hipStream_t s) {
    const size_t lds = sizeof(float) * NTB * a.hidden;
    const int iters = (a.hidden + 511) / 512;
    const dim3 grid(static_cast<unsigned>(items)), block(kThreads);
    switch (iters) {
        case 1: hipLaunchKernelGGL((gemv_gateup_kernel<1, NTB>), grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL((gemv_gateup_kernel<2, NTB>), grid, block, lds, s, a); break;
        case 3: hipLaunchKernelGGL((gemv_gateup_kernel<3, NTB>), grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL((gemv_gateup_kernel<4, NTB>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((gemv_gateup_kernel<0, NTB>), grid, block, lds, s, a); break;
    }
    return hipGetLastError();
}

template <int NTB>
hipError_t down_dispatch(const ExpertArgs& a, int64_t items, hipStream_t s) {
    const int widest = a.shared_inter_p > a.inter_p ? a.shared_inter_p : a.inter_p;
    const size_t lds = sizeof(float) * NTB * widest;
    const int iters = (widest + 511) / 512;
    const dim3 grid(static_cast<unsigned>(items)), block(kThreads);
    switch (iters) {
        case 1: hipLaunchKernelGGL((gemv_down_kernel<1, NTB>), grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL((gemv_down_kernel<2, NTB>), grid, block, lds, s, a); break;
        case 3: hipLaunchKernelGGL((gemv_down_kernel<3, NTB>), grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL((gemv_down_kernel<4, NTB>), grid, block, lds, s, a); break;
        case 5: hipLaunchKernelGGL((gemv_down_kernel<5, NTB>), grid, block, lds, s, a); break;
        case 6: hipLaunchKernelGGL((gemv_down_kernel<6, NTB>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((gemv_down_kernel<0, NTB>), grid, block, lds, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

// Token batch: 1 for single-token decode, else 4.
hipError_t launch_gemv_gateup(const ExpertArgs& a, int64_t max_items, hipStream_t s) {
    if (a.tokens <= 0 || max_items <= 0) {
        return hipSuccess;
    }
    return a.tokens == 1 ? gateup_dispatch<1>(a, max_items, s) : gateup_dispatch<4>(a, max_items, s);
}

hipError_t launch_gemv_down(const ExpertArgs& a, int64_t max_items, hipStream_t s) {
    if (a.tokens <= 0 || max_items <= 0) {
        return hipSuccess;
    }
    // A 4-token batch of activations must fit the 64 KB of LDS a workgroup may
    // request without opting in; wider FFNs (the dense layer) use single tokens.
    const int widest = a.shared_inter_p > a.inter_p ? a.shared_inter_p : a.inter_p;
    const bool batch4 = a.tokens > 1 && 4 * widest * static_cast<int>(sizeof(float)) <= 65536;
    return batch4 ? down_dispatch<4>(a, max_items, s) : down_dispatch<1>(a, max_items, s);
}

}  // namespace lm
