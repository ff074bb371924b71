// k_gemv.hip -- grouped SwiGLU for small token counts (weight streaming, fp32 math).
//
// Reference: DeepSeekRunner::Impl::feed_forward (src/DeepSeekRunner.cpp:228-240).
// At small T every routed expert has a handful of tokens, so the kernels are
// bound by streaming expert weights from HBM.  A work item is a block of weight
// rows of one group (a routed expert, or the shared expert / dense FFN as the
// last group); each wavefront holds its rows in registers and applies them to
// all of the group's tokens (see gemv_items.h).
#include "gemv_items.h"

namespace lm {
namespace {

using gemv::dot_rows;
using gemv::dot_rows_stream;
using gemv::fma8;
using gemv::load_act;
using gemv::load_rows;
using gemv::log2c;
using gemv::transpose_reduce;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kGuRpw = 2;                    // gate rows (and as many up rows) per wave
constexpr int kDownRpw = 2;                  // output rows per wave
constexpr int kGuRows = kGuRpw * kWaves;     // gate rows per gate/up item
constexpr int kDownRows = kDownRpw * kWaves; // output rows per down item

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

// Stages the activation rows of tokens [tb, tb + nt) into LDS ([NTB][width]).
template <int NTB, typename RowOf>
__device__ inline void stage_rows(float* lds, int width, int nt, RowOf row_of) {
    lds_barrier();
    for (int idx = threadIdx.x * 4; idx < NTB * width; idx += kThreads * 4) {
        const int k = idx / width, c = idx - k * width;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (k < nt) {
            v = *reinterpret_cast<const float4*>(row_of(k) + c);
        }
        *reinterpret_cast<float4*>(lds + k * width + c) = v;
    }
    lds_barrier();
}

template <int R, int ITERS, int NTB>
__device__ inline void dot_rows_lds(const uint4 (&w)[R][ITERS], const float* lds, int width, int lane,
                                    float (&acc)[R * NTB]) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int c = it * 512 + lane * 8;
        if (c < width) {
#pragma unroll
            for (int k = 0; k < NTB; ++k) {
                const float4 x0 = *reinterpret_cast<const float4*>(lds + k * width + c);
                const float4 x1 = *reinterpret_cast<const float4*>(lds + k * width + c + 4);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    fma8(acc[r + R * k], w[r][it], x0, x1);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ---------------------------------------------------------------------------
// gate/up.  ITERS = ceil(hidden / 512) steps cached in registers (0: streamed).
// NTB = 1 keeps the token's activations in registers (no LDS, no barrier).
// ---------------------------------------------------------------------------
template <int ITERS, int NTB>
__global__ __launch_bounds__(kThreads) void gemv_gateup_kernel(ExpertArgs a) {
    extern __shared__ float xs[];  // [NTB][hidden] when staged
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int g, chunk;
    if (!decode_item(a, blockIdx.x, a.inter_p / kGuRows, a.shared_inter_p / kGuRows, g, chunk)) {
        return;
    }
    const GroupInfo gi = group_info(a, g);
    const int H = a.hidden;
    const uint16_t* gu = a.groups.gu[g];
    constexpr int R = 2 * kGuRpw;  // kGuRpw gate rows, then the matching up rows
    const uint16_t* rows[R];
    const int j0 = chunk * kGuRows + wave * kGuRpw;
#pragma unroll
    for (int r = 0; r < kGuRpw; ++r) {
        const int j = j0 + r;
        const int64_t gate_row = static_cast<int64_t>(j / kGroupRows) * (2 * kGroupRows) + (j % kGroupRows);
        rows[r] = gu + gate_row * a.hidden_p;
        rows[kGuRpw + r] = gu + (gate_row + kGroupRows) * a.hidden_p;
    }
    constexpr bool CACHE = ITERS > 0;
    constexpr bool DIRECT = CACHE && NTB == 1;
    constexpr int CI = CACHE ? ITERS : 1;
    constexpr int V = R * NTB;
    constexpr int L = log2c<V>();
    if (DIRECT) {
        // Single-token decode: every group holds at most this one token.
        if (gi.rows <= 0) {
            return;
        }
        float4 xr[1][CI][2];
        load_act<CI>(a.x + token_of(a, gi, 0) * H, H, lane, xr[0]);
        uint4 w[R][CI];
        load_rows<R, CI>(rows, H, lane, w);
        float acc[R];
#pragma unroll
        for (int i = 0; i < R; ++i) {
            acc[i] = 0.0f;
        }
        dot_rows<R, CI, 1>(w, xr, acc);
        const float sum = transpose_reduce<R>(acc, lane);
        constexpr int L1 = log2c<R>();
        const int vi = lane >> (6 - L1);
        const float up = __shfl_xor(sum, kGuRpw << (6 - L1));
        if ((lane & ((1 << (6 - L1)) - 1)) == 0 && (vi & kGuRpw) == 0) {
            gi.act_rows[j0 + (vi & (kGuRpw - 1))] = silu_mul_ref(sum, up);
        }
        return;
    }
    uint4 w[R][CI];
    if (CACHE) {
        load_rows<R, CI>(rows, H, lane, w);
    }

    for (int64_t tb = 0; tb < gi.rows; tb += NTB) {
        const int nt = gi.rows - tb < NTB ? static_cast<int>(gi.rows - tb) : NTB;
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
            acc[i] = 0.0f;
        }
        stage_rows<NTB>(xs, H, nt, [&](int k) { return a.x + token_of(a, gi, tb + k) * H; });
        if (CACHE) {
            dot_rows_lds<R, CI, NTB>(w, xs, H, lane, acc);
        } else {
            dot_rows_stream<R, NTB>(rows, xs, H, lane, acc);
        }
        // Value index vi = r + R k: r < kGuRpw gate rows, then the matching up rows.
        const float sum = transpose_reduce<V>(acc, lane);
        const int vi = lane >> (6 - L);
        const float up = __shfl_xor(sum, kGuRpw << (6 - L));
        const bool writer = (lane & ((1 << (6 - L)) - 1)) == 0 && (vi & kGuRpw) == 0;
        const int k = vi / R;
        if (writer && k < nt) {
            const int j = j0 + (vi & (kGuRpw - 1));
            gi.act_rows[(tb + k) * gi.width_p + j] = silu_mul_ref(sum, up);
        }
    }
}

// ---------------------------------------------------------------------------
// down.  ITERS = ceil(widest / 512) steps cached in registers (0: streamed);
// groups narrower than the widest skip the steps they do not have.
// ---------------------------------------------------------------------------
template <int ITERS, int NTB>
__global__ __launch_bounds__(kThreads) void gemv_down_kernel(ExpertArgs a) {
    extern __shared__ float hs[];  // [NTB][width] when staged
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int H = a.hidden;
    int g, chunk;
    if (!decode_item(a, blockIdx.x, H / kDownRows, H / kDownRows, g, chunk)) {
        return;
    }
    const GroupInfo gi = group_info(a, g);
    const int W = gi.width_p;
    const uint16_t* down = a.groups.down[g];
    constexpr int R = kDownRpw;
    const int h0 = chunk * kDownRows + wave * R;
    const uint16_t* rows[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        rows[r] = down + static_cast<int64_t>(h0 + r) * W;
    }
    constexpr bool CACHE = ITERS > 0;
    constexpr bool DIRECT = CACHE && NTB == 1;
    constexpr int CI = CACHE ? ITERS : 1;
    const int need = (W + 511) / 512;
    if (DIRECT && gi.rows <= 0) {
        return;
    }
    float4 hr[1][CI][2];
    uint4 w[R][CI];
    if (DIRECT) {
#pragma unroll
        for (int it = 0; it < CI; ++it) {
            const int c = it * 512 + lane * 8;
            const int cc = c < W ? c : W - 8;
            hr[0][it][0] = make_float4(0.f, 0.f, 0.f, 0.f);
            hr[0][it][1] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (it < need) {
                const float4 v0 = *reinterpret_cast<const float4*>(gi.act_rows + cc);
                const float4 v1 = *reinterpret_cast<const float4*>(gi.act_rows + cc + 4);
                if (c < W) {
                    hr[0][it][0] = v0;
                    hr[0][it][1] = v1;
                }
            }
        }
    }
    if (CACHE) {
#pragma unroll
        for (int it = 0; it < CI; ++it) {
            const int c = it * 512 + lane * 8;
            const int cc = c < W ? c : W - 8;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                w[r][it] = it < need ? load_stream16(rows[r] + cc) : make_uint4(0, 0, 0, 0);
            }
        }
    }

    constexpr int V = R * NTB;
    constexpr int L = log2c<V>();
    for (int64_t tb = 0; tb < gi.rows; tb += NTB) {
        const int nt = gi.rows - tb < NTB ? static_cast<int>(gi.rows - tb) : NTB;
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) {
            acc[i] = 0.0f;
        }
        if (DIRECT) {
            // Single-token decode: the group's one activation row is in registers.
            dot_rows<R, CI, 1>(w, hr, *reinterpret_cast<float(*)[R]>(acc));
        } else {
            stage_rows<NTB>(hs, W, nt, [&](int k) { return gi.act_rows + (tb + k) * W; });
            if (CACHE) {
                dot_rows_lds<R, CI, NTB>(w, hs, W, lane, acc);
            } else {
                dot_rows_stream<R, NTB>(rows, hs, W, lane, acc);
            }
        }
        const float sum = transpose_reduce<V>(acc, lane);
        const int vi = lane >> (6 - L);
        const bool writer = (lane & ((1 << (6 - L)) - 1)) == 0;
        const int k = vi / R;
        if (writer && k < nt) {
            a.down_out[(gi.slot0 + tb + k) * H + h0 + (vi % R)] = sum;
        }
    }
}

template <int NTB>
hipError_t gateup_dispatch(const ExpertArgs& a, int64_t items, hipStream_t s) {
    const int iters = (a.hidden + 511) / 512;
    // Activations are staged in LDS unless one token is held in registers.
    const bool staged = NTB > 1 || iters > 4;
    const size_t lds = staged ? sizeof(float) * NTB * a.hidden : 0;
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
    const int iters = (widest + 511) / 512;
    const bool staged = NTB > 1 || iters > 8;
    const size_t lds = staged ? sizeof(float) * NTB * widest : 0;
    const dim3 grid(static_cast<unsigned>(items)), block(kThreads);
    switch (iters) {
        case 1: hipLaunchKernelGGL((gemv_down_kernel<1, NTB>), grid, block, lds, s, a); break;
        case 2: hipLaunchKernelGGL((gemv_down_kernel<2, NTB>), grid, block, lds, s, a); break;
        case 3: hipLaunchKernelGGL((gemv_down_kernel<3, NTB>), grid, block, lds, s, a); break;
        case 4: hipLaunchKernelGGL((gemv_down_kernel<4, NTB>), grid, block, lds, s, a); break;
        case 5: hipLaunchKernelGGL((gemv_down_kernel<5, NTB>), grid, block, lds, s, a); break;
        case 6: hipLaunchKernelGGL((gemv_down_kernel<6, NTB>), grid, block, lds, s, a); break;
        case 7: hipLaunchKernelGGL((gemv_down_kernel<7, NTB>), grid, block, lds, s, a); break;
        case 8: hipLaunchKernelGGL((gemv_down_kernel<8, NTB>), grid, block, lds, s, a); break;
        default: hipLaunchKernelGGL((gemv_down_kernel<0, NTB>), grid, block, lds, s, a); break;
    }
    return hipGetLastError();
}

}  // namespace

// Grids: one item per workgroup; max_groups bounds the routed experts that
// can hold tokens (min(E, T*k)).  Token batch: 1 for single-token decode, else 4.
hipError_t launch_gemv_gateup(const ExpertArgs& a, int64_t max_groups, hipStream_t s) {
    const int64_t items = max_groups * (a.inter_p / kGuRows) + (a.has_shared ? a.shared_inter_p / kGuRows : 0);
    if (a.tokens <= 0 || items <= 0) {
        return hipSuccess;
    }
    return a.tokens == 1 ? gateup_dispatch<1>(a, items, s) : gateup_dispatch<4>(a, items, s);
}

hipError_t launch_gemv_down(const ExpertArgs& a, int64_t max_groups, hipStream_t s) {
    const int64_t items = (max_groups + (a.has_shared ? 1 : 0)) * (a.hidden / kDownRows);
    if (a.tokens <= 0 || items <= 0) {
        return hipSuccess;
    }
    // A 4-token batch of activations must fit the 64 KB of LDS a workgroup may
    // request without opting in; wider FFNs (the dense layer) use single tokens.
    const int widest = a.shared_inter_p > a.inter_p ? a.shared_inter_p : a.inter_p;
    const bool batch4 = a.tokens > 1 && 4 * widest * static_cast<int>(sizeof(float)) <= 65536;
    return batch4 ? down_dispatch<4>(a, items, s) : down_dispatch<1>(a, items, s);
}

}  // namespace lm
