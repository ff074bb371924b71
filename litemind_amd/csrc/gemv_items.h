// gemv_items.h -- one wavefront's share of a grouped-SwiGLU work item (small T).
//
// Reference: DeepSeekRunner::Impl::feed_forward (src/DeepSeekRunner.cpp:228-240):
// gate = W_g x, up = W_u x (gemm::matvec_bf16, src/Gemm.cpp:139-154),
// act = silu(gate) * up in fp32 (src/Gemm.cpp:225-231), then the down projection
// (src/Gemm.cpp:156-175).  Activations stay fp32 as in LiteMind; BF16 weights
// are widened exactly and accumulated with fp32 FMAs.
//
// A wave loads its rows once into registers with 16-byte coalesced,
// non-temporal loads (64 lanes x 16 B = 1 KB per instruction), then applies them
// to every token of the group in batches of NTB.  Lane l covers columns
// it * 512 + 8 l .. +7 for it < ITERS = ceil(width / 512).  Lanes past the row
// end clamp their weight address (always in bounds, no branch, no select on the
// weights) and use zero activations, so their products vanish.  Row sums are
// finished with a transposing butterfly: V values per lane are reduced in
// log2(V) exchange steps instead of 6 V.
#pragma once

#include "lm_internal.h"

namespace lm {
namespace gemv {

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

template <int V>
constexpr int log2c() {
    return V <= 1 ? 0 : 1 + log2c<V / 2>();
}

// Reduces V per-lane partial sums (V a power of two, <= 64) across the wave.
// Afterwards every lane holds the full sum of value index lane >> (6 - log2 V).
// The halves are exchanged with a bit mask rather than `upper ? v[a] : v[b]`,
// which the compiler may turn into a dynamically indexed (scratch) array.
template <int V>
__device__ inline float transpose_reduce(float (&v)[V], int lane) {
    int off = 32;
#pragma unroll
    for (int half = V / 2; half >= 1; half >>= 1) {
        const uint32_t m = (lane & off) != 0 ? 0xffffffffu : 0u;
#pragma unroll
        for (int i = 0; i < half; ++i) {
            const uint32_t lo = float_bits(v[i]), hi = float_bits(v[i + half]);
            const float keep = bits_float((hi & m) | (lo & ~m));
            const float send = bits_float((lo & m) | (hi & ~m));
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

// Activations of lane columns for one row of width `width`: zero past the end.
template <int ITERS>
__device__ inline void load_act(const float* row, int width, int lane, float4 (&x)[ITERS][2]) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int c = it * 512 + lane * 8;
        const int cc = c < width ? c : width - 8;
        x[it][0] = *reinterpret_cast<const float4*>(row + cc);
        x[it][1] = *reinterpret_cast<const float4*>(row + cc + 4);
        if (c >= width) {
            x[it][0] = make_float4(0.f, 0.f, 0.f, 0.f);
            x[it][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

// Loads R rows x ITERS column steps of BF16 weights (clamped addresses).
template <int R, int ITERS>
__device__ inline void load_rows(const uint16_t* const (&rows)[R], int width, int lane, uint4 (&w)[R][ITERS]) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int c = it * 512 + lane * 8;
        const int cc = c < width ? c : width - 8;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            w[r][it] = load_stream16(rows[r] + cc);
        }
    }
}

// acc[r + R k] += W[r] . x[k] for NTB activation rows.
template <int R, int ITERS, int NTB>
__device__ inline void dot_rows(const uint4 (&w)[R][ITERS], const float4 (&x)[NTB][ITERS][2], float (&acc)[R * NTB]) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
#pragma unroll
        for (int k = 0; k < NTB; ++k) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                fma8(acc[r + R * k], w[r][it], x[k][it][0], x[k][it][1]);
            }
        }
        // Keep each step's widening next to its FMAs (hoisting them all would
        // double the live registers and halve occupancy).
        __builtin_amdgcn_sched_barrier(0);
    }
}

// acc[r + R k] += W[r] . x[k] streaming the rows (no register cache; any width).
// U steps' loads are issued before their products (the same order of
// additions): one step at a time left a lane with R loads in flight, and a
// long row (the dense layer's down, width 10944) waited on every one.
template <int R, int NTB, int U = 4>
__device__ inline void dot_rows_stream(const uint16_t* const (&rows)[R], const float* lds, int width, int lane,
                                       float (&acc)[R * NTB]) {
    int c = lane * 8;
    for (; c + (U - 1) * 512 < width; c += U * 512) {
        uint4 wu[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wu[u][r] = load_stream16(rows[r] + c + u * 512);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int k = 0; k < NTB; ++k) {
                const float4 x0 = *reinterpret_cast<const float4*>(lds + k * width + c + u * 512);
                const float4 x1 = *reinterpret_cast<const float4*>(lds + k * width + c + u * 512 + 4);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    fma8(acc[r + R * k], wu[u][r], x0, x1);
                }
            }
        }
    }
    for (; c < width; c += 512) {
        uint4 w[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            w[r] = load_stream16(rows[r] + c);
        }
#pragma unroll
        for (int k = 0; k < NTB; ++k) {
            const float4 x0 = *reinterpret_cast<const float4*>(lds + k * width + c);
            const float4 x1 = *reinterpret_cast<const float4*>(lds + k * width + c + 4);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                fma8(acc[r + R * k], w[r], x0, x1);
            }
        }
    }
}

}  // namespace gemv
}  // namespace lm
