// k_router.hip -- fused router: gate matvec, softmax, (group mask), top-k, weights.
//
// Reference: gemm::matvec_f32 (src/Gemm.cpp:132-137, :183-189), gemm::softmax
// (:209-223) and MoeRouter::select (src/MoeRouter.cpp:14-107).
//
// One wavefront routes TPW tokens; lane e owns expert e.  Each logit is LiteMind's
// dot product as its GCC build executes it: every product rounded to fp32, then
// added strictly left to right.  This file is compiled with -ffp-contract=off
// so neither the products nor the additions are fused.  The router gate is
// stored transposed ([H, E]) so the 64 lanes read one 256-byte row per step;
// the token's activations are wave-uniform scalar loads.
#include "lm_internal.h"

namespace lm {
namespace {

constexpr int kWaves = 4;

__device__ inline float wave_max_f32(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float other = __shfl_xor(v, o);
        v = other > v ? other : v;
    }
    return v;
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t other = __shfl_xor(v, o);
        v = other > v ? other : v;
    }
    return v;
}

// MoeRouter::select for one token whose logit for expert `lane` is `logit`.
__device__ void route_token(float logit, bool valid, int lane, int64_t t, const RouterArgs& a) {
    const int E = a.experts;
    // softmax (src/Gemm.cpp:209-223): max, exp(v - max), left-to-right sum, reciprocal.
    const float maximum = wave_max_f32(valid ? logit : -__builtin_inff());
    const float s = valid ? expf_ref(logit - maximum) : 0.0f;
    float total = 0.0f;
    for (int e = 0; e < E; ++e) {
        total = total + __shfl(s, e);
    }
    const float inverse = total > 0.0f ? 1.0f / total : 0.0f;
    const float score = s * inverse;

    // Group-limited mask (src/MoeRouter.cpp:67-84), with the constructor's
    // fallback to greedy when the groups do not divide the experts (:46-51).
    bool allowed = true;
    if (a.group_limited && a.n_group > 1 && E % a.n_group == 0) {
        const int per_group = E / a.n_group;
        const int my_group = lane / per_group;
        // Lane j < n_group computes the maximum score of group j.
        float gmax = -__builtin_inff();
        for (int q = 0; q < per_group; ++q) {
            const int src = (lane < a.n_group ? lane : 0) * per_group + q;
            const float v = __shfl(score, src);
            gmax = v > gmax ? v : gmax;
        }
        // top_k_indices over the group scores (no mask): higher score, then lower index.
        const int take = a.topk_group < a.n_group ? a.topk_group : a.n_group;
        uint64_t gkey = lane < a.n_group
                            ? ((static_cast<uint64_t>(float_bits(gmax)) << 8) | static_cast<uint64_t>(255 - lane))
                            : 0;
        uint64_t chosen_groups_lo = 0, chosen_groups_hi = 0;  // bitset over 128 groups
        for (int r = 0; r < take; ++r) {
            const uint64_t best = wave_max_u64(gkey);
            const int gsel = 255 - static_cast<int>(best & 255u);
            if (lane == gsel) {
                gkey = 0;
            }
            if (gsel < 64) {
                chosen_groups_lo |= 1ull << gsel;
            } else {
                chosen_groups_hi |= 1ull << (gsel - 64);
            }
        }
        allowed = my_group < 64 ? ((chosen_groups_lo >> my_group) & 1u) != 0
                                : ((chosen_groups_hi >> (my_group - 64)) & 1u) != 0;
    }

    // top_k_indices (src/MoeRouter.cpp:14-34): allowed first, then score
    // descending, then index ascending.  Scores are non-negative, so their bit
    // patterns order like the values.
    uint64_t key = valid ? ((static_cast<uint64_t>(allowed ? 1u : 0u) << 40) |
                            (static_cast<uint64_t>(float_bits(score)) << 8) | static_cast<uint64_t>(255 - lane))
                         : 0;
    const int K = a.top_k < E ? a.top_k : E;
    // Lane r keeps the r-th selection; the running sum is wave-uniform.
    int my_idx = 0;
    float my_w = 0.0f;
    float selected_sum = 0.0f;
    for (int r = 0; r < K; ++r) {
        const uint64_t best = wave_max_u64(key);
        const int e = 255 - static_cast<int>(best & 255u);
        if (lane == e) {
            key = 0;
        }
        const float w = __shfl(score, e);
        if (lane == r) {
            my_idx = e;
            my_w = w;
        }
        selected_sum = selected_sum + w;
    }
    // Normalise XOR scale (src/MoeRouter.cpp:96-106).
    if (a.top_k > 1 && a.normalize) {
        const float denominator = selected_sum + 1e-20f;
        my_w = my_w / denominator;
    } else if (a.scale != 1.0f) {
        my_w = my_w * a.scale;
    }
    if (lane < K) {
        a.idx[t * a.top_k + lane] = my_idx;
        a.wts[t * a.top_k + lane] = my_w;
    }
}

// Rows of the transposed gate staged per step: [kChunk/4][64 experts] float4,
// component j of entry (q, e) holding gate row i0 + 4q + j of expert e.
constexpr int kChunk = 64;

template <int TPW>
__global__ __launch_bounds__(kWaves * 64) void router_kernel(RouterArgs a, const float* __restrict__ x,
                                                             const float* __restrict__ wt) {
    __shared__ float4 stage[2][kChunk / 4][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kWaves + wave) * TPW;
    const bool active = t0 < a.tokens;  // wave-uniform; idle waves still help stage the gate
    const int E = a.experts;
    const int H = a.hidden;
    const bool valid = lane < E;

    float acc[TPW];
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        acc[k] = 0.0f;
    }
    if (a.do_matvec) {
        const float* xr[TPW];
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const int64_t t = t0 + k < a.tokens ? t0 + k : a.tokens - 1;
            xr[k] = x + t * H;
        }
        // Each thread stages 16 values per chunk: row r = idx / 64, expert e = idx % 64.
        constexpr int kPer = kChunk * 64 / (kWaves * 64);
        float pre[kPer];
        auto fetch = [&](int i0) {
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const int idx = threadIdx.x + j * kWaves * 64;
                const int r = idx >> 6, e = idx & 63;
                pre[j] = (i0 + r < H && e < E) ? wt[static_cast<int64_t>(i0 + r) * E + e] : 0.0f;
            }
        };
        auto store = [&](int buf) {
#pragma unroll
            for (int j = 0; j < kPer; ++j) {
                const int idx = threadIdx.x + j * kWaves * 64;
                const int r = idx >> 6, e = idx & 63;
                reinterpret_cast<float*>(&stage[buf][r >> 2][e])[r & 3] = pre[j];
            }
        };
        const int nchunks = (H + kChunk - 1) / kChunk;
        fetch(0);
        store(0);
        __syncthreads();
        for (int c = 0; c < nchunks; ++c) {
            const int i0 = c * kChunk;
            if (c + 1 < nchunks) {
                fetch(i0 + kChunk);
            }
            if (active) {
                const int rows = H - i0 < kChunk ? H - i0 : kChunk;  // H % 4 == 0
                for (int q = 0; q < rows / 4; ++q) {
                    const float4 w = stage[c & 1][q][lane];
                    const int i = i0 + 4 * q;
#pragma unroll
                    for (int k = 0; k < TPW; ++k) {
                        float p = w.x * xr[k][i];
                        acc[k] = acc[k] + p;
                        p = w.y * xr[k][i + 1];
                        acc[k] = acc[k] + p;
                        p = w.z * xr[k][i + 2];
                        acc[k] = acc[k] + p;
                        p = w.w * xr[k][i + 3];
                        acc[k] = acc[k] + p;
                    }
                }
            }
            if (c + 1 < nchunks) {
                store((c + 1) & 1);
            }
            __syncthreads();
        }
    } else if (active) {
        // Select-only mode: x holds logits [T, E].
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const int64_t t = t0 + k;
            acc[k] = (valid && t < a.tokens) ? x[t * E + lane] : 0.0f;
        }
    }
    if (!active) {
        return;
    }

#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        const int64_t t = t0 + k;
        if (t >= a.tokens) {
            break;
        }
        float logit = acc[k];
        if (a.bias != nullptr && valid) {
            logit = logit + a.bias[lane];
        }
        if (a.logits != nullptr && valid) {
            a.logits[t * E + lane] = logit;
        }
        route_token(logit, valid, lane, t, a);

        // fp16 copy of the activations for the MFMA path, zero-padded to hidden_p.
        if (a.x16 != nullptr) {
            const float* xt = x + t * H;
            _Float16* dst = a.x16 + t * a.hidden_p;
            for (int c = lane; c < a.hidden_p; c += 64) {
                dst[c] = c < H ? static_cast<_Float16>(xt[c]) : static_cast<_Float16>(0.0f);
            }
        }
    }
}

}  // namespace

hipError_t launch_router(const RouterArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    int tpw = 1;
    if (a.do_matvec) {
        if (a.tokens >= 4096) {
            tpw = 4;
        } else if (a.tokens >= 2048) {
            tpw = 2;
        }
    }
    const int64_t waves = (a.tokens + tpw - 1) / tpw;
    const dim3 grid(static_cast<unsigned>((waves + kWaves - 1) / kWaves));
    const dim3 block(kWaves * 64);
    switch (tpw) {
        case 4: hipLaunchKernelGGL(router_kernel<4>, grid, block, 0, s, a, a.x, a.wt); break;
        case 2: hipLaunchKernelGGL(router_kernel<2>, grid, block, 0, s, a, a.x, a.wt); break;
        default: hipLaunchKernelGGL(router_kernel<1>, grid, block, 0, s, a, a.x, a.wt); break;
    }
    return hipGetLastError();
}

}  // namespace lm
