// lm_select.h -- MoeRouter::select on one wavefront (one lane per expert).
//
// Reference: gemm::softmax (src/Gemm.cpp:209-223) and MoeRouter::select /
// top_k_indices (src/MoeRouter.cpp:14-107).
#pragma once

#include "lm_internal.h"

namespace lm {

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const uint64_t other = __shfl_xor(v, o);
        v = other > v ? other : v;
    }
    return v;
}

__device__ inline float lane_value(float v, int e) {
    return bits_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(float_bits(v)), e)));
}

// MoeRouter::select for one token whose logit for expert `lane` is `logit`
// (lanes >= experts pass valid = false).  On return `rank` is the lane's place
// in the selection (>= top_k when not selected) and `weight` its routing weight.
// Values are broadcast with v_readlane so the sequential reductions LiteMind
// performs (max, left-to-right sum) run on uniform registers without LDS
// round trips; the top-k order is found by counting, in every lane, how many
// keys beat its own.
__device__ inline void select_token(float logit, bool valid, int lane, const SelectPolicy& a, int& rank,
                                    float& weight) {
    const int E = a.experts;
    // softmax (src/Gemm.cpp:209-223): max (std::max_element keeps the first of
    // equal values; only the value matters), exp(v - max), left-to-right sum.
    float maximum = lane_value(logit, 0);
#pragma unroll
    for (int e = 1; e < kMaxExperts; ++e) {
        if (e < E) {
            const float v = lane_value(logit, e);
            maximum = maximum < v ? v : maximum;
        }
    }
    const float s = valid ? expf_ref(logit - maximum) : 0.0f;
    float total = 0.0f;
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) {
        if (e < E) {
            total = total + lane_value(s, e);
        }
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
        uint64_t chosen_groups = 0;  // n_group <= 64
        for (int r = 0; r < take; ++r) {
            const uint64_t best = wave_max_u64(gkey);
            const int gsel = 255 - static_cast<int>(best & 255u);
            if (lane == gsel) {
                gkey = 0;
            }
            chosen_groups |= 1ull << gsel;
        }
        allowed = ((chosen_groups >> my_group) & 1u) != 0;
    }

    // top_k_indices (src/MoeRouter.cpp:14-34): allowed first, then score
    // descending, then index ascending.  Scores are non-negative, so their bit
    // patterns order like the values; keys are unique through the index.
    const uint32_t key_hi = valid ? ((allowed ? 0x80000000u : 0u) | (float_bits(score) >> 1)) : 0u;
    const uint32_t key_lo = valid ? ((float_bits(score) << 31) | static_cast<uint32_t>(255 - lane)) : 0u;
    rank = 0;
#pragma unroll
    for (int e = 0; e < kMaxExperts; ++e) {
        if (e < E) {
            const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key_hi), e));
            const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(key_lo), e));
            rank += (hi > key_hi || (hi == key_hi && lo > key_lo)) ? 1 : 0;
        }
    }
    const int K = a.top_k < E ? a.top_k : E;
    // Weights in rank order; the selected sum runs left to right as in :91-94.
    float selected_sum = 0.0f;
    for (int r = 0; r < K; ++r) {
        const uint64_t who = __ballot(valid && rank == r);
        const int src = static_cast<int>(__builtin_ctzll(who));
        selected_sum = selected_sum + lane_value(score, src);
    }
    float my_w = score;
    // Normalise XOR scale (src/MoeRouter.cpp:96-106).
    if (a.top_k > 1 && a.normalize) {
        const float denominator = selected_sum + 1e-20f;
        my_w = my_w / denominator;
    } else if (a.scale != 1.0f) {
        my_w = my_w * a.scale;
    }
    weight = my_w;
}


// Per-wave LDS scratch of select_token_lds, in floats (16-byte aligned).
constexpr int kSelectScratch = 64 + 128 + kMaxTopK;

// The same selection as select_token, with the all-to-all steps done through
// the wave's own LDS scratch instead of v_readlane chains: each lane reads the
// 64 values with broadcast loads and reduces them in registers.  Identical
// results (max is exact in any order; the sum runs left to right over experts,
// invalid lanes adding +0; the rank counts beating keys).  Group-limited
// routing takes select_token.
__device__ inline void select_token_lds(float logit, bool valid, int lane, const SelectPolicy& a, float* sh,
                                        int& rank, float& weight) {
    if (a.group_limited && a.n_group > 1 && a.experts % a.n_group == 0) {
        select_token(logit, valid, lane, a, rank, weight);
        return;
    }
    float4* sh4 = reinterpret_cast<float4*>(sh);
    // max over valid logits (lanes past E repeat expert 0's logit)
    const float first = lane_value(logit, 0);
    sh[lane] = valid ? logit : first;
    __builtin_amdgcn_wave_barrier();
    float m[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 v = sh4[i];
        const float a01 = v.x < v.y ? v.y : v.x;
        const float a23 = v.z < v.w ? v.w : v.z;
        m[i] = a01 < a23 ? a23 : a01;
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
        for (int i = 0; i < w; ++i) {
            m[i] = m[i] < m[i + w] ? m[i + w] : m[i];
        }
    }
    const float maximum = m[0];
    const float s = valid ? expf_ref(logit - maximum) : 0.0f;
    __builtin_amdgcn_wave_barrier();
    sh[lane] = s;
    __builtin_amdgcn_wave_barrier();
    // LiteMind's left-to-right total (src/Gemm.cpp:216-218); +0 for lanes past E.
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 v = sh4[i];
        total = total + v.x;
        total = total + v.y;
        total = total + v.z;
        total = total + v.w;
    }
    const float inverse = total > 0.0f ? 1.0f / total : 0.0f;
    const float score = s * inverse;
    // top_k_indices order: score descending, then index ascending (all allowed).
    const uint64_t key = valid ? ((static_cast<uint64_t>(float_bits(score)) << 8) | static_cast<uint64_t>(255 - lane))
                               : 0ull;
    uint64_t* keys = reinterpret_cast<uint64_t*>(sh + 64);
    keys[lane] = key;
    __builtin_amdgcn_wave_barrier();
    int beaten = 0;
    const ulonglong2* keys2 = reinterpret_cast<const ulonglong2*>(keys);
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const ulonglong2 k2 = keys2[i];
        beaten += k2.x > key ? 1 : 0;
        beaten += k2.y > key ? 1 : 0;
    }
    rank = beaten;
    const int K = a.top_k < a.experts ? a.top_k : a.experts;
    float* picked = sh + 192;
    if (valid && rank < K) {
        picked[rank] = score;
    }
    __builtin_amdgcn_wave_barrier();
    float selected_sum = 0.0f;
    for (int r = 0; r < K; ++r) {
        selected_sum = selected_sum + picked[r];
    }
    float my_w = score;
    if (a.top_k > 1 && a.normalize) {
        const float denominator = selected_sum + 1e-20f;
        my_w = my_w / denominator;
    } else if (a.scale != 1.0f) {
        my_w = my_w * a.scale;
    }
    weight = my_w;
}

// ---- more than 64 experts ----------------------------------------------------
//
// MoeRouter takes any expert count (DeepSeek-V2 routes over 160 experts in 8
// groups, V3 over 256).  Above 64 experts a lane owns experts lane + 64 j,
// j < EPL.  The softmax total goes through the wave's own LDS scratch: every
// lane reads the E values in expert order, so the sum runs left to right as
// LiteMind's; the maximum and the top-k are wave reductions whose results do
// not depend on the order (see below).
// Per-wave scratch of select_token_multi, in 32-bit words: values, group
// maxima and group flags [64 EPL] each, picked weights [kMaxTopK].
__host__ __device__ constexpr int select_multi_words(int epl) { return 64 * epl * 3 + kMaxTopK; }

template <int EPL>
__device__ inline void select_token_multi(const float (&logit)[EPL], int lane, const SelectPolicy& a, float* sh,
                                          int (&rank)[EPL], float (&weight)[EPL]) {
    constexpr int NE = 64 * EPL;
    const int E = a.experts;
    float* val = sh;
    float* gval = sh + NE;
    int* gflag = reinterpret_cast<int*>(sh + 2 * NE);
    float* picked = sh + 3 * NE;
    bool valid[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        valid[j] = lane + 64 * j < E;
        if (valid[j]) {
            val[lane + 64 * j] = logit[j];
        }
    }
    __builtin_amdgcn_wave_barrier();
    // softmax (src/Gemm.cpp:209-223).  std::max_element's maximum: only its
    // value matters (the sign of a zero maximum cannot change logit - max),
    // and a NaN takes part only at index 0, where it stays the maximum (no
    // comparison with it holds); elsewhere a NaN never replaces it.  So the
    // lanes' maxima of their other values, by compare and select (exact bit
    // patterns, NaNs never enter), then a butterfly over the wave, then the
    // rule for a NaN first value (a chain over the E values in LDS: 2.6 us at
    // 160 experts).
    float lane_max = -__builtin_inff();
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        if (valid[j]) {
            lane_max = lane_max < logit[j] ? logit[j] : lane_max;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float other = __shfl_xor(lane_max, o);
        lane_max = lane_max < other ? other : lane_max;
    }
    const float first = val[0];
    const float maximum = first != first ? first : lane_max;
    float s[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        s[j] = valid[j] ? expf_ref(logit[j] - maximum) : 0.0f;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        if (valid[j]) {
            val[lane + 64 * j] = s[j];
        }
    }
    __builtin_amdgcn_wave_barrier();
    float total = 0.0f;
#pragma unroll 8  // the eight reads of a step go out together; the adds stay in expert order
    for (int e = 0; e < E; ++e) {
        total = total + val[e];
    }
    const float inverse = total > 0.0f ? 1.0f / total : 0.0f;
    float score[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        score[j] = s[j] * inverse;
    }
    // Group-limited mask (src/MoeRouter.cpp:67-84), with the constructor's
    // fallback to greedy when the groups do not divide the experts (:46-51):
    // a group's score is its first maximum, and the topk_group groups with the
    // highest scores (lower index first on equal scores) stay allowed.
    bool allowed[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        allowed[j] = true;
    }
    const int G = a.n_group;
    if (a.group_limited && G > 1 && E % G == 0) {
        const int per_group = E / G;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            if (valid[j]) {
                val[lane + 64 * j] = score[j];
            }
        }
        __builtin_amdgcn_wave_barrier();
        for (int g = lane; g < G; g += 64) {
            float best = val[g * per_group];
#pragma unroll 8
            for (int q = 1; q < per_group; ++q) {
                const float v = val[g * per_group + q];
                best = best < v ? v : best;
            }
            gval[g] = best;
        }
        __builtin_amdgcn_wave_barrier();
        const int take = a.topk_group < G ? a.topk_group : G;
        for (int g = lane; g < G; g += 64) {
            const float mine = gval[g];
            int beaten = 0;
#pragma unroll 8
            for (int h = 0; h < G; ++h) {
                const float other = gval[h];
                beaten += (other > mine || (other == mine && h < g)) ? 1 : 0;
            }
            gflag[g] = beaten < take ? 1 : 0;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            allowed[j] = valid[j] && gflag[(lane + 64 * j) / per_group] != 0;
        }
    }
    // top_k_indices (src/MoeRouter.cpp:14-34): allowed first, then score
    // descending, then index ascending.  Scores are non-negative, so their bit
    // patterns order like the values; the index makes every key unique.
    // The K largest keys in K rounds of a wave maximum over the keys not yet
    // taken: round r's key has rank r, the others keep rank K (not
    // selected).  Valid keys are non-zero and unique, and K <= E of them exist.
    const int K = a.top_k < E ? a.top_k : E;
    uint64_t key[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        key[j] = valid[j] ? ((allowed[j] ? (1ull << 62) : 0ull) | (static_cast<uint64_t>(float_bits(score[j])) << 16) |
                             static_cast<uint64_t>(0xffff - e))
                          : 0ull;
        rank[j] = K;
    }
    for (int r = 0; r < K; ++r) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            best = rank[j] == K && key[j] > best ? key[j] : best;
        }
        best = wave_max_u64(best);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            rank[j] = rank[j] == K && key[j] == best ? r : rank[j];
        }
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        if (valid[j] && rank[j] < K) {
            picked[rank[j]] = score[j];
        }
    }
    __builtin_amdgcn_wave_barrier();
    // Weights in rank order; the selected sum runs left to right as in :91-94.
    float selected_sum = 0.0f;
    for (int r = 0; r < K; ++r) {
        selected_sum = selected_sum + picked[r];
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        float w = score[j];
        if (a.top_k > 1 && a.normalize) {
            const float denominator = selected_sum + 1e-20f;
            w = w / denominator;
        } else if (a.scale != 1.0f) {
            w = w * a.scale;
        }
        weight[j] = w;
        if (!valid[j]) {
            rank[j] = E;  // never selected
        }
    }
    __builtin_amdgcn_wave_barrier();  // the scratch may be reused right after
}

}  // namespace lm
