// k_permute.hip -- expert histogram, exclusive scan and stable permutation.
//
// LiteMind evaluates one token at a time and visits its selections in rank
// order (src/DeepSeekRunner.cpp:277-284), so it has no permutation.  The grouped
// kernels need one, and it is defined canonically: assignment a = t*k + r goes
// to expert idx[a]'s bucket, buckets in expert order, and within a bucket in
// increasing a (token, then rank).  Positions come from ballots and prefix sums,
// never from atomic arrival order, so the permutation is deterministic.
//
// One workgroup of 16 waves.  Wave w owns a contiguous segment of the
// assignment list, walked in 64-entry steps.  In each step every lane finds the
// lanes holding the same expert as itself from six ballots (one per bit of the
// expert id); its rank among them is the number of such lanes below it, and the
// lowest of them updates the wave's running count for that expert in LDS.
// Pass 1 counts; the counts are scanned (waves in order within an expert,
// experts in order) into each wave's first position per expert; pass 2 repeats
// the walk and places every entry at its running position plus its rank.
#include "lm_internal.h"

namespace lm {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kBatch = 16;  // 64-entry steps per batch of loads

__global__ __launch_bounds__(kThreads) void permute_kernel(PermuteArgs a) {
    __shared__ int wave_count[kWaves][kMaxExperts];
    __shared__ int wave_base[kWaves][kMaxExperts];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int E = a.experts;
    const int64_t total = a.tokens * a.top_k;
    const int64_t steps = (total + 63) / 64;
    const int64_t per_wave = (steps + kWaves - 1) / kWaves;
    const int64_t first = per_wave * wave * 64;
    const int64_t last = first + per_wave * 64 < total ? first + per_wave * 64 : total;
    const uint64_t below = (1ull << lane) - 1ull;

    // Lanes of this step holding the same (valid) expert as this lane.
    auto same_expert = [&](int v) -> uint64_t {
        const bool valid = v >= 0 && v < E;
        uint64_t m = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 6; ++bit) {  // experts < 64
            const uint64_t plane = __ballot(((v >> bit) & 1) != 0);
            m &= ((v >> bit) & 1) != 0 ? plane : ~plane;
        }
        return valid ? m : 0ull;
    };
    // The segment is walked in batches of kBatch steps whose loads are all
    // issued before any is used (one memory latency per batch, not per step).
    auto load_batch = [&](int64_t b0, int (&v)[kBatch]) {
#pragma unroll
        for (int st = 0; st < kBatch; ++st) {
            const int64_t i = b0 + st * 64 + lane;
            v[st] = i < last ? a.idx[i] : -1;
        }
    };
    int* const my_count = wave_count[wave];
    for (int j = lane; j < kMaxExperts; j += 64) {
        my_count[j] = 0;
    }
    __builtin_amdgcn_wave_barrier();
    for (int64_t b0 = first; b0 < last; b0 += 64 * kBatch) {
        int v[kBatch];
        load_batch(b0, v);
#pragma unroll
        for (int st = 0; st < kBatch; ++st) {
            const uint64_t m = same_expert(v[st]);
            if (m != 0 && (m & below) == 0) {  // lowest lane of its expert in this step
                my_count[v[st]] += __popcll(m);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        // Lane e: expert e's total, then the exclusive scan over experts.
        int tot = 0;
        if (lane < E) {
            for (int w = 0; w < kWaves; ++w) {
                tot += wave_count[w][lane];
            }
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int up = __shfl_up(incl, o);
            if (lane >= o) {
                incl += up;
            }
        }
        const int off = incl - tot;
        if (lane < E) {
            int run = off;
            for (int w = 0; w < kWaves; ++w) {
                wave_base[w][lane] = run;
                run += wave_count[w][lane];
            }
            a.rb.counts[lane] = tot;
            a.rb.offsets[lane] = off;
        }
        if (lane == E - 1) {
            a.rb.offsets[E] = incl;
        }
        // Experts with tokens, ascending, and their number.
        const uint64_t has = __ballot(lane < E && tot > 0);
        if (lane < E && tot > 0) {
            a.rb.active[__popcll(has & below)] = lane;
        }
        if (lane == 0) {
            a.rb.active[E] = __popcll(has);
        }
    }
    __syncthreads();
    int* const my_pos = wave_base[wave];  // next slot of each expert for this wave
    for (int64_t b0 = first; b0 < last; b0 += 64 * kBatch) {
        int v[kBatch];
        load_batch(b0, v);
#pragma unroll
        for (int st = 0; st < kBatch; ++st) {
            const int64_t i = b0 + st * 64 + lane;
            const uint64_t m = same_expert(v[st]);
            if (m != 0) {
                const int at = my_pos[v[st]] + __popcll(m & below);
                a.rb.perm[at] = static_cast<int32_t>(i);
                a.rb.slot_of[i] = at;
            }
            __builtin_amdgcn_wave_barrier();  // every lane has read its expert's position
            if (m != 0 && (m & below) == 0) {
                my_pos[v[st]] += __popcll(m);
            }
            __builtin_amdgcn_wave_barrier();
        }
    }
}

}  // namespace

hipError_t launch_permute(const PermuteArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.experts <= 0 || a.experts > kMaxExperts) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace lm
