// k_permute.hip -- expert histogram, exclusive scan and stable permutation.
//
// LiteMind evaluates one token at a time and visits its selections in rank
// order (src/DeepSeekRunner.cpp:277-284), so it has no permutation.  The grouped
// kernels need one, and it is defined canonically: assignment a = t*k + r goes
// to expert idx[a]'s bucket, buckets in expert order, and within a bucket in
// increasing a (token, then rank).  Positions come from ballots and prefix sums,
// never from atomic arrival order, so the permutation is deterministic.
//
// Grid: one workgroup per expert.  Every workgroup builds the full histogram in
// LDS (the index list is at most a few hundred KB and L2-resident), scans it,
// then places its own expert's assignments: each of the 4 waves counts matches
// in a contiguous quarter of the list, the quarters are prefix-summed, and a
// second pass writes perm / slot_of.
#include "lm_internal.h"

namespace lm {
namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void permute_kernel(PermuteArgs a) {
    __shared__ int hist[kMaxExperts];
    __shared__ int offs[kMaxExperts + 1];
    __shared__ int wave_count[kThreads / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int E = a.experts;
    const int e = blockIdx.x;
    const int64_t total = a.tokens * a.top_k;

    for (int j = tid; j < E; j += kThreads) {
        hist[j] = 0;
    }
    __syncthreads();
    for (int64_t i = tid; i < total; i += kThreads) {
        const int v = a.idx[i];
        if (v >= 0 && v < E) {
            atomicAdd(&hist[v], 1);
        }
    }
    __syncthreads();
    if (tid == 0) {
        int run = 0;
        for (int j = 0; j < E; ++j) {
            offs[j] = run;
            run += hist[j];
        }
        offs[E] = run;
    }
    __syncthreads();
    if (e == 0) {
        for (int j = tid; j <= E; j += kThreads) {
            a.rb.offsets[j] = offs[j];
            if (j < E) {
                a.rb.counts[j] = hist[j];
            }
        }
        if (tid == 0) {
            int n = 0;
            for (int j = 0; j < E; ++j) {
                if (hist[j] > 0) {
                    a.rb.active[n++] = j;
                }
            }
            a.rb.active[E] = n;
        }
    }

    // Contiguous quarter of the assignment list per wave, in 64-entry steps.
    const int64_t steps = (total + 63) / 64;
    const int64_t per_wave = (steps + (kThreads / 64) - 1) / (kThreads / 64);
    const int64_t first = per_wave * wave * 64;
    const int64_t last = first + per_wave * 64 < total ? first + per_wave * 64 : total;
    int count = 0;
    for (int64_t base = first; base < last; base += 64) {
        const int64_t i = base + lane;
        const bool match = i < last && a.idx[i] == e;
        count += __popcll(__ballot(match));
    }
    if (lane == 0) {
        wave_count[wave] = count;
    }
    __syncthreads();
    int pos = offs[e];
    for (int w = 0; w < wave; ++w) {
        pos += wave_count[w];
    }
    const uint64_t below = (1ull << lane) - 1ull;
    for (int64_t base = first; base < last; base += 64) {
        const int64_t i = base + lane;
        const bool match = i < last && a.idx[i] == e;
        const uint64_t bal = __ballot(match);
        if (match) {
            const int at = pos + __popcll(bal & below);
            a.rb.perm[at] = static_cast<int32_t>(i);
            a.rb.slot_of[i] = at;
        }
        pos += __popcll(bal);
    }
}

}  // namespace

hipError_t launch_permute(const PermuteArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(permute_kernel, dim3(a.experts), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace lm
