// k_permute.hip -- expert histogram, exclusive scan and stable permutation.
//
// LiteMind evaluates one token at a time and visits its selections in rank
// order (src/DeepSeekRunner.cpp:277-284), so it has no permutation.  The grouped
// kernels need one, and it is defined canonically: assignment a = t*k + r goes
// to expert idx[a]'s bucket, buckets in expert order, and within a bucket in
// increasing a (token, then rank).  Positions come from ballots and prefix sums,
// never from atomic arrival order, so the permutation is deterministic.
//
// The assignment list is cut into segments of kSegment entries, one per
// workgroup of 16 waves, one 64-entry step per wave.  In a step every lane finds
// the lanes holding the same expert as itself from six ballots (one per bit of
// the expert id); its rank among them is the number of such lanes below it, and
// the lowest of them records the step's count for that expert.  Two launches:
//   count:   every workgroup stores its per-expert counts; the last one to
//            finish (an arrival ticket, so no workgroup ever waits for another)
//            scans them into each segment's first position per expert
//            (segments in order within an expert, experts in order) and writes
//            counts, offsets and the list of experts with tokens;
//   scatter: every workgroup recounts its steps, adds the waves before it to
//            its segment's base, and places every entry at its position plus
//            its rank.
// One segment (up to 1024 assignments) takes a single launch of one
// workgroup that does all three.
#include "lm_internal.h"

namespace lm {
namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kSegment = kThreads;  // assignments per workgroup, one step per wave

// Device-scope accesses: the segment counts cross XCDs within the count launch.
__device__ inline void store_agent(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline int32_t load_agent(const int32_t* p) {
    return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Lanes of this step holding the same (valid) expert as this lane, from one
// ballot per bit of the expert id (BITS = 6 below 64 experts).
template <int BITS>
__device__ inline uint64_t same_expert(int v, int E) {
    const bool valid = v >= 0 && v < E;
    uint64_t m = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < BITS; ++bit) {
        const uint64_t plane = __ballot(((v >> bit) & 1) != 0);
        m &= ((v >> bit) & 1) != 0 ? plane : ~plane;
    }
    return valid ? m : 0ull;
}

// Experts per lane (EPL, lane owns experts lane + 64 j) and id bits.
template <int EPL>
struct Wide {
    static constexpr int NE = 64 * EPL;
    static constexpr int BITS = EPL == 1 ? 6 : (EPL == 2 ? 7 : (EPL == 4 ? 8 : 9));
};

// This wave's step: its entry (-1 past the end), the lanes sharing its expert,
// and the step's count per expert into count[] (one LDS row per wave).
template <int EPL>
__device__ inline void count_step(const PermuteArgs& a, int64_t i, int lane, int& v, uint64_t& m, int* count) {
    const int64_t total = a.tokens * a.top_k;
    v = i < total ? a.idx[i] : -1;
    m = same_expert<Wide<EPL>::BITS>(v, a.experts);
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        count[lane + 64 * j] = 0;
    }
    __builtin_amdgcn_wave_barrier();
    const uint64_t below = (1ull << lane) - 1ull;
    if (m != 0 && (m & below) == 0) {  // lowest lane of its expert in this step
        count[v] = __popcll(m);
    }
}

// scratch: [0] the arrival ticket (0 between launches), [16, 16 + NE G) the
// segment counts, replaced by the segment bases.
constexpr int kTicketWords = 16;

template <int EPL>
__global__ __launch_bounds__(kThreads) void permute_count_kernel(PermuteArgs a) {
    constexpr int NE = Wide<EPL>::NE;
    __shared__ int wave_count[kWaves][NE];
    __shared__ uint32_t arrived;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int E = a.experts;
    const int g = blockIdx.x;
    const int G = gridDim.x;
    int v;
    uint64_t m;
    count_step<EPL>(a, static_cast<int64_t>(g) * kSegment + wave * 64 + lane, lane, v, m, wave_count[wave]);
    __syncthreads();
    int32_t* seg = a.scratch + kTicketWords;
    if (threadIdx.x < 64) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            int c = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                c += wave_count[w][e];
            }
            if (e < E) {
                store_agent(seg + g * NE + e, c);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the counts are out before the ticket
    __syncthreads();
    if (threadIdx.x == 0) {
        // release: this segment's counts; acquire: every earlier segment's
        arrived = __hip_atomic_fetch_add(reinterpret_cast<uint32_t*>(a.scratch), 1u, __ATOMIC_ACQ_REL,
                                         __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (arrived != static_cast<uint32_t>(G - 1) || threadIdx.x >= 64) {
        return;
    }
    // The last workgroup: lane e scans expert e's counts over the segments,
    // then the totals over the experts in expert order.  Up to kScanRegs
    // segments the counts are loaded at once (clamped, unconditional loads) and
    // the bases kept in registers, so every base is stored once, offset
    // included; beyond that in batches of 8 loads, the relative bases stored
    // and then offset.
    constexpr int kScanRegs = 32;
    const bool in_regs = G <= kScanRegs;
    int carry = 0, carry_active = 0;
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        const bool valid = e < E;
        int tot = 0;
        int rel[kScanRegs];
        if (in_regs) {
            // lanes past E read words of their own column that no one wrote
            // (inside the segment table) and count them as zero
            int c[kScanRegs];
#pragma unroll
            for (int q = 0; q < kScanRegs; ++q) {
                c[q] = load_agent(seg + (q < G ? q : G - 1) * NE + e);
            }
#pragma unroll
            for (int q = 0; q < kScanRegs; ++q) {
                rel[q] = tot;
                tot += valid && q < G ? c[q] : 0;
            }
        }
        for (int g0 = 0; !in_regs && g0 < G; g0 += 8) {
            int c[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                c[q] = valid && g0 + q < G ? load_agent(seg + (g0 + q) * NE + e) : 0;
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (valid && g0 + q < G) {
                    seg[(g0 + q) * NE + e] = tot;  // relative base, offset added below
                    tot += c[q];
                }
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
        const int off = carry + incl - tot;
        if (valid && in_regs) {
#pragma unroll
            for (int q = 0; q < kScanRegs; ++q) {
                if (q < G) {
                    seg[q * NE + e] = rel[q] + off;
                }
            }
        } else if (valid) {
            for (int sg = 0; sg < G; ++sg) {
                seg[sg * NE + e] += off;
            }
        }
        if (valid) {
            a.rb.counts[e] = tot;
            a.rb.offsets[e] = off;
        }
        carry += __shfl(incl, 63);
        // Experts with tokens, ascending.
        const uint64_t has = __ballot(valid && tot > 0);
        if (valid && tot > 0) {
            a.rb.active[carry_active + __popcll(has & below)] = e;
        }
        carry_active += __popcll(has);
    }
    if (lane == 0) {
        a.rb.offsets[E] = carry;
        a.rb.active[E] = carry_active;
        a.scratch[0] = 0;  // the ticket, for the next launch
    }
}

template <int EPL>
__global__ __launch_bounds__(kThreads) void permute_scatter_kernel(PermuteArgs a) {
    constexpr int NE = Wide<EPL>::NE;
    __shared__ int wave_count[kWaves][NE];
    __shared__ int wave_base[kWaves][NE];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int g = blockIdx.x;
    const int64_t i = static_cast<int64_t>(g) * kSegment + wave * 64 + lane;
    int v;
    uint64_t m;
    count_step<EPL>(a, i, lane, v, m, wave_count[wave]);
    __syncthreads();
    if (threadIdx.x < 64) {
        // First position of each expert for every wave of the segment.
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            int run = e < a.experts ? a.scratch[kTicketWords + g * NE + e] : 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                wave_base[w][e] = run;
                run += wave_count[w][e];
            }
        }
    }
    __syncthreads();
    if (m != 0) {
        const uint64_t below = (1ull << lane) - 1ull;
        const int at = wave_base[wave][v] + __popcll(m & below);
        a.rb.perm[at] = static_cast<int32_t>(i);
        a.rb.slot_of[i] = at;
    }
}

// One segment (T k <= 1024 assignments): the count, the scan and the scatter
// in one workgroup and one launch (no ticket; the scratch is not touched).
template <int EPL>
__global__ __launch_bounds__(kThreads) void permute_single_kernel(PermuteArgs a) {
    constexpr int NE = Wide<EPL>::NE;
    __shared__ int wave_count[kWaves][NE];  // counts, then each wave's first position per expert
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int E = a.experts;
    const int64_t i = wave * 64 + lane;
    int v;
    uint64_t m;
    count_step<EPL>(a, i, lane, v, m, wave_count[wave]);
    __syncthreads();
    if (threadIdx.x < 64) {
        int carry = 0, carry_active = 0;
        const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            const bool valid = e < E;
            int tot = 0;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                tot += valid ? wave_count[w][e] : 0;
            }
            int incl = tot;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int up = __shfl_up(incl, o);
                if (lane >= o) {
                    incl += up;
                }
            }
            int run = carry + incl - tot;
            if (valid) {
                a.rb.counts[e] = tot;
                a.rb.offsets[e] = run;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const int c = wave_count[w][e];
                    wave_count[w][e] = run;
                    run += c;
                }
            }
            carry += __shfl(incl, 63);
            const uint64_t has = __ballot(valid && tot > 0);
            if (valid && tot > 0) {
                a.rb.active[carry_active + __popcll(has & below)] = e;
            }
            carry_active += __popcll(has);
        }
        if (lane == 0) {
            a.rb.offsets[E] = carry;
            a.rb.active[E] = carry_active;
        }
    }
    __syncthreads();
    if (m != 0) {
        const uint64_t below = (1ull << lane) - 1ull;
        const int at = wave_count[wave][v] + __popcll(m & below);
        a.rb.perm[at] = static_cast<int32_t>(i);
        a.rb.slot_of[i] = at;
    }
}

template <int EPL>
hipError_t launch_epl(const PermuteArgs& a, int64_t segments, hipStream_t s) {
    if (segments == 1) {
        hipLaunchKernelGGL(permute_single_kernel<EPL>, dim3(1), dim3(kThreads), 0, s, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(permute_count_kernel<EPL>, dim3(static_cast<unsigned>(segments)), dim3(kThreads), 0, s, a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    hipLaunchKernelGGL(permute_scatter_kernel<EPL>, dim3(static_cast<unsigned>(segments)), dim3(kThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace

int64_t permute_scratch_words(int64_t assignments) {
    return kTicketWords + (assignments + kSegment - 1) / kSegment * kMaxExpertsWide;
}

hipError_t launch_permute(const PermuteArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.experts <= 0 || a.experts > kMaxExpertsWide || a.scratch == nullptr) {
        return hipErrorInvalidValue;
    }
    const int64_t segments = (a.tokens * a.top_k + kSegment - 1) / kSegment;
    if (a.experts <= 64) {
        return launch_epl<1>(a, segments, s);
    }
    if (a.experts <= 128) {
        return launch_epl<2>(a, segments, s);
    }
    if (a.experts <= 256) {
        return launch_epl<4>(a, segments, s);
    }
    return launch_epl<8>(a, segments, s);
}

}  // namespace lm
