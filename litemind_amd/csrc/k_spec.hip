// k_spec.hip -- one token over more than 64 experts on the GEMV path: the
// router and the gate/up projections in one launch, the routed experts
// started from a speculative selection.
//
// Reference: the MoE branch of DeepSeekRunner::Impl::forward
// (src/DeepSeekRunner.cpp:273-290): the router's matvec_f32
// (src/Gemm.cpp:183-189), MoeRouter::select (src/MoeRouter.cpp:55-113), and
// feed_forward's gate / up and silu_multiply for each selected expert and the
// shared expert (src/DeepSeekRunner.cpp:228-240).
//
// Every exact logit is LiteMind's chain of H dependent fp32 adds (~18 us at
// H = 5120), and a routed expert's rows cannot be requested before the expert
// is known.  One grid, roles by workgroup index:
//
//   [partial sums | exact router | shared gate/up | routed gate/up | repair]
//
// The partial-sum workgroups add the gate's products over slices of the rows
// in any order; the last of them to arrive adds the slices and ranks the
// experts by these reassociated logits (the softmax keeps the order; the group
// mask ranks groups by their largest logit) and publishes the speculative
// experts.  The routed gate/up items stream those experts' rows at once, the
// shared items from the start, while the exact router's chains run.  The last
// exact router workgroup selects with MoeRouter::select, writes the selection
// and the permutation the down and combine launches read, and publishes
// whether the exact set of experts differs from the speculated one (near-ties
// only).  The activations are indexed by the slot of the expert among the
// selected ones, which depends on the set alone; where the sets differ, the
// repair workgroups recompute every routed activation row from the exact
// experts once all routed items are done.  The outputs therefore always
// follow the exact selection.
//
// A workgroup waits only for workgroups with lower indices, which the
// dispatcher places first, so every wait ends; each is bounded all the same
// and sets the error word when it gives up.
#include "gemv_items.h"
#include "handoff.h"
#include "lm_select.h"
#include "router_chunks.h"

namespace lm {
namespace {

using gemv::dot_rows_stream;
using gemv::log2c;
using gemv::transpose_reduce;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRpw = 2;                   // gate rows (and as many up rows) per wave, as the GEMV items
constexpr int kItemRows = kRpw * kWaves;  // gate rows per gate/up item
constexpr int kSliceRows = 4 * kThreads;  // hidden rows per partial-sum workgroup: one row quad per thread
constexpr int kMaxSlices = 16;
constexpr int kRepairBlocks = 64;
constexpr uint32_t kMaxSpins = 1u << 16;  // ~50 ms of polling
// Counters of one launch: the two arrival tickets in one line each, the routed
// items' completion count spread over kLanes lines.
constexpr int kLanes = 16;
constexpr int kSlotStride = 16;  // words
enum : int { kPartialTicket = 0, kRouterTicket, kRoutedDone, kCounters };
constexpr int kSetWords = kCounters * kLanes * kSlotStride;
static_assert(2 * kSetWords <= kSpecCounterWords, "spec scratch layout");
static_assert(kChunkThreads == kThreads, "one block shape for every role");

struct SpecArgs {
    RouterArgs r;      // token, gate layouts, bias, outputs (idx, wts, logits), exact logit hand-off, permutation
    ExpertArgs e;      // groups, token, activations; e.rb is not used
    uint32_t* sync;    // this launch's counter set
    uint32_t* clear;   // the other launch parity's set, cleared by the grid's last workgroup
    uint32_t* error;
    uint64_t* spec;    // [kMaxTopK] tagged speculative experts by rank
    uint64_t* exact;   // [1] tagged: 1 when the exact set of experts differs from the speculated one
    float* partial;    // [slices][E] reassociated partial logits
    uint32_t seq;      // this launch's tag (nonzero, differs from the last launch's)
    int32_t perturb;   // testing: the speculation's last rank takes the next expert (a wrong set)
    uint32_t max_spins;
    int32_t slices, n_partial, n_router, n_shared, n_routed;
};

__device__ inline uint32_t* counter_slot(uint32_t* set, int counter, int slot) {
    return set + (counter * kLanes + slot) * kSlotStride;
}

// Arrival ticket of one workgroup once its stores are acknowledged: returns
// how many arrived before it (every thread).  Stores that another workgroup
// reads are device-scope (handoff.h); vmcnt(0) and the barrier put the add
// after all of them.
__device__ inline uint32_t arrive(uint32_t* ticket, uint32_t* arrived) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
        *arrived = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return *arrived;
}

// Waits until the routed items' count reaches target (wave 0 polls every slot
// at once), then releases the workgroup.
__device__ inline void wait_routed(const SpecArgs& f, uint32_t target) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        uint32_t spins = 0;
        for (;;) {
            uint32_t v = lane < kLanes ? __hip_atomic_load(counter_slot(f.sync, kRoutedDone, lane), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0u;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                v += __shfl_xor(v, o);
            }
            if (v >= target) {
                break;
            }
            if (++spins > f.max_spins) {
                if (lane == 0) {
                    __hip_atomic_store(f.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                break;
            }
            __builtin_amdgcn_s_sleep(8);
        }
    }
    __syncthreads();
}

// Orders floats as unsigned integers (NaNs aside).
__device__ inline uint32_t float_order(float v) {
    const uint32_t u = float_bits(v);
    return (u & 0x80000000u) != 0 ? ~u : (u | 0x80000000u);
}

// The token into LDS (xs, hidden floats) for the items' dot products.
__device__ inline void stage_token(const ExpertArgs& a, float* xs) {
    for (int c = static_cast<int>(threadIdx.x) * 4; c < a.hidden; c += kThreads * 4) {
        *reinterpret_cast<float4*>(xs + c) = *reinterpret_cast<const float4*>(a.x + c);
    }
    lds_barrier();
}

// Gate/up rows [8 chunk, 8 chunk + 8) of one FFN (gu: its interleaved gate/up
// matrix) for the token in xs: act_row[j] = silu(gate_j . x) * (up_j . x),
// the GEMV kernel's item (k_gemv.hip, gemv_gateup_kernel for one token with
// streamed rows): the same loads, products and additions in the same order.
__device__ inline void gateup_item(const ExpertArgs& a, const uint16_t* gu, int chunk, float* act_row,
                                   const float* xs) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int R = 2 * kRpw;
    const uint16_t* rows[R];
    const int j0 = chunk * kItemRows + wave * kRpw;
#pragma unroll
    for (int r = 0; r < kRpw; ++r) {
        const int j = j0 + r;
        const int64_t gate_row = static_cast<int64_t>(j / kGroupRows) * (2 * kGroupRows) + (j % kGroupRows);
        rows[r] = gu + gate_row * a.hidden_p;
        rows[kRpw + r] = gu + (gate_row + kGroupRows) * a.hidden_p;
    }
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        acc[i] = 0.0f;
    }
    // five steps per batch: DeepSeek-V2's ten 512-column steps in two round
    // trips instead of four (4 + 4 + 1 + 1); 75.5 against 76.3 us per layer
    dot_rows_stream<R, 1, 5>(rows, xs, a.hidden, lane, acc);
    const float sum = transpose_reduce<R>(acc, lane);
    constexpr int L = log2c<R>();
    const int vi = lane >> (6 - L);
    const float up = __shfl_xor(sum, kRpw << (6 - L));
    if ((lane & ((1 << (6 - L)) - 1)) == 0 && (vi & kRpw) == 0) {
        store_coherent(act_row + j0 + (vi & (kRpw - 1)), silu_mul_ref(sum, up));
    }
}

// Wave 0 of the last partial-sum workgroup: the speculative selection from the
// reassociated logits val [E] (LDS).  MoeRouter::select's group mask and top k
// in the logits' order (the softmax is monotone in the logit), ties to the
// lower index; publishes spec[r] for r < K.
template <int EPL>
__device__ void speculate(const SpecArgs& f, const float* val) {
    const int lane = threadIdx.x & 63;
    const RouterArgs& a = f.r;
    const int E = a.experts;
    bool valid[EPL], allowed[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        valid[j] = lane + 64 * j < E;
        allowed[j] = valid[j];
    }
    const int G = a.n_group;
    if (a.group_limited && G > 1 && E % G == 0) {  // G <= 64 (spec_gateup_supported)
        const int per = E / G;
        uint64_t gkey = 0;
        if (lane < G) {
            float m = val[lane * per];
#pragma unroll 8
            for (int q = 1; q < per; ++q) {
                const float v = val[lane * per + q];
                m = m < v ? v : m;
            }
            gkey = (static_cast<uint64_t>(float_order(m)) << 8) | static_cast<uint64_t>(255 - lane);
        }
        const int take = a.topk_group < G ? a.topk_group : G;
        uint64_t chosen = 0;
        for (int r = 0; r < take; ++r) {
            const uint64_t best = wave_max_u64(gkey);
            const int g = 255 - static_cast<int>(best & 255u);
            if (lane == g) {
                gkey = 0;
            }
            chosen |= 1ull << g;
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            allowed[j] = valid[j] && ((chosen >> ((lane + 64 * j) / per)) & 1u) != 0;
        }
    }
    // allowed first, then the logit descending, then the index ascending
    const int K = a.top_k < E ? a.top_k : E;
    const bool wrong = f.perturb != 0 && K < E;
    const int picks = wrong ? K + 1 : K;
    uint64_t key[EPL];
    int rank[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        const float v = valid[j] ? val[e] : 0.0f;
        key[j] = valid[j] ? ((allowed[j] ? (1ull << 62) : 0ull) | (static_cast<uint64_t>(float_order(v)) << 16) |
                             static_cast<uint64_t>(0xffff - e))
                          : 0ull;
        rank[j] = picks;
    }
    for (int r = 0; r < picks; ++r) {
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            best = rank[j] == picks && key[j] > best ? key[j] : best;
        }
        best = wave_max_u64(best);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            rank[j] = rank[j] == picks && key[j] == best ? r : rank[j];
        }
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        // testing: rank K - 1 takes the (K + 1)-th expert
        const int at = !wrong ? rank[j] : (rank[j] == K - 1 ? picks : (rank[j] == K ? K - 1 : rank[j]));
        if (at < K) {
            publish(f.spec + at, f.seq, static_cast<uint32_t>(lane + 64 * j));
        }
    }
}

// Wave 0 of the last exact router workgroup: MoeRouter::select on the exact
// logits (select_token_multi), the selection and the token's permutation as
// select_one_multi_kernel writes them (k_router.hip), then whether the exact
// set of experts differs from the speculated one.
template <int EPL>
__device__ void select_exact(const SpecArgs& f, float* sel, int* ranked) {
    const int lane = threadIdx.x & 63;
    const RouterArgs& a = f.r;
    const int E = a.experts;
    float logit[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        logit[j] = e < E ? load_coherent(a.logits_scratch + e) : 0.0f;
        if (a.bias != nullptr && e < E) {
            logit[j] = logit[j] + a.bias[e];
        }
        if (a.logits != nullptr && e < E) {
            a.logits[e] = logit[j];
        }
    }
    const SelectPolicy p{a.experts, a.top_k, a.normalize, a.group_limited, a.n_group, a.topk_group, a.scale};
    const int K = a.top_k < E ? a.top_k : E;
    int rank[EPL];
    float weight[EPL];
    select_token_multi<EPL>(logit, lane, p, sel, rank, weight);
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        if (rank[j] < K) {
            a.wts[rank[j]] = weight[j];
            ranked[rank[j]] = lane + 64 * j;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the ranks are in LDS
    __builtin_amdgcn_wave_barrier();
    int chosen[kMaxTopK];
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r) {
        chosen[r] = r < K ? ranked[r] : 0x7fffffff;
    }
    for (int e = lane; e < E; e += 64) {
        int count = 0, offset = 0;
#pragma unroll
        for (int r = 0; r < kMaxTopK; ++r) {
            count += chosen[r] == e ? 1 : 0;
            offset += chosen[r] < e ? 1 : 0;
        }
        a.rb.counts[e] = count;
        a.rb.offsets[e] = offset;
    }
    if (lane == 0) {
        a.rb.offsets[E] = K;
        a.rb.active[E] = K;
    }
    if (lane < K) {
        const int e = ranked[lane];
        int pos = 0;
#pragma unroll
        for (int r = 0; r < kMaxTopK; ++r) {
            pos += chosen[r] < e ? 1 : 0;
        }
        a.rb.perm[pos] = lane;
        a.rb.slot_of[lane] = pos;
        a.rb.active[pos] = e;
    }
    // The sets: every exact expert among the speculated ones?
    const uint32_t s = wait_tagged(f.spec, K, f.seq, f.error, f.max_spins);
    const int mine = lane < K ? ranked[lane] : -1;
    bool found = lane >= K;
#pragma unroll
    for (int r = 0; r < kMaxTopK; ++r) {
        const int other = __shfl(static_cast<int>(s), r);
        found = found || (r < K && other == mine);
    }
    const uint32_t differs = __ballot(!found) != 0 ? 1u : 0u;
    // idx is also read by the repair workgroups of this launch
    if (lane < K) {
        store_coherent(a.idx + lane, mine);
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): idx is out before the word that releases its readers
    if (lane == 0) {
        publish(f.exact, f.seq, differs);
    }
}

template <int EPL>
__global__ __launch_bounds__(kThreads) void spec_gateup_kernel(SpecArgs f) {
    extern __shared__ float4 lds4[];  // the router's chunks, the token, or selection scratch
    float* lds = reinterpret_cast<float*>(lds4);
    __shared__ float part[kWaves][8];
    __shared__ int ranked[kMaxTopK];
    __shared__ uint32_t arrived;
    __shared__ uint32_t flag;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const RouterArgs& a = f.r;
    const int E = a.experts;
    const int H = a.hidden;
    const int K = a.top_k < E ? a.top_k : E;
    const int chunks = f.e.inter_p / kItemRows;
    int b = static_cast<int>(blockIdx.x);
    if (blockIdx.x == gridDim.x - 1) {
        // the last workgroup, off the critical path, clears the next launch's counters
        for (int i = tid; i < kCounters * kLanes; i += kThreads) {
            __hip_atomic_store(f.clear + i * kSlotStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (b < f.n_partial) {
        // Reassociated partial logits of experts [e0, e0 + 8) over row quads
        // [256 s, 256 s + 256): one quad per thread ([H/4][E][4] gate layout).
        const int groups = E / 8;
        const int s = b / groups;
        const int e0 = (b - s * groups) * 8;
        const int q = s * (kSliceRows / 4) + tid;
        float sum[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sum[j] = 0.0f;
        }
        if (q < H / 4) {
            const float4 xv = reinterpret_cast<const float4*>(a.x)[q];
            float4 w[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                w[j] = *reinterpret_cast<const float4*>(a.wq4 + (static_cast<int64_t>(q) * E + e0 + j) * 4);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                sum[j] = (w[j].x * xv.x + w[j].y * xv.y) + (w[j].z * xv.z + w[j].w * xv.w);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                sum[j] += __shfl_xor(sum[j], o);
            }
        }
        if (lane < 8) {
            float v = sum[0];
#pragma unroll
            for (int j = 1; j < 8; ++j) {
                v = lane == j ? sum[j] : v;
            }
            part[wave][lane] = v;
        }
        __syncthreads();
        if (tid < 8) {
            store_coherent(f.partial + static_cast<int64_t>(s) * E + e0 + tid,
                           (part[0][tid] + part[1][tid]) + (part[2][tid] + part[3][tid]));
        }
        if (arrive(counter_slot(f.sync, kPartialTicket, 0), &arrived) != static_cast<uint32_t>(f.n_partial - 1) ||
            tid >= 64) {
            return;
        }
        // the last to arrive: the slices' sums (each slice's loads in flight together), the bias
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            if (e < E) {
                float v[kMaxSlices];
#pragma unroll
                for (int u = 0; u < kMaxSlices; ++u) {
                    v[u] = u < f.slices ? load_coherent(f.partial + static_cast<int64_t>(u) * E + e) : 0.0f;
                }
                float t = a.bias != nullptr ? a.bias[e] : 0.0f;
#pragma unroll
                for (int u = 0; u < kMaxSlices; ++u) {
                    t += v[u];
                }
                lds[e] = t;
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_wave_barrier();
        speculate<EPL>(f, lds);
        return;
    }
    b -= f.n_partial;
    if (b < f.n_router) {
        // Exact logits of experts [8 b, 8 b + 8): LiteMind's chains.
        const int e0 = b * 8;
        const float acc = chunked_logit(H, E, a.x, a.wt, e0, lds4);
        if (tid < 8) {
            store_coherent(a.logits_scratch + e0 + tid, acc);
        }
        if (arrive(counter_slot(f.sync, kRouterTicket, 0), &arrived) != static_cast<uint32_t>(f.n_router - 1) ||
            tid >= 64) {
            return;
        }
        select_exact<EPL>(f, lds, ranked);
        return;
    }
    b -= f.n_router;
    if (b < f.n_shared) {
        stage_token(f.e, lds);
        gateup_item(f.e, f.e.groups.gu[E], b, f.e.act + static_cast<int64_t>(K) * f.e.inter_p, lds);
        return;
    }
    b -= f.n_shared;
    if (b < f.n_routed) {
        // Routed gate/up of the speculated expert of rank r, into its slot
        // among the speculated experts.
        stage_token(f.e, lds);
        if (tid < 64) {
            const uint32_t v = wait_tagged(f.spec, K, f.seq, f.error, f.max_spins);
            if (lane < K) {
                ranked[lane] = static_cast<int>(v < static_cast<uint32_t>(E) ? v : 0u);  // clamped after a timeout
            }
        }
        __syncthreads();
        const int r = b / chunks;
        const int g = ranked[r];
        int slot = 0;
        for (int i = 0; i < K; ++i) {
            slot += ranked[i] < g ? 1 : 0;
        }
        gateup_item(f.e, f.e.groups.gu[g], b - r * chunks, f.e.act + static_cast<int64_t>(slot) * f.e.inter_p, lds);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the activations are out before the count
        __syncthreads();
        if (tid == 0) {
            (void)__hip_atomic_fetch_add(counter_slot(f.sync, kRoutedDone, b % kLanes), 1u, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    b -= f.n_routed;
    // Repair: nothing to do unless the exact set differs from the speculated one.
    if (tid < 64) {
        const uint32_t m = wait_tagged(f.exact, 1, f.seq, f.error, f.max_spins);
        if (lane == 0) {
            flag = m;
        }
    }
    __syncthreads();
    if (flag == 0) {
        return;
    }
    wait_routed(f, static_cast<uint32_t>(f.n_routed));
    if (tid < K) {
        const int e = load_coherent(a.idx + tid);
        ranked[tid] = e >= 0 && e < E ? e : 0;
    }
    stage_token(f.e, lds);  // its barrier also publishes ranked
    for (int i = b; i < K * chunks; i += kRepairBlocks) {
        const int r = i / chunks;
        const int g = ranked[r];
        int slot = 0;
        for (int u = 0; u < K; ++u) {
            slot += ranked[u] < g ? 1 : 0;
        }
        gateup_item(f.e, f.e.groups.gu[g], i - r * chunks, f.e.act + static_cast<int64_t>(slot) * f.e.inter_p, lds);
    }
}

}  // namespace

bool spec_gateup_supported(int experts, int hidden, int top_k, int n_group, int group_limited, int inter_p,
                           int shared_inter_p) {
    return experts > kMaxExperts && experts <= kMaxExpertsWide && experts % 8 == 0 && hidden % 8 == 0 &&
           hidden <= kMaxSlices * kSliceRows && top_k >= 1 && top_k <= kMaxTopK && top_k < experts &&
           (!group_limited || n_group <= 64) && inter_p > 0 && inter_p % kItemRows == 0 &&
           shared_inter_p % kItemRows == 0;
}

hipError_t launch_spec_gateup(const RouterArgs& r, const ExpertArgs& e, uint32_t* spec_sync, uint32_t* error,
                              int parity, uint32_t seq, int perturb, uint32_t max_spins, hipStream_t s) {
    const int E = r.experts, H = r.hidden;
    if (r.tokens != 1 || e.tokens != 1 || r.x != e.x || r.x16 != nullptr || r.wt == nullptr || r.wq4 == nullptr ||
        r.logits_scratch == nullptr || r.rb.counts == nullptr || r.idx == nullptr || r.wts == nullptr ||
        e.experts != E || e.top_k != r.top_k || e.hidden != H || spec_sync == nullptr || error == nullptr ||
        seq == 0 || !spec_gateup_supported(E, H, r.top_k, r.n_group, r.group_limited, e.inter_p, e.shared_inter_p)) {
        return hipErrorInvalidValue;
    }
    SpecArgs f{};
    f.r = r;
    f.e = e;
    f.sync = spec_sync + (parity & 1) * kSetWords;
    f.clear = spec_sync + (1 - (parity & 1)) * kSetWords;
    f.error = error;
    f.spec = reinterpret_cast<uint64_t*>(spec_sync + kSpecTagWord);
    f.exact = f.spec + kMaxTopK;
    f.partial = reinterpret_cast<float*>(spec_sync + kSpecPartialWord);
    f.seq = seq;
    f.perturb = perturb;
    f.max_spins = max_spins != 0 ? max_spins : kMaxSpins;
    f.slices = (H + kSliceRows - 1) / kSliceRows;
    f.n_partial = (E / 8) * f.slices;
    f.n_router = E / 8;
    f.n_shared = e.has_shared ? e.shared_inter_p / kItemRows : 0;
    f.n_routed = r.top_k * (e.inter_p / kItemRows);
    const int blocks = f.n_partial + f.n_router + f.n_shared + f.n_routed + kRepairBlocks;
    const int epl = (E + 63) / 64;
    const size_t lds = std::max<size_t>({sizeof(float4) * kChunkFloat4s, sizeof(float) * static_cast<size_t>(H),
                                         sizeof(float) * static_cast<size_t>(select_multi_words(epl))});
    const dim3 grid(static_cast<unsigned>(blocks)), block(kThreads);
    switch (epl) {
        case 2: hipLaunchKernelGGL(spec_gateup_kernel<2>, grid, block, lds, s, f); break;
        case 3: hipLaunchKernelGGL(spec_gateup_kernel<3>, grid, block, lds, s, f); break;
        case 4: hipLaunchKernelGGL(spec_gateup_kernel<4>, grid, block, lds, s, f); break;
        case 5: hipLaunchKernelGGL(spec_gateup_kernel<5>, grid, block, lds, s, f); break;
        case 6: hipLaunchKernelGGL(spec_gateup_kernel<6>, grid, block, lds, s, f); break;
        case 7: hipLaunchKernelGGL(spec_gateup_kernel<7>, grid, block, lds, s, f); break;
        default: hipLaunchKernelGGL(spec_gateup_kernel<8>, grid, block, lds, s, f); break;
    }
    return hipGetLastError();
}

}  // namespace lm
