// lm_internal.h -- shared definitions of the gfx950 MoE library (not part of the ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lm_math.h"

struct lm_context;

namespace lm {

// Weight rows are stored with gate and up interleaved in groups of kGroupRows:
// rows [2*g*G, 2*g*G + G) are gate rows [g*G, (g+1)*G) and the next G rows are
// the matching up rows.  One 32-wide MFMA column block therefore holds only gate
// or only up, and its partner block holds the same output columns.
constexpr int kGroupRows = 32;
// Padding granularity of the intermediate (reduction) and hidden dimensions in
// the resident layout; padded rows and columns are zero.
constexpr int kPad = 64;
constexpr int kMaxExperts = 64;   // one lane per expert: the single-token kernel and the fast router paths
constexpr int kMaxExpertsWide = 512;  // the general router, selection and permutation (lane owns experts lane + 64 j)
// Up to this many tokens, layers of more than 64 experts form their logits
// over E / 8 workgroups per token (into the [tokens, E] logits scratch) before
// the per-token selection.
#ifndef LM_ROUTER_SPLIT_TOKENS
#define LM_ROUTER_SPLIT_TOKENS 256
#endif
constexpr int kRouterSplitTokens = LM_ROUTER_SPLIT_TOKENS;
constexpr int kMaxTopK = 16;

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Panel layout of the fp16 operands of the MFMA path: a [rows, cols] matrix
// (cols a multiple of kPanel) is stored as cols / kPanel panels of
// [rows, kPanel], so the 32-column K slice of any run of rows is one contiguous
// block (rows x 64 bytes).  Element (r, c) sits at panel_index(r, c, rows).
constexpr int kPanel = 32;
__host__ __device__ inline int64_t panel_index(int64_t r, int64_t c, int64_t rows) {
    return (c / kPanel) * rows * kPanel + r * kPanel + (c % kPanel);
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(1))) const u32x4 global_u32x4;

// Workgroup barrier that orders LDS only: waits for this wave's LDS operations
// (lgkmcnt(0); vmcnt and expcnt left at their maxima) and then s_barrier.
// __syncthreads() also fences global memory, which makes every wave wait for
// its outstanding global loads and defeats register prefetching across it.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_s_barrier();
}

// 16-byte load of streamed weights: global address space (pointers read from a
// table would otherwise compile to flat loads) and non-temporal, since every
// weight byte is used once per step.
__device__ inline uint4 load_stream16(const void* p) {
    const u32x4 v = __builtin_nontemporal_load((global_u32x4*)(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// One FFN (routed expert, the fused shared expert or a dense layer) resident in HBM.
//   gu:   [2 * inter_p, hidden_p] BF16, gate/up interleaved as above
//   down: [hidden, inter_p] BF16 (columns >= inter are zero)
//   *_h:  the same matrices re-encoded as fp16 in panel layout for the MFMA path
//   down_t: [inter_p, hidden_p] BF16, the down matrix transposed (the shared
//         expert of a layer the single-token kernel runs; null otherwise)
struct FfnDev {
    uint16_t* gu = nullptr;
    uint16_t* down = nullptr;
    uint16_t* down_t = nullptr;
    _Float16* gu_h = nullptr;
    _Float16* down_h = nullptr;
    int32_t inter = 0;    // logical intermediate width
    int32_t inter_p = 0;  // padded to kPad
};

// Per-group tables the expert kernels index by group id: group g < E is routed
// expert g, group E is the shared expert.  Device arrays of pointers.
struct GroupTable {
    const uint16_t* const* gu;       // [E+1]
    const uint16_t* const* down;     // [E+1]
    const _Float16* const* gu_h;     // [E+1]
    const _Float16* const* down_h;   // [E+1]
};

// Routing results and the permutation, in device memory.
struct RouteBufs {
    int32_t* idx;        // [T*K]
    float* wt;           // [T*K]
    int32_t* counts;     // [E]
    int32_t* offsets;    // [E+1]
    int32_t* perm;       // [T*K]   assignment id at each permuted slot
    int32_t* slot_of;    // [T*K]   permuted slot of each assignment
    int32_t* active;     // [E+1]   routed experts with tokens, ascending; [E] = their number
};

struct RouterArgs {
    const float* x;          // [T, H]
    const float* wt;         // [H, E] router gate, transposed
    const float* wq4;        // [H/4][E][4] the same gate, four rows of an expert together
    const float* bias;       // [E] or null
    float* logits;           // [T, E] or null
    int32_t* idx;            // [T, K]
    float* wts;              // [T, K]
    _Float16* x16;           // [T, Hp] fp16 in panel layout, or null
    int64_t tokens;
    int32_t hidden, hidden_p, experts, top_k;
    int32_t normalize, group_limited, n_group, topk_group;
    float scale;
    int32_t do_matvec;       // 0: x holds logits [T, E] already (select only)
    // Single-token path: fused selection and permutation by the last workgroup.
    float* logits_scratch;   // [E] logits handed to the last workgroup
    uint32_t* ticket;        // arrival counter, 0 between launches (the last workgroup resets it)
    RouteBufs rb;            // permutation outputs (counts, offsets, perm, slot_of, active)
};

struct PermuteArgs {
    const int32_t* idx;
    int64_t tokens;
    int32_t top_k, experts;
    RouteBufs rb;
    int32_t* scratch;        // permute_scratch_words(T*K) words, word 0 zero between launches
};

// Grouped expert kernels.  Slot space: routed slots [0, T*K) in permuted order,
// shared slots [T*K, T*K + T) in token order.
struct ExpertArgs {
    GroupTable groups;
    RouteBufs rb;
    const float* x;          // [T, H] fp32 (GEMV path)
    const _Float16* x16;     // [T, Hp] fp16 in panel layout (MFMA path)
    float* act;              // GEMV: activations fp32, routed [T*K, Ip] then shared [T, Sp]
    _Float16* act16;         // MFMA: fp16 panels, routed [T*K, Ip] then shared [T, Sp]
    float* down_out;         // [T*K + T, H] fp32 down-projection per slot
    int64_t tokens;
    int32_t hidden, hidden_p, experts, top_k;
    int32_t inter_p, shared_inter_p;   // padded widths (shared 0 = none)
    int32_t has_shared;
    // Down GEMM of a layer without routed experts only: K split into ksplit
    // chunks (0 or 1: none), chunk c's partial sums [T, hidden] at
    // partial + c T hidden instead of down_out.
    int32_t ksplit;
    float* partial;
};

struct CombineArgs {
    const float* down_out;   // [T*K + T, H]
    const int32_t* slot_of;  // [T*K]
    const float* wts;        // [T*K]
    float* y;                // [T, H]
    const float* residual;   // [T, H] or null: y = residual + ffn
    int64_t tokens;
    int32_t hidden, top_k, has_shared;
    // The next stack layer's RMSNorm applied to y in the same pass (null: none):
    // xnorm [T, H] = rms_norm(y, next_norm), and x16 (or null) its fp16 copy in
    // panel layout [T, hidden_p].
    const float* next_norm;
    float* xnorm;
    _Float16* x16;
    int32_t hidden_p;
    float eps;
};

// The routing policy of MoeRouter (src/MoeRouter.cpp:38-52).
struct SelectPolicy {
    int32_t experts, top_k;
    int32_t normalize, group_limited, n_group, topk_group;
    float scale;
};

// The single-token MoE block (k_decode.hip).
struct DecodeLaunch {
    const float* x;             // [H] the token, or the hidden state when norm is set
    const float* norm;          // [H] RMSNorm weight applied inside the launch, or null
    float eps;
    float* xnorm;               // [H] scratch: the normalised token (needed when norm is set)
    const float* wq;            // [E/4][H][4] router gate, four experts per contiguous slice
    const float* bias;          // [E] or null
    float* logits;              // [E] scratch
    float* logits_out;          // [E] or null
    int32_t* idx;               // [K] out, rank order
    float* wts;                 // [K] out
    const uint16_t* routed;     // expert 0's resident FFN (gate/up then down)
    int64_t routed_stride;      // elements from one expert's FFN to the next
    const uint16_t* shared_gu;  // shared expert (null: none)
    const uint16_t* shared_down;
    const uint16_t* shared_t;   // the shared expert's down matrix transposed [Sp, Hp]
    float* shared_part;         // [Sp / 16, H] the shared items' partial down projections
    float* act;                 // [K * Ip + Sp]
    float* y;                   // [H]
    const float* residual;      // [H] or null
    int32_t hidden, hidden_p, inter_p, shared_inter_p;
    SelectPolicy policy;
    uint32_t* sync;             // kDecodeSyncWords words, zeroed once
    int32_t parity;             // alternates between consecutive launches
    uint32_t seq;               // nonzero, different in consecutive launches: tags the hand-off words
    int32_t perturb;            // testing: the speculative selection disagrees with every rank
    uint32_t max_spins;         // polls before a wait gives up (0: the kernel's default bound)
};

// Kernel launchers (implemented in the .hip files).
hipError_t launch_router(const RouterArgs& a, hipStream_t s, bool* permuted);
// True when the single-token forward has a one-launch kernel for this shape.
bool decode_supported(int hidden, int experts, int top_k, int inter_p, int shared_inter_p);
hipError_t launch_decode(const DecodeLaunch& d, hipStream_t s);
// Floats of the shared items' partial down projections of the single-token kernel.
int64_t decode_shared_part_floats(int hidden, int shared_inter_p);
// Single-launch decode scratch, in 32-bit words: two sets of 4 counters x 16
// slots x 64 B, the error word, approximate logits [64] and speculative experts
// [16] as tagged 64-bit words, and the mask of ranks the speculation got wrong.
constexpr int kDecodeCounterWords = 2 * 4 * 16 * 16;
constexpr int kDecodeErrorWord = kDecodeCounterWords;
constexpr int kDecodeApproxWord = kDecodeErrorWord + 16;
constexpr int kDecodeSpecWord = kDecodeApproxWord + 2 * kMaxExperts;
constexpr int kDecodeMaskWord = kDecodeSpecWord + 2 * kMaxTopK;
// per-XCD copies of the speculative experts: 8 slots of 128 bytes (one L2 line each)
constexpr int kDecodeXcdSpecWord = (kDecodeMaskWord + 16 + 31) / 32 * 32;
constexpr int kDecodeXcdSlotWords = 32;
constexpr int kDecodeSyncWords = kDecodeXcdSpecWord + 8 * kDecodeXcdSlotWords;
// One token over more than 64 experts on the GEMV path (k_spec.hip): the
// router (selection and permutation into r's outputs) and the gate/up
// projections of the selected and the shared experts into e.act, in one
// launch that starts the routed experts from a speculative selection.  The
// down and combine launches follow as on the multi-launch path.  spec_sync:
// kSpecSyncWords words, zeroed once (counters of the two launch parities,
// tagged hand-off words, partial logits); error: a word that a bounded wait
// which gave up sets; parity alternates and seq (nonzero) differs between
// consecutive launches on spec_sync.  perturb (testing) makes the speculated
// set of experts wrong, so the repair runs.
constexpr int kSpecCounterWords = 2 * 3 * 16 * 16;
constexpr int kSpecTagWord = kSpecCounterWords;
constexpr int kSpecPartialWord = kSpecTagWord + 64;
constexpr int kSpecSyncWords = kSpecPartialWord + 16 * kMaxExpertsWide;
bool spec_gateup_supported(int experts, int hidden, int top_k, int n_group, int group_limited, int inter_p,
                           int shared_inter_p);
hipError_t launch_spec_gateup(const RouterArgs& r, const ExpertArgs& e, uint32_t* spec_sync, uint32_t* error,
                              int parity, uint32_t seq, int perturb, uint32_t max_spins, hipStream_t s);
hipError_t launch_permute(const PermuteArgs& a, hipStream_t s);
// LM head (k_head.hip): logits [tokens, rows] = w [rows, in_dim] . x [tokens, in_dim]
// with gemm::dot_bf16's association, tokens <= kHeadTokens, in_dim % 8 == 0; and
// the greedy choice per token (first maximum of the non-NaN logits).
constexpr int kHeadTokens = 4;
struct HeadBest {
    float v;
    int32_t i;
    int32_t have;
};
// Blocks of the head launch; partial holds kHeadTokens * head_blocks(rows) candidates.
int64_t head_blocks(int64_t rows);
// token may be null (logits only).
hipError_t launch_head(const uint16_t* w, const float* x, float* logits, HeadBest* partial, int32_t* token,
                       int64_t rows, int32_t in_dim, int32_t tokens, hipStream_t s);
// The same kernel as one bit-exact gemm::matvec_bf16 (or _accumulate) of a
// row-major [rows, in_dim] matrix (16-byte aligned), for in_dim % 8 == 0 and
// in_dim <= 16384.
bool matvec_rows_supported(int64_t rows, int64_t in_dim);
hipError_t launch_matvec_rows(const uint16_t* w, const float* x, float* out, int64_t rows, int64_t in_dim, float scale,
                              int32_t accumulate, hipStream_t s);
// The same kernel over T tokens x [T, in_dim] -> out [T, rows] (or out +=
// fma(scale, ., out)), one wave per 16 rows, in launches of up to kHeadTokens
// tokens; conditions as matvec_rows_supported.
hipError_t launch_matvec_tokens(const uint16_t* w, const float* x, float* out, int64_t rows, int64_t in_dim,
                                int64_t tokens, float scale, int32_t accumulate, hipStream_t s);
// gemm::rms_norm (src/Gemm.cpp:197-207) adds the exact double squares in
// element order; the kernels add them in a thread-strided tree (below), whose
// double sum can differ in its last bits, and the inverse float(1 / sqrt(sum /
// n + eps)) then by one ulp for inputs whose double inverse lies near a float
// rounding boundary (rows of a few large and many tiny elements reach it at
// will).  Both sums lie within (n - 1) 2^-53 of the exact sum of the n
// non-negative squares, so the two double inverses lie within a relative
// (n + 8) 2^-53 of each other (half the sums' difference through the root,
// plus the roundings of the division, root and reciprocal).  rms_inverse_exact
// returns the tree's float inverse when it lies farther than (n + 64) 2^-52 of
// itself from both rounding boundaries around it (then both round alike: all
// but about one row in 10^5 of N(0, 1) data); otherwise every thread runs
// stage() (which may copy the thread's elements to where src points) and
// thread 0 adds the squares of src[0], src[1], ... in order, eight loads in
// flight, and the inverse comes from that sum.  Either way the float is
// gemm::rms_norm's, bit for bit.  Every thread of the workgroup calls it with
// the same `total`; `barrier` orders LDS (`part`, 4 doubles, and the stage)
// between its readers and writers.
template <class Stage, class Barrier>
__device__ inline float rms_inverse_exact(double total, int n, float eps, double* part, const float* src, Stage stage,
                                          Barrier barrier) {
    const double r = 1.0 / __builtin_sqrt(total / static_cast<double>(n) + static_cast<double>(eps));
    const float f = static_cast<float>(r);
    const double below = 0.5 * (static_cast<double>(f) + static_cast<double>(nextafterf(f, 0.0f)));
    const double above = 0.5 * (static_cast<double>(f) + static_cast<double>(nextafterf(f, __builtin_inff())));
    const double margin = r * (static_cast<double>(n) + 64.0) * 0x1p-52;
    if (r - below >= margin && above - r >= margin) {
        return f;
    }
    barrier();  // every thread has read the tree's parts
    stage();
    barrier();
    if (threadIdx.x == 0) {
        double sum = 0.0;
        int i = 0;
        for (; i + 8 <= n; i += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                v[u] = src[i + u];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const double d = static_cast<double>(v[u]);
                sum = sum + d * d;
            }
        }
        for (; i < n; ++i) {
            const double d = static_cast<double>(src[i]);
            sum = sum + d * d;
        }
        part[0] = sum;
    }
    barrier();
    const double sum = part[0];
    barrier();  // read before a later call writes `part` or the stage again
    return static_cast<float>(1.0 / __builtin_sqrt(sum / static_cast<double>(n) + static_cast<double>(eps)));
}

// gemm::rms_norm's inverse for x[0 .. n) with 256 threads: thread t sums the
// exact squares of elements t, t + 256, ... in double, in that order; the
// wave's butterfly; then (w0 + w1) + (w2 + w3) over the four waves, made
// LiteMind's by rms_inverse_exact.  The loads are issued eight at a time (a
// loop of one load per step waits a round trip per element).  Every thread of
// the 256-thread workgroup calls it; `part` is 4 doubles of LDS.
// The same inverse from a thread's elements already in registers: v[u] is
// element threadIdx.x + 256 u (n <= 2048; past n ignored); `stage_lds` (n
// floats of LDS, free during the call) receives them for the rare in-order sum.
__device__ inline float rms_inverse_256_regs(const float (&v)[8], int n, float eps, double* part, float* stage_lds) {
    double sq = 0.0;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        if (static_cast<int>(threadIdx.x) + 256 * u < n) {
            const double d = static_cast<double>(v[u]);
            sq = sq + d * d;
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        sq += __shfl_xor(sq, o);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = sq;
    }
    __syncthreads();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    return rms_inverse_exact(
        total, n, eps, part, stage_lds,
        [&] {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int e = static_cast<int>(threadIdx.x) + 256 * u;
                if (e < n) {
                    stage_lds[e] = v[u];
                }
            }
        },
        [] { __syncthreads(); });
}

__device__ inline float rms_inverse_256(const float* __restrict__ x, int n, float eps, double* part) {
    double sq = 0.0;
    for (int e0 = static_cast<int>(threadIdx.x); e0 < n; e0 += 8 * 256) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = e0 + 256 * u;
            v[u] = x[e < n ? e : n - 1];  // unconditional (a conditional load becomes a branch and a wait)
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (e0 + 256 * u < n) {
                const double d = static_cast<double>(v[u]);
                sq = sq + d * d;
            }
        }
    }
    for (int o = 32; o >= 1; o >>= 1) {
        sq += __shfl_xor(sq, o);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = sq;
    }
    __syncthreads();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    return rms_inverse_exact(total, n, eps, part, x, [] {}, [] { __syncthreads(); });
}

// gemm::dot_bf16 of one weight row over 32 lanes (lane c = 0..31 of a half
// wave): lane c runs chain c (elements c, c + 32, ... in order, kOneAhead of
// them requested before the first is added), then chains 0..7 over the 8-wide
// remainder; the 32 lanes then reduce by shuffles in LiteMind's association,
// (a[l] + a[8 + l]) + (a[16 + l] + a[24 + l]), lanes j and j + 4,
// (h0 + h2) + (h1 + h3).  Every lane of the half wave returns the total.
// `xat(e)` gives input element e.  in_dim % 8 == 0.  With `pre`, the lane's
// weights of the first kOneAhead steps were loaded by the caller, earlier
// (only when in_dim >= 32 kOneAhead): word u is the aligned 32-bit word
// holding element 32 u + c (pre_weights), so no instruction touches it before
// the FMA that uses it.
constexpr int kOneAhead = 16;

// The words dot_bf16_lanes32 takes as `pre`: for u < kOneAhead, the aligned
// 32-bit word of row wr holding element 32 u + c (wr 4-byte aligned).
__device__ inline void pre_weights(const uint16_t* __restrict__ wr, int c, uint32_t (&pre)[kOneAhead]) {
    const uint32_t* w32 = reinterpret_cast<const uint32_t*>(wr);
#pragma unroll
    for (int u = 0; u < kOneAhead; ++u) {
        pre[u] = w32[(32 * u + c) >> 1];
    }
}

template <bool PRE, class X>
__device__ inline float dot_bf16_lanes32_impl(const uint16_t* __restrict__ wr, X xat, int in_dim, int c,
                                              const uint32_t (&pre)[kOneAhead]) {
    const int steps = in_dim / 32;
    float acc = 0.0f;
    int k = 0;
    if (PRE) {
        float xv[kOneAhead];
#pragma unroll
        for (int u = 0; u < kOneAhead; ++u) {
            xv[u] = xat(32 * u + c);
        }
#pragma unroll
        for (int u = 0; u < kOneAhead; ++u) {
            const uint32_t word = pre[u];
            acc = __builtin_fmaf(bits_float((c & 1) != 0 ? (word & 0xffff0000u) : (word << 16)), xv[u], acc);
        }
        k = kOneAhead;
    }
    for (; k + kOneAhead <= steps; k += kOneAhead) {
        uint16_t wv[kOneAhead];
        float xv[kOneAhead];
#pragma unroll
        for (int u = 0; u < kOneAhead; ++u) {
            wv[u] = wr[32 * (k + u) + c];
            xv[u] = xat(32 * (k + u) + c);
        }
#pragma unroll
        for (int u = 0; u < kOneAhead; ++u) {
            acc = __builtin_fmaf(widen_bf16(wv[u]), xv[u], acc);
        }
    }
    for (; k < steps; ++k) {
        acc = __builtin_fmaf(widen_bf16(wr[32 * k + c]), xat(32 * k + c), acc);
    }
    if (c < 8) {
        for (int e = steps * 32 + c; e < in_dim; e += 8) {
            acc = __builtin_fmaf(widen_bf16(wr[e]), xat(e), acc);
        }
    }
    const float t1 = acc + __shfl_xor(acc, 8);
    const float t2 = t1 + __shfl_xor(t1, 16);
    const float t3 = t2 + __shfl_xor(t2, 4);
    const float t4 = t3 + __shfl_xor(t3, 2);
    return t4 + __shfl_xor(t4, 1);
}

template <class X>
__device__ inline float dot_bf16_lanes32(const uint16_t* __restrict__ wr, X xat, int in_dim, int c) {
    const uint32_t none[kOneAhead] = {};
    return dot_bf16_lanes32_impl<false>(wr, xat, in_dim, c, none);
}

// The same with the first kOneAhead steps' weights already in registers.
template <class X>
__device__ inline float dot_bf16_lanes32(const uint16_t* __restrict__ wr, X xat, int in_dim, int c,
                                         const uint32_t (&pre)[kOneAhead]) {
    return dot_bf16_lanes32_impl<true>(wr, xat, in_dim, c, pre);
}

// ---- multi-head latent attention (k_attn.hip) ----
// Shapes of one attention launch; cos_t / sin_t are the rotary tables
// [max_positions, rope / 2] in HBM.
struct AttnShape {
    int32_t heads = 0, nope = 0, rope = 0, vh = 0, rank = 0;
    int64_t cap = 0;            // KV cache capacity (token stride of key_nope and key_rope)
    int64_t max_positions = 0;  // rotary table rows
    const float* cos_t = nullptr;
    const float* sin_t = nullptr;
};
// One layer's KV cache: key_nope [heads][nope][cap], key_rope [rope][cap],
// value [heads][cap][vh], fp32.
struct KvCacheDev {
    float* key_nope = nullptr;
    float* key_rope = nullptr;
    float* value = nullptr;
};
bool attention_shape_supported(const AttnShape& a);
hipError_t launch_rope_query(const AttnShape& a, float* q, int64_t T, int64_t pos0, hipStream_t s);
hipError_t launch_kv_prep(const AttnShape& a, const KvCacheDev& c, const float* lat, const float* norm_w, float* kvn,
                          int64_t T, int64_t slot0, int64_t pos0, float eps, hipStream_t s);
hipError_t launch_kv_append(const AttnShape& a, const KvCacheDev& c, const float* kvx, int64_t T, int64_t slot0,
                            hipStream_t s);
// One token (decode): the query projection (rows heads * (nope + rope), or
// q_b's) with the rotary step of launch_rope_query applied to its output rows
// in the same launch; nope % 2 == 0 and matvec_rows_supported.  With w2, a
// second projection of the same x (rows2 rows, no rotary step, into out2)
// runs in the same launch.  With norm_w (in_dim <= 2048), x is normalised
// inside the launch first, bit for bit as launch_rms_norm would (eps as there).
bool query_rope_one_supported(const AttnShape& a, int64_t in_dim);
hipError_t launch_query_rope_one(const AttnShape& a, const uint16_t* w, const float* x, float* q, int64_t in_dim,
                                 int64_t pos, hipStream_t s, const uint16_t* w2 = nullptr, float* out2 = nullptr,
                                 int64_t rows2 = 0, const float* norm_w = nullptr, float eps = 0.0f);
// One token: launch_kv_prep, kv_b's projection of its output and
// launch_kv_append in one launch (every workgroup forms the normalised latent
// itself); the cache slot `slot`, rotary position `pos`.
bool kv_one_supported(const AttnShape& a);
hipError_t launch_kv_one(const AttnShape& a, const KvCacheDev& c, const uint16_t* kv_b, const float* lat,
                         const float* norm_w, float eps, int64_t slot, int64_t pos, hipStream_t s);
// scores -> softmax -> context for T tokens in slots n0 .. n0 + T - 1 (already
// appended); S holds T * heads * (n0 + T) floats, ctx [T, heads * vh].
hipError_t launch_attention_core(const AttnShape& a, const KvCacheDev& c, const float* q, float* S, float* ctx,
                                 int64_t T, int64_t n0, float scale, hipStream_t s);
// The attention core on MFMA (fp16 operands, fp32 accumulation) for T query
// tokens at cache slots n0 .. n0 + T - 1 over the first `keys` cached tokens
// (n0 + T <= keys), Kp = keys rounded up to 32.  Buffers:
struct AttnMfmaBufs {
    _Float16* k16;   // [heads][Kp][qk] panels (launch_pack_kv16)
    _Float16* v16;   // [heads][vh][Kp] panels (launch_pack_kv16)
    _Float16* q16;   // [heads T][qk] panels
    float* S;        // [heads T][Kp] raw scores
    _Float16* p16;   // [heads T][Kp] panels, probabilities
    float* c32;      // [heads T][vh] context per head
    void* meta;      // mfma_heads_meta_bytes(heads): the per-head group table
};
bool attention_mfma_supported(const AttnShape& a);
// fp16 panel copies of keys 0 .. keys - 1 (zero rows / columns up to Kp).
hipError_t launch_pack_kv16(const AttnShape& a, const KvCacheDev& c, int64_t keys, _Float16* k16, _Float16* v16,
                            hipStream_t s);
// q [T][heads][qk] (rotary applied) -> the context in fp16 panels
// ctx16 [ctx_rows][heads vh], rows row0 .. row0 + T - 1 (the output
// projection's input).
hipError_t launch_attention_core_mfma(const AttnShape& a, const float* q, const AttnMfmaBufs& b, int64_t T,
                                      int64_t n0, int64_t keys, float scale, _Float16* ctx16, int64_t row0,
                                      int64_t ctx_rows, hipStream_t s);

// ---- services of the context (lm_capi.hip) to the attention translation unit ----
struct AttnState;
struct ContextInfo {
    int device = 0;
    hipStream_t stream = nullptr;
    int32_t hidden = 0;
    int32_t layers = 0;
};
ContextInfo context_info(const lm_context* ctx);
AttnState*& context_attention(lm_context* ctx);
// h += FFN_l(rms_norm(h, post_attention_layernorm_l)) for T rows of hidden
// (src/DeepSeekRunner.cpp:264-290), as one layer of lm_stack_forward.
int ffn_sublayer(lm_context* ctx, int32_t layer, float* hidden, int64_t T, int32_t path);
// Frees what lm_attention_configure allocated (lm_attn.hip); null is a no-op.
void attention_release(AttnState* st);

// Words of the permutation's scratch for T*K assignments (zeroed once at allocation).
int64_t permute_scratch_words(int64_t assignments);
hipError_t launch_gemv_gateup(const ExpertArgs& a, int64_t max_groups, hipStream_t s);
hipError_t launch_gemv_down(const ExpertArgs& a, int64_t max_groups, hipStream_t s);
// Grouped SwiGLU on MFMA (k_mfma.hip): fp16 panel operands, fp32 accumulation.
hipError_t launch_mfma_gateup(const ExpertArgs& a, hipStream_t s);
hipError_t launch_mfma_down(const ExpertArgs& a, hipStream_t s);
// out [M, N] = a16 . W^T (accumulate: out += a16 . W^T) for a16 [M, Kp] and W
// [N, Kp] fp16 panels (*w, a device pointer to the matrix), fp32 accumulation,
// on the down kernel as one group of M rows.  With few tiles the K range is
// split (partial sums, then added in chunk order).  scratch: floats for the
// partial sums (at least M N when accumulating; up to 4 M N are used).
hipError_t launch_mfma_gemm(const _Float16* a16, const _Float16* const* w, float* out, int64_t M, int32_t N, int32_t Kp,
                            int32_t accumulate, float* scratch, int64_t scratch_floats, hipStream_t s);
// Per-head GEMMs on the grouped MFMA kernel: out[g rows + m, n] =
// a16[g rows + m] . w16[g w_stride + n] for heads groups of `rows` rows; a16
// [heads rows][Kp] and each w16 block [N][Kp] in panel layout, out fp32
// [heads rows][N].  meta: device scratch of mfma_heads_meta_bytes(heads) for the
// group table (written by a kernel on s before the GEMM).
inline int64_t mfma_heads_meta_bytes(int64_t heads) { return round_up(4 * (2 * heads + 1), 8) + 8 * heads; }
hipError_t launch_mfma_heads(const _Float16* a16, const _Float16* w16, int64_t w_stride, float* out, int32_t heads,
                             int64_t rows, int32_t N, int32_t Kp, void* meta, hipStream_t s);
hipError_t launch_combine(const CombineArgs& a, hipStream_t s);
// out[i] += y[i] for n floats.
hipError_t launch_add_rows(float* out, const float* y, int64_t n, hipStream_t s);
// out [T*K + T, H]: the down projection of each routed assignment in
// assignment order (down_out[slot_of[a]]), then the T shared rows (zero
// without a shared expert).  hidden % 4 == 0.
hipError_t launch_gather_slots(const float* down_out, const int32_t* slot_of, float* out, int64_t assignments,
                               int64_t tokens, int32_t hidden, int32_t has_shared, hipStream_t s);
// True when launch_combine can apply the next layer's norm (CombineArgs::next_norm).
bool combine_norm_supported(int32_t hidden, int32_t hidden_p);
// dst = fp16 panels of the BF16 matrix src [rows, cols] (cols % kPanel == 0);
// counts values outside the fp16 range into *overflow.
hipError_t launch_bf16_to_f16_panels(const uint16_t* src, _Float16* dst, int64_t rows, int64_t cols, int* overflow,
                                     unsigned long long* inexact, hipStream_t s);
// x16 = fp16 panels of x [rows, cols], zero-padded to cols_p columns.
hipError_t launch_to_f16_rows(const float* x, _Float16* x16, int64_t rows, int32_t cols, int32_t cols_p,
                              hipStream_t s);
// dst [cols, dst_stride] = src [rows, src_stride] transposed (16-bit elements).
hipError_t launch_transpose_u16(const uint16_t* src, uint16_t* dst, int64_t rows, int64_t cols, int64_t src_stride,
                               int64_t dst_stride, hipStream_t s);
hipError_t launch_clock_probe(uint64_t* out, int32_t max_pairs, int64_t period_ticks, int64_t total_ticks,
                              hipStream_t s);
hipError_t launch_rms_norm(const float* in, const float* w, float* out, int64_t rows, int32_t cols, float eps,
                           hipStream_t s);
hipError_t launch_matvec_f32_ref(const float* w, const float* x, float* out, int64_t out_dim, int64_t in_dim,
                                 hipStream_t s);
hipError_t launch_vector_op(int op, const void* a, const float* b, float* out, int64_t n, float scalar,
                            hipStream_t s);
hipError_t launch_gemv_plain(const uint16_t* w, const float* x, float* out, int64_t out_dim, int64_t in_dim,
                             float scale, int32_t accumulate, hipStream_t s);

}  // namespace lm
