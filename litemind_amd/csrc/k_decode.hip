// k_decode.hip -- the MoE block for a single token (decode) in one launch.
//
// Reference: the MoE branch of DeepSeekRunner::Impl::forward
// (src/DeepSeekRunner.cpp:273-290): router matvec_f32, MoeRouter::select,
// feed_forward for each selected expert in rank order, then the shared expert,
// accumulated into the layer output.
//
// At T = 1 the block streams ~139 MB of weights; what it computes is small.  Its
// critical path would be the router's 2048-long dependent add chain (~7 us on
// gfx950: every logit is LiteMind's strictly sequential fp32 sum) followed by
// the routed experts, which cannot start before the selection is known.  One
// launch runs every part as a role of its workgroups, ordered so that work
// waits only on workgroups with lower indices (see decode_fused_kernel), and
// the routed experts start from a speculative selection while the exact
// logits are still being summed.
#include <algorithm>

#include "gemv_items.h"
#include "handoff.h"
#include "lm_select.h"


// Timeline hooks: a build with LM_DECODE_TRACE defined records, per workgroup,
// four s_memrealtime stamps (100 MHz) into lm_decode_trace, read back with
// lm_decode_trace_read: 0 the start, 1 the speculation known (routed, down),
// 2 the weights consumed (gate/up) or every wait passed (down), 3 the end.  The
// library's own build compiles them out.
#ifdef LM_DECODE_TRACE
__device__ unsigned long long lm_decode_trace[4 * 4096];
#define LM_TRACE(k)                                                                   \
    do {                                                                              \
        if (threadIdx.x == 0 && blockIdx.x < 4096) {                                  \
            lm_decode_trace[4 * blockIdx.x + (k)] = __builtin_amdgcn_s_memrealtime(); \
        }                                                                             \
    } while (0)
#else
#define LM_TRACE(k) \
    do {            \
    } while (0)
#endif

namespace lm {
namespace {

typedef __attribute__((address_space(1))) const void decode_global_void;
typedef __attribute__((address_space(3))) void decode_lds_void;

using gemv::dot_rows;
using gemv::fma8;
using gemv::load_rows;
using gemv::log2c;
using gemv::transpose_reduce;

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRouterExperts = 4;            // experts per router workgroup
constexpr int kRpw = 4;                      // gate rows (and as many up rows) per wave
constexpr int kItemRows = kRpw * kWaves;     // gate rows per gate/up item

struct DecodeArgs {
    const float* x;            // [H] the token (the hidden state when norm is set)
    const float* norm;         // [H] RMSNorm weight applied to x first, or null (x is already normalised)
    float eps;
    float* xnorm;              // [H] the normalised token (written by router workgroup 0 when norm is set)
    const float* wq;           // [E/4][H][4] router gate, four experts per contiguous slice
    const float* bias;         // [E] or null
    float* logits;             // [E] exact logits (hand-off to the selecting workgroup)
    float* logits_out;         // [E] or null
    int32_t* idx;              // [K] selection in rank order
    float* wts;                // [K]
    const uint16_t* routed;    // expert 0's FFN; expert e at routed + e * routed_stride
    int64_t routed_stride;     // elements between consecutive experts
    const uint16_t* shared_gu;
    const uint16_t* shared_down;
    const uint16_t* shared_t;  // [Sp, Hp] the shared expert's down matrix transposed
    float* shared_part;        // [Sp / 16, H] the shared items' partial down projections
    float* act;                // [K, Ip] routed activations in rank order
    float* y;                  // [H]
    const float* residual;     // [H] or null
    int32_t hidden, hidden_p, experts, top_k, inter_p, shared_inter_p, has_shared;
    SelectPolicy policy;
};

// Device-scope accesses (`sc1`): stores write through the XCD's L2 to memory
// and loads bypass it, so a value written by a workgroup on one XCD is seen by
// a workgroup on another within the same launch without an L2 writeback or
// invalidate.  Everything one workgroup hands to another goes through these.
// (store_coherent / load_coherent: handoff.h)
__device__ inline float4 load_coherent4(const float* p) {
    uint64_t* q = reinterpret_cast<uint64_t*>(const_cast<float*>(p));
    const uint64_t lo = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t hi = __hip_atomic_load(q + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(bits_float(static_cast<uint32_t>(lo)), bits_float(static_cast<uint32_t>(lo >> 32)),
                       bits_float(static_cast<uint32_t>(hi)), bits_float(static_cast<uint32_t>(hi >> 32)));
}

// Activations of lane columns of one row (device-scope loads): zero past the end.
template <int ITERS>
__device__ inline void load_act_coherent(const float* row, int width, int lane, float4 (&x)[ITERS][2]) {
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
        const int c = it * 512 + lane * 8;
        const int cc = c < width ? c : width - 8;
        x[it][0] = load_coherent4(row + cc);
        x[it][1] = load_coherent4(row + cc + 4);
        if (c >= width) {
            x[it][0] = make_float4(0.f, 0.f, 0.f, 0.f);
            x[it][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

// RMSNorm of the token inside the launch (the stack's T = 1 step): the inverse
// of gemm::rms_norm (src/Gemm.cpp:197-207) with the arithmetic of
// rms_norm_kernel (thread-strided double sums of exact squares, wave
// butterfly, then (w0 + w1) + (w2 + w3), made LiteMind's by rms_inverse_exact),
// so the normalised token is the same bits as the separate kernel's.  The token's elements are loaded first
// (norm_load: issue them before any weight stream, so waiting for them waits
// for nothing else) and reduced by norm_reduce, which every thread of the
// workgroup calls; its barrier orders LDS only.  `stage`: hidden floats of LDS
// that are free during the call (the rare in-order sum copies the token there).
static_assert(kWaves == 4, "norm_reduce combines four wave sums");
template <int N>
__device__ inline void norm_load(const DecodeArgs& a, float (&v)[N]) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const int c = static_cast<int>(threadIdx.x) + k * kThreads;
        v[k] = c < a.hidden ? a.x[c] : 0.0f;
    }
}

template <int N>
__device__ inline float norm_reduce(const DecodeArgs& a, const float (&v)[N], float* stage) {
    __shared__ double part[kWaves];
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        if (static_cast<int>(threadIdx.x) + k * kThreads < a.hidden) {
            const double d = static_cast<double>(v[k]);
            s = s + d * d;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        s += __shfl_xor(s, o);
    }
    if ((threadIdx.x & 63) == 0) {
        part[threadIdx.x >> 6] = s;
    }
    lds_barrier();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    return rms_inverse_exact(
        total, a.hidden, a.eps, part, stage,
        [&] {
#pragma unroll
            for (int k = 0; k < N; ++k) {
                const int c = static_cast<int>(threadIdx.x) + k * kThreads;
                if (c < a.hidden) {
                    stage[c] = v[k];
                }
            }
        },
        [] { lds_barrier(); });
}

// Elements per thread of norm_load for a hidden width covered by GI 512-column steps.
template <int GI>
constexpr int norm_elems() { return 2 * GI; }

// ---- roles -------------------------------------------------------------------

// Logits of experts [e0, e0 + 4) with LiteMind's dot (src/Gemm.cpp:183-189):
// all threads form the rounded products into LDS ([H/4][4] float4, four
// consecutive rows of one expert per float4) from the slice's contiguous
// [H][4] weights; then lane e adds its expert's products strictly left to
// right, at raised wave priority (the chain shares its SIMD with streaming
// waves).  after_load runs on every thread once the products are in LDS.
// With the norm fused and no logit bias, the approximate logits come earlier,
// from the unnormalised products w (x nw): the norm's inverse is one positive
// factor of every expert's logit, so it does not change their order, and the
// speculation then waits for neither the norm's reduction nor the products'
// LDS round; `early(e, t)` runs on threads e < 4 with expert e0 + e's sum, and
// after_load is not called.
template <int GI, typename AfterLoad, typename Early>
__device__ __forceinline__ void router_slice(const DecodeArgs& a, int e0, float4* prod, AfterLoad after_load,
                                             Early early) {
    const int tid = threadIdx.x;
    const int H = a.hidden;
    const float4* slice = reinterpret_cast<const float4*>(a.wq) + static_cast<int64_t>(e0 / 4) * H;
    float* pf = reinterpret_cast<float*>(prod);
    auto load_block = [&](int hb, float4 (&w)[8]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int h = hb + j * kThreads + tid;
            w[j] = slice[h < H ? h : H - 1];
        }
    };
    // With the norm fused, the token's elements and their norm weights are
    // requested first and the slice's rows right after them: results return in
    // issue order, so the reduction runs while the slice is still arriving.
    // The elements the norm reduces are the ones this thread multiplies
    // (element tid + kThreads k), so nothing is loaded after the reduction.
    constexpr int kBlocks = (GI + 3) / 4;  // passes of kThreads * 8 rows
    constexpr int KB = kBlocks * 8;
    float4 w[8];
    float v[KB], nw[KB];
    float inverse = 1.0f;
    if (a.norm != nullptr) {
        norm_load(a, v);
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const int c = tid + k * kThreads;
            nw[k] = c < H ? a.norm[c] : 0.0f;
        }
    }
    load_block(0, w);
    const bool early_spec = kBlocks == 1 && a.norm != nullptr && a.bias == nullptr;
    if (early_spec) {
        float p[kRouterExperts] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (j * kThreads + tid < H) {
                const float u = v[j] * nw[j];
                p[0] = __builtin_fmaf(w[j].x, u, p[0]);
                p[1] = __builtin_fmaf(w[j].y, u, p[1]);
                p[2] = __builtin_fmaf(w[j].z, u, p[2]);
                p[3] = __builtin_fmaf(w[j].w, u, p[3]);
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
#pragma unroll
            for (int e = 0; e < kRouterExperts; ++e) {
                p[e] += __shfl_xor(p[e], o);
            }
        }
        __shared__ float early_red[kWaves][kRouterExperts];
        if ((tid & 63) == 0) {
#pragma unroll
            for (int e = 0; e < kRouterExperts; ++e) {
                early_red[tid >> 6][e] = p[e];
            }
        }
        lds_barrier();
        if (tid < kRouterExperts) {
            early(tid, (early_red[0][tid] + early_red[1][tid]) + (early_red[2][tid] + early_red[3][tid]));
        }
    }
    if (a.norm != nullptr) {
        inverse = norm_reduce(a, v, pf);  // the products are formed after it
    }
#pragma unroll
    for (int blk = 0; blk < kBlocks; ++blk) {
        const int hb = blk * kThreads * 8;
        if (blk > 0) {
            load_block(hb, w);
        }
        float xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int h = hb + j * kThreads + tid;
            const int hc = h < H ? h : H - 1;
            if (a.norm != nullptr) {
                const float scaled = v[blk * 8 + j] * inverse;  // rms_norm's (x * inverse) * w
                xv[j] = scaled * nw[blk * 8 + j];
            } else {
                xv[j] = a.x[hc];
            }
            if (a.norm != nullptr && e0 == 0 && h < H) {
                // the repair path's copy: y may overwrite x (the stack updates the
                // hidden state in place) once every router and gate/up item is done
                store_coherent(a.xnorm + h, xv[j]);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int h = hb + j * kThreads + tid;
            if (h < H) {
                float* q = pf + (h >> 2) * 16 + (h & 3);
                q[0] = w[j].x * xv[j];
                q[4] = w[j].y * xv[j];
                q[8] = w[j].z * xv[j];
                q[12] = w[j].w * xv[j];
            }
        }
    }
    lds_barrier();
    if (!early_spec) {
        after_load();
    }
    if (tid >= kRouterExperts) {
        return;
    }
    __builtin_amdgcn_s_setprio(3);
    const int quads = H / 4;
    float acc = 0.0f;
    int q = 0;
    if (quads >= 16) {
        float4 A[8], B[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            A[u] = prod[u * kRouterExperts + tid];
        }
        for (; q + 16 <= quads; q += 16) {
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                B[u] = prod[(q + 8 + u) * kRouterExperts + tid];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc = acc + A[u].x;
                acc = acc + A[u].y;
                acc = acc + A[u].z;
                acc = acc + A[u].w;
            }
            const int nq = q + 16 + 8 <= quads ? q + 16 : q;  // next A batch (re-read harmlessly at the end)
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                A[u] = prod[(nq + u) * kRouterExperts + tid];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc = acc + B[u].x;
                acc = acc + B[u].y;
                acc = acc + B[u].z;
                acc = acc + B[u].w;
            }
        }
    }
    for (; q < quads; ++q) {
        const float4 p = prod[q * kRouterExperts + tid];
        acc = acc + p.x;
        acc = acc + p.y;
        acc = acc + p.z;
        acc = acc + p.w;
    }
    __builtin_amdgcn_s_setprio(0);
    const int e = e0 + tid;
    if (a.bias != nullptr) {
        acc = acc + a.bias[e];
    }
    store_coherent(a.logits + e, acc);
    if (a.logits_out != nullptr) {
        a.logits_out[e] = acc;
    }
}

// Gate/up rows [16 chunk, 16 chunk + 16) of one FFN for the token, act =
// silu(gate) * up (src/Gemm.cpp:225-231), four gate rows and the matching up
// rows per wave.  The token's activations are staged once per workgroup in LDS
// (xs, hidden floats) rather than held by every wave, which leaves the registers
// to weight rows in flight; their loads are issued before the weights' so that
// waiting for them does not wait for the weights.
template <int GI>
__device__ __forceinline__ void gateup_item(const uint16_t* gu, const DecodeArgs& a, int chunk, float* act_row,
                                            float* xs) {
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
    uint4 w[R][GI];
    constexpr int XS = (GI * 128 + kThreads - 1) / kThreads;  // float4 per thread
    const int n4 = a.hidden / 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    float4 xv[XS];
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        const int f = static_cast<int>(threadIdx.x) + i * kThreads;
        xv[i] = x4[f < n4 ? f : n4 - 1];
    }
    // With the norm fused, its elements and the norm weights of this thread's
    // staging columns are requested before the weight rows too: results return
    // in issue order, so anything requested after the rows would wait for them.
    float nv[norm_elems<GI>()];
    float4 nw[XS];
    if (a.norm != nullptr) {
        norm_load(a, nv);
        const float4* n4w = reinterpret_cast<const float4*>(a.norm);
#pragma unroll
        for (int i = 0; i < XS; ++i) {
            const int f = static_cast<int>(threadIdx.x) + i * kThreads;
            nw[i] = n4w[f < n4 ? f : n4 - 1];
        }
    }
    load_rows<R, GI>(rows, a.hidden, lane, w);
    const float inverse = a.norm != nullptr ? norm_reduce(a, nv, xs) : 1.0f;
    float4* xs4 = reinterpret_cast<float4*>(xs);
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        const int f = static_cast<int>(threadIdx.x) + i * kThreads;
        if (f < n4) {
            float4 t = xv[i];
            if (a.norm != nullptr) {  // rms_norm's (x * inverse) * w, on the preloaded weights
                t.x = (t.x * inverse) * nw[i].x;
                t.y = (t.y * inverse) * nw[i].y;
                t.z = (t.z * inverse) * nw[i].z;
                t.w = (t.w * inverse) * nw[i].w;
            }
            xs4[f] = t;
        }
    }
    lds_barrier();
#pragma unroll
    for (int it = 0; it < GI; ++it) {
        const int c = it * 512 + lane * 8;
        const bool in = c < a.hidden;
        const int cc = in ? c : 0;
        float4 x0 = xs4[cc / 4];
        float4 x1 = xs4[cc / 4 + 1];
        if (!in) {
            x0 = make_float4(0.f, 0.f, 0.f, 0.f);
            x1 = make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            fma8(acc[r], w[r][it], x0, x1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    LM_TRACE(2);
    const float sum = transpose_reduce<R>(acc, lane);
    constexpr int L = log2c<R>();
    const int vi = lane >> (6 - L);
    const float up = __shfl_xor(sum, kRpw << (6 - L));
    if ((lane & ((1 << (6 - L)) - 1)) == 0 && (vi & kRpw) == 0) {
        store_coherent(act_row + j0 + (vi & (kRpw - 1)), silu_mul_ref(sum, up));
    }
}

// A shared-expert item: gate/up rows [16 chunk, 16 chunk + 16) as gateup_item
// forms them (LiteMind's roundings), and then the item's share of the shared
// expert's down projection of every output row, p[h] = sum_j act_j down[h][j]
// over its 16 rows j, from the transposed down matrix (row j of it is column j
// of down, contiguous).  Gate, up and down rows (192 KB) are requested
// together.  The four waves' sums go through LDS to part with device-scope
// stores, two floats per lane.  Layout [H / 8][items][8]: output rows 8b ..
// 8b + 7 of every item form one contiguous run, which is what one down
// workgroup reads (four lanes fill one 32-byte piece).  The shared items run from the launch's start, while the router
// still decides, so this moves the shared expert's down stream (11.5 MB on
// V2-Lite) out of the down workgroups' late phase.  LDS: xs (hidden floats),
// red (4 hidden floats).
template <int GI>
__device__ __forceinline__ void shared_item(const DecodeArgs& a, int chunk, float* xs, float* red) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    constexpr int R = 2 * kRpw;
    const uint16_t* rows[R];
    const uint16_t* drows[kRpw];
    const int j0 = chunk * kItemRows + wave * kRpw;
#pragma unroll
    for (int r = 0; r < kRpw; ++r) {
        const int j = j0 + r;
        const int64_t gate_row = static_cast<int64_t>(j / kGroupRows) * (2 * kGroupRows) + (j % kGroupRows);
        rows[r] = a.shared_gu + gate_row * a.hidden_p;
        rows[kRpw + r] = a.shared_gu + (gate_row + kGroupRows) * a.hidden_p;
        drows[r] = a.shared_t + static_cast<int64_t>(j) * a.hidden_p;
    }
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        acc[i] = 0.0f;
    }
    uint4 w[R][GI];
    uint4 dw[kRpw][GI];
    constexpr int XS = (GI * 128 + kThreads - 1) / kThreads;  // float4 per thread
    const int n4 = a.hidden / 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    float4 xv[XS];
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        const int f = static_cast<int>(threadIdx.x) + i * kThreads;
        xv[i] = x4[f < n4 ? f : n4 - 1];
    }
    // the norm's inputs are requested before the weight rows (results return
    // in issue order)
    float nv[norm_elems<GI>()];
    float4 nw[XS];
    if (a.norm != nullptr) {
        norm_load(a, nv);
        const float4* n4w = reinterpret_cast<const float4*>(a.norm);
#pragma unroll
        for (int i = 0; i < XS; ++i) {
            const int f = static_cast<int>(threadIdx.x) + i * kThreads;
            nw[i] = n4w[f < n4 ? f : n4 - 1];
        }
    }
    load_rows<R, GI>(rows, a.hidden, lane, w);
    load_rows<kRpw, GI>(drows, a.hidden, lane, dw);
    const float inverse = a.norm != nullptr ? norm_reduce(a, nv, xs) : 1.0f;
    float4* xs4 = reinterpret_cast<float4*>(xs);
#pragma unroll
    for (int i = 0; i < XS; ++i) {
        const int f = static_cast<int>(threadIdx.x) + i * kThreads;
        if (f < n4) {
            float4 t = xv[i];
            if (a.norm != nullptr) {  // rms_norm's (x * inverse) * w
                t.x = (t.x * inverse) * nw[i].x;
                t.y = (t.y * inverse) * nw[i].y;
                t.z = (t.z * inverse) * nw[i].z;
                t.w = (t.w * inverse) * nw[i].w;
            }
            xs4[f] = t;
        }
    }
    lds_barrier();
#pragma unroll
    for (int it = 0; it < GI; ++it) {
        const int c = it * 512 + lane * 8;
        const bool in = c < a.hidden;
        const int cc = in ? c : 0;
        float4 x0 = xs4[cc / 4];
        float4 x1 = xs4[cc / 4 + 1];
        if (!in) {
            x0 = make_float4(0.f, 0.f, 0.f, 0.f);
            x1 = make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            fma8(acc[r], w[r][it], x0, x1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    LM_TRACE(2);
    const float sum = transpose_reduce<R>(acc, lane);
    constexpr int L = log2c<R>();
    // lanes r << (6 - L), r < kRpw, hold gate row j0 + r; its up row is 32 lanes up
    const float up = __shfl_xor(sum, kRpw << (6 - L));
    const float act = silu_mul_ref(sum, up);
    float av[kRpw];
#pragma unroll
    for (int r = 0; r < kRpw; ++r) {
        av[r] = __shfl(act, r << (6 - L));
    }
    // This wave's four rows of the down projection for the lane's columns.
    float4* red4 = reinterpret_cast<float4*>(red);
    const int H = a.hidden;
#pragma unroll
    for (int it = 0; it < GI; ++it) {
        const int c = it * 512 + lane * 8;
        float p[8];
#pragma unroll
        for (int r = 0; r < kRpw; ++r) {
            const uint4 d = dw[r][it];
            const float dv[8] = {bits_float(d.x << 16), bits_float(d.x & 0xffff0000u), bits_float(d.y << 16),
                                 bits_float(d.y & 0xffff0000u), bits_float(d.z << 16), bits_float(d.z & 0xffff0000u),
                                 bits_float(d.w << 16), bits_float(d.w & 0xffff0000u)};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                p[e] = r == 0 ? av[0] * dv[e] : __builtin_fmaf(av[r], dv[e], p[e]);
            }
        }
        if (c < H) {
            red4[(wave * H + c) / 4] = make_float4(p[0], p[1], p[2], p[3]);
            red4[(wave * H + c) / 4 + 1] = make_float4(p[4], p[5], p[6], p[7]);
        }
    }
    lds_barrier();
    const float2* red2 = reinterpret_cast<const float2*>(red);
    const int64_t n_items = a.shared_inter_p / kItemRows;
    for (int h2 = threadIdx.x; h2 < H / 2; h2 += kThreads) {
        float2 v[kWaves];
#pragma unroll
        for (int u = 0; u < kWaves; ++u) {
            v[u] = red2[u * (H / 2) + h2];
        }
        const float o0 = (v[0].x + v[1].x) + (v[2].x + v[3].x);
        const float o1 = (v[0].y + v[1].y) + (v[2].y + v[3].y);
        const int h = 2 * h2;
        uint64_t* dst = reinterpret_cast<uint64_t*>(a.shared_part + ((h >> 3) * n_items + chunk) * 8 + (h & 7));
        __hip_atomic_store(dst, static_cast<uint64_t>(float_bits(o0)) | (static_cast<uint64_t>(float_bits(o1)) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---- the single launch --------------------------------------------------------
//
// One grid, roles by workgroup index, in dependency order:
//   [routers | shared gate/up | routed gate/up | down + combine]
// (the down workgroups also project the shared expert for their rows).
// A workgroup waits only for workgroups with lower indices.  The dispatcher
// places workgroups on the GPU in index order, so when one waits, everything it
// waits for is resident or finished, and every wait ends; each wait is bounded
// all the same and reports a timeout through the error word.  Counters come in
// two sets used by alternating launches; each launch clears the set the next one
// uses (the launch before it, which used that set, has completed).
constexpr uint32_t kMaxSpins = 1u << 16;  // ~50 ms of polling (the default limit of every wait)
// Each logical counter is spread over kLanes slots, one 64-byte line apart, so
// hundreds of workgroups neither add to nor poll one address.
constexpr int kLanes = 16;
constexpr int kSlotStride = 16;  // words
enum : int {
    kRouterDone = 0, kSelectReady, kSharedGuDone, kRoutedDone, kCounters
};
constexpr int kSetWords = kCounters * kLanes * kSlotStride;
constexpr int kDownRows = 2;                   // down + combine: output rows per wave
constexpr int kFusedRows = kWaves * kDownRows;  // output rows per down workgroup

struct FusedArgs {
    DecodeArgs a;
    uint32_t* sync;     // [2][kSetWords] counters, then the error word
    uint64_t* approx;   // [E] fast (reassociated) logits for the speculative selection, tagged
    uint64_t* spec;     // [K] speculative experts by rank, tagged
    uint64_t* spec_xcd; // [8][16] the same per XCD, one 128-byte L2 line each (kDecodeXcdSpecWord)
    uint32_t* mask;     // ranks whose speculative expert differs from the exact one
    int32_t parity;
    uint32_t seq;       // this launch's tag of the approx / spec words (nonzero, changes every launch)
    int32_t perturb;    // testing: make the speculation disagree with every rank
    uint32_t max_spins; // polls before a wait gives up and sets the error word
    int32_t n_router, n_shared_gu, n_routed;
};

__device__ inline uint32_t* counter_slot(uint32_t* set, int counter, int slot) {
    return set + (counter * kLanes + slot) * kSlotStride;
}

// Counters that at most the 16 router workgroups (or one workgroup) add to live
// in one slot: a waiter then reads a single line, and the previous value of an
// add tells the last arriver.  The per-item counters of the streaming roles
// spread over kLanes slots.
__device__ constexpr bool single_slot(int counter) {
    return counter == kRouterDone || counter == kSelectReady;
}

// Counts this workgroup done once every wave's stores are acknowledged.  The
// add returns nothing, so the workgroup ends (and frees its slot for a later
// workgroup) without waiting for it.
//
// Ordering of the hand-offs.  Every value one workgroup hands to another is
// written with an agent-scope atomic store (global_store ... sc1: written
// through the XCD's L2 to memory) and read with an agent-scope atomic load
// (global_load ... sc1: read from memory, never from an L2 copy), so no cache
// can hold a stale copy of it.  The writer's vmcnt(0) waits until memory has
// acknowledged each of the wave's stores and the barrier waits for every wave,
// so the counter's add is issued after all of the workgroup's data is in
// memory; the reader issues its data loads only after its poll has returned
// the count (the loop exit depends on the loaded value) and behind a barrier
// the compiler does not move memory operations across.  An agent-scope
// release / acquire pair states the same order in the memory model but adds
// an L2 write-back (buffer_wbl2) per signal and an L2 invalidate (buffer_inv)
// per wait, for data that never sits in L2: measured, it doubles the launch
// (35 to 70 us per V2-Lite block).
__device__ inline void signal_done(uint32_t* set, int counter) {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __syncthreads();
    if (threadIdx.x == 0) {
        const int slot = single_slot(counter) ? 0 : static_cast<int>(blockIdx.x % kLanes);
        (void)__hip_atomic_fetch_add(counter_slot(set, counter, slot), 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Waits until the counter's slots sum to `target` (wave 0 polls all slots at
// once, backing off while far from done), then releases the workgroup.
__device__ inline void wait_count(uint32_t* set, int counter, uint32_t target, uint32_t* error, uint32_t limit) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        uint32_t spins = 0;
        const int polled = single_slot(counter) ? 1 : kLanes;
        for (;;) {
            uint32_t v = lane < polled ? __hip_atomic_load(counter_slot(set, counter, lane), __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT)
                                       : 0u;
            // every lane of the wave must see the total, or the lanes would leave
            // the loop at different times
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                v += __shfl_xor(v, o);
            }
            if (v >= target) {
                break;
            }
            if (++spins > limit) {
                if (lane == 0) {
                    __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                break;
            }
            if (single_slot(counter)) {
                __builtin_amdgcn_s_sleep(4);  // one line polled: check often
            } else if (target - v > target / 4) {
                __builtin_amdgcn_s_sleep(32);
            } else {
                __builtin_amdgcn_s_sleep(4);
            }
        }
    }
    __syncthreads();
}

// (publish / wait_tagged, the tagged hand-off words: handoff.h)

// Speculative experts of every rank into LDS (all waves read them afterwards).
// A wait that gave up returns a word of an earlier launch (or zero); the index
// is clamped all the same, so no weight address can leave the layer.
__device__ inline void load_spec(const FusedArgs& f, uint32_t* error, int* spec_lds) {
    if (threadIdx.x < 64) {
        const uint32_t v = wait_tagged(f.spec, f.a.top_k, f.seq, error, f.max_spins);
        if (static_cast<int>(threadIdx.x) < f.a.top_k) {
            spec_lds[threadIdx.x] = static_cast<int>(v < static_cast<uint32_t>(f.a.experts) ? v : 0u);
        }
    }
    __syncthreads();
}

// The XCD this workgroup runs on (HW_REG_XCC_ID, bits 0..3; eight per device).
__device__ inline int xcd_id() { return static_cast<int>(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 7); }

// Per-XCD copies of the speculative experts.  The selectors (the first routed
// workgroups, kXcdSelectors of them) each store the tagged words into the slot
// of their own XCD with `sc0` stores: written through the CU's L1 into the
// XCD's L2 and kept there.  The routed workgroups poll their XCD's slot with
// `sc0` loads, which miss L1 and read that L2 (the scope the memory model
// uses for a workgroup split over the CUs of one XCD), so the hand-off costs an
// L2 round trip instead of a device-scope one through memory.  They poll the
// device-scope words as well, alternately: a slot no selector of this launch
// reached (workgroups placed on XCDs otherwise than round robin) never
// delays them past the device-scope hand-off.  Slots hold words of earlier
// launches, which their tags reject.
constexpr int kXcdSelectors = 8;
constexpr int kXcdSlotBytes = kDecodeXcdSlotWords * 4;
constexpr int kAuxSc0 = 1;  // buffer instruction cache policy: sc0

__device__ inline void publish_xcd(const FusedArgs& f, int rank, uint32_t bits) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(f.spec_xcd, 0, 8 * kXcdSlotBytes, 0x00020000);
    const uint64_t word = (static_cast<uint64_t>(f.seq) << 32) | bits;
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 v = {static_cast<unsigned>(word), static_cast<unsigned>(word >> 32)};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, xcd_id() * kXcdSlotBytes + rank * 8, 0, kAuxSc0);
}

__device__ inline void load_spec_xcd(const FusedArgs& f, uint32_t* error, int* spec_lds) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const int n = f.a.top_k;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(f.spec_xcd, 0, 8 * kXcdSlotBytes, 0x00020000);
        const int off = xcd_id() * kXcdSlotBytes + (lane < n ? lane : 0) * 8;
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        uint32_t spins = 0, v = 0;
        for (;;) {
            const u32x2 l = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kAuxSc0);
            if (__ballot(lane < n && l.y != f.seq) == 0) {
                v = l.x;
                break;
            }
            // the device-scope words every 8th poll (a poll of them waits a
            // round trip through memory; the slot's, one through L2)
            if ((spins & 7) == 7) {
                const uint64_t g = lane < n ? __hip_atomic_load(f.spec + lane, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT)
                                            : static_cast<uint64_t>(f.seq) << 32;
                if (__ballot(static_cast<uint32_t>(g >> 32) != f.seq) == 0) {
                    v = static_cast<uint32_t>(g);
                    break;
                }
                v = static_cast<uint32_t>(g);
            }
            if (++spins > f.max_spins) {
                if (lane == 0) {
                    __hip_atomic_store(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (lane < n) {
            spec_lds[lane] = static_cast<int>(v < static_cast<uint32_t>(f.a.experts) ? v : 0u);
        }
    }
    __syncthreads();
}

// Router workgroups, once their products are in LDS: publish the approximate
// logits of the slice.
__device__ __forceinline__ void speculate(const FusedArgs& f, int e0, const float4* lds) {
    const DecodeArgs& a = f.a;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // Approximate logit of expert e0 + wave: the same products, tree order.
    const int quads = a.hidden / 4;
    float t = 0.0f;
    for (int q = lane; q < quads; q += 64) {
        const float4 p = lds[q * kRouterExperts + wave];
        t += (p.x + p.y) + (p.z + p.w);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        t += __shfl_xor(t, o);
    }
    if (lane == 0) {
        publish(f.approx + e0 + wave, f.seq, float_bits(a.bias != nullptr ? t + a.bias[e0 + wave] : t));
    }
}

// Speculative rank of expert `lane` from the approximate logits.  A softmax
// score is non-decreasing in its logit, so ordering by logit (higher first,
// then lower index) is MoeRouter::select's order unless two different logits
// round to the same score; the exact selection corrects any such rank.  This
// skips the exponentials, the sequential total and the weights, which the
// speculation does not use.  Group-limited routing takes the full selection.
__device__ inline int speculative_rank(float logit, bool valid, int lane, const SelectPolicy& p, float* sh) {
    if (p.group_limited && p.n_group > 1 && p.experts % p.n_group == 0) {
        int rank;
        float weight;
        select_token_lds(logit, valid, lane, p, sh, rank, weight);
        return rank;
    }
    // logit bits mapped so unsigned order is float order
    const uint32_t bits = float_bits(logit);
    const uint32_t ordered = (bits & 0x80000000u) != 0 ? ~bits : (bits | 0x80000000u);
    const uint64_t key = valid ? ((static_cast<uint64_t>(ordered) << 8) | static_cast<uint64_t>(255 - lane)) : 0ull;
    uint64_t* keys = reinterpret_cast<uint64_t*>(sh + 64);
    keys[lane] = key;
    __builtin_amdgcn_wave_barrier();
    const ulonglong2* keys2 = reinterpret_cast<const ulonglong2*>(keys);
    int beaten = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const ulonglong2 k2 = keys2[i];
        beaten += k2.x > key ? 1 : 0;
        beaten += k2.y > key ? 1 : 0;
    }
    return beaten;
}

// Recomputes, in LDS, the activation row of rank r for expert e (rare path:
// the speculative selection put another expert at this rank).  Plain loops,
// few registers: it runs once in tens of thousands of tokens.
__device__ void repair_act_row(const DecodeArgs& a, int e, float* act_row) {
    const uint16_t* gu = a.routed + static_cast<int64_t>(e) * a.routed_stride;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    for (int j = threadIdx.x; j < a.inter_p; j += blockDim.x) {
        const int64_t gate_row = static_cast<int64_t>(j / kGroupRows) * (2 * kGroupRows) + (j % kGroupRows);
        const uint16_t* g = gu + gate_row * a.hidden_p;
        const uint16_t* u = g + static_cast<int64_t>(kGroupRows) * a.hidden_p;
        float gate = 0.0f, up = 0.0f;
        for (int c = 0; c < a.hidden; c += 8) {
            const uint4 wg = *reinterpret_cast<const uint4*>(g + c);
            const uint4 wu = *reinterpret_cast<const uint4*>(u + c);
            // with the norm fused, the normalised copy (x itself may be overwritten)
            const float4 x0 = a.norm != nullptr ? load_coherent4(a.xnorm + c) : x4[c / 4];
            const float4 x1 = a.norm != nullptr ? load_coherent4(a.xnorm + c + 4) : x4[c / 4 + 1];
            fma8(gate, wg, x0, x1);
            fma8(up, wu, x0, x1);
        }
        act_row[j] = silu_mul_ref(gate, up);
    }
}

// Down projection and combine for output row h (one per wave) in the single
// launch.  The down rows are fetched for the speculative experts as soon as
// those are known; the exact selection then decides: ranks it confirms use the
// rows in registers and the activations the routed workgroups wrote, the others
// (rare) are recomputed here from the exact expert's weights.
template <int KM, int DI, int SI, int RW>
__device__ __forceinline__ void down_fused(const FusedArgs& f, uint32_t* sync, uint32_t* error, int h0,
                                           float* acts) {
    constexpr int KP = KM <= 2 ? 2 : (KM <= 4 ? 4 : 8);  // reduction width per row (power of two)
    __shared__ float fixed_dot[kWaves][RW][kMaxTopK];
    const DecodeArgs& a = f.a;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    static_assert(RW == 2, "a wave's two rows are one 8-byte pair of the shared partial sums");
    static_assert(kFusedRows == 8, "a down workgroup's rows are one 8-row block of the shared partial sums");
    const int K = a.top_k;
    const int W = a.inter_p;
    const int n_sitems = a.shared_inter_p / kItemRows;
    // Rows h0 .. h0 + RW - 1 of the output (h0 even).
    __shared__ int spec_lds[kMaxTopK];
    load_spec(f, error, spec_lds);
    LM_TRACE(1);
    const int64_t down_base = static_cast<int64_t>(2) * W * a.hidden_p;
    uint4 w[RW][KM][DI];
    {
        int ex[KM];
#pragma unroll
        for (int r = 0; r < KM; ++r) {
            ex[r] = spec_lds[r < K ? r : 0];
        }
#pragma unroll
        for (int j = 0; j < RW; ++j) {
#pragma unroll
            for (int it = 0; it < DI; ++it) {
                const int c = it * 512 + lane * 8;
                const int cc = c < W ? c : W - 8;
#pragma unroll
                for (int r = 0; r < KM; ++r) {
                    w[j][r][it] = load_stream16(a.routed + static_cast<int64_t>(ex[r]) * a.routed_stride + down_base +
                                                static_cast<int64_t>(h0 + j) * W + cc);
                }
            }
        }
    }
    // The shared expert's projection of the two rows: its items' partial sums.
    // The workgroup's eight rows of every item are one contiguous run
    // (n_sitems x 32 B), staged once into LDS behind the activations' region
    // with direct-to-LDS loads past the XCD's L2 (the items ran on other
    // XCDs), whole 256-byte pieces (the buffer has the slack); then each lane
    // adds items lane, lane + 64, ... in order, and the wave's butterfly.
    wait_count(sync, kSharedGuDone, f.n_shared_gu, error, f.max_spins);
    float shared_h[RW] = {0.0f, 0.0f};
    {
        float* staged = acts + K * W;
        const float* src = a.shared_part + static_cast<int64_t>(h0 >> 3) * n_sitems * 8;
        const int nf = (n_sitems * 8 + 63) / 64 * 64;
        for (int c = wave; c < nf / 256; c += kWaves) {
            __builtin_amdgcn_global_load_lds((decode_global_void*)(src + c * 256 + 4 * lane),
                                             (decode_lds_void*)(staged + c * 256), 16, 0, 16);
        }
        for (int g = wave; g < (nf % 256) / 64; g += kWaves) {
            const int o = nf / 256 * 256 + g * 64;
            __builtin_amdgcn_global_load_lds((decode_global_void*)(src + o + lane), (decode_lds_void*)(staged + o), 4, 0,
                                             16);
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        lds_barrier();
        constexpr int kPer = (SI * 512 / kItemRows + 63) / 64;  // items per lane at most
#pragma unroll
        for (int u = 0; u < kPer; ++u) {
            const int i = lane + 64 * u;
            if (i < n_sitems) {
                const float2 v = *reinterpret_cast<const float2*>(staged + i * 8 + (h0 & 7));
                shared_h[0] = shared_h[0] + v.x;
                shared_h[1] = shared_h[1] + v.y;
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
#pragma unroll
            for (int j = 0; j < RW; ++j) {
                shared_h[j] += __shfl_xor(shared_h[j], o);
            }
        }
    }
    wait_count(sync, kRoutedDone, f.n_routed, error, f.max_spins);
    wait_count(sync, kSelectReady, 1, error, f.max_spins);
    LM_TRACE(2);
    const uint32_t m = __hip_atomic_load(f.mask, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float wk[KM];
#pragma unroll
    for (int r = 0; r < KM; ++r) {
        wk[r] = load_coherent(a.wts + (r < K ? r : 0));
    }
    // The routed ranks' activations, once per workgroup, into LDS in one round
    // trip: direct-to-LDS loads that read memory past the XCD's L2 (sc1, like
    // load_coherent), 1 KB per wave instruction, then 256 B ones for the rest
    // (W is a multiple of 64).  A rank the speculation got wrong is staged too
    // and overwritten by the repair below.
    {
        const int n = K * W;
        const int full = n / 256;
        for (int c = wave; c < full; c += kWaves) {
            __builtin_amdgcn_global_load_lds((decode_global_void*)(a.act + c * 256 + 4 * lane),
                                             (decode_lds_void*)(acts + c * 256), 16, 0, 16);
        }
        for (int g = wave; g < (n - full * 256) / 64; g += kWaves) {
            const int o = full * 256 + g * 64;
            __builtin_amdgcn_global_load_lds((decode_global_void*)(a.act + o + lane), (decode_lds_void*)(acts + o), 4, 0,
                                             16);
        }
    }
    float residual[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        residual[j] = a.residual != nullptr ? a.residual[h0 + j] : 0.0f;
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the staged activations are in
    lds_barrier();
    // acc[j KP + r]: row j, rank r (ranks past K read valid data and are never
    // combined).
    float acc[RW * KP];
#pragma unroll
    for (int i = 0; i < RW * KP; ++i) {
        acc[i] = 0.0f;
    }
#pragma unroll
    for (int it = 0; it < DI; ++it) {
        const int c = it * 512 + lane * 8;
        if (c < W) {
#pragma unroll
            for (int r = 0; r < KM; ++r) {
                const int rr = r < K ? r : 0;
                const float4 x0 = *reinterpret_cast<const float4*>(acts + rr * W + c);
                const float4 x1 = *reinterpret_cast<const float4*>(acts + rr * W + c + 4);
#pragma unroll
                for (int j = 0; j < RW; ++j) {
                    fma8(acc[j * KP + r], w[j][r][it], x0, x1);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    const float sum = transpose_reduce<RW * KP>(acc, lane);
    if (m != 0) {
        // Ranks the speculation got wrong: their activation rows and down dot
        // products from the exact experts (the sums above are discarded).
        for (int r = 0; r < K; ++r) {
            if (((m >> r) & 1u) == 0) {
                continue;
            }
            // clamped: after a wait that gave up, idx may hold anything
            const int e_read = load_coherent(a.idx + r);
            const int e = e_read >= 0 && e_read < a.experts ? e_read : 0;
            lds_barrier();
            repair_act_row(a, e, acts + r * W);
            lds_barrier();
            for (int j = 0; j < RW; ++j) {
                const uint16_t* down = a.routed + static_cast<int64_t>(e) * a.routed_stride + down_base +
                                       static_cast<int64_t>(h0 + j) * W;
                float d = 0.0f;
                for (int c = lane * 8; c < W; c += 512) {
                    const float4 x0 = *reinterpret_cast<const float4*>(acts + r * W + c);
                    const float4 x1 = *reinterpret_cast<const float4*>(acts + r * W + c + 4);
                    fma8(d, *reinterpret_cast<const uint4*>(down + c), x0, x1);
                }
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) {
                    d += __shfl_xor(d, o);
                }
                if (lane == 0) {
                    fixed_dot[wave][j][r] = d;
                }
            }
        }
        lds_barrier();
    }
    constexpr int L = log2c<RW * KP>();
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        float out = 0.0f;
#pragma unroll
        for (int r = 0; r < KM; ++r) {
            if (r < K) {
                const float d =
                    ((m >> r) & 1u) != 0 ? fixed_dot[wave][j][r] : lane_value(sum, (j * KP + r) << (6 - L));
                out = __builtin_fmaf(wk[r], d, out);
            }
        }
        if (a.has_shared) {
            out = out + shared_h[j];
        }
        if (a.residual != nullptr) {
            out = residual[j] + out;
        }
        if (lane == 0) {
            a.y[h0 + j] = out;
        }
    }
}

// The routed experts start from a speculative selection: each router workgroup
// first sums its products in a fast tree order (approximate logits), the last
// one to finish selects from those, and the routed gate/up rows of the
// speculated experts stream while the exact, strictly sequential logits are
// still being added.  The exact selection decides everything that is output;
// ranks where the speculation picked another expert are recomputed by the down
// workgroups (almost never: only a near-tie between two experts' scores can
// order them differently).
template <int GI, int SI, int KM, int DI>
__global__ __launch_bounds__(kThreads) void decode_fused_kernel(FusedArgs f) {
    extern __shared__ float4 lds[];  // router products or the down stage's activations
    __shared__ __align__(16) float sel[kSelectScratch];
    __shared__ int expert_of_rank[kMaxTopK];
    __shared__ uint32_t arrived;
    const DecodeArgs& a = f.a;
    uint32_t* sync = f.sync + f.parity * kSetWords;
    uint32_t* error = f.sync + kDecodeErrorWord;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int b = blockIdx.x;
    LM_TRACE(0);
    if (b == static_cast<int>(gridDim.x) - 1) {
        // the last workgroup, off the critical path, clears the next launch's counters
        uint32_t* next = f.sync + (1 - f.parity) * kSetWords;
        for (int i = threadIdx.x; i < kCounters * kLanes; i += kThreads) {
            __hip_atomic_store(next + i * kSlotStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (b < f.n_router) {
        const int e0 = b * kRouterExperts;
        router_slice<GI>(a, e0, lds, [&] { speculate(f, e0, lds); },
                         [&](int e, float t) { publish(f.approx + e0 + e, f.seq, float_bits(t)); });
        // The last router workgroup to finish its exact logits selects for the output.
        __builtin_amdgcn_s_waitcnt(0x0F70);
        __syncthreads();
        if (threadIdx.x == 0) {
            arrived = __hip_atomic_fetch_add(counter_slot(sync, kRouterDone, 0), 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (arrived != static_cast<uint32_t>(f.n_router - 1)) {
            return;
        }
        if (threadIdx.x < 64) {
            const bool valid = lane < a.experts;
            const float logit = valid ? load_coherent(a.logits + lane) : 0.0f;
            int rank;
            float weight;
            select_token_lds(logit, valid, lane, a.policy, sel, rank, weight);
            const bool chosen = valid && rank < a.top_k;
            if (chosen) {
                store_coherent(a.idx + rank, lane);
                store_coherent(a.wts + rank, weight);
            }
            const int spec_of_rank = __shfl(static_cast<int>(wait_tagged(f.spec, a.top_k, f.seq, error, f.max_spins)),
                                            chosen ? rank : 0);
            const uint64_t wrong = __ballot(chosen && spec_of_rank != lane);
            // bit r of the mask: rank r must be recomputed
            uint32_t m = 0;
            if (chosen && ((wrong >> lane) & 1u) != 0) {
                m = 1u << rank;
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                m |= static_cast<uint32_t>(__shfl_xor(static_cast<int>(m), o));
            }
            if (lane == 0) {
                __hip_atomic_store(f.mask, m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        signal_done(sync, kSelectReady);
        LM_TRACE(3);
        return;
    }
    b -= f.n_router;
    if (b < f.n_shared_gu) {
        // Streams from the start: nothing here depends on the router (held
        // until the router's loads were in, the launch measured 0.2 us longer).
        shared_item<GI>(a, b, reinterpret_cast<float*>(lds), reinterpret_cast<float*>(lds) + a.hidden);
        signal_done(sync, kSharedGuDone);
        LM_TRACE(3);
        return;
    }
    b -= f.n_shared_gu;
    const int chunks = a.inter_p / kItemRows;
    if (b < kXcdSelectors && b < f.n_routed) {
        // The first routed workgroups select speculatively from the approximate
        // logits and publish the experts into their XCD's slot; the first also
        // into the device-scope words the down workgroups read.
        if (threadIdx.x < 64) {
            const bool valid = lane < a.experts;
            const float logit = bits_float(wait_tagged(f.approx, a.experts, f.seq, error, f.max_spins));
            const int rank = speculative_rank(valid ? logit : 0.0f, valid, lane, a.policy, sel);
            if (valid && rank < a.top_k) {
                const int slot = f.perturb ? (rank + 1) % a.top_k : rank;
                publish_xcd(f, slot, static_cast<uint32_t>(lane));
                if (b == 0) {
                    publish(f.spec + slot, f.seq, static_cast<uint32_t>(lane));
                }
            }
        }
    }
    b -= f.n_routed;
    if (b < 0) {
        // Routed gate/up of the speculative experts.
        const int item = b + f.n_routed;
        const int r = item / chunks;
        load_spec_xcd(f, error, expert_of_rank);
        LM_TRACE(1);
        gateup_item<GI>(a.routed + static_cast<int64_t>(expert_of_rank[r]) * a.routed_stride, a,
                        item - r * chunks, a.act + static_cast<int64_t>(r) * a.inter_p,
                        reinterpret_cast<float*>(lds));
        signal_done(sync, kRoutedDone);
        LM_TRACE(3);
        return;
    }
    down_fused<KM, DI, SI, kDownRows>(f, sync, error, b * kFusedRows + wave * kDownRows,
                                      reinterpret_cast<float*>(lds));
    LM_TRACE(3);
}

int iters_of(int width) { return (width + 511) / 512; }

int km_of(int top_k) { return top_k <= 2 ? 2 : (top_k <= 4 ? 4 : (top_k <= 6 ? 6 : 8)); }

// (GI, SI, KM, DI) instantiations: DeepSeek-V2-Lite (hidden 2048, routed 1408,
// shared 2816, k 6) and LiteMind's tiny test model (hidden 32, routed 16,
// shared 16, k 2).  Other shapes take the general path.
int fused_shape(int hidden, int top_k, int inter_p, int shared_inter_p) {
    const int gi = iters_of(hidden), si = iters_of(shared_inter_p), km = km_of(top_k), di = iters_of(inter_p);
    if (gi == 4 && si == 6 && km == 6 && di == 3) {
        return 0;
    }
    if (gi == 1 && si == 1 && km == 2 && di == 1) {
        return 1;
    }
    return -1;
}

}  // namespace

bool decode_supported(int hidden, int experts, int top_k, int inter_p, int shared_inter_p) {
    return experts % kRouterExperts == 0 && experts >= 2 && experts <= kMaxExperts && top_k >= 1 &&
           top_k <= 8 && top_k <= experts && shared_inter_p > 0 && shared_inter_p % 4 == 0 &&
           hidden % kFusedRows == 0 && hidden * 16 <= 65536 &&
           (top_k * inter_p + (shared_inter_p / kItemRows * 8 + 63) / 64 * 64) * 4 <= 65536 &&
           inter_p % 64 == 0 && shared_inter_p % kItemRows == 0 &&  // activations staged in 256-byte pieces
           fused_shape(hidden, top_k, inter_p, shared_inter_p) >= 0;
}

int64_t decode_shared_part_floats(int hidden, int shared_inter_p) {
    // + 64: the down workgroups stage whole 256-byte pieces of their run
    return static_cast<int64_t>(hidden) * (shared_inter_p / kItemRows) + 64;
}

hipError_t launch_decode(const DecodeLaunch& d, hipStream_t s) {
    const int hidden = d.hidden, top_k = d.policy.top_k, inter_p = d.inter_p;
    if (d.sync == nullptr || d.shared_gu == nullptr || d.shared_t == nullptr || d.shared_part == nullptr ||
        (d.norm != nullptr && d.xnorm == nullptr) ||
        !decode_supported(hidden, d.policy.experts, top_k, inter_p, d.shared_inter_p)) {
        return hipErrorInvalidValue;
    }
    FusedArgs f{};
    DecodeArgs& a = f.a;
    a.x = d.x;
    a.norm = d.norm;
    a.eps = d.eps;
    a.xnorm = d.xnorm;
    a.wq = d.wq;
    a.bias = d.bias;
    a.logits = d.logits;
    a.logits_out = d.logits_out;
    a.idx = d.idx;
    a.wts = d.wts;
    a.routed = d.routed;
    a.routed_stride = d.routed_stride;
    a.shared_gu = d.shared_gu;
    a.shared_down = d.shared_down;
    a.shared_t = d.shared_t;
    a.shared_part = d.shared_part;
    a.act = d.act;
    a.y = d.y;
    a.residual = d.residual;
    a.hidden = hidden;
    a.hidden_p = d.hidden_p;
    a.experts = d.policy.experts;
    a.top_k = top_k;
    a.inter_p = inter_p;
    a.shared_inter_p = d.shared_inter_p;
    a.has_shared = 1;
    a.policy = d.policy;
    static_assert(2 * kSetWords == kDecodeCounterWords, "decode scratch layout");
    f.sync = d.sync;
    f.approx = reinterpret_cast<uint64_t*>(d.sync + kDecodeApproxWord);
    f.spec = reinterpret_cast<uint64_t*>(d.sync + kDecodeSpecWord);
    f.spec_xcd = reinterpret_cast<uint64_t*>(d.sync + kDecodeXcdSpecWord);
    f.seq = d.seq;
    f.mask = d.sync + kDecodeMaskWord;
    f.parity = d.parity & 1;
    f.perturb = d.perturb;
    f.max_spins = d.max_spins != 0 ? d.max_spins : kMaxSpins;
    f.n_router = a.experts / kRouterExperts;
    f.n_shared_gu = a.shared_inter_p / kItemRows;
    f.n_routed = top_k * (inter_p / kItemRows);
    const int n_down = hidden / kFusedRows;
    const dim3 grid(static_cast<unsigned>(f.n_router + f.n_shared_gu + f.n_routed + n_down));
    const size_t router_lds = sizeof(float) * static_cast<size_t>(hidden) * kRouterExperts;
    const size_t down_lds =
        sizeof(float) * (static_cast<size_t>(top_k) * inter_p + (d.shared_inter_p / kItemRows * 8 + 63) / 64 * 64);
    const size_t shared_lds = sizeof(float) * static_cast<size_t>(hidden) * (1 + kWaves);
    const size_t lds = std::max(router_lds, std::max(down_lds, shared_lds));
    if (fused_shape(hidden, top_k, inter_p, d.shared_inter_p) == 0) {
        hipLaunchKernelGGL((decode_fused_kernel<4, 6, 6, 3>), grid, dim3(kThreads), lds, s, f);
    } else {
        hipLaunchKernelGGL((decode_fused_kernel<1, 1, 2, 1>), grid, dim3(kThreads), lds, s, f);
    }
    return hipGetLastError();
}

}  // namespace lm

#ifdef LM_DECODE_TRACE
extern "C" int lm_decode_trace_read(unsigned long long* host, int n) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(lm_decode_trace), sizeof(unsigned long long) * n) == hipSuccess ? 0 : -1;
}
#endif
