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
#include "lm_select.h"
#include "router_chunks.h"

namespace lm {
namespace {

constexpr int kWaves = 4;

// Selects for token t and writes its experts and weights in rank order.
__device__ void route_token(float logit, bool valid, int lane, int64_t t, const RouterArgs& a) {
    const SelectPolicy p{a.experts, a.top_k, a.normalize, a.group_limited, a.n_group, a.topk_group, a.scale};
    int rank;
    float weight;
    select_token(logit, valid, lane, p, rank, weight);
    const int K = a.top_k < a.experts ? a.top_k : a.experts;
    if (valid && rank < K) {
        a.idx[t * a.top_k + rank] = lane;
        a.wts[t * a.top_k + rank] = weight;
    }
}

// Rows of the transposed gate staged per step: [kChunk/4][64 experts] float4,
// component j of entry (q, e) holding gate row i0 + 4q + j of expert e.
constexpr int kChunk = 64;

// One workgroup routes kWaves * TPW tokens.  All threads stage the next chunk
// of the transposed gate and of the tokens' activations into LDS while the
// waves run the current chunk; each wave reads a whole chunk into registers
// before its dependent add chain starts, so the chain runs at VALU issue rate.
template <int TPW>
__global__ __launch_bounds__(kWaves * 64) void router_kernel(RouterArgs a, const float* __restrict__ x,
                                                             const float* __restrict__ wt) {
    __shared__ float4 wstage[2][kChunk / 4][64];
    __shared__ float4 xstage[2][kWaves * TPW][kChunk / 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tb0 = static_cast<int64_t>(blockIdx.x) * kWaves * TPW;  // first token of the block
    const int64_t t0 = tb0 + static_cast<int64_t>(wave) * TPW;
    const bool active = t0 < a.tokens;  // wave-uniform; idle waves still help stage
    const int E = a.experts;
    const int H = a.hidden;
    const bool valid = lane < E;

    float acc[TPW];
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        acc[k] = 0.0f;
    }
    if (a.do_matvec) {
        // Per chunk each thread stages 16 gate values (row r = idx / 64, expert
        // e = idx % 64) and TPW activation values (token idx / 64, row idx % 64).
        constexpr int kPerW = kChunk * 64 / (kWaves * 64);
        float wpre[kPerW];
        float xpre[TPW];
        auto fetch = [&](int i0) {
#pragma unroll
            for (int j = 0; j < kPerW; ++j) {
                const int idx = threadIdx.x + j * kWaves * 64;
                const int r = idx >> 6, e = idx & 63;
                wpre[j] = (i0 + r < H && e < E) ? wt[static_cast<int64_t>(i0 + r) * E + e] : 0.0f;
            }
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                const int idx = threadIdx.x + k * kWaves * 64;
                const int tk = idx >> 6, r = idx & 63;
                const int64_t t = tb0 + tk;
                xpre[k] = (t < a.tokens && i0 + r < H) ? x[t * H + i0 + r] : 0.0f;
            }
        };
        auto store = [&](int buf) {
#pragma unroll
            for (int j = 0; j < kPerW; ++j) {
                const int idx = threadIdx.x + j * kWaves * 64;
                const int r = idx >> 6, e = idx & 63;
                reinterpret_cast<float*>(&wstage[buf][r >> 2][e])[r & 3] = wpre[j];
            }
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                const int idx = threadIdx.x + k * kWaves * 64;
                const int tk = idx >> 6, r = idx & 63;
                reinterpret_cast<float*>(&xstage[buf][tk][r >> 2])[r & 3] = xpre[k];
            }
        };
        const int nchunks = (H + kChunk - 1) / kChunk;
        fetch(0);
        store(0);
        lds_barrier();
        for (int c = 0; c < nchunks; ++c) {
            const int i0 = c * kChunk;
            const int b = c & 1;
            if (c + 1 < nchunks) {
                fetch(i0 + kChunk);
            }
            if (active) {
                if (H - i0 >= kChunk) {
                    float4 w[kChunk / 4];
#pragma unroll
                    for (int q = 0; q < kChunk / 4; ++q) {
                        w[q] = wstage[b][q][lane];
                    }
#pragma unroll
                    for (int k = 0; k < TPW; ++k) {
                        float4 xv[kChunk / 4];
#pragma unroll
                        for (int q = 0; q < kChunk / 4; ++q) {
                            xv[q] = xstage[b][wave * TPW + k][q];
                        }
#pragma unroll
                        for (int q = 0; q < kChunk / 4; ++q) {
                            float p = w[q].x * xv[q].x;
                            acc[k] = acc[k] + p;
                            p = w[q].y * xv[q].y;
                            acc[k] = acc[k] + p;
                            p = w[q].z * xv[q].z;
                            acc[k] = acc[k] + p;
                            p = w[q].w * xv[q].w;
                            acc[k] = acc[k] + p;
                        }
                    }
                } else {
                    const int quads = (H - i0) / 4;  // H % 4 == 0
                    for (int q = 0; q < quads; ++q) {
                        const float4 w = wstage[b][q][lane];
#pragma unroll
                        for (int k = 0; k < TPW; ++k) {
                            const float4 xv = xstage[b][wave * TPW + k][q];
                            float p = w.x * xv.x;
                            acc[k] = acc[k] + p;
                            p = w.y * xv.y;
                            acc[k] = acc[k] + p;
                            p = w.z * xv.z;
                            acc[k] = acc[k] + p;
                            p = w.w * xv.w;
                            acc[k] = acc[k] + p;
                        }
                    }
                }
            }
            if (c + 1 < nchunks) {
                store((c + 1) & 1);
            }
            lds_barrier();
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

        // fp16 copy of the activations for the MFMA path (panel layout),
        // zero-padded to hidden_p.
        if (a.x16 != nullptr) {
            const float* xt = x + t * H;
            for (int c = lane; c < a.hidden_p; c += 64) {
                a.x16[panel_index(t, c, a.tokens)] = c < H ? static_cast<_Float16>(xt[c]) : static_cast<_Float16>(0.0f);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// More than 64 experts (up to 64 EPL): lane owns experts lane + 64 j.  One
// workgroup of 4 waves routes 4 TPW tokens; per chunk of R = 64 / EPL gate rows
// all threads stage the rows of the transposed gate ([H, E]) and the tokens'
// activations in LDS (16 KB of gate per chunk whatever EPL), and every lane
// runs EPL x TPW of LiteMind's sequential chains (src/Gemm.cpp:183-189).  With
// do_matvec = 0, x holds the logits [T, E] (select only).
// ---------------------------------------------------------------------------
template <int EPL, int TPW>
__global__ __launch_bounds__(kWaves * 64) void router_multi_kernel(RouterArgs a, const float* __restrict__ x,
                                                                   const float* __restrict__ wt) {
    constexpr int R = 64 / EPL;
    constexpr int NE = 64 * EPL;
    constexpr int XT = kWaves * TPW;  // tokens of the workgroup
    __shared__ float wstage[2][R][NE];
    __shared__ float xstage[2][XT][R];
    __shared__ __align__(16) float sel[kWaves][select_multi_words(EPL)];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tb0 = static_cast<int64_t>(blockIdx.x) * XT;
    const int64_t t0 = tb0 + static_cast<int64_t>(wave) * TPW;
    const bool active = t0 < a.tokens;
    const int E = a.experts;
    const int H = a.hidden;

    float acc[TPW][EPL];
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            acc[k][j] = 0.0f;
        }
    }
    if (a.do_matvec) {
        constexpr int kPerW = R * NE / (kWaves * 64);  // 16 gate values per thread and chunk
        float wpre[kPerW];
        float xpre[(XT * R + kWaves * 64 - 1) / (kWaves * 64)];
        auto fetch = [&](int i0) {
#pragma unroll
            for (int q = 0; q < kPerW; ++q) {
                const int idx = threadIdx.x + q * kWaves * 64;
                const int r = idx / NE, e = idx % NE;
                wpre[q] = (i0 + r < H && e < E) ? wt[static_cast<int64_t>(i0 + r) * E + e] : 0.0f;
            }
#pragma unroll
            for (int q = 0; q * kWaves * 64 < XT * R; ++q) {
                const int idx = threadIdx.x + q * kWaves * 64;
                const int tk = idx / R, r = idx % R;
                const int64_t t = tb0 + tk;
                xpre[q] = (idx < XT * R && t < a.tokens && i0 + r < H) ? x[t * H + i0 + r] : 0.0f;
            }
        };
        auto store = [&](int buf) {
#pragma unroll
            for (int q = 0; q < kPerW; ++q) {
                const int idx = threadIdx.x + q * kWaves * 64;
                wstage[buf][idx / NE][idx % NE] = wpre[q];
            }
#pragma unroll
            for (int q = 0; q * kWaves * 64 < XT * R; ++q) {
                const int idx = threadIdx.x + q * kWaves * 64;
                if (idx < XT * R) {
                    xstage[buf][idx / R][idx % R] = xpre[q];
                }
            }
        };
        const int nchunks = (H + R - 1) / R;
        fetch(0);
        store(0);
        lds_barrier();
        for (int c = 0; c < nchunks; ++c) {
            const int i0 = c * R;
            const int b = c & 1;
            if (c + 1 < nchunks) {
                fetch(i0 + R);
            }
            if (active) {
                const int rows = H - i0 < R ? H - i0 : R;
                for (int r = 0; r < rows; ++r) {
                    float w[EPL];
#pragma unroll
                    for (int j = 0; j < EPL; ++j) {
                        w[j] = wstage[b][r][lane + 64 * j];
                    }
#pragma unroll
                    for (int k = 0; k < TPW; ++k) {
                        const float xv = xstage[b][wave * TPW + k][r];
#pragma unroll
                        for (int j = 0; j < EPL; ++j) {
                            const float p = w[j] * xv;
                            acc[k][j] = acc[k][j] + p;
                        }
                    }
                }
            }
            if (c + 1 < nchunks) {
                store((c + 1) & 1);
            }
            lds_barrier();
        }
    } else if (active) {
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const int64_t t = t0 + k;
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const int e = lane + 64 * j;
                acc[k][j] = (e < E && t < a.tokens) ? x[t * E + e] : 0.0f;
            }
        }
    }
    if (!active) {
        return;
    }
    const SelectPolicy p{a.experts, a.top_k, a.normalize, a.group_limited, a.n_group, a.topk_group, a.scale};
    const int K = a.top_k < E ? a.top_k : E;
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        const int64_t t = t0 + k;
        if (t >= a.tokens) {
            break;
        }
        float logit[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            logit[j] = acc[k][j];
            if (a.bias != nullptr && e < E) {
                logit[j] = logit[j] + a.bias[e];
            }
            if (a.logits != nullptr && e < E) {
                a.logits[t * E + e] = logit[j];
            }
        }
        int rank[EPL];
        float weight[EPL];
        select_token_multi<EPL>(logit, lane, p, sel[wave], rank, weight);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            if (rank[j] < K) {
                a.idx[t * a.top_k + rank[j]] = lane + 64 * j;
                a.wts[t * a.top_k + rank[j]] = weight[j];
            }
        }
        if (a.x16 != nullptr) {
            const float* xt = x + t * H;
            for (int c = lane; c < a.hidden_p; c += 64) {
                a.x16[panel_index(t, c, a.tokens)] = c < H ? static_cast<_Float16>(xt[c]) : static_cast<_Float16>(0.0f);
            }
        }
    }
}

template <int EPL>
void launch_multi(const RouterArgs& a, hipStream_t s) {
    const int tpw = a.do_matvec && a.tokens >= 1024 ? 2 : 1;
    const int64_t per_block = static_cast<int64_t>(kWaves) * tpw;
    const dim3 grid(static_cast<unsigned>((a.tokens + per_block - 1) / per_block));
    if (tpw == 2) {
        hipLaunchKernelGGL((router_multi_kernel<EPL, 2>), grid, dim3(kWaves * 64), 0, s, a, a.x, a.wt);
    } else {
        hipLaunchKernelGGL((router_multi_kernel<EPL, 1>), grid, dim3(kWaves * 64), 0, s, a, a.x, a.wt);
    }
}

// Few-token router (T <= 4) for shapes the wide kernel below does not take
// (E != 64, or H not a multiple of 256): one workgroup of 16 waves.  The tokens' activations
// are staged in LDS once; all 1024 threads stream the transposed gate with a
// kDepth-chunk register prefetch (one float4 per thread per chunk) into a
// double-buffered LDS ring, and wave t runs token t's sequential chains.
constexpr int kDecodeThreads = 1024;
constexpr int kDecodeMaxTokens = 4;
constexpr int kDepth = 4;

__global__ __launch_bounds__(kDecodeThreads) void router_decode_kernel(RouterArgs a, const float* __restrict__ x,
                                                                        const float* __restrict__ wt) {
    __shared__ float4 wstage[2][kChunk / 4][64];                    // 32 KB
    extern __shared__ float4 xs[];                                   // [T][H / 4]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int E = a.experts;
    const int H = a.hidden;
    const int T = static_cast<int>(a.tokens);
    const bool valid = lane < E;
    const bool chain = wave < T;

    for (int i = tid; i < T * (H / 4); i += kDecodeThreads) {
        const int t = i / (H / 4), q = i - t * (H / 4);
        xs[i] = *reinterpret_cast<const float4*>(x + static_cast<int64_t>(t) * H + 4 * q);
    }
    // Thread tid owns float4 slot tid of a chunk: gate row r = tid / 16 of the
    // chunk, experts 4 * (tid % 16) .. +3 (all of them below E or zero).
    const int r = tid >> 4;
    const int e4 = (tid & 15) * 4;
    // Straight-line fetch with a clamped address and no masking: rows past H
    // are never read by the chains (a partial chunk reads only its valid
    // quads) and lanes past E are discarded.  Branches or selects here would
    // make the compiler wait for every outstanding prefetch.
    const int e_load = e4 < E ? e4 : 0;  // E % 4 == 0 for this kernel
    auto fetch = [&](int c) -> float4 {
        const int i = c * kChunk + r;
        const int i_load = i < H ? i : H - 1;
        return *reinterpret_cast<const float4*>(wt + static_cast<int64_t>(i_load) * E + e_load);
    };
    auto store = [&](int buf, float4 v) {
        float* base = reinterpret_cast<float*>(&wstage[buf][r >> 2][0]);
        base[(e4 + 0) * 4 + (r & 3)] = v.x;
        base[(e4 + 1) * 4 + (r & 3)] = v.y;
        base[(e4 + 2) * 4 + (r & 3)] = v.z;
        base[(e4 + 3) * 4 + (r & 3)] = v.w;
    };
    // H % (kChunk * kDepth) == 0 for this kernel: the pipeline below has no
    // conditionals, so the compiler can wait for exactly the oldest prefetch.
    // Fetches past the last chunk are clamped to row H - 1 and never used.
    const int nchunks = H / kChunk;
    float4 pre[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
        pre[d] = fetch(d);
    }
    float acc = 0.0f;
    for (int c0 = 0; c0 < nchunks; c0 += kDepth) {
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const int c = c0 + d;
            store(c & 1, pre[d]);
            pre[d] = fetch(c + kDepth);
            lds_barrier();
            if (chain) {
                const int i0 = c * kChunk;
                constexpr int kHalf = kChunk / 8;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    float4 w[kHalf], xv[kHalf];
#pragma unroll
                    for (int q = 0; q < kHalf; ++q) {
                        w[q] = wstage[c & 1][h * kHalf + q][lane];
                        xv[q] = xs[wave * (H / 4) + i0 / 4 + h * kHalf + q];
                    }
#pragma unroll
                    for (int q = 0; q < kHalf; ++q) {
                        float p = w[q].x * xv[q].x;
                        acc = acc + p;
                        p = w[q].y * xv[q].y;
                        acc = acc + p;
                        p = w[q].z * xv[q].z;
                        acc = acc + p;
                        p = w[q].w * xv[q].w;
                        acc = acc + p;
                    }
                }
            }
        }
    }
    if (!chain) {
        return;
    }
    const int64_t t = wave;
    float logit = acc;
    if (a.bias != nullptr && valid) {
        logit = logit + a.bias[lane];
    }
    if (a.logits != nullptr && valid) {
        a.logits[t * E + lane] = logit;
    }
    route_token(logit, valid, lane, t, a);
    if (a.x16 != nullptr) {
        for (int c = lane; c < a.hidden_p; c += 64) {
            a.x16[panel_index(t, c, a.tokens)] = c < H ? static_cast<_Float16>(x[t * H + c]) : static_cast<_Float16>(0.0f);
        }
    }
}

// ---------------------------------------------------------------------------
// Batched router for many tokens (E == 64, H % 256 == 0).  A workgroup of 4
// waves routes 4 * TPW tokens; lane e owns expert e and runs TPW sequential
// chains.  Each chunk of 64 gate rows (16 KB of the [H/4][E][4] layout: lane e
// reads four consecutive rows of its expert with one ds_read_b128) and the
// tokens' activations for those rows go from global memory straight into a
// 4-deep LDS ring with global_load_lds, so three chunks are always in flight
// behind the one the chains consume; every step waits for a constant count and
// always issues (a chunk past the end reloads the last one into a buffer that
// is never read), so the waits stay exact.  The selection uses the LDS variant.
// The fp16 copy of the activations (MFMA path) is a separate, fully parallel
// conversion launch rather than a loop of dependent loads at the end of each
// wave.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(1))) const void router_global_void;
typedef __attribute__((address_space(3))) void router_lds_void;

constexpr int kWideRows = 64;
constexpr int kWideDepth = 4;
constexpr int kWideWaves = 4;
constexpr int64_t kWideTpw2Tokens = 2048;  // above this, two tokens per wave
constexpr int64_t kWideTpw4Tokens = 4096;  // above this, four
#ifndef LM_WIDE8_TOKENS
#define LM_WIDE8_TOKENS 2048
#endif
constexpr int64_t kWide8Tokens = LM_WIDE8_TOKENS;  // from this on, 8-wave workgroups (one token per wave)
// ... and with two tokens per wave from this on (224 or more workgroups of 16
// tokens; with fewer, more CUs stay busy with 4-wave workgroups)
constexpr int64_t kWide8Tpw2Tokens = 3584;

// NW waves per workgroup.  With 4 waves a lane's token values come in one
// 16-byte load (1 KB per wave, TPW * 256 B used); with 8 (one token per wave,
// one workgroup per CU) in one 4-byte load per lane (256 B per wave), which
// leaves LDS for an 8-deep ring.
template <int TPW, int NW>
struct WideShape {
    static constexpr int kWBytes = kWideRows * 64 * 4;                    // 16 KB of gate rows
    static constexpr int kXWave = NW == 4 ? 1024 : 256 * TPW;             // activation bytes per wave
    static constexpr int kXBytes = NW * kXWave;
    static constexpr int kStage = kWBytes + kXBytes;
    static constexpr int kWLoads = kWBytes / 1024 / NW;                   // gate wave instructions per chunk
    static constexpr int kLoads = kWLoads + (NW == 4 ? 1 : TPW);          // wave instructions per chunk
};

__device__ inline void route_token_lds(float logit, bool valid, int lane, int64_t t, const RouterArgs& a,
                                       float* sh) {
    const SelectPolicy p{a.experts, a.top_k, a.normalize, a.group_limited, a.n_group, a.topk_group, a.scale};
    int rank;
    float weight;
    select_token_lds(logit, valid, lane, p, sh, rank, weight);
    const int K = a.top_k < a.experts ? a.top_k : a.experts;
    if (valid && rank < K) {
        a.idx[t * a.top_k + rank] = lane;
        a.wts[t * a.top_k + rank] = weight;
    }
}

template <int TPW, int NW, int DEPTH>
__global__ __launch_bounds__(NW * 64) void router_wide_kernel(RouterArgs a, const float* __restrict__ x,
                                                               const float* __restrict__ wq4) {
    using S = WideShape<TPW, NW>;
    static_assert(DEPTH == 4 || DEPTH == 8, "ring depth");
    static_assert(DEPTH * S::kStage <= 160 * 1024, "LDS");
    constexpr int kS4 = DEPTH > 4 ? S::kStage : 16;
    __shared__ __attribute__((aligned(1024))) char r0[S::kStage], r1[S::kStage], r2[S::kStage], r3[S::kStage];
    __shared__ __attribute__((aligned(1024))) char r4[kS4], r5[kS4], r6[kS4], r7[kS4];
    char* const ring[8] = {r0, r1, r2, r3, r4, r5, r6, r7};
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int H = a.hidden;
    const int64_t tb0 = static_cast<int64_t>(blockIdx.x) * NW * TPW;
    const int nchunks = H / kWideRows;

    // With 4 waves, this lane's activation row segment: token wave * TPW +
    // (lane / 16) % TPW of the workgroup (clamped to the last token), rows
    // 4 (lane % 16) .. +3.  Every lane loads (lanes past TPW * 16 repeat a token
    // into the unused part of the wave's slot), so the issue has no divergent
    // branch.  With 8 waves, row lane of each of the wave's tokens.
    int64_t xt = tb0 + wave * TPW + (NW == 4 ? ((lane >> 4) % TPW) : 0);
    xt = xt < a.tokens ? xt : a.tokens - 1;
    const float* xsrc = x + xt * H + (NW == 4 ? 4 * (lane & 15) : lane);
    const float* wsrc = wq4 + static_cast<int64_t>(wave) * 256 + 4 * lane;
    auto issue = [&](int c, char* buf) {
        c = c < nchunks ? c : nchunks - 1;
        const int64_t i0 = static_cast<int64_t>(c) * kWideRows;
#pragma unroll
        for (int j = 0; j < S::kWLoads; ++j) {
            const int n = j * NW + wave;  // 1 KB block n of the chunk's gate rows
            __builtin_amdgcn_global_load_lds((router_global_void*)(wsrc + i0 * 64 + j * NW * 256),
                                             (router_lds_void*)(buf + n * 1024), 16, 0, 0);
        }
        if constexpr (NW == 4) {
            __builtin_amdgcn_global_load_lds((router_global_void*)(xsrc + i0),
                                             (router_lds_void*)(buf + S::kWBytes + wave * S::kXWave), 16, 0, 0);
        } else {
            // token k of the wave: tokens past the batch end repeat the last one
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                const int64_t step = tb0 + wave * TPW + k < a.tokens ? static_cast<int64_t>(k) * H : 0;
                __builtin_amdgcn_global_load_lds((router_global_void*)(xsrc + step + i0),
                                                 (router_lds_void*)(buf + S::kWBytes + wave * S::kXWave + k * 256), 4,
                                                 0, 0);
            }
        }
    };

    float acc[TPW];
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        acc[k] = 0.0f;
    }
    // Rows 4q .. 4q + 3 of a chunk: the four gate values of this lane's expert
    // (one 16-byte read) and the activations of its tokens (broadcast reads).
    // The reads of a batch of kBatch rows are issued together and the
    // additions then run from registers: while LDS-DMA writes are pending the
    // compiler can only wait for all LDS reads at once, so one wait per batch
    // is the cheapest arrangement.
    constexpr int kBatch = 32;
    auto compute = [&](const char* buf) {
        const float4* wb = reinterpret_cast<const float4*>(buf);
        const float* xb = reinterpret_cast<const float*>(buf + S::kWBytes + wave * S::kXWave);
#pragma unroll
        for (int r0 = 0; r0 < kWideRows; r0 += kBatch) {
            float4 w[kBatch / 4];
            float4 xv[kBatch / 4][TPW];
#pragma unroll
            for (int q = 0; q < kBatch / 4; ++q) {
                w[q] = wb[(r0 / 4 + q) * 64 + lane];
#pragma unroll
                for (int k = 0; k < TPW; ++k) {
                    xv[q][k] = *reinterpret_cast<const float4*>(xb + k * kWideRows + r0 + 4 * q);
                }
            }
#pragma unroll
            for (int q = 0; q < kBatch / 4; ++q) {
                // Products first (independent), then the TPW chains' additions
                // interleaved so consecutive adds never depend on each other.
                float p[4][TPW];
#pragma unroll
                for (int k = 0; k < TPW; ++k) {
                    p[0][k] = w[q].x * xv[q][k].x;
                    p[1][k] = w[q].y * xv[q][k].y;
                    p[2][k] = w[q].z * xv[q][k].z;
                    p[3][k] = w[q].w * xv[q][k].w;
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
#pragma unroll
                    for (int k = 0; k < TPW; ++k) {
                        acc[k] = acc[k] + p[j][k];
                    }
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // Chunk c lives in ring[c % depth]; before consuming it, wait until at
    // most the depth - 2 chunks issued after it are in flight (and this wave's
    // LDS reads of the previous chunk are done); the barrier then also frees the
    // buffer consumed in the previous step for chunk c + depth - 1.
    constexpr int kVm = (DEPTH - 2) * S::kLoads;
    static_assert(kVm < 64, "vmcnt immediate");
    constexpr int kWait = 0x0070 | (kVm & 15) | ((kVm >> 4) << 14);  // vmcnt(kVm) lgkmcnt(0)
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d) {
        issue(d, ring[d]);
    }
    for (int c0 = 0; c0 < nchunks; c0 += DEPTH) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) {
            __builtin_amdgcn_s_waitcnt(kWait);
            __builtin_amdgcn_s_barrier();
            issue(c0 + j + DEPTH - 1, ring[(j + DEPTH - 1) % DEPTH]);
            compute(ring[j]);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);  // drain the clamped reloads
    __builtin_amdgcn_s_barrier();

    // With a.x16, the fp16 panel copy of the wave's tokens for the MFMA path
    // (to_f16_rows_kernel's conversion), from rows the loop above has just
    // brought into L2.  After the loop: a global store inside it makes the
    // compiler keep far more registers live (256 VGPRs + 256 AGPRs against 100).
    if (a.x16 != nullptr) {
        typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int k = 0; k < TPW; ++k) {
            const int64_t t = tb0 + wave * TPW + k;
            if (t < a.tokens) {
                for (int c = 4 * lane; c < H; c += 256) {
                    const float4 v = *reinterpret_cast<const float4*>(x + t * H + c);
                    *reinterpret_cast<half4_t*>(a.x16 + panel_index(t, c, a.tokens)) =
                        half4_t{static_cast<_Float16>(v.x), static_cast<_Float16>(v.y), static_cast<_Float16>(v.z),
                                static_cast<_Float16>(v.w)};
                }
            }
        }
    }

    float* sh = reinterpret_cast<float*>(r0) + wave * kSelectScratch;
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        const int64_t t = tb0 + wave * TPW + k;
        if (t >= a.tokens) {
            break;
        }
        float logit = acc[k];
        if (a.bias != nullptr) {
            logit = logit + a.bias[lane];
        }
        if (a.logits != nullptr) {
            a.logits[t * 64 + lane] = logit;
        }
        route_token_lds(logit, true, lane, t, a, sh);
        __builtin_amdgcn_wave_barrier();
    }
}

// ---------------------------------------------------------------------------
// More than 64 experts at batches above kRouterSplitTokens: router_wide_kernel's
// direct-to-LDS ring, DEPTH slots deep (8 fill the CU's LDS where the grid has
// one workgroup per CU, 4 let two share a CU), with lane l owning experts
// l + 64 j (j < EPL).  The slots are separate LDS variables, each indexed by a
// constant in the unrolled loop: the compiler can then tell the slot a read
// uses from the ones the loads in flight fill, and waits only for its own
// chunk (with one array it waits for every load in flight before each chunk's
// first read).  A
// chunk is R = 32 / 16 / 8 gate rows (EPL 2 / 4 / 8): their block of the
// [H/4][E][4] layout, R / 4 x E x 16 bytes <= 16 KB and contiguous, loaded as
// 16 wave instructions of 1 KB (those past the block reload its start into
// LDS that is never read, so every chunk issues the same loads and the waits
// stay exact), and the tokens' R activations each.  Each lane runs EPL x TPW
// of LiteMind's sequential chains (src/Gemm.cpp:183-189), rows in order; then
// select_token_multi per token.  H % R == 0.
// ---------------------------------------------------------------------------
template <int EPL>
constexpr int wide_multi_rows() { return EPL <= 2 ? 32 : (EPL <= 4 ? 16 : 8); }
constexpr int kWideMultiGate = 16 * 1024;  // gate bytes per ring slot

// NW waves per workgroup.  With 8 (one token per wave, one workgroup per CU, an
// 8-deep ring) each lane loads one 4-byte token value per chunk (256 B per
// wave), so each gate chunk serves 8 tokens in 144 KB of LDS.
template <int NW>
constexpr int wide_multi_slot() {
    return kWideMultiGate + NW * (NW == 4 ? 1024 : 256);
}

template <int EPL, int TPW, int DEPTH, int NW = kWideWaves>
__global__ __launch_bounds__(NW * 64) void router_wide_multi_kernel(RouterArgs a, const float* __restrict__ x,
                                                                     const float* __restrict__ wq4) {
    static_assert(DEPTH == 4 || DEPTH == 8, "ring depth");
    static_assert(NW == 4 || (NW == 8 && TPW == 1 && DEPTH == 8), "8 waves: one token per wave, 8-deep ring");
    constexpr int kWideMultiSlot = wide_multi_slot<NW>();
    constexpr int kXWave = NW == 4 ? 1024 : 256;
    constexpr int R = wide_multi_rows<EPL>();
    constexpr int kGateLoads = kWideMultiGate / 1024 / NW;  // 4 (2) per wave
    constexpr int kLoads = kGateLoads + 1;
    constexpr int kHi = DEPTH > 4 ? kWideMultiSlot : 16;
    __shared__ __attribute__((aligned(1024))) char r0[kWideMultiSlot], r1[kWideMultiSlot], r2[kWideMultiSlot],
        r3[kWideMultiSlot];
    __shared__ __attribute__((aligned(1024))) char r4[kHi], r5[kHi], r6[kHi], r7[kHi];
    char* const ring[8] = {r0, r1, r2, r3, r4, r5, r6, r7};
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int H = a.hidden;
    const int E = a.experts;
    const int64_t tb0 = static_cast<int64_t>(blockIdx.x) * NW * TPW;
    const int nchunks = H / R;
    const int chunk_bytes = R / 4 * E * 16;

    // activations, 4 waves: lane -> token (lane / (R / 4)) % TPW of the wave,
    // rows 4 (lane % (R / 4)) .. + 3; 8 waves: the wave's token, row lane of
    // the chunk (lanes past R read rows of later chunks, clamped to the last row)
    int64_t xt = tb0 + wave * TPW + (NW == 4 ? ((lane / (R / 4)) % TPW) : 0);
    xt = xt < a.tokens ? xt : a.tokens - 1;
    const float* xsrc = x + xt * H + (NW == 4 ? 4 * (lane % (R / 4)) : 0);
    const char* wbase = reinterpret_cast<const char*>(wq4);
    auto issue = [&](int c, char* buf) {
        c = c < nchunks ? c : nchunks - 1;
        const char* chunk = wbase + static_cast<int64_t>(c) * chunk_bytes;
#pragma unroll
        for (int j = 0; j < kGateLoads; ++j) {
            const int n = j * NW + wave;  // 1 KB block n of the slot
            const int off = n * 1024 + lane * 16;
            __builtin_amdgcn_global_load_lds((router_global_void*)(chunk + (off < chunk_bytes ? off : 0)),
                                             (router_lds_void*)(buf + n * 1024), 16, 0, 0);
        }
        if constexpr (NW == 4) {
            __builtin_amdgcn_global_load_lds((router_global_void*)(xsrc + static_cast<int64_t>(c) * R),
                                             (router_lds_void*)(buf + kWideMultiGate + wave * kXWave), 16, 0, 0);
        } else {
            const int row = c * R + lane;
            __builtin_amdgcn_global_load_lds((router_global_void*)(xsrc + (row < H ? row : H - 1)),
                                             (router_lds_void*)(buf + kWideMultiGate + wave * kXWave), 4, 0, 0);
        }
    };

    float acc[TPW][EPL];
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            acc[k][j] = 0.0f;
        }
    }
    int ecl[EPL];  // this lane's experts, clamped for the reads (results past E are discarded)
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        ecl[j] = lane + 64 * j < E ? lane + 64 * j : E - 1;
    }
    auto compute = [&](const char* buf) {
        const float4* wb = reinterpret_cast<const float4*>(buf);
        const float* xb = reinterpret_cast<const float*>(buf + kWideMultiGate + wave * kXWave);
#pragma unroll
        for (int q = 0; q < R / 4; ++q) {
            float4 w[EPL];
            float4 xv[TPW];
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                w[j] = wb[q * E + ecl[j]];
            }
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
                xv[k] = *reinterpret_cast<const float4*>(xb + k * R + 4 * q);
            }
#pragma unroll
            for (int k = 0; k < TPW; ++k) {
#pragma unroll
                for (int j = 0; j < EPL; ++j) {
                    const float p0 = w[j].x * xv[k].x, p1 = w[j].y * xv[k].y;
                    const float p2 = w[j].z * xv[k].z, p3 = w[j].w * xv[k].w;
                    acc[k][j] = acc[k][j] + p0;
                    acc[k][j] = acc[k][j] + p1;
                    acc[k][j] = acc[k][j] + p2;
                    acc[k][j] = acc[k][j] + p3;
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // chunk c in ring[c % DEPTH] with DEPTH - 2 chunks in flight behind it:
    // wait for c, barrier (every wave is past c - 1), refill c - 1's slot with
    // c + DEPTH - 1, compute c
    constexpr int kVm = (DEPTH - 2) * kLoads;
    static_assert(kVm < 64, "vmcnt field");
    constexpr int kWait = 0x0070 | (kVm & 15) | ((kVm >> 4) << 14);  // vmcnt(kVm) lgkmcnt(0)
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d) {
        issue(d, ring[d]);
    }
    for (int c0 = 0; c0 < nchunks; c0 += DEPTH) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) {
            __builtin_amdgcn_s_waitcnt(kWait);
            __builtin_amdgcn_s_barrier();
            issue(c0 + j + DEPTH - 1, ring[(j + DEPTH - 1) % DEPTH]);
            if (c0 + j < nchunks) {
                compute(ring[j]);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070);  // drain the clamped reloads
    __builtin_amdgcn_s_barrier();

    const SelectPolicy p{a.experts, a.top_k, a.normalize, a.group_limited, a.n_group, a.topk_group, a.scale};
    const int K = a.top_k < E ? a.top_k : E;
    // one slot per wave (selected, not indexed: ring[] is only ever indexed by constants)
    char* slot = wave == 0 ? r0 : (wave == 1 ? r1 : (wave == 2 ? r2 : r3));
    if constexpr (NW == 8) {
        slot = wave < 4 ? slot : (wave == 4 ? r4 : (wave == 5 ? r5 : (wave == 6 ? r6 : r7)));
    }
    float* sh = reinterpret_cast<float*>(slot);
    static_assert(select_multi_words(EPL) * 4 <= kWideMultiSlot, "selection scratch in the ring");
#pragma unroll
    for (int k = 0; k < TPW; ++k) {
        const int64_t t = tb0 + wave * TPW + k;
        if (t >= a.tokens) {
            break;
        }
        float logit[EPL];
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const int e = lane + 64 * j;
            logit[j] = acc[k][j];
            if (a.bias != nullptr && e < E) {
                logit[j] = logit[j] + a.bias[e];
            }
            if (a.logits != nullptr && e < E) {
                a.logits[t * E + e] = logit[j];
            }
        }
        int rank[EPL];
        float weight[EPL];
        select_token_multi<EPL>(logit, lane, p, sh, rank, weight);
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            if (rank[j] < K) {
                a.idx[t * a.top_k + rank[j]] = lane + 64 * j;
                a.wts[t * a.top_k + rank[j]] = weight[j];
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

#ifndef LM_RING_TPW2_TOKENS
#define LM_RING_TPW2_TOKENS 2048
#endif
#ifndef LM_RING_TPW4_TOKENS
#define LM_RING_TPW4_TOKENS 4096
#endif
// Tokens per wave: each gate value read from LDS feeds TPW chains.
constexpr int64_t kRingTpw2Tokens = LM_RING_TPW2_TOKENS;
constexpr int64_t kRingTpw4Tokens = LM_RING_TPW4_TOKENS;
#ifndef LM_RING_DEEP_BLOCKS
#define LM_RING_DEEP_BLOCKS 256
#endif
// Grids of up to this many workgroups (one per CU) take the 8-deep ring.
constexpr int64_t kRingDeepBlocks = LM_RING_DEEP_BLOCKS;
#ifndef LM_RING_WIDE8
#define LM_RING_WIDE8 1
#endif
// Above that, one token per wave in workgroups of 8 waves (0: of 4, 4-deep).
constexpr bool kRingWide8 = LM_RING_WIDE8 != 0;
#ifndef LM_SMALL_SPLIT_TOKENS
#define LM_SMALL_SPLIT_TOKENS 64
#endif
// Up to 64 experts: batches of 2 .. kSmallSplitTokens tokens take the logits
// over E / 8 workgroups per token (router_chunked_kernel).
constexpr int64_t kSmallSplitTokens = LM_SMALL_SPLIT_TOKENS;
static_assert(kSmallSplitTokens <= kRouterSplitTokens, "the logits scratch holds kRouterSplitTokens tokens");

template <int EPL, int TPW>
void launch_wide_multi_tpw(const RouterArgs& a, hipStream_t s) {
    constexpr int64_t per_block = static_cast<int64_t>(kWideWaves) * TPW;
    const int64_t blocks = (a.tokens + per_block - 1) / per_block;
    const dim3 grid(static_cast<unsigned>(blocks));
    if constexpr (TPW == 1) {  // more tokens per wave only above kRingTpw2Tokens: more than one workgroup per CU
        if (blocks <= kRingDeepBlocks) {
            hipLaunchKernelGGL((router_wide_multi_kernel<EPL, 1, 8>), grid, dim3(kWideWaves * 64), 0, s, a, a.x,
                               a.wq4);
            return;
        }
        // more workgroups than CUs: 8 waves per workgroup instead, so each gate
        // chunk serves 8 tokens (at most one workgroup per CU either way)
        if (kRingWide8) {
            const dim3 grid8(static_cast<unsigned>((a.tokens + 7) / 8));
            hipLaunchKernelGGL((router_wide_multi_kernel<EPL, 1, 8, 8>), grid8, dim3(8 * 64), 0, s, a, a.x, a.wq4);
            return;
        }
    }
    hipLaunchKernelGGL((router_wide_multi_kernel<EPL, TPW, 4>), grid, dim3(kWideWaves * 64), 0, s, a, a.x, a.wq4);
}

template <int EPL>
void launch_wide_multi(const RouterArgs& a, hipStream_t s) {
    if (a.tokens > kRingTpw4Tokens) {
        launch_wide_multi_tpw<EPL, 4>(a, s);
    } else if (a.tokens > kRingTpw2Tokens) {
        launch_wide_multi_tpw<EPL, 2>(a, s);
    } else {
        launch_wide_multi_tpw<EPL, 1>(a, s);
    }
}

// The ring router for 65..512 experts when the hidden size is a multiple of
// a chunk's rows; false (nothing launched) otherwise.
bool launch_ring_router(const RouterArgs& a, hipStream_t s) {
    const int epl = (a.experts + 63) / 64;
    const int rows = epl <= 2 ? wide_multi_rows<2>() : (epl <= 4 ? wide_multi_rows<4>() : wide_multi_rows<8>());
    if (epl < 2 || epl > 8 || a.hidden % rows != 0) {
        return false;
    }
    switch (epl) {
        case 2: launch_wide_multi<2>(a, s); break;
        case 3: launch_wide_multi<3>(a, s); break;
        case 4: launch_wide_multi<4>(a, s); break;
        case 5: launch_wide_multi<5>(a, s); break;
        case 6: launch_wide_multi<6>(a, s); break;
        case 7: launch_wide_multi<7>(a, s); break;
        default: launch_wide_multi<8>(a, s); break;
    }
    return true;
}

// ---------------------------------------------------------------------------
// Single-token router (T = 1): the experts are split over kSplit workgroups so
// each one loads its whole slice of the transposed gate (H x 8 fp32, 64 KB at
// H = 2048) at once, forms every product fl(w * x) in parallel into LDS, and
// leaves only the ordered additions to the chain lanes (one lane per expert,
// 4 rows per ds_read_b128).  A second single-workgroup launch performs the
// selection and the (trivial) permutation.
// ---------------------------------------------------------------------------
constexpr int kSplitExperts = 8;
constexpr int kSplitThreads = 256;

__device__ void permute_one_token(const RouterArgs& a) {
    // Canonical permutation for T = 1: the k selections, bucketed by expert.
    const int E = a.experts, K = a.top_k;
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += static_cast<int>(blockDim.x)) {
        int count = 0;
        for (int r = 0; r < K; ++r) {
            count += a.idx[r] == e ? 1 : 0;
        }
        a.rb.counts[e] = count;
        int offset = 0;
        for (int r = 0; r < K; ++r) {
            offset += a.idx[r] < e ? 1 : 0;
        }
        a.rb.offsets[e] = offset;
    }
    if (tid == 0) {
        a.rb.offsets[E] = K;
        a.rb.active[E] = K;
    }
    if (tid < K) {
        const int e = a.idx[tid];
        int pos = 0;
        for (int r = 0; r < K; ++r) {
            pos += a.idx[r] < e ? 1 : 0;  // experts are distinct within a token
        }
        a.rb.perm[pos] = tid;
        a.rb.slot_of[tid] = pos;
        a.rb.active[pos] = e;
    }
}

__global__ __launch_bounds__(kSplitThreads) void router_single_kernel(RouterArgs a, const float* __restrict__ x,
                                                                       const float* __restrict__ wt) {
    extern __shared__ float4 prod[];  // [H / 4][kSplitExperts] float4: 4 consecutive rows of one expert
    const int tid = threadIdx.x;
    const int H = a.hidden;
    const int E = a.experts;
    const int e0 = blockIdx.x * kSplitExperts;
    // float4 f covers row f / 2, experts e0 + 4 (f % 2) .. +3 of the slice.
    const int nf = H * (kSplitExperts / 4);
    for (int f0 = 0; f0 < nf; f0 += kSplitThreads * 8) {
        float4 w[8];
        float xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int f = f0 + j * kSplitThreads + tid;
            const int fl = f < nf ? f : nf - 1;
            const int i = fl >> 1;
            w[j] = *reinterpret_cast<const float4*>(wt + static_cast<int64_t>(i) * E + e0 + 4 * (fl & 1));
            xv[j] = x[i];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int f = f0 + j * kSplitThreads + tid;
            if (f < nf) {
                const int i = f >> 1;
                const int el = 4 * (f & 1);
                float* base = reinterpret_cast<float*>(&prod[(i >> 2) * kSplitExperts]);
                base[(el + 0) * 4 + (i & 3)] = w[j].x * xv[j];
                base[(el + 1) * 4 + (i & 3)] = w[j].y * xv[j];
                base[(el + 2) * 4 + (i & 3)] = w[j].z * xv[j];
                base[(el + 3) * 4 + (i & 3)] = w[j].w * xv[j];
            }
        }
    }
    lds_barrier();
    if (tid < kSplitExperts) {
        // LiteMind's dot: the rounded products added strictly left to right.
        float acc = 0.0f;
        const int quads = H / 4;
        int q = 0;
        for (; q + 8 <= quads; q += 8) {
            float4 p[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                p[u] = prod[(q + u) * kSplitExperts + tid];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                acc = acc + p[u].x;
                acc = acc + p[u].y;
                acc = acc + p[u].z;
                acc = acc + p[u].w;
            }
        }
        for (; q < quads; ++q) {
            const float4 p = prod[q * kSplitExperts + tid];
            acc = acc + p.x;
            acc = acc + p.y;
            acc = acc + p.z;
            acc = acc + p.w;
        }
        const int e = e0 + tid;
        if (a.bias != nullptr) {
            acc = acc + a.bias[e];
        }
        a.logits_scratch[e] = acc;
        if (a.logits != nullptr) {
            a.logits[e] = acc;
        }
    }
}

// Raw logits (bias not added) of experts [e0, e0 + 8) for token blockIdx.y
// (chunked_logit).  Grid (E / 8, T); hidden % 4 == 0, E % 8 == 0.
static_assert(kChunkExperts == kSplitExperts && kChunkThreads == kSplitThreads, "router chunk shape");
__global__ __launch_bounds__(kSplitThreads) void router_chunked_kernel(RouterArgs a, const float* __restrict__ x,
                                                                        const float* __restrict__ wt) {
    __shared__ float4 prod[kChunkFloat4s];
    const int e0 = blockIdx.x * kSplitExperts;
    const int64_t t = blockIdx.y;
    const float acc = chunked_logit(a.hidden, a.experts, x + t * a.hidden, wt, e0, prod);
    if (threadIdx.x < kSplitExperts) {
        a.logits_scratch[t * a.experts + e0 + threadIdx.x] = acc;
    }
}

// Token t's fp16 panel copy (x16 [tokens, hidden_p]) by one wave: lane l
// writes columns 8 q .. 8 q + 7 (one 16-byte run of a panel row) from two
// float4 loads, four chunks' loads in flight together (one element per lane
// per step waited a load round trip per step).  hidden % 8 == 0,
// hidden_p % 32 == 0.
__device__ inline void store_f16_row(const RouterArgs& a, int64_t t, int lane) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    const float* xt = a.x + t * a.hidden;
    const int full = a.hidden / 8;  // chunks of the row; the rest of hidden_p is padding
    for (int q0 = lane; q0 < full; q0 += 256) {
        float4 v[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u) {  // every load first (clamped addresses), then the stores
            const int q = q0 + 64 * u < full ? q0 + 64 * u : full - 1;
            v[u][0] = *reinterpret_cast<const float4*>(xt + 8 * q);
            v[u][1] = *reinterpret_cast<const float4*>(xt + 8 * q + 4);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int q = q0 + 64 * u;
            if (q < full) {
                const h8 h = {static_cast<_Float16>(v[u][0].x), static_cast<_Float16>(v[u][0].y),
                              static_cast<_Float16>(v[u][0].z), static_cast<_Float16>(v[u][0].w),
                              static_cast<_Float16>(v[u][1].x), static_cast<_Float16>(v[u][1].y),
                              static_cast<_Float16>(v[u][1].z), static_cast<_Float16>(v[u][1].w)};
                *reinterpret_cast<h8*>(a.x16 + panel_index(t, 8 * q, a.tokens)) = h;
            }
        }
    }
    const h8 zero = {};
    for (int q = full + lane; q < a.hidden_p / 8; q += 64) {
        *reinterpret_cast<h8*>(a.x16 + panel_index(t, 8 * q, a.tokens)) = zero;
    }
}

// One token over more than 64 experts, after router_chunked_kernel: the bias
// added to the raw logits, the selection (lane owns experts lane + 64 j), the
// token's permutation and its fp16 copy in one launch.
template <int EPL>
__global__ __launch_bounds__(64) void select_one_multi_kernel(RouterArgs a) {
    __shared__ __align__(16) float sel[select_multi_words(EPL)];
    __shared__ int ranked[kMaxTopK];  // the expert of each rank
    const int lane = threadIdx.x;
    const int E = a.experts;
    float logit[EPL];
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const int e = lane + 64 * j;
        logit[j] = e < E ? a.logits_scratch[e] : 0.0f;
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
            a.idx[rank[j]] = lane + 64 * j;
            a.wts[rank[j]] = weight[j];
            ranked[rank[j]] = lane + 64 * j;
        }
    }
    if (a.rb.counts != nullptr) {
        // permute_one_token's permutation from the ranks in LDS (the experts of
        // one token are distinct): counts 0 / 1, offsets and positions count
        // the selected experts below
        __syncthreads();
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
    }
    if (a.x16 != nullptr) {
        store_f16_row(a, 0, lane);
    }
}

// Up to 64 experts, after router_chunked_kernel: one wave per token adds the
// bias to its raw logits, selects (route_token) and writes the token's fp16
// panel copy.
__global__ __launch_bounds__(256) void select_tokens_kernel(RouterArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (t >= a.tokens) {
        return;
    }
    const bool valid = lane < a.experts;
    float logit = valid ? a.logits_scratch[t * a.experts + lane] : 0.0f;
    if (valid && a.bias != nullptr) {
        logit = logit + a.bias[lane];
    }
    if (valid && a.logits != nullptr) {
        a.logits[t * a.experts + lane] = logit;
    }
    route_token(logit, valid, lane, t, a);
    if (a.x16 != nullptr) {
        store_f16_row(a, t, lane);
    }
}

hipError_t launch_select_one_multi(const RouterArgs& a, hipStream_t s) {
    switch ((a.experts + 63) / 64) {
        case 2: hipLaunchKernelGGL(select_one_multi_kernel<2>, dim3(1), dim3(64), 0, s, a); break;
        case 3: hipLaunchKernelGGL(select_one_multi_kernel<3>, dim3(1), dim3(64), 0, s, a); break;
        case 4: hipLaunchKernelGGL(select_one_multi_kernel<4>, dim3(1), dim3(64), 0, s, a); break;
        case 5: hipLaunchKernelGGL(select_one_multi_kernel<5>, dim3(1), dim3(64), 0, s, a); break;
        case 6: hipLaunchKernelGGL(select_one_multi_kernel<6>, dim3(1), dim3(64), 0, s, a); break;
        case 7: hipLaunchKernelGGL(select_one_multi_kernel<7>, dim3(1), dim3(64), 0, s, a); break;
        default: hipLaunchKernelGGL(select_one_multi_kernel<8>, dim3(1), dim3(64), 0, s, a); break;
    }
    return hipGetLastError();
}

// Selection and permutation for one token from the logits of router_single_kernel
// (a separate launch: the kernel boundary orders the hand-off across XCDs).
__global__ __launch_bounds__(64) void select_single_kernel(RouterArgs a) {
    const int lane = threadIdx.x;
    const bool valid = lane < a.experts;
    const float logit = valid ? a.logits_scratch[lane] : 0.0f;
    route_token(logit, valid, lane, 0, a);
    if (a.rb.counts != nullptr) {
        __syncthreads();
        permute_one_token(a);
    }
    if (a.x16 != nullptr) {  // one token: the panel layout is the row itself
        for (int c = lane; c < a.hidden_p; c += 64) {
            a.x16[c] = c < a.hidden ? static_cast<_Float16>(a.x[c]) : static_cast<_Float16>(0.0f);
        }
    }
}

}  // namespace

hipError_t launch_router(const RouterArgs& a, hipStream_t s, bool* permuted) {
    if (permuted != nullptr) {
        *permuted = false;
    }
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.experts > kMaxExperts) {
        if (a.experts > kMaxExpertsWide) {
            return hipErrorInvalidValue;
        }
        RouterArgs k = a;
        // few tokens: the logits over E / 8 workgroups per token first, then
        // the per-token kernel selects from them (bias added there)
        const bool split = a.do_matvec && a.tokens <= kRouterSplitTokens && a.experts % kSplitExperts == 0 &&
                           a.hidden % 4 == 0 && a.logits_scratch != nullptr;
        if (split) {
            hipLaunchKernelGGL(router_chunked_kernel,
                               dim3(static_cast<unsigned>(a.experts / kSplitExperts), static_cast<unsigned>(a.tokens)),
                               dim3(kSplitThreads), 0, s, a, a.x, a.wt);
            hipError_t err = hipGetLastError();
            if (err != hipSuccess) {
                return err;
            }
            if (a.tokens == 1) {
                err = launch_select_one_multi(a, s);
                if (err == hipSuccess && permuted != nullptr) {
                    *permuted = a.rb.counts != nullptr;
                }
                return err;
            }
            k.do_matvec = 0;
            k.x = a.logits_scratch;
            k.x16 = nullptr;
        }
        // larger batches: the direct-to-LDS ring (the per-token kernel waits a
        // round trip per 16 gate rows: 694 us at T = 2048 on DeepSeek-V2's layer)
        const bool wide = !split && a.do_matvec && a.wq4 != nullptr && launch_ring_router(a, s);
        if (!wide) {
            if (a.experts <= 128) {
                launch_multi<2>(k, s);
            } else if (a.experts <= 256) {
                launch_multi<4>(k, s);
            } else {
                launch_multi<8>(k, s);
            }
        }
        hipError_t err = hipGetLastError();
        if (err == hipSuccess && (split || wide) && a.x16 != nullptr) {
            err = launch_to_f16_rows(a.x, a.x16, a.tokens, a.hidden, a.hidden_p, s);
        }
        return err;
    }
    const size_t split_lds = sizeof(float) * static_cast<size_t>(a.hidden) * kSplitExperts;
    if (a.do_matvec && a.tokens == 1 && a.experts % kSplitExperts == 0 && a.logits_scratch != nullptr &&
        split_lds <= 65536) {
        hipLaunchKernelGGL(router_single_kernel, dim3(a.experts / kSplitExperts), dim3(kSplitThreads), split_lds, s,
                           a, a.x, a.wt);
        hipLaunchKernelGGL(select_single_kernel, dim3(1), dim3(64), 0, s, a);
        if (permuted != nullptr) {
            *permuted = a.rb.counts != nullptr;
        }
        return hipGetLastError();
    }
    // 2 .. 64 tokens: each token's logits over E / 8 workgroups (one chain
    // per expert, ~3.5 ns per row), then one wave per token selects: the
    // wide kernel below runs few workgroups there, each through every chunk
    // of the gate in turn.  V2-Lite's router, T = 2 .. 32: 19.3-19.5 against
    // 23.2-24.1 us; T = 64 21.1 against 24.4; T = 128 even; T = 256 36.8
    // against 24.4.
    if (a.do_matvec && a.tokens >= 2 && a.tokens <= kSmallSplitTokens && a.experts % kSplitExperts == 0 &&
        a.hidden % 4 == 0 && a.logits_scratch != nullptr) {
        hipLaunchKernelGGL(router_chunked_kernel,
                           dim3(static_cast<unsigned>(a.experts / kSplitExperts), static_cast<unsigned>(a.tokens)),
                           dim3(kSplitThreads), 0, s, a, a.x, a.wt);
        hipLaunchKernelGGL(select_tokens_kernel, dim3(static_cast<unsigned>((a.tokens + 3) / 4)), dim3(256), 0, s, a);
        return hipGetLastError();
    }
    // Every batch the wide kernel's shape allows: even a few tokens keep its
    // 4-deep DMA ring fed (T = 2: 126 us per MoE block against 140 us with the
    // decode router; T = 16: 241 against 273 us with router_kernel).
    if (a.do_matvec && a.wq4 != nullptr && a.experts == 64 && a.hidden % (kWideRows * kWideDepth) == 0) {
        const int tpw = a.tokens > kWideTpw4Tokens ? 4 : (a.tokens > kWideTpw2Tokens ? 2 : 1);
        // From kWide8Tokens on, one or two tokens per wave in workgroups of 8
        // waves (one per CU) with an 8-deep ring: each gate chunk serves 8 or 16
        // tokens.
        const bool eight = ((tpw == 1 && a.tokens >= kWide8Tokens) || (tpw == 2 && a.tokens >= kWide8Tpw2Tokens)) &&
                           a.hidden % (kWideRows * 8) == 0;
        const int64_t per_block = static_cast<int64_t>(eight ? 8 : kWideWaves) * tpw;
        const dim3 grid(static_cast<unsigned>((a.tokens + per_block - 1) / per_block));
        // the kernel writes the fp16 copy itself when it covers every column
        RouterArgs k = a;
        const bool separate_x16 = a.x16 != nullptr && a.hidden_p != a.hidden;
        if (separate_x16) {
            k.x16 = nullptr;
        }
        if (eight && tpw == 2) {
            hipLaunchKernelGGL((router_wide_kernel<2, 8, 8>), grid, dim3(8 * 64), 0, s, k, a.x, a.wq4);
        } else if (eight) {
            hipLaunchKernelGGL((router_wide_kernel<1, 8, 8>), grid, dim3(8 * 64), 0, s, k, a.x, a.wq4);
        } else {
            switch (tpw) {
                case 4: hipLaunchKernelGGL((router_wide_kernel<4, 4, 4>), grid, dim3(kWideWaves * 64), 0, s, k, a.x, a.wq4); break;
                case 2: hipLaunchKernelGGL((router_wide_kernel<2, 4, 4>), grid, dim3(kWideWaves * 64), 0, s, k, a.x, a.wq4); break;
                default: hipLaunchKernelGGL((router_wide_kernel<1, 4, 4>), grid, dim3(kWideWaves * 64), 0, s, k, a.x, a.wq4); break;
            }
        }
        hipError_t err = hipGetLastError();
        if (err == hipSuccess && separate_x16) {
            err = launch_to_f16_rows(a.x, a.x16, a.tokens, a.hidden, a.hidden_p, s);
        }
        return err;
    }
    if (a.do_matvec && a.tokens <= kDecodeMaxTokens && a.experts % 4 == 0 && a.hidden % (kChunk * kDepth) == 0) {
        const size_t lds = sizeof(float) * static_cast<size_t>(a.tokens) * a.hidden;
        hipLaunchKernelGGL(router_decode_kernel, dim3(1), dim3(kDecodeThreads), lds, s, a, a.x, a.wt);
        return hipGetLastError();
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
