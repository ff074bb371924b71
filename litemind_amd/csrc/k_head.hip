// k_head.hip -- the LM head and the greedy choice of the next token.
//
// Reference: the end of DeepSeekRunner::Impl::forward (src/DeepSeekRunner.cpp:
// 296-300): rms_norm with the final norm weight, then gemm::matvec_bf16 over
// the [V, H] head; and Sampler::select_next's greedy branch
// (src/Sampler.cpp:117-126), std::max_element over the logits.
//
// The logits follow gemm::dot_bf16's association (src/Gemm.cpp:46-82) bit for
// bit, like gemv_plain_kernel: 32 sequential fused chains over the elements
// i = c (mod 32), chains 0..7 continuing over the 8-wide remainder, then
// (a0+a1)+(a2+a3) per lane, lanes j and j+4 added, (h0+h2)+(h1+h3) (no scalar
// tail: the width is a multiple of 8).  A chain's elements lie 64 bytes apart;
// a lane that owns 8 consecutive chains reads one 16-byte piece per step, so
// the loads stay wide and every chain stays in one lane, in order.  The head
// streams 420 MB at V = 102400, H = 2048: the kernel is bound by HBM.
#include "lm_internal.h"

#include <algorithm>

namespace lm {
namespace {

constexpr int kThreads = 256;                            // the head: 4 waves per block
constexpr int kRowsPerWave = 16;                         // 4 lanes per row
constexpr int kRows = kRowsPerWave * (kThreads / 64);    // head rows per block
constexpr int kUnroll = 8;                               // 16-byte loads in flight per lane
// Projections with few rows (attention: 576 to 4096) take one wave per block,
// so that a launch still spreads over the CUs.
constexpr int kSmallThreads = 64;

// Combines two candidates of the greedy choice: the larger value, the lower
// index between equal values (IEEE equality: -0 equals +0), NaN never chosen.
// Associative, so the order of the reduction does not matter.
__device__ inline HeadBest better(HeadBest a, HeadBest b) {
    if (!b.have) {
        return a;
    }
    if (!a.have || b.v > a.v || (b.v == a.v && b.i < a.i)) {
        return b;
    }
    return a;
}

__device__ inline HeadBest wave_better(HeadBest b) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const HeadBest other{__shfl_xor(b.v, o), __shfl_xor(b.i, o), __shfl_xor(b.have, o)};
        b = better(b, other);
    }
    return b;
}

// Four lanes per row: lane q of a row owns chains 8q .. 8q + 7, so one 16-byte
// load gives it the next element of each of its chains (elements 32 s + 8 q ..
// + 7), and a wave's load covers 64 contiguous bytes of 16 rows.  The tokens
// (tokens x in_dim floats, dynamic LDS) are staged once per block.  Lane 0 of a
// row also owns chains 0..7's continuation over the 8-wide remainder.  Then
// each block's best row per token goes to `partial` (when given).
template <int THREADS>
__global__ __launch_bounds__(THREADS) void head_logits_kernel(const uint16_t* __restrict__ w,
                                                              const float* __restrict__ x, float* logits,
                                                              HeadBest* partial, int64_t rows, int32_t in_dim,
                                                              int32_t tokens, float scale, int32_t accumulate) {
    constexpr int ROWS = kRowsPerWave * (THREADS / 64);
    extern __shared__ float4 xs4[];  // [tokens][in_dim / 4]
    __shared__ HeadBest wave_best[THREADS / 64];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int q = lane & 3;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS + (tid >> 2);
    const bool live = row < rows;
    const int n32 = in_dim / 32 * 32;
    const int n8 = n32 + (in_dim - n32) / 8 * 8;  // == in_dim: the launch requires in_dim % 8 == 0
    const int q4 = in_dim / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    for (int i = tid; i < tokens * q4; i += THREADS) {
        xs4[i] = x4[i];
    }
    __syncthreads();
    const uint16_t* wr = w + (live ? row : rows - 1) * in_dim;
    float acc[kHeadTokens][8];
#pragma unroll
    for (int t = 0; t < kHeadTokens; ++t) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[t][j] = 0.0f;
        }
    }
    auto step = [&](const uint4 wv, int e) {
        // elements e .. e + 7 of the row, chains (e % 32) .. + 7
        float wf[8];
        wf[0] = widen_bf16(static_cast<uint16_t>(wv.x));
        wf[1] = widen_bf16(static_cast<uint16_t>(wv.x >> 16));
        wf[2] = widen_bf16(static_cast<uint16_t>(wv.y));
        wf[3] = widen_bf16(static_cast<uint16_t>(wv.y >> 16));
        wf[4] = widen_bf16(static_cast<uint16_t>(wv.z));
        wf[5] = widen_bf16(static_cast<uint16_t>(wv.z >> 16));
        wf[6] = widen_bf16(static_cast<uint16_t>(wv.w));
        wf[7] = widen_bf16(static_cast<uint16_t>(wv.w >> 16));
#pragma unroll
        for (int t = 0; t < kHeadTokens; ++t) {
            if (t < tokens) {
                const float4 xa = xs4[t * q4 + e / 4];
                const float4 xb = xs4[t * q4 + e / 4 + 1];
                acc[t][0] = __builtin_fmaf(wf[0], xa.x, acc[t][0]);
                acc[t][1] = __builtin_fmaf(wf[1], xa.y, acc[t][1]);
                acc[t][2] = __builtin_fmaf(wf[2], xa.z, acc[t][2]);
                acc[t][3] = __builtin_fmaf(wf[3], xa.w, acc[t][3]);
                acc[t][4] = __builtin_fmaf(wf[4], xb.x, acc[t][4]);
                acc[t][5] = __builtin_fmaf(wf[5], xb.y, acc[t][5]);
                acc[t][6] = __builtin_fmaf(wf[6], xb.z, acc[t][6]);
                acc[t][7] = __builtin_fmaf(wf[7], xb.w, acc[t][7]);
            }
        }
    };
    const int steps = n32 / 32;
    int s = 0;
    for (; s + kUnroll <= steps; s += kUnroll) {
        uint4 wv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            wv[u] = load_stream16(wr + 32 * (s + u) + 8 * q);
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            step(wv[u], 32 * (s + u) + 8 * q);
        }
    }
    for (; s < steps; ++s) {
        step(load_stream16(wr + 32 * s + 8 * q), 32 * s + 8 * q);
    }
    if (q == 0) {
        // chains 0..7 continue over the remainder, element n32 + 8 k + j on chain j
        for (int e = n32; e < n8; e += 8) {
            step(load_stream16(wr + e), e);
        }
    }
#pragma unroll
    for (int t = 0; t < kHeadTokens; ++t) {
        if (t >= tokens) {
            break;
        }
        // lane sums (a[l] + a[8 + l]) + (a[16 + l] + a[24 + l]) over the row's 4 lanes
        float ls[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const float v01 = acc[t][l] + __shfl_xor(acc[t][l], 1);
            ls[l] = v01 + __shfl_xor(v01, 2);
        }
        const float h0 = ls[0] + ls[4];
        const float h1 = ls[1] + ls[5];
        const float h2 = ls[2] + ls[6];
        const float h3 = ls[3] + ls[7];
        const float total = (h0 + h2) + (h1 + h3);
        if (live && q == 0) {
            // gemm::matvec_bf16_accumulate folds the row as fma(scale, dot, out) (src/Gemm.cpp:156-175)
            float* o = logits + static_cast<int64_t>(t) * rows + row;
            *o = accumulate ? __builtin_fmaf(scale, total, *o) : total;
        }
        if (partial == nullptr) {
            continue;
        }
        HeadBest b{total, static_cast<int32_t>(row), live && q == 0 && total == total ? 1 : 0};
        b = wave_better(b);
        if (lane == 0) {
            wave_best[tid >> 6] = b;
        }
        __syncthreads();
        if (tid == 0) {
            HeadBest r = wave_best[0];
            for (int k = 1; k < THREADS / 64; ++k) {
                r = better(r, wave_best[k]);
            }
            partial[static_cast<int64_t>(t) * gridDim.x + blockIdx.x] = r;
        }
        __syncthreads();
    }
}

// Weight rows read through the scalar cache (uniform across the lanes).
typedef const __attribute__((address_space(4))) uint32_t const_u32;

// The same dot products for many tokens, with each token's inputs read from
// memory once per workgroup rather than once per wave: 64 tokens (one per
// lane) and four waves of kTokRows rows.  The tokens' inputs pass through LDS in
// tiles of 64 elements, a kTokStages-slot ring filled by direct-to-LDS buffer
// loads (each wave a quarter of each tile) and read by all four waves; the rows
// come through the scalar cache, 16 elements per step.  The steps are
// pipelined on one wait: at the start of a step everything requested so far is
// in (lgkmcnt(0)), then the next step's LDS reads and scalar loads are issued,
// then this step's FMAs run while they land (a scalar load can complete out of
// order, so no finer wait on the shared counter would be exact).  Every
// (token, row) pair keeps its 32 chains in one lane and reduces them as
// head_logits_kernel does, bit for bit.  in_dim % 64 == 0.
constexpr int kTokRows = 3;    // rows per wave
constexpr int kTokTile = 64;   // input elements per LDS slot
constexpr int kTokStages = 4;
constexpr int kTokStep = 16;   // elements per weight step
typedef __attribute__((address_space(3))) void head_lds_void;
constexpr int kHeadBufferWord3 = 0x00020000;  // buffer descriptor word 3, raw 32-bit access
// s_waitcnt immediates (vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
constexpr int kWaitLgkm0 = 0xC07F;             // lgkmcnt(0), the others unconstrained
constexpr int kWaitVm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x0070 | 0x0F00; }

__global__ __launch_bounds__(256) void matvec_tokens_kernel(const uint16_t* __restrict__ w,
                                                            const float* __restrict__ x, float* out, int64_t rows,
                                                            int32_t in_dim, int64_t tokens, float scale,
                                                            int32_t accumulate) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    // slot: 64 tokens x 16 units of 4 elements; unit q of token t at position
    // t * 16 + (q ^ (t % 16)), so the 16 lanes of each quarter-wave read 16
    // distinct bank groups.  One array per slot, so the compiler's waits
    // tell the slots apart.
    __shared__ __align__(16) float s0[64 * kTokTile], s1[64 * kTokTile], s2[64 * kTokTile], s3[64 * kTokTile];
    float* const ring[kTokStages] = {s0, s1, s2, s3};
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int64_t t0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int64_t ntok = std::min<int64_t>(64, tokens - t0);
    const int64_t row0 = (static_cast<int64_t>(blockIdx.y) * 4 + wave) * kTokRows;
    const_u32* wr[kTokRows];
#pragma unroll
    for (int r = 0; r < kTokRows; ++r) {
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;  // rows past the end load the last, store nothing
        wr[r] = (const_u32*)(w + row * in_dim);
    }
    const int ntiles = in_dim / kTokTile;
    // this wave's four loads of a tile: load j covers positions (4 wave + j) 64
    // + lane, i.e. token u / 16 and unit (u % 16) ^ (token % 16); tokens past
    // the last read the last
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(x + t0 * in_dim), 0, static_cast<int>(ntok * in_dim * 4), kHeadBufferWord3);
    unsigned src[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int u = (4 * wave + j) * 64 + lane;
        const int tt = u >> 4;
        const int q = (u & 15) ^ (tt & 15);
        const int ttc = tt < ntok ? tt : static_cast<int>(ntok) - 1;
        src[j] = static_cast<unsigned>((ttc * in_dim + 4 * q) * 4);
    }
    auto issue = [&](int tile, float* slot) {
        tile = tile < ntiles ? tile : ntiles - 1;  // past the end: reload the last tile (every step issues alike)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(xres, (head_lds_void*)(slot + (4 * wave + j) * 256), 16,
                                                     src[j] + static_cast<unsigned>(tile * kTokTile * 4), 0, 0, 0);
        }
    };
    float acc[kTokRows][32];
#pragma unroll
    for (int r = 0; r < kTokRows; ++r) {
#pragma unroll
        for (int c = 0; c < 32; ++c) {
            acc[r][c] = 0.0f;
        }
    }
    f4v xa[4], xb[4];
    uint32_t wa[kTokRows][8], wb[kTokRows][8];
    const int sw = lane & 15;
    // step `st` (0..3) of `tile` from `slot`: the lane's token's 16 inputs and
    // each row's 16 weights (8 bf16 pairs)
    auto read = [&](const float* slot, int tile, int st, f4v (&xv)[4], uint32_t (&wv)[kTokRows][8]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xv[i] = *reinterpret_cast<const f4v*>(slot + (lane * 16 + ((4 * st + i) ^ sw)) * 4);
        }
        const int e = (tile < ntiles ? tile : ntiles - 1) * kTokTile + st * kTokStep;
#pragma unroll
        for (int r = 0; r < kTokRows; ++r) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                wv[r][k] = wr[r][e / 2 + k];
            }
        }
    };
    // elements e .. e + 15 of a step with parity `half` (e % 32 == 16 half):
    // element e + m on chain 16 half + m
    auto fma_step = [&](int half, const f4v (&xv)[4], const uint32_t (&wv)[kTokRows][8]) {
#pragma unroll
        for (int r = 0; r < kTokRows; ++r) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const uint32_t pair = wv[r][2 * i + j];
                    const int c = 16 * half + 4 * i + 2 * j;
                    acc[r][c] = __builtin_fmaf(bits_float(pair << 16), xv[i][2 * j], acc[r][c]);
                    acc[r][c + 1] = __builtin_fmaf(bits_float(pair & 0xffff0000u), xv[i][2 * j + 1], acc[r][c + 1]);
                }
            }
        }
    };
    auto wait_all_lgkm = [] {
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
        __builtin_amdgcn_sched_barrier(0);
    };
#pragma unroll
    for (int d = 0; d < kTokStages - 1; ++d) {
        issue(d, ring[d]);
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm(4 * (kTokStages - 2)));  // tile 0 is in
    __builtin_amdgcn_s_barrier();
    read(ring[0], 0, 0, xa, wa);
    for (int tb = 0; tb < ntiles; tb += kTokStages) {
#pragma unroll
        for (int j = 0; j < kTokStages; ++j) {
            const int tile = tb + j;  // tiles past the end load alike and add nothing
            const float* slot = ring[j];
            const bool live = tile < ntiles;
            wait_all_lgkm();
            read(slot, tile, 1, xb, wb);
            __builtin_amdgcn_sched_barrier(0);
            if (live) {
                fma_step(0, xa, wa);
            }
            wait_all_lgkm();
            read(slot, tile, 2, xa, wa);
            __builtin_amdgcn_sched_barrier(0);
            if (live) {
                fma_step(1, xb, wb);
            }
            wait_all_lgkm();
            read(slot, tile, 3, xb, wb);
            __builtin_amdgcn_sched_barrier(0);
            if (live) {
                fma_step(0, xa, wa);
            }
            wait_all_lgkm();
            // tile + 1 is in (the one issued after it may still be in flight),
            // and every wave has read all of tile - 1: its slot takes tile + 3
            __builtin_amdgcn_s_waitcnt(kWaitVm(4 * (kTokStages - 3)));
            __builtin_amdgcn_s_barrier();
            issue(tile + kTokStages - 1, ring[(j + kTokStages - 1) % kTokStages]);
            read(ring[(j + 1) % kTokStages], tile + 1, 0, xa, wa);
            __builtin_amdgcn_sched_barrier(0);
            if (live) {
                fma_step(1, xb, wb);
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // every load to LDS has landed before the workgroup ends
    const int64_t t = t0 + lane;
#pragma unroll
    for (int r = 0; r < kTokRows; ++r) {
        // (a[l] + a[8 + l]) + (a[16 + l] + a[24 + l]), lanes j and j + 4, (h0 + h2) + (h1 + h3)
        float ls[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            ls[l] = (acc[r][l] + acc[r][8 + l]) + (acc[r][16 + l] + acc[r][24 + l]);
        }
        const float h0 = ls[0] + ls[4];
        const float h1 = ls[1] + ls[5];
        const float h2 = ls[2] + ls[6];
        const float h3 = ls[3] + ls[7];
        const float total = (h0 + h2) + (h1 + h3);
        if (t < tokens && row0 + r < rows) {
            float* o = out + t * rows + row0 + r;
            *o = accumulate ? __builtin_fmaf(scale, total, *o) : total;
        }
    }
}

// The same dot product for one token (the projections of a decode step): 32
// lanes per row (dot_bf16_lanes32), two rows per wave, so even a 576-row
// projection spreads over 72 workgroups.
// STEPS > 0: in_dim == 32 STEPS, and every step's weight word and activation
// is loaded before the first multiply-add (the whole matrix in flight at once
// when there are few rows); the chain and the lane reduction are
// dot_bf16_lanes32's.
template <int STEPS>
__global__ __launch_bounds__(256) void matvec_one_kernel(const uint16_t* __restrict__ w, const float* __restrict__ x,
                                                         float* out, int64_t rows, int32_t in_dim, float scale,
                                                         int32_t accumulate) {
    const int lane = threadIdx.x & 63;
    const int c = lane & 31;
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
    const bool live = row < rows;
    const uint16_t* wr = w + (live ? row : rows - 1) * in_dim;
    float total;
    if constexpr (STEPS > 0) {
        uint32_t word[STEPS];
        float xv[STEPS];
        const uint32_t* w32 = reinterpret_cast<const uint32_t*>(wr) + (c >> 1);
#pragma unroll
        for (int u = 0; u < STEPS; ++u) {
            word[u] = w32[16 * u];
            xv[u] = x[32 * u + c];
        }
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < STEPS; ++u) {
            acc = __builtin_fmaf(bits_float((c & 1) != 0 ? (word[u] & 0xffff0000u) : (word[u] << 16)), xv[u], acc);
        }
        const float t1 = acc + __shfl_xor(acc, 8);
        const float t2 = t1 + __shfl_xor(t1, 16);
        const float t3 = t2 + __shfl_xor(t2, 4);
        const float t4 = t3 + __shfl_xor(t3, 2);
        total = t4 + __shfl_xor(t4, 1);
    } else {
        total = dot_bf16_lanes32(wr, [&](int e) { return x[e]; }, in_dim, c);
    }
    if (live && c == 0) {
        out[row] = accumulate ? __builtin_fmaf(scale, total, out[row]) : total;
    }
}

// Sampler::select_next's greedy branch over the blocks' candidates:
// std::max_element keeps the first of equal values and moves only on a strictly
// larger one, so a NaN never becomes the choice, except at index 0, which
// nothing after it can replace.  That is the first maximum of the non-NaN
// logits, or 0 when logit 0 is NaN.
__global__ __launch_bounds__(1024) void argmax_first_kernel(const HeadBest* __restrict__ partial, int32_t blocks,
                                                            const float* __restrict__ logits, int64_t vocab,
                                                            int32_t* out) {
    __shared__ HeadBest wave_best[16];
    const HeadBest* p = partial + static_cast<int64_t>(blockIdx.x) * blocks;
    HeadBest b{0.0f, 0, 0};
    for (int i = threadIdx.x; i < blocks; i += 1024) {
        b = better(b, p[i]);
    }
    b = wave_better(b);
    if ((threadIdx.x & 63) == 0) {
        wave_best[threadIdx.x >> 6] = b;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        HeadBest r = wave_best[0];
        for (int k = 1; k < 16; ++k) {
            r = better(r, wave_best[k]);
        }
        const float first = logits[static_cast<int64_t>(blockIdx.x) * vocab];
        out[blockIdx.x] = (first != first || !r.have) ? 0 : r.i;
    }
}

}  // namespace

int64_t head_blocks(int64_t rows) { return (rows + kRows - 1) / kRows; }

hipError_t launch_head(const uint16_t* w, const float* x, float* logits, HeadBest* partial, int32_t* token,
                       int64_t rows, int32_t in_dim, int32_t tokens, hipStream_t s) {
    if (rows <= 0 || tokens <= 0) {
        return hipSuccess;
    }
    if (tokens > kHeadTokens || in_dim <= 0 || in_dim % 8 != 0 || rows > INT32_MAX) {
        return hipErrorInvalidValue;
    }
    const int64_t blocks = head_blocks(rows);
    const size_t lds = sizeof(float) * static_cast<size_t>(tokens) * static_cast<size_t>(in_dim);
    if (lds > 64 * 1024) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(head_logits_kernel<kThreads>, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), lds, s, w,
                       x, logits, partial, rows, in_dim, tokens, 1.0f, 0);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || token == nullptr) {
        return err;
    }
    hipLaunchKernelGGL(argmax_first_kernel, dim3(static_cast<unsigned>(tokens)), dim3(1024), 0, s, partial,
                       static_cast<int32_t>(blocks), logits, rows, token);
    return hipGetLastError();
}

bool matvec_rows_supported(int64_t rows, int64_t in_dim) {
    return rows > 0 && rows <= INT32_MAX && in_dim > 0 && in_dim % 8 == 0 && in_dim <= 16384;
}

hipError_t launch_matvec_rows(const uint16_t* w, const float* x, float* out, int64_t rows, int64_t in_dim, float scale,
                              int32_t accumulate, hipStream_t s) {
    if (!matvec_rows_supported(rows, in_dim)) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(head_logits_kernel<kThreads>, dim3(static_cast<unsigned>(head_blocks(rows))), dim3(kThreads),
                       sizeof(float) * static_cast<size_t>(in_dim), s, w, x, out, nullptr, rows,
                       static_cast<int32_t>(in_dim), 1, scale, accumulate);
    return hipGetLastError();
}

hipError_t launch_matvec_tokens(const uint16_t* w, const float* x, float* out, int64_t rows, int64_t in_dim,
                                int64_t tokens, float scale, int32_t accumulate, hipStream_t s) {
    if (tokens <= 0) {
        return hipSuccess;
    }
    if (!matvec_rows_supported(rows, in_dim)) {
        return hipErrorInvalidValue;
    }
    if (tokens == 1) {
        if (in_dim == 2048) {
            hipLaunchKernelGGL(matvec_one_kernel<64>, dim3(static_cast<unsigned>((rows + 7) / 8)), dim3(256), 0, s, w,
                               x, out, rows, static_cast<int32_t>(in_dim), scale, accumulate);
        } else {
            hipLaunchKernelGGL(matvec_one_kernel<0>, dim3(static_cast<unsigned>((rows + 7) / 8)), dim3(256), 0, s, w, x,
                               out, rows, static_cast<int32_t>(in_dim), scale, accumulate);
        }
        return hipGetLastError();
    }
    if (tokens > kHeadTokens && in_dim % 64 == 0) {
        const dim3 grid(static_cast<unsigned>((tokens + 63) / 64),
                        static_cast<unsigned>((rows + 4 * kTokRows - 1) / (4 * kTokRows)));
        hipLaunchKernelGGL(matvec_tokens_kernel, grid, dim3(256), 0, s, w, x, out, rows,
                           static_cast<int32_t>(in_dim), tokens, scale, accumulate);
        return hipGetLastError();
    }
    // tokens per launch: at most kHeadTokens, and their rows must fit 64 KiB of LDS
    const int64_t per = std::min<int64_t>(kHeadTokens, std::max<int64_t>(1, 16384 / in_dim));
    const int64_t rows_per_block = kRowsPerWave * (kSmallThreads / 64);
    const unsigned blocks = static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block);
    for (int64_t t0 = 0; t0 < tokens; t0 += per) {
        const int32_t n = static_cast<int32_t>(std::min<int64_t>(per, tokens - t0));
        hipLaunchKernelGGL(head_logits_kernel<kSmallThreads>, dim3(blocks), dim3(kSmallThreads),
                           sizeof(float) * static_cast<size_t>(n) * static_cast<size_t>(in_dim), s, w,
                           x + t0 * in_dim, out + t0 * rows, nullptr, rows, static_cast<int32_t>(in_dim), n, scale,
                           accumulate);
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) {
            return err;
        }
    }
    return hipSuccess;
}

}  // namespace lm
