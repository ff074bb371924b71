// router_chunks.h -- the exact router logits of eight experts for one token
// by one 256-thread workgroup, the gate rows streamed in chunks through LDS
// (router_chunked_kernel, and the one-token launch of router and gate/up for
// more than 64 experts).
//
// Reference: gemm::matvec_f32 / dot (src/Gemm.cpp:183-189), one strictly
// left-to-right fp32 sum per logit.
#pragma once

#include "lm_internal.h"

namespace lm {

// Raw logit (bias not added) of expert e0 + threadIdx.x for threads 0..7 (0
// on the others) of one token xt, for any hidden width: the gate rows in
// chunks of kChunkRows, each chunk's
// rounded products formed by all threads into one of two LDS buffers while
// lanes 0..7 of wave 0 add the previous chunk's products to their expert's
// chain, strictly left to right over the whole row (LiteMind's dot,
// src/Gemm.cpp:183-189), as router_single_kernel does for a row that fits LDS
// whole.  For more than 64 experts, where the per-token router gives one wave
// every expert of a token (a chain per expert, one after another).  256
// threads; hidden % 4 == 0, E % 8 == 0; wt is the gate transposed [H, E];
// prod: kChunkFloat4s float4 of LDS.
constexpr int kChunkExperts = 8;
constexpr int kChunkThreads = 256;
constexpr int kChunkRows = 512;
constexpr int kChunkFloat4s = 2 * kChunkRows / 4 * kChunkExperts;
__device__ inline float chunked_logit(int H, int E, const float* __restrict__ xt, const float* __restrict__ wt, int e0,
                                      float4* prod_lds) {
    constexpr int kSplitExperts = kChunkExperts;
    constexpr int kSplitThreads = kChunkThreads;
    float4 (*prod)[kChunkRows / 4 * kSplitExperts] =
        reinterpret_cast<float4 (*)[kChunkRows / 4 * kSplitExperts]>(prod_lds);
    const int tid = threadIdx.x;
    const int nchunks = (H + kChunkRows - 1) / kChunkRows;
    constexpr int kPer = kChunkRows * (kSplitExperts / 4) / kSplitThreads;  // float4 loads per thread per chunk
    float4 w[kPer];
    float xv[kPer];
    auto fetch = [&](int c) {
        const int i0 = c * kChunkRows;
        const int nf = (H - i0 < kChunkRows ? H - i0 : kChunkRows) * (kSplitExperts / 4);
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int f = j * kSplitThreads + tid;
            const int fl = f < nf ? f : nf - 1;
            const int i = i0 + (fl >> 1);
            w[j] = *reinterpret_cast<const float4*>(wt + static_cast<int64_t>(i) * E + e0 + 4 * (fl & 1));
            xv[j] = xt[i];
        }
    };
    auto store = [&](int c) {
        const int i0 = c * kChunkRows;
        const int nf = (H - i0 < kChunkRows ? H - i0 : kChunkRows) * (kSplitExperts / 4);
        float4* buf = prod[c & 1];
#pragma unroll
        for (int j = 0; j < kPer; ++j) {
            const int f = j * kSplitThreads + tid;
            if (f < nf) {
                const int i = f >> 1;  // row within the chunk
                const int el = 4 * (f & 1);
                float* base = reinterpret_cast<float*>(&buf[(i >> 2) * kSplitExperts]);
                base[(el + 0) * 4 + (i & 3)] = w[j].x * xv[j];
                base[(el + 1) * 4 + (i & 3)] = w[j].y * xv[j];
                base[(el + 2) * 4 + (i & 3)] = w[j].z * xv[j];
                base[(el + 3) * 4 + (i & 3)] = w[j].w * xv[j];
            }
        }
    };
    fetch(0);
    store(0);
    lds_barrier();
    float acc = 0.0f;
    for (int c = 0; c < nchunks; ++c) {
        if (c + 1 < nchunks) {
            fetch(c + 1);  // in flight while the chains run
        }
        if (tid < kSplitExperts) {
            const float4* buf = prod[c & 1];
            const int quads = (H - c * kChunkRows < kChunkRows ? H - c * kChunkRows : kChunkRows) / 4;
            auto add8 = [&](const float4 (&p)[8]) {
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    acc = acc + p[u].x;
                    acc = acc + p[u].y;
                    acc = acc + p[u].z;
                    acc = acc + p[u].w;
                }
            };
            int q = 0;
            if (quads == kChunkRows / 4) {
                // a whole chunk fully unrolled, two register sets in turn: one
                // batch's reads are in flight while the other batch is added,
                // so the chain (a dependent add every ~3.5 ns) never waits for
                // LDS (a loop over the batches costs register copies and a
                // full wait per batch)
                constexpr int kBatches = kChunkRows / 32;
                float4 p[2][8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    p[0][u] = buf[u * kSplitExperts + tid];
                }
#pragma unroll
                for (int b = 0; b < kBatches; ++b) {
                    if (b + 1 < kBatches) {
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            p[(b + 1) & 1][u] = buf[(8 * (b + 1) + u) * kSplitExperts + tid];
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the adds
                    add8(p[b & 1]);
                    __builtin_amdgcn_sched_barrier(0);
                }
                q = quads;
            }
            for (; q + 8 <= quads; q += 8) {  // eight reads in flight, then their adds in order
                float4 p[8];
#pragma unroll
                for (int u = 0; u < 8; ++u) {
                    p[u] = buf[(q + u) * kSplitExperts + tid];
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
                const float4 p = buf[q * kSplitExperts + tid];
                acc = acc + p.x;
                acc = acc + p.y;
                acc = acc + p.z;
                acc = acc + p.w;
            }
        }
        if (c + 1 < nchunks) {
            store(c + 1);  // the other buffer: its last readers passed the previous barrier
        }
        lds_barrier();
    }
    return acc;
}


}  // namespace lm
