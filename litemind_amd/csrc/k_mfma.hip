// k_mfma.hip -- grouped SwiGLU on MFMA for large token counts.
//
// Reference: DeepSeekRunner::Impl::feed_forward (src/DeepSeekRunner.cpp:228-240)
// applied to every (token, expert) assignment; LiteMind evaluates each token
// separately, here the assignments of one expert form the rows of a GEMM.
//
// Operands are fp16 (activations converted once; BF16 weights re-encoded to
// fp16 at upload, exact for |w| in [2^-17, 65504]) with fp32 accumulation on
// v_mfma_f32_32x32x16_f16.  Two kernels:
//   gate/up: act16[slot, j] = silu(x . Wg[j]) * (x . Wu[j]), the x rows gathered
//            through the permutation; Wgu rows are gate/up interleaved in 32-row
//            groups, so a wave's two 32-wide column blocks are the gate and the
//            up of the same outputs and the epilogue pairs them in registers.
//   down:    down_out[slot, h] = act16[slot] . Wd[h] (fp32 out, combined later).
// Block tile 128 x 128, K step 64, 4 waves of 64 x 64 (2 x 2 MFMA blocks).
// Tiles of one weight column block are consecutive (M fastest) and tile ids
// are remapped so consecutive tiles run on the same XCD and share its L2.
#include "lm_internal.h"

namespace lm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;
constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int kLdsRow = BK + 8;          // halves per LDS row (16 B padding)
constexpr int kTileHalves = BM * kLdsRow;
constexpr int kXcds = 8;

enum Mode { kGateUp = 0, kDown = 1 };

struct TileInfo {
    int g;        // group
    int mt, nt;   // tile coordinates inside the group
    int rows;     // tokens in the group
    int64_t slot0;
};

// Finds the tile's group from per-group tile counts (routed experts in expert
// order, then the shared expert).  Wave 0 scans; the result goes through LDS.
__device__ bool decode_tile(const ExpertArgs& a, int64_t tile, int nt_routed, int nt_shared, TileInfo& ti) {
    __shared__ int s_info[4];
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64) {
        const int g = lane;
        const int n = g < a.experts ? a.rb.counts[g] : 0;
        const int mts = (n + BM - 1) / BM;
        const int tiles = mts * nt_routed;
        int incl = tiles;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int v = __shfl_up(incl, o);
            if (lane >= o) {
                incl += v;
            }
        }
        const int excl = incl - tiles;
        const int routed_total = __shfl(incl, 63);
        int found = -1, local = 0, found_mts = 0;
        if (tile < routed_total) {
            const uint64_t hit = __ballot(tile >= excl && tile < incl && tiles > 0);
            const int gl = static_cast<int>(__builtin_ctzll(hit));
            found = gl;
            local = static_cast<int>(tile) - __shfl(excl, gl);
            found_mts = __shfl(mts, gl);
        } else if (a.has_shared) {
            const int mts_s = static_cast<int>((a.tokens + BM - 1) / BM);
            const int64_t l = tile - routed_total;
            if (l < static_cast<int64_t>(mts_s) * nt_shared) {
                found = a.experts;
                local = static_cast<int>(l);
                found_mts = mts_s;
            }
        }
        if (lane == 0) {
            s_info[0] = found;
            s_info[1] = found >= 0 ? local % found_mts : 0;
            s_info[2] = found >= 0 ? local / found_mts : 0;
        }
    }
    __syncthreads();
    ti.g = s_info[0];
    if (ti.g < 0) {
        return false;
    }
    ti.mt = s_info[1];
    ti.nt = s_info[2];
    if (ti.g < a.experts) {
        ti.rows = a.rb.counts[ti.g];
        ti.slot0 = a.rb.offsets[ti.g];
    } else {
        ti.rows = static_cast<int>(a.tokens);
        ti.slot0 = a.tokens * a.top_k;
    }
    return true;
}

// 16-byte load through the global address space (operand pointers are read
// from tables, which would otherwise compile to flat loads).
__device__ inline uint4 load16(const void* p) {
    const u32x4 v = *(global_u32x4*)(p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ inline float silu_fast(float g, float u) {
    // The fp16-operand path is checked against a tolerance; the hardware exp
    // and reciprocal are accurate to a few ulp, far below the fp16 rounding.
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

template <int MODE>
__global__ __launch_bounds__(kThreads) void mfma_kernel(ExpertArgs a, int64_t grid_tiles) {
    __shared__ _Float16 lds[2][2][kTileHalves];  // [buffer][A, B][row * kLdsRow + k]
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware remap: workgroup b runs on XCD b % 8; give each XCD a
    // contiguous range of tiles (grid_tiles is a multiple of 8).
    const int64_t b = blockIdx.x;
    const int64_t tile = (b % kXcds) * (grid_tiles / kXcds) + b / kXcds;

    const int inter_p = a.inter_p;
    const int nt_routed = MODE == kGateUp ? 2 * inter_p / BN : (a.hidden + BN - 1) / BN;
    const int nt_shared = MODE == kGateUp ? 2 * a.shared_inter_p / BN : (a.hidden + BN - 1) / BN;
    TileInfo ti;
    if (!decode_tile(a, tile, nt_routed, nt_shared, ti)) {
        return;
    }
    const bool shared = ti.g >= a.experts;
    const int width_p = shared ? a.shared_inter_p : inter_p;
    const int K = MODE == kGateUp ? a.hidden_p : width_p;
    const _Float16* act_base =
        a.act16 + (shared ? a.tokens * a.top_k * static_cast<int64_t>(inter_p) : ti.slot0 * inter_p);

    // Global -> register staging: each thread moves 4 x 16 B of A and of B per K step.
    // Chunk c = tid + 256 q (q = 0..3): row c / 8, 16-byte column c % 8.
    const _Float16* arow[4];
    const _Float16* brow[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int c = tid + q * kThreads;
        const int r = c >> 3;
        int m = ti.mt * BM + r;
        m = m < ti.rows ? m : ti.rows - 1;  // padding rows repeat the last row; never stored
        if (MODE == kGateUp) {
            const int64_t token = shared ? m : a.rb.perm[ti.slot0 + m] / a.top_k;
            arow[q] = a.x16 + token * a.hidden_p + (c & 7) * 8;
            brow[q] = a.groups.gu_h[ti.g] + static_cast<int64_t>(ti.nt * BN + r) * a.hidden_p + (c & 7) * 8;
        } else {
            // Output rows past H (hidden not a multiple of 128) repeat row H - 1; never stored.
            const int h = ti.nt * BN + r < a.hidden ? ti.nt * BN + r : a.hidden - 1;
            arow[q] = act_base + static_cast<int64_t>(m) * width_p + (c & 7) * 8;
            brow[q] = a.groups.down_h[ti.g] + static_cast<int64_t>(h) * width_p + (c & 7) * 8;
        }
    }
    // Staging registers, written out per chunk so they stay in registers.
    uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
    const int off0 = ((tid + 0 * kThreads) >> 3) * kLdsRow + (tid & 7) * 8;
    const int off1 = ((tid + 1 * kThreads) >> 3) * kLdsRow + (tid & 7) * 8;
    const int off2 = ((tid + 2 * kThreads) >> 3) * kLdsRow + (tid & 7) * 8;
    const int off3 = ((tid + 3 * kThreads) >> 3) * kLdsRow + (tid & 7) * 8;
#define LM_MFMA_FETCH(k0)               \
    ra0 = load16(arow[0] + (k0));       \
    rb0 = load16(brow[0] + (k0));       \
    ra1 = load16(arow[1] + (k0));       \
    rb1 = load16(brow[1] + (k0));       \
    ra2 = load16(arow[2] + (k0));       \
    rb2 = load16(brow[2] + (k0));       \
    ra3 = load16(arow[3] + (k0));       \
    rb3 = load16(brow[3] + (k0));
#define LM_MFMA_STORE(buf)                                        \
    *reinterpret_cast<uint4*>(&lds[(buf)][0][off0]) = ra0;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][1][off0]) = rb0;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][0][off1]) = ra1;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][1][off1]) = rb1;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][0][off2]) = ra2;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][1][off2]) = rb2;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][0][off3]) = ra3;        \
    *reinterpret_cast<uint4*>(&lds[(buf)][1][off3]) = rb3;

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[i][j] = floatx16{};
        }
    }
    const int nk = K / BK;
    LM_MFMA_FETCH(0)
    LM_MFMA_STORE(0)
    lds_barrier();
    for (int ks = 0; ks < nk; ++ks) {
        const int buf = ks & 1;
        if (ks + 1 < nk) {
            LM_MFMA_FETCH((ks + 1) * BK)
        }
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = wm * 64 + i * 32 + (lane & 31);
                af[i] = *reinterpret_cast<const half8*>(&lds[buf][0][row * kLdsRow + kk * 16 + (lane >> 5) * 8]);
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = wn * 64 + j * 32 + (lane & 31);
                bf[j] = *reinterpret_cast<const half8*>(&lds[buf][1][row * kLdsRow + kk * 16 + (lane >> 5) * 8]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (ks + 1 < nk) {
            LM_MFMA_STORE(buf ^ 1)
        }
        lds_barrier();
    }
#undef LM_MFMA_FETCH
#undef LM_MFMA_STORE

    // Epilogue.  Lane l holds column n = l % 32 of each 32 x 32 block, rows
    // m = 8 (r / 4) + 4 (l / 32) + r % 4 for registers r = 0..15.
    const int n = lane & 31;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m_local = wm * 64 + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int m = ti.mt * BM + m_local;
            if (m >= ti.rows) {
                continue;
            }
            if (MODE == kGateUp) {
                // Interleaved columns: block j = 0 is gate, j = 1 the matching up.
                const int jcol = (ti.nt * BN) / 2 + wn * 32 + n;
                const float h = silu_fast(acc[i][0][r], acc[i][1][r]);
                a.act16[(shared ? a.tokens * a.top_k * static_cast<int64_t>(inter_p) : ti.slot0 * inter_p) +
                        static_cast<int64_t>(m) * width_p + jcol] = static_cast<_Float16>(h);
            } else {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int h = ti.nt * BN + wn * 64 + j * 32 + n;
                    if (h < a.hidden) {
                        a.down_out[(ti.slot0 + m) * a.hidden + h] = acc[i][j][r];
                    }
                }
            }
        }
    }
}

int64_t tile_bound(const ExpertArgs& a, int nt_routed, int nt_shared) {
    const int64_t TK = a.tokens * a.top_k;
    const int64_t groups = a.experts < TK ? a.experts : TK;
    int64_t tiles = ((TK + BM - 1) / BM + groups) * nt_routed;
    if (a.has_shared) {
        tiles += (a.tokens + BM - 1) / BM * nt_shared;
    }
    return (tiles + kXcds - 1) / kXcds * kXcds;
}

}  // namespace

hipError_t launch_mfma_gateup(const ExpertArgs& a, int64_t, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.hidden_p % BK != 0 || (2 * a.inter_p) % BN != 0 || (2 * a.shared_inter_p) % BN != 0) {
        return hipErrorInvalidValue;
    }
    const int64_t grid = tile_bound(a, 2 * a.inter_p / BN, 2 * a.shared_inter_p / BN);
    hipLaunchKernelGGL((mfma_kernel<kGateUp>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, a, grid);
    return hipGetLastError();
}

hipError_t launch_mfma_down(const ExpertArgs& a, int64_t, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.inter_p % BK != 0 || a.shared_inter_p % BK != 0) {
        return hipErrorInvalidValue;
    }
    const int nt = (a.hidden + BN - 1) / BN;
    const int64_t grid = tile_bound(a, nt, nt);
    hipLaunchKernelGGL((mfma_kernel<kDown>), dim3(static_cast<unsigned>(grid)), dim3(kThreads), 0, s, a, grid);
    return hipGetLastError();
}

}  // namespace lm
