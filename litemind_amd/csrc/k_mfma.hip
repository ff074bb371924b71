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
//
// Every operand is stored in panel layout (32-column panels of [rows, 32]), so
// the K slice of a stage is one contiguous block per operand: 64 bytes per row,
// consecutive rows adjacent.  Loads go from global memory straight into LDS
// with global_load_lds_dwordx4 (no staging registers); each wave instruction
// fills 1 KB of LDS, 16 rows of 64 bytes, lane l writing bytes [16 l, 16 l + 16).
// The lane chooses which 16-byte chunk of its row it loads, so rows are stored
// in LDS with their chunks permuted (row_swizzle), which keeps the MFMA fragment
// reads free of bank conflicts.
//
// Per workgroup: a WM x WN grid of waves, each computing MI x NJ MFMA blocks of
// 32 x 32, over a BM x 256 tile (BM = 32 WM MI), K step 32, and a STAGES-deep
// pipeline: while stage k is multiplied, stages k + 1 .. k + STAGES - 1 are in
// flight, each in its own LDS array so the compiler can track the asynchronous
// writes per buffer.  Rows past the end of a group (tokens) or of a matrix
// (weight rows) load a clamped row and are never stored.  Two shapes:
//   128 x 256, 2 x 2 waves of 64 x 128, 3 stages (24 KB each): large groups;
//    64 x 256, 1 x 4 waves of 64 x 64, 4 stages (20 KB each): groups of a few
//    dozen rows, where the kernel streams weights and the bytes in flight
//    per CU (two workgroups x (STAGES - 1) x 16 KB of weights) set its rate.
#include "lm_internal.h"

namespace lm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(1))) const void global_void;
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BN = 256;
constexpr int BK = kPanel;                   // halves: 64-byte rows, 4 chunks of 16 B
constexpr int kRowBytes = BK * 2;
constexpr int kBBytes = BN * kRowBytes;      // 16 KB
constexpr int kXcds = 8;

template <int WM, int WN, int MI, int NJ, int STAGES>
struct Shape {
    static constexpr int WAVES = WM * WN;
    static constexpr int kThreads = 64 * WAVES;
    static constexpr int BM = 32 * WM * MI;
    static constexpr int kABytes = BM * kRowBytes;
    static constexpr int kALoads = kABytes / 1024 / WAVES;  // wave instructions per stage
    static constexpr int kBLoads = kBBytes / 1024 / WAVES;
    static constexpr int kLoadsPerStage = kALoads + kBLoads;
    static_assert(32 * WN * NJ == BN, "the waves cover the 256 columns");
    static_assert(kALoads * 1024 * WAVES == kABytes && kALoads >= 1, "whole A instructions per wave");
    static_assert(NJ % 2 == 0, "gate/up column blocks come in pairs");
    static_assert((STAGES - 2) * kLoadsPerStage < 16, "vmcnt immediate");
};

// Launches whose average routed group fits one 64-row tile (T k <= 64 E; a
// dense layer: T <= 64) take the 64-row shape.  Measured on V2-Lite (one MoE block, 64 experts, k 6): 8-12%
// faster from T = 8 to T = 512, 4-13% slower from T = 768 on, where groups
// span several 64-row tiles and each re-streams the expert's weights.
constexpr int64_t kNarrowRows = 64;

enum Mode { kGateUp = 0, kDown = 1 };

struct TileInfo {
    int g;        // group
    int mt, nt;   // tile coordinates inside the group
    int rows;     // tokens in the group
    int64_t slot0;
};

// Maps workgroup `blk` to a tile and finds the tile's group from per-group tile
// counts (routed experts in expert order, then the shared expert); M tiles of
// one column block are consecutive.  Workgroup b runs on XCD b % 8.  With
// `split` (the down projection, whose shared tiles have a longer K than the
// routed ones: 2816 against 1408 on V2-Lite) every XCD gets an equal share
// (within one) of the shared expert's tiles and of the routed tiles, each a
// contiguous range, its shared tiles first; one contiguous split of all tiles
// left the XCD that holds the shared tiles with twice the work of the others
// (measured: down at T = 2048 222 -> 179 us, T = 4096 351 -> 261 us).  Without
// it (gate/up: every tile has the same K) XCD x takes the x-th of eight
// contiguous, equal ranges of all tiles; dealing column blocks round robin over
// the XCDs instead (every XCD a share of every expert) measured 8% slower at
// T = 2048 and 5% at T = 4096.  M tiles of a column block share one L2.
// s_info: 3 ints of LDS for the hand-off from wave 0 (the caller lends a
// pipeline buffer that no load writes before every wave has passed a later
// barrier).
__device__ bool decode_tile(const ExpertArgs& a, int BM, int64_t blk, int nt_routed, int nt_shared, bool split,
                            TileInfo& ti, int* s_info) {
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64) {
        // Tiles of the routed groups in expert order, 64 experts per pass.
        int routed_total = 0;
        for (int g0 = 0; g0 < a.experts; g0 += 64) {
            const int g = g0 + lane;
            const int n = g < a.experts ? a.rb.counts[g] : 0;
            const int tiles = (n + BM - 1) / BM * nt_routed;
            int incl = tiles;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int v = __shfl_up(incl, o);
                if (lane >= o) {
                    incl += v;
                }
            }
            routed_total += __shfl(incl, 63);
        }
        const int mts_s = a.has_shared ? static_cast<int>((a.tokens + BM - 1) / BM) : 0;
        const int64_t shared_total = static_cast<int64_t>(mts_s) * nt_shared;
        const int64_t xcd = blk % kXcds, idx = blk / kXcds;
        // this XCD's contiguous share of n tiles: [first, first + count)
        auto share = [&](int64_t n, int64_t& first, int64_t& count) {
            const int64_t per = n / kXcds, extra = n % kXcds;
            count = per + (xcd < extra ? 1 : 0);
            first = xcd * per + (xcd < extra ? xcd : extra);
        };
        int64_t tile = -1;  // routed tile index, or shared tile routed_total + i
        if (split) {
            int64_t s_first, s_count, r_first, r_count;
            share(shared_total, s_first, s_count);
            share(routed_total, r_first, r_count);
            if (idx < s_count) {
                tile = routed_total + s_first + idx;
            } else if (idx - s_count < r_count) {
                tile = r_first + (idx - s_count);
            }
        } else {
            int64_t first, count;
            share(routed_total + shared_total, first, count);
            if (idx < count) {
                tile = first + idx;
            }
        }
        int found = -1, local = 0, found_mts = 0;
        if (tile >= 0 && tile < routed_total) {
            int carry = 0;
            for (int g0 = 0; g0 < a.experts; g0 += 64) {
                const int g = g0 + lane;
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
                const int excl = carry + incl - tiles;
                const uint64_t hit = __ballot(tile >= excl && tile < carry + incl && tiles > 0);
                if (hit != 0) {
                    const int gl = static_cast<int>(__builtin_ctzll(hit));
                    found = g0 + gl;
                    local = static_cast<int>(tile) - __shfl(excl, gl);
                    found_mts = __shfl(mts, gl);
                    break;
                }
                carry += __shfl(incl, 63);
            }
        } else if (tile >= routed_total) {
            found = a.experts;
            local = static_cast<int>(tile - routed_total);
            found_mts = mts_s;
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

__device__ inline float silu_fast(float g, float u) {
    // The fp16-operand path is checked against a tolerance; the hardware exp
    // and reciprocal are accurate to a few ulp, far below the fp16 rounding.
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// Chunk permutation of row r (row bits 1..3 only).  A ds_read_b128 serves 16
// lanes per cycle from 64 banks: lanes 0..15 read rows r0..r0+15 (r0 a
// multiple of 16) at one logical chunk, and the rows that share a bank phase
// (r mod 4) get four different chunk positions; the same holds for 8-lane
// groups over 32 banks.
__device__ inline int row_swizzle(int r) { return ((r >> 2) & 3) ^ (r & 2); }
// LDS byte offset of the 16-byte chunk c of row r.
__device__ inline int chunk_offset(int r, int c) { return r * kRowBytes + ((c ^ row_swizzle(r)) << 4); }

template <int MODE, int WM, int WN, int MI, int NJ, int STAGES>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_grouped_kernel(
    ExpertArgs a) {
    using S = Shape<WM, WN, MI, NJ, STAGES>;
    constexpr int WAVES = S::WAVES;
    constexpr int BM = S::BM;
    // One LDS array per stage (A tile, then B tile): the compiler tracks the
    // asynchronous LDS writes per array and only a few arrays individually.
    constexpr int kA = S::kABytes;
    constexpr int kStage = kA + kBBytes;
    constexpr int kStage3 = STAGES > 3 ? kStage : 16;
    __shared__ __attribute__((aligned(1024))) char s0[kStage], s1[kStage], s2[kStage], s3[kStage3];
    char* const As[4] = {s0, s1, s2, s3};
    char* const Bs[4] = {s0 + kA, s1 + kA, s2 + kA, s3 + kA};
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const int inter_p = a.inter_p;
    const int n_routed = MODE == kGateUp ? 2 * inter_p : a.hidden;  // weight rows
    const int n_shared = MODE == kGateUp ? 2 * a.shared_inter_p : a.hidden;
    TileInfo ti;
    // The last stage buffer holds the tile hand-off: the prologue never loads
    // into it, and the first load that does follows the main loop's first
    // barrier, after every wave has read its tile.
    if (!decode_tile(a, BM, blockIdx.x, (n_routed + BN - 1) / BN, (n_shared + BN - 1) / BN, MODE == kDown, ti,
                     reinterpret_cast<int*>(As[STAGES - 1]))) {
        return;
    }
    const bool shared = ti.g >= a.experts;
    const int width_p = shared ? a.shared_inter_p : inter_p;
    const int n_rows = shared ? n_shared : n_routed;
    const int K = MODE == kGateUp ? a.hidden_p : width_p;
    // act16: routed panels [T*K, Ip], then the shared expert's panels [T, Sp].
    const int64_t TK = a.tokens * a.top_k;
    const int64_t act_rows = shared ? a.tokens : TK;
    const int64_t act_slot0 = shared ? 0 : ti.slot0;
    _Float16* const act_base = a.act16 + (shared ? TK * static_cast<int64_t>(inter_p) : 0);

    // Rows this lane loads: A block q covers rows 16 (WAVES q + wave) + lane / 4,
    // B block q likewise over the 256 B rows.  The chunk follows the permutation.
    const int chunk = (lane & 3) ^ row_swizzle(lane >> 2);  // the lane's row is 16 k + lane / 4
    const _Float16* pa[S::kALoads];
    const _Float16* pb[S::kBLoads];
    // Halves between consecutive K panels of each operand.
    const int64_t a_step = (MODE == kGateUp ? a.tokens : act_rows) * kPanel;
    const int64_t b_step = static_cast<int64_t>(n_rows) * kPanel;
#pragma unroll
    for (int q = 0; q < S::kALoads; ++q) {
        const int r = 16 * (WAVES * q + wave) + (lane >> 2);
        int m = ti.mt * BM + r;
        m = m < ti.rows ? m : ti.rows - 1;  // padding rows repeat the last row; never stored
        if (MODE == kGateUp) {
            const int64_t token = shared ? m : a.rb.perm[ti.slot0 + m] / a.top_k;
            pa[q] = a.x16 + token * kPanel + chunk * 8;
        } else {
            pa[q] = act_base + (act_slot0 + m) * kPanel + chunk * 8;
        }
    }
    const _Float16* const wbase = MODE == kGateUp ? a.groups.gu_h[ti.g] : a.groups.down_h[ti.g];
#pragma unroll
    for (int q = 0; q < S::kBLoads; ++q) {
        const int r = 16 * (WAVES * q + wave) + (lane >> 2);
        int row = ti.nt * BN + r;
        row = row < n_rows ? row : n_rows - 1;  // rows past the matrix: never stored
        pb[q] = wbase + static_cast<int64_t>(row) * kPanel + chunk * 8;
    }

    auto issue = [&](int ks, char* as, char* bs) {
#pragma unroll
        for (int q = 0; q < S::kALoads; ++q) {
            __builtin_amdgcn_global_load_lds((global_void*)(pa[q] + ks * a_step),
                                             (lds_void*)(as + (WAVES * q + wave) * 1024), 16, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < S::kBLoads; ++q) {
            __builtin_amdgcn_global_load_lds((global_void*)(pb[q] + ks * b_step),
                                             (lds_void*)(bs + (WAVES * q + wave) * 1024), 16, 0, 0);
        }
    };

    floatx16 acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            acc[i][j] = floatx16{};
        }
    }
    auto compute = [&](const char* as, const char* bs) {
#pragma unroll
        for (int kk = 0; kk < BK / 16; ++kk) {
            const int c = 2 * kk + (lane >> 5);
            half8 af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int r = wm * (32 * MI) + i * 32 + (lane & 31);
                af[i] = *reinterpret_cast<const half8*>(as + chunk_offset(r, c));
            }
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int r = wn * (32 * NJ) + j * 32 + (lane & 31);
                bf[j] = *reinterpret_cast<const half8*>(bs + chunk_offset(r, c));
            }
#pragma unroll
            for (int i = 0; i < MI; ++i) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    // Stage ks lives in buffer ks % STAGES and was issued STAGES - 1 steps
    // earlier.  Before multiplying it, wait for this wave's loads of it (the
    // loads of the stages after it may remain in flight) and for its own LDS
    // reads of the previous step; the barrier then makes every wave's part
    // visible and guarantees that buffer (ks - 1) % STAGES, read in the previous
    // step, is free for stage ks + STAGES - 1.
    constexpr int L = S::kLoadsPerStage;
    const int nk = K / BK;
    auto step_full = [&](int ks, char* as, char* bs, char* an, char* bn) {
        __builtin_amdgcn_s_waitcnt(0x0070 | ((STAGES - 2) * L));  // vmcnt((STAGES - 2) L) lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        issue(ks + STAGES - 1, an, bn);
        compute(as, bs);
    };
    // The last steps: fewer stages remain in flight behind stage ks.
    auto step_tail = [&](int ks, char* as, char* bs, char* an, char* bn) {
        const int later = nk - 1 - ks;
        if (STAGES > 3 && later >= 2) {
            __builtin_amdgcn_s_waitcnt(0x0070 | (2 * L));
        } else if (later >= 1) {
            __builtin_amdgcn_s_waitcnt(0x0070 | L);
        } else {
            __builtin_amdgcn_s_waitcnt(0x0070);
        }
        __builtin_amdgcn_s_barrier();
        if (ks + STAGES - 1 < nk) {
            issue(ks + STAGES - 1, an, bn);
        }
        compute(as, bs);
    };
    // The prologue always issues STAGES - 1 stages (a stage past the end
    // reloads the last one into a buffer that is never read), so every path
    // into the main loop has the same loads in flight and the compiler's own
    // wait tracking needs no extra vmcnt(0).
#pragma unroll
    for (int d = 0; d < STAGES - 1; ++d) {
        issue(d < nk ? d : nk - 1, As[d], Bs[d]);
    }
    // Main loop: every step has STAGES - 2 stages behind it and issues one.
    int ks = 0;
    for (; ks + 2 * STAGES - 1 <= nk; ks += STAGES) {
#pragma unroll
        for (int j = 0; j < STAGES; ++j) {
            step_full(ks + j, As[j], Bs[j], As[(j + STAGES - 1) % STAGES], Bs[(j + STAGES - 1) % STAGES]);
        }
    }
#pragma unroll
    for (int j = 0; j < 2 * STAGES - 1; ++j) {
        if (ks + j < nk) {
            step_tail(ks + j, As[j % STAGES], Bs[j % STAGES], As[(j + STAGES - 1) % STAGES],
                      Bs[(j + STAGES - 1) % STAGES]);
        }
    }

    // Epilogue.  Lane l holds column n = l % 32 of each 32 x 32 block, rows
    // m = 8 (r / 4) + 4 (l / 32) + r % 4 for registers r = 0..15.
    const int n = lane & 31;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m_local = wm * (32 * MI) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const int m = ti.mt * BM + m_local;
            if (m >= ti.rows) {
                continue;
            }
            if (MODE == kGateUp) {
                // Blocks (2p, 2p + 1) are the gate and up of one 32-column group.
#pragma unroll
                for (int p = 0; p < NJ / 2; ++p) {
                    const int jcol = (ti.nt * BN) / 2 + wn * (16 * NJ) + p * 32 + n;
                    if (jcol < width_p) {
                        const float h = silu_fast(acc[i][2 * p][r], acc[i][2 * p + 1][r]);
                        act_base[panel_index(act_slot0 + m, jcol, act_rows)] = static_cast<_Float16>(h);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int h = ti.nt * BN + wn * (32 * NJ) + j * 32 + n;
                    if (h < a.hidden) {
                        a.down_out[(ti.slot0 + m) * a.hidden + h] = acc[i][j][r];
                    }
                }
            }
        }
    }
}

// Upper bound of the workgroups the tile walk needs (the kernel maps
// workgroups onto the tiles that exist and the rest return at once): per XCD
// at most ceil(routed / 8) + ceil(shared / 8) tiles.
int64_t tile_bound(const ExpertArgs& a, int BM, int nt_routed, int nt_shared) {
    const int64_t TK = a.tokens * a.top_k;
    const int64_t groups = a.experts < TK ? a.experts : TK;
    const int64_t routed = ((TK + BM - 1) / BM + groups) * nt_routed;
    const int64_t shared = a.has_shared ? (a.tokens + BM - 1) / BM * nt_shared : 0;
    return ((routed + kXcds - 1) / kXcds + (shared + kXcds - 1) / kXcds) * kXcds;
}

template <int MODE, int WM, int WN, int MI, int NJ, int STAGES>
hipError_t launch_shape(const ExpertArgs& a, hipStream_t s) {
    using S = Shape<WM, WN, MI, NJ, STAGES>;
    const int nr = MODE == kGateUp ? 2 * a.inter_p : a.hidden;
    const int ns = MODE == kGateUp ? 2 * a.shared_inter_p : a.hidden;
    const int64_t grid = tile_bound(a, S::BM, (nr + BN - 1) / BN, (ns + BN - 1) / BN);
    hipLaunchKernelGGL((mfma_grouped_kernel<MODE, WM, WN, MI, NJ, STAGES>), dim3(static_cast<unsigned>(grid)),
                       dim3(S::kThreads), 0, s, a);
    return hipGetLastError();
}

template <int MODE>
hipError_t launch(const ExpertArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.hidden_p % BK != 0 || a.inter_p % BK != 0 || (a.has_shared && a.shared_inter_p % BK != 0)) {
        return hipErrorInvalidValue;
    }
    // A layer without routed experts (the dense FFN) is one group of T rows.
    const bool narrow = a.experts > 0 ? a.tokens * a.top_k <= kNarrowRows * a.experts : a.tokens <= kNarrowRows;
    if (narrow) {
        return launch_shape<MODE, 1, 4, 2, 2, 4>(a, s);
    }
    return launch_shape<MODE, 2, 2, 2, 4, 3>(a, s);
}

}  // namespace

hipError_t launch_mfma_gateup(const ExpertArgs& a, hipStream_t s) { return launch<kGateUp>(a, s); }

hipError_t launch_mfma_down(const ExpertArgs& a, hipStream_t s) { return launch<kDown>(a, s); }

}  // namespace lm
