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
// with buffer_load_dwordx4 ... lds (no staging registers; a buffer load, unlike
// a global load to LDS, does not make the compiler wait for every LDS read);
// each wave instruction fills 1 KB of LDS, 16 rows of 64 bytes, lane l writing
// bytes [16 l, 16 l + 16).  The lane chooses which 16-byte chunk of its row it
// loads, so rows are stored in LDS with their chunks permuted (row_swizzle),
// which keeps the MFMA fragment reads free of bank conflicts.
//
// Per workgroup: a WM x WN grid of waves, each computing MI x NJ MFMA blocks of
// 32 x 32, over a BM x 256 tile (BM = 32 WM MI), K step 32, and a STAGES-deep
// pipeline: while stage k is multiplied, stages k + 1 .. k + STAGES - 2 are in
// flight, each in its own LDS array so the compiler can track the asynchronous
// writes per buffer.  Two workgroups share a CU, so one's memory waits are
// covered by the other's MFMAs.  Rows past the end of a group (tokens) or of a
// matrix (weight rows) load a clamped row and are never stored.  Two shapes:
//   128 x 256, 2 x 2 waves of 64 x 128, 3 stages (24 KB each): large groups;
//    64 x 256, 1 x 4 waves of 64 x 64, 4 stages (20 KB each): groups of a few
//    dozen rows, where the kernel streams weights and the bytes in flight
//    per CU (two workgroups x (STAGES - 1) x 16 KB of weights) set its rate.
//
// Measured alternatives, not kept (T = 2048 skewed / T = 4096 MoE layer, gate/up
// µs on one box): 256 x 256 or 192 x 256 tiles of one workgroup per CU with the
// next half step's fragments prefetched, four or five stages (1.17 against
// 0.94 PFLOP/s for this kernel's previous version on a dense 4096^3 GEMM, but
// 307-343 against 284 on the grouped layer, where one workgroup per CU cannot
// cover the memory waits of gathered token rows); those tiles for the groups
// of 96 rows and more with the small groups in a separate 64-row launch
// (343: the second launch's tail).
#include "lm_internal.h"

#include <algorithm>

namespace lm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr int BN = 256;
constexpr int BK = kPanel;                   // halves: 64-byte rows, 4 chunks of 16 B
constexpr int kRowBytes = BK * 2;
constexpr int kBBytes = BN * kRowBytes;      // 16 KB
constexpr int kXcds = 8;
constexpr int kBufferWord3 = 0x00020000;     // buffer descriptor word 3: raw 32-bit access

template <int WM, int WN, int MI, int NJ, int STAGES>
struct Shape {
    static constexpr int WAVES = WM * WN;
    static constexpr int kThreads = 64 * WAVES;
    static constexpr int BM = 32 * WM * MI;
    static constexpr int kABytes = BM * kRowBytes;
    static constexpr int kStageBytes = kABytes + kBBytes;
    static constexpr int AL = kABytes / 1024 / WAVES;  // A loads (1 KB wave instructions) per wave per stage
    static constexpr int BL = kBBytes / 1024 / WAVES;
    static constexpr int L = AL + BL;
    static constexpr int NR = MI + NJ;                 // fragment reads per half step
    static constexpr int NP = MI * NJ / 2;             // MFMA pairs per half step
    static_assert(32 * WN * NJ == BN, "the waves cover the 256 columns");
    static_assert(AL * 1024 * WAVES == kABytes && AL >= 1, "whole A instructions per wave");
    static_assert(NJ % 2 == 0, "gate/up column blocks come in pairs");
    static_assert(NR <= 2 * NP && L <= 4 * NP, "reads and loads spread over the MFMA pairs");
    static_assert(STAGES >= 3 && STAGES <= 4 && (STAGES - 2) * L < 64, "pipeline depth, vmcnt");
    static_assert(STAGES * kStageBytes <= 80 * 1024, "two workgroups per CU");
};

// Launches whose average routed group fits one 64-row tile (T k <= 64 E; a
// dense layer: T <= 64) take the 64-row shape.  Measured on V2-Lite (one MoE block, 64 experts, k 6): 8-12%
// faster from T = 8 to T = 512, 4-13% slower from T = 768 on, where groups
// span several 64-row tiles and each re-streams the expert's weights.
constexpr int64_t kNarrowRows = 64;

enum Mode { kGateUp = 0, kDown = 1 };

// Tile order inside a group: gate/up takes the M tiles of a column block
// consecutively; down takes groups of kDownGroupM M tiles, each over every
// column block (its activation tiles are read by up to 4 M tiles' worth of
// concurrent workgroups while the weight tiles stream).  Measured (MoE layer,
// down µs): T = 2048 skewed 156.6 -> 153.3, T = 4096 232.1 -> 226.5; groups of
// 2, 3, 4 or 8 for gate/up gave 270-278 against 270.
constexpr int kDownGroupM = 4;

struct TileInfo {
    int g;        // group
    int mt, nt;   // tile coordinates inside the group
    int rows;     // tokens in the group
    int64_t slot0;
};

// Maps workgroup `blk` to a tile and finds the tile's group from per-group tile
// counts (routed experts in expert order, then the shared expert); inside a
// group the M tiles of one column block are consecutive, or with group_m > 0
// groups of group_m M tiles are, each over every column block.  Workgroup b
// runs on XCD b % 8.  With
// `split` (the down projection, whose shared tiles have a longer K than the
// routed ones: 2816 against 1408 on V2-Lite) every XCD gets an equal share
// (within one) of the shared expert's tiles and of the routed tiles, each a
// contiguous range, its shared tiles first; one contiguous split of all tiles
// left the XCD that holds the shared tiles with twice the work of the others
// (measured: down at T = 2048 222 -> 179 us, T = 4096 351 -> 261 us).  Without
// it (gate/up: every tile has the same K) XCD x takes the x-th of eight
// contiguous, equal ranges of all tiles; dealing column blocks round robin over
// the XCDs instead (every XCD a share of every expert) measured 8% slower at
// T = 2048 and 5% at T = 4096, and spreading the tiles of single-tile groups
// (weight streams) evenly among each XCD's other tiles changed nothing
// (273 against 272 us for gate/up at T = 2048).  M tiles of a column block
// share one L2.
// s_info: 3 ints of LDS for the hand-off from wave 0 (the caller lends a
// pipeline buffer that no load writes before every wave has passed a later
// barrier).
__device__ bool decode_tile(const ExpertArgs& a, int BM, int64_t blk, int nt_routed, int nt_shared, bool split,
                            int group_m, TileInfo& ti, int* s_info) {
    const int lane = threadIdx.x & 63;
    if (threadIdx.x < 64) {
        auto inclusive = [&](int v) {
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int u = __shfl_up(v, o);
                if (lane >= o) {
                    v += u;
                }
            }
            return v;
        };
        // Tiles of the routed groups in expert order, 64 experts per pass.
        int64_t routed_total = 0;
        for (int g0 = 0; g0 < a.experts; g0 += 64) {
            const int g = g0 + lane;
            const int n = g < a.experts ? a.rb.counts[g] : 0;
            routed_total += __shfl(inclusive((n + BM - 1) / BM * nt_routed), 63);
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
            int64_t carry = 0;
            for (int g0 = 0; g0 < a.experts; g0 += 64) {
                const int g = g0 + lane;
                const int n = g < a.experts ? a.rb.counts[g] : 0;
                const int mts = (n + BM - 1) / BM;
                const int tiles = mts * nt_routed;
                const int incl = inclusive(tiles);
                const int64_t excl = carry + incl - tiles;
                const uint64_t hit = __ballot(tile >= excl && tile < carry + incl && tiles > 0);
                if (hit != 0) {
                    const int gl = static_cast<int>(__builtin_ctzll(hit));
                    found = g0 + gl;
                    local = static_cast<int>(tile - __shfl(excl, gl));
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
            int mt = 0, nt = 0;
            if (found >= 0) {
                if (group_m > 0) {
                    // groups of group_m M tiles, each over every column block
                    const int nts = found < a.experts ? nt_routed : nt_shared;
                    const int g = local / (group_m * nts);
                    const int in = local - g * group_m * nts;
                    const int rows_g = found_mts - g * group_m < group_m ? found_mts - g * group_m : group_m;
                    mt = g * group_m + in % rows_g;
                    nt = in / rows_g;
                } else {
                    mt = local % found_mts;
                    nt = local / found_mts;
                }
            }
            s_info[1] = mt;
            s_info[2] = nt;
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

// s_waitcnt with only vmcnt (expcnt and lgkmcnt at their maxima)
#define LM_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | 0x0F70)

// The per-wave state of a tile and the steps of its pipeline.  One type per
// kernel instantiation (MODE is a parameter): hipcc's host pass left out the
// launch stub of a second kernel whose body instantiated the same member
// functions.
template <int MODE, int WM, int WN, int MI, int NJ, int STAGES>
struct Tile {
    using Z = Shape<WM, WN, MI, NJ, STAGES>;
    __amdgpu_buffer_rsrc_t ra, rb;  // operand A (token rows / activations), operand B (weight rows)
    unsigned va[Z::AL], vb[Z::BL];  // this lane's byte offset of its row chunk in stage 0
    unsigned a_step, b_step;        // bytes between consecutive K panels
    int lane, wave, wm, wn;
    int blocks;                     // this wave's 32-row blocks holding group rows (0..MI); the rest skip their MFMAs
    half8 fa[2][MI], fb[2][NJ];     // fragments of the two half steps of a stage
    floatx16 acc[MI][NJ];

    // Load q of this wave's stage loads (A first, then B): 1 KB, 16 rows of 64
    // bytes, into LDS by a buffer load (the stage offset is a scalar).
    __device__ void load1(int ks, char* buf, int q) {
        if (q < Z::AL) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_void*)(buf + (Z::WAVES * q + wave) * 1024), 16, va[q],
                                                     static_cast<unsigned>(ks) * a_step, 0, 0);
        } else {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rb, (lds_void*)(buf + Z::kABytes + (Z::WAVES * (q - Z::AL) + wave) * 1024), 16, vb[q - Z::AL],
                static_cast<unsigned>(ks) * b_step, 0, 0);
        }
    }
    // Fragment r of half step kk: A blocks 0..MI-1, then B blocks 0..NJ-1.
    __device__ void read1(const char* buf, int kk, int r) {
        const int c = 2 * kk + (lane >> 5);
        if (r < MI) {
            fa[kk][r] = *reinterpret_cast<const half8*>(buf + chunk_offset(wm * 32 * MI + 32 * r + (lane & 31), c));
        } else {
            fb[kk][r - MI] = *reinterpret_cast<const half8*>(
                buf + Z::kABytes + chunk_offset(wn * 32 * NJ + 32 * (r - MI) + (lane & 31), c));
        }
    }
    // MFMAs t and t + 1 of half step kk (one A block: NJ is even), skipped for
    // a block past the group's rows (its accumulators are never stored).
    __device__ void mma2(int t, int kk) {
        const int i = t / NJ, j = t % NJ;
        if (i < blocks) {
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
            acc[i][j + 1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[kk][i], fb[kk][j + 1], acc[i][j + 1], 0, 0, 0);
        }
    }
    // s_waitcnt vmcnt(n L): n later stages of this wave's loads may stay in flight.
    __device__ void wait_stages(int n) {
        if (n >= 2) {
            LM_WAIT_VM(2 * Z::L);
        } else if (n == 1) {
            LM_WAIT_VM(Z::L);
        } else {
            LM_WAIT_VM(0);
        }
    }
    // Stage ks: wait for this wave's loads of it (`behind` later stages stay in
    // flight), barrier (every wave's loads visible; the buffer of stage ks - 1,
    // which the loads of stage ks + STAGES - 1 overwrite, read by every wave),
    // the first half step's fragments, then its MFMAs with the second half
    // step's fragment reads and the stage's loads between them, then the second
    // half step's MFMAs with the remaining loads.  With one read or load
    // between two MFMAs the wave's MFMA issue never waits for a run of memory
    // instructions to be accepted (measured on a dense 4096^3 GEMM: 1,150 cycles
    // per stage against 1,561 with the loads and reads issued in runs).
    __device__ void stage(int ks, const char* cur, char* tgt, bool issue, int behind) {
        wait_stages(behind);
        __builtin_amdgcn_s_barrier();
#pragma unroll
        for (int r = 0; r < Z::NR; ++r) {
            read1(cur, 0, r);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < 2 * Z::NP; ++p) {
            if (p < Z::NP) {
#pragma unroll
                for (int r = 2 * p; r < 2 * p + 2; ++r) {
                    if (r < Z::NR) {
                        read1(cur, 1, r);
                    }
                }
            }
#pragma unroll
            for (int q = p * Z::L / (2 * Z::NP); q < (p + 1) * Z::L / (2 * Z::NP); ++q) {
                if (issue) {
                    load1(ks + STAGES - 1, tgt, q);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            mma2(2 * (p % Z::NP), p / Z::NP);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

template <int MODE, int WM, int WN, int MI, int NJ, int STAGES>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(2, 2))) void mfma_grouped_kernel(
    ExpertArgs a) {
    using Z = Shape<WM, WN, MI, NJ, STAGES>;
    constexpr int BM = Z::BM;
    // One LDS array per stage: the compiler tracks the asynchronous LDS writes
    // per array.
    constexpr int kStage3 = STAGES > 3 ? Z::kStageBytes : 16;
    __shared__ __attribute__((aligned(1024))) char s0[Z::kStageBytes], s1[Z::kStageBytes], s2[Z::kStageBytes],
        s3[kStage3];
    char* const bufs[4] = {s0, s1, s2, s3};
    Tile<MODE, WM, WN, MI, NJ, STAGES> t;
    t.lane = threadIdx.x & 63;
    t.wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    t.wm = t.wave / WN;
    t.wn = t.wave % WN;
    const int lane = t.lane, wave = t.wave;

    const int inter_p = a.inter_p;
    const int n_routed = MODE == kGateUp ? 2 * inter_p : a.hidden;  // weight rows
    const int n_shared = MODE == kGateUp ? 2 * a.shared_inter_p : a.hidden;
    TileInfo ti;
    // The last stage buffer holds the tile hand-off: the prologue never loads
    // into it, and its first load follows the first stage's barrier, after
    // every wave has read its tile.  A split K multiplies the shared group's
    // column blocks: block nt + c * blocks is chunk c of column block nt.
    const int nt_shared = (n_shared + BN - 1) / BN;
    const int ksplit = MODE == kDown && a.ksplit > 1 ? a.ksplit : 1;
    if (!decode_tile(a, BM, blockIdx.x, (n_routed + BN - 1) / BN, nt_shared * ksplit, MODE == kDown,
                     MODE == kDown ? kDownGroupM : 0, ti, reinterpret_cast<int*>(bufs[STAGES - 1]))) {
        return;
    }
    int kc = 0;
    if (ksplit > 1) {
        kc = ti.nt / nt_shared;
        ti.nt -= kc * nt_shared;
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

    // Operand A: token rows (gate/up, gathered through the permutation) or the
    // slots' activations (down); operand B: the group's weight rows.  Lane l of
    // a load covers row 16 k + l / 4 and loads the chunk of it that the row's
    // LDS swizzle puts at byte 16 (l % 4) of the row.  Rows past the end of a
    // group (tokens) or of a matrix (weight rows) load a clamped row and are
    // never stored.  32-bit offsets: the launcher checks the operand sizes.
    const int chunk = (lane & 3) ^ row_swizzle(lane >> 2);
    const _Float16* const a_base = MODE == kGateUp ? a.x16 : act_base;
    const int64_t a_rows = MODE == kGateUp ? a.tokens : act_rows;
    t.ra = __builtin_amdgcn_make_buffer_rsrc((void*)a_base, 0, static_cast<int>(a_rows * K * 2), kBufferWord3);
    const _Float16* const wbase = MODE == kGateUp ? a.groups.gu_h[ti.g] : a.groups.down_h[ti.g];
    t.rb = __builtin_amdgcn_make_buffer_rsrc((void*)wbase, 0, static_cast<int>(static_cast<int64_t>(n_rows) * K * 2),
                                             kBufferWord3);
#pragma unroll
    for (int q = 0; q < Z::AL; ++q) {
        int m = ti.mt * BM + 16 * (Z::WAVES * q + wave) + (lane >> 2);
        m = m < ti.rows ? m : ti.rows - 1;  // padding rows repeat the last row; never stored
        int64_t row;
        if (MODE == kGateUp) {
            row = shared ? m : a.rb.perm[ti.slot0 + m] / a.top_k;
        } else {
            row = act_slot0 + m;
        }
        t.va[q] = static_cast<unsigned>((row * kPanel + chunk * 8) * 2);
    }
#pragma unroll
    for (int q = 0; q < Z::BL; ++q) {
        int n = ti.nt * BN + 16 * (Z::WAVES * q + wave) + (lane >> 2);
        n = n < n_rows ? n : n_rows - 1;  // rows past the matrix: never stored
        t.vb[q] = static_cast<unsigned>((static_cast<int64_t>(n) * kPanel + chunk * 8) * 2);
    }
    t.a_step = static_cast<unsigned>(a_rows * kRowBytes);
    t.b_step = static_cast<unsigned>(n_rows) * kRowBytes;
    // this tile's K stages [k0, k0 + nk): all of K, or chunk kc of the split
    const int nk_all = K / BK;
    const int kchunk = (nk_all + ksplit - 1) / ksplit;
    const int k0 = kc * kchunk;
    const int nk = nk_all - k0 < kchunk ? nk_all - k0 : kchunk;  // >= 1: the launcher's choice of ksplit
#pragma unroll
    for (int q = 0; q < Z::AL; ++q) {
        t.va[q] += static_cast<unsigned>(k0) * t.a_step;
    }
#pragma unroll
    for (int q = 0; q < Z::BL; ++q) {
        t.vb[q] += static_cast<unsigned>(k0) * t.b_step;
    }
    {
        const int left = ti.rows - (ti.mt * BM + t.wm * 32 * MI);
        t.blocks = __builtin_amdgcn_readfirstlane(left <= 0 ? 0 : (left >= 32 * MI ? MI : (left + 31) / 32));
    }
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            t.acc[i][j] = floatx16{};
        }
    }
    // Stages 0 .. STAGES - 2 in flight before the first stage; stage ks lives in
    // buffer ks % STAGES and the loads of stage ks + STAGES - 1 go to buffer
    // (ks - 1) % STAGES.  A K shorter than STAGES - 1 stages reloads the last
    // stage into buffers that are never read, so every path has the same loads
    // in flight.
#pragma unroll
    for (int d = 0; d < STAGES - 1; ++d) {
#pragma unroll
        for (int q = 0; q < Z::L; ++q) {
            t.load1(d < nk ? d : nk - 1, bufs[d], q);
        }
    }
    int ks = 0;
    for (; ks + 2 * STAGES - 1 <= nk; ks += STAGES) {
#pragma unroll
        for (int j = 0; j < STAGES; ++j) {
            t.stage(ks + j, bufs[j], bufs[(j + STAGES - 1) % STAGES], true, STAGES - 2);
        }
    }
#pragma unroll
    for (int j = 0; j < 2 * STAGES - 1; ++j) {
        const int kj = ks + j;
        if (kj < nk) {
            const int later = nk - 1 - kj;
            t.stage(kj, bufs[j % STAGES], bufs[(j + STAGES - 1) % STAGES], kj + STAGES - 1 < nk,
                    later < STAGES - 2 ? later : STAGES - 2);
        }
    }

    // Epilogue.  Lane l holds column n = l % 32 of each 32 x 32 block, rows
    // m = 8 (r / 4) + 4 (l / 32) + r % 4 for registers r = 0..15.
    const int n = lane & 31;
#pragma unroll
    for (int i = 0; i < MI; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = ti.mt * BM + t.wm * (32 * MI) + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (m >= ti.rows) {
                continue;
            }
            if (MODE == kGateUp) {
                // Blocks (2p, 2p + 1) are the gate and up of one 32-column group.
#pragma unroll
                for (int p = 0; p < NJ / 2; ++p) {
                    const int jcol = (ti.nt * BN) / 2 + t.wn * (16 * NJ) + p * 32 + n;
                    if (jcol < width_p) {
                        const float h = silu_fast(t.acc[i][2 * p][r], t.acc[i][2 * p + 1][r]);
                        act_base[panel_index(act_slot0 + m, jcol, act_rows)] = static_cast<_Float16>(h);
                    }
                }
            } else {
                float* const dst = ksplit > 1 ? a.partial + static_cast<int64_t>(kc) * a.tokens * a.hidden : a.down_out;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const int h = ti.nt * BN + t.wn * (32 * NJ) + j * 32 + n;
                    if (h < a.hidden) {
                        dst[(ti.slot0 + m) * a.hidden + h] = t.acc[i][j][r];
                    }
                }
            }
        }
    }
}
#undef LM_WAIT_VM

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
    const int ksplit = MODE == kDown && a.ksplit > 1 ? a.ksplit : 1;
    const int64_t grid = tile_bound(a, S::BM, (nr + BN - 1) / BN, (ns + BN - 1) / BN * ksplit);
    hipLaunchKernelGGL((mfma_grouped_kernel<MODE, WM, WN, MI, NJ, STAGES>), dim3(static_cast<unsigned>(grid)),
                       dim3(S::kThreads), 0, s, a);
    return hipGetLastError();
}

// Operands the kernels' 32-bit buffer offsets reach: the fp16 token copy
// [T, Hp], the activations [T K Ip + T Sp] and the widest gate/up matrix.
bool offsets_fit(const ExpertArgs& a) {
    const int64_t limit = 0x7fffffff;
    const int64_t widest = a.inter_p > a.shared_inter_p ? a.inter_p : a.shared_inter_p;
    const int64_t TK = a.tokens * a.top_k;
    return a.tokens * a.hidden_p * 2 <= limit && (TK * a.inter_p + a.tokens * a.shared_inter_p) * 2 <= limit &&
           2 * widest * a.hidden_p * 2 <= limit && static_cast<int64_t>(a.hidden) * widest * 2 <= limit;
}

template <int MODE>
hipError_t launch(const ExpertArgs& a, hipStream_t s) {
    if (a.tokens <= 0) {
        return hipSuccess;
    }
    if (a.hidden_p % BK != 0 || a.inter_p % BK != 0 || (a.has_shared && a.shared_inter_p % BK != 0) ||
        !offsets_fit(a)) {
        return hipErrorInvalidValue;
    }
    // A layer without routed experts (the dense FFN) is one group of T rows.
    const bool narrow = a.experts > 0 ? a.tokens * a.top_k <= kNarrowRows * a.experts : a.tokens <= kNarrowRows;
    if (narrow) {
        return launch_shape<MODE, 1, 4, 2, 2, 4>(a, s);
    }
    return launch_shape<MODE, 2, 2, 2, 4, 3>(a, s);
}

// out[i] = (accumulate ? out[i] : 0) + (p_0[i] + p_1[i] + ... + p_{n-1}[i]), the
// chunks in order.
__global__ __launch_bounds__(256) void splitk_sum_kernel(const float* __restrict__ partial, float* __restrict__ out,
                                                         int64_t count, int32_t chunks, int32_t accumulate) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (i >= count) {
        return;
    }
    float sum = partial[i];
    for (int c = 1; c < chunks; ++c) {
        sum = sum + partial[c * count + i];
    }
    out[i] = accumulate ? out[i] + sum : sum;
}

}  // namespace

hipError_t launch_mfma_gemm(const _Float16* a16, const _Float16* const* w, float* out, int64_t M, int32_t N, int32_t Kp,
                            int32_t accumulate, float* scratch, int64_t scratch_floats, hipStream_t s) {
    if (M <= 0 || N <= 0) {
        return hipSuccess;
    }
    if (Kp <= 0 || Kp % BK != 0 || (accumulate && scratch_floats < M * N)) {
        return hipErrorInvalidValue;
    }
    ExpertArgs ea{};
    ea.groups.down_h = w;
    ea.groups.gu_h = w;
    ea.act16 = const_cast<_Float16*>(a16);
    ea.down_out = out;
    ea.tokens = M;
    ea.hidden = N;
    ea.hidden_p = static_cast<int32_t>(round_up(N, kPanel));
    ea.experts = 0;
    ea.top_k = 0;
    ea.inter_p = 0;
    ea.shared_inter_p = Kp;
    ea.has_shared = 1;
    // Split K while the tiles fill less than half of the workgroup slots (two
    // per CU), keeping at least 8 stages per chunk and at most 4 chunks.
    const int64_t bm = M <= kNarrowRows ? 64 : 128;
    const int64_t tiles = (M + bm - 1) / bm * ((N + BN - 1) / BN);
    const int nk = Kp / BK;
    int ks = 1;
    if (tiles < 256) {
        ks = static_cast<int>(std::min<int64_t>({(256 + tiles - 1) / tiles, 4, nk / 8}));
        ks = ks < 1 ? 1 : ks;
        const int chunk = (nk + ks - 1) / ks;
        ks = (nk + chunk - 1) / chunk;  // every chunk holds at least one stage
        if (static_cast<int64_t>(ks) * M * N > scratch_floats) {
            ks = 1;
        }
    }
    const bool via_scratch = ks > 1 || accumulate;
    if (via_scratch) {
        ea.down_out = scratch;
        ea.ksplit = ks;
        ea.partial = scratch;
    }
    hipError_t e = launch<kDown>(ea, s);
    if (e != hipSuccess || !via_scratch) {
        return e;
    }
    const int64_t count = M * N;
    hipLaunchKernelGGL(splitk_sum_kernel, dim3(static_cast<unsigned>((count + 255) / 256)), dim3(256), 0, s, scratch,
                       out, count, ks, accumulate);
    return hipGetLastError();
}

namespace {
// The group table of launch_mfma_heads: every head a group of `rows` rows.
__global__ __launch_bounds__(64) void heads_table_kernel(int32_t* counts, int32_t* offsets, const _Float16** ptrs,
                                                         const _Float16* w16, int64_t w_stride, int32_t heads,
                                                         int32_t rows) {
    const int g = blockIdx.x * 64 + threadIdx.x;
    if (g < heads) {
        counts[g] = rows;
        offsets[g] = g * rows;
        ptrs[g] = w16 + g * w_stride;
    } else if (g == heads) {
        offsets[g] = heads * rows;
    }
}
}  // namespace

hipError_t launch_mfma_heads(const _Float16* a16, const _Float16* w16, int64_t w_stride, float* out, int32_t heads,
                             int64_t rows, int32_t N, int32_t Kp, void* meta, hipStream_t s) {
    if (rows <= 0 || heads <= 0 || N <= 0) {
        return hipSuccess;
    }
    if (Kp <= 0 || Kp % BK != 0 || heads * rows > 0x7fffffff) {
        return hipErrorInvalidValue;
    }
    int32_t* const counts = static_cast<int32_t*>(meta);
    int32_t* const offsets = counts + heads;
    const _Float16** const ptrs =
        reinterpret_cast<const _Float16**>(static_cast<char*>(meta) + round_up(4 * (2 * heads + 1), 8));
    hipLaunchKernelGGL(heads_table_kernel, dim3(static_cast<unsigned>(heads / 64 + 1)), dim3(64), 0, s, counts,
                       offsets, ptrs, w16, w_stride, heads, static_cast<int32_t>(rows));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return e;
    }
    ExpertArgs ea{};
    ea.groups.down_h = ptrs;
    ea.rb.counts = counts;
    ea.rb.offsets = offsets;
    ea.act16 = const_cast<_Float16*>(a16);
    ea.down_out = out;
    ea.tokens = rows;
    ea.top_k = heads;  // the kernel's routed rows: tokens * top_k = every head's rows
    ea.experts = heads;
    ea.hidden = N;
    ea.hidden_p = static_cast<int32_t>(round_up(N, kPanel));
    ea.inter_p = Kp;
    ea.shared_inter_p = 0;
    ea.has_shared = 0;
    return launch<kDown>(ea, s);
}

hipError_t launch_mfma_gateup(const ExpertArgs& a, hipStream_t s) { return launch<kGateUp>(a, s); }

hipError_t launch_mfma_down(const ExpertArgs& a, hipStream_t s) { return launch<kDown>(a, s); }

}  // namespace lm
