// k_attn.hip -- multi-head latent attention over a resident KV cache.
//
// Reference: Attention::forward (src/Attention.cpp:22-103), RotaryEmbedding::
// apply (src/Rope.cpp:96-118), KvCache (include/KvCache.hpp, src/KvCache.cpp)
// and gemm::{dot, softmax, axpy, rms_norm} (src/Gemm.cpp:183-231).  The
// projections run through the LM head's bit-exact matvec (k_head.hip); this
// file holds everything between them, for T tokens at once:
//
//   rope_query     each head's rotary channels of q, in place
//   kv_prep        RMSNorm of the latent's first kv_lora_rank channels, the
//                  rotary key tail rotated and stored in the cache
//   kv_append      kv_b_proj's [key_nope | value] per head into the cache
//   scores         scale * (dot(q_nope, k_nope) + dot(q_rope, k_rope)) for every
//                  (token, head, cached key) the token may see
//   softmax_rows   gemm::softmax per (token, head) row
//   context        gemm::axpy over the cached values, in token order
//
// Cache layout in HBM, per layer, fp32 (capacity C tokens):
//   key_nope  [heads][qk_nope][C]   keys of one (head, channel) contiguous, so
//                                   the score lanes (one key each) read coalesced
//   key_rope  [qk_rope][C]          the rotary key, shared by the heads
//   value     [heads][C][v_head]    one token's values of a head contiguous, so
//                                   the context lanes (one channel each) read
//                                   coalesced while walking the tokens in order
//
// Every sum keeps LiteMind's order: the score dots add rounded products left to
// right (a fused tail past the last multiple of four, as GCC's vector loop
// leaves it), the softmax total is one left-to-right chain per row, and each
// context channel is one fused chain over the cached tokens.  Those chains are
// sequential by definition; the kernels parallelise across them (heads,
// channels, tokens, keys), never within one.
#include "lm_internal.h"

#include <algorithm>

namespace lm {
namespace {

constexpr int kKeyTile = 256;   // keys per score block (one per lane)
constexpr int kQueries = 8;     // tokens per score / context block when T > 1
constexpr int kChunk = 1024;    // probabilities staged in LDS per context step (T > 1)

// RotaryEmbedding::apply on one channel pair: the first output is
// even*cos - odd*sin and the second odd*cos + even*sin, each contracted to one
// fused multiply-add whose addend is the other product rounded (GCC's
// contraction of the reference's expressions).
__device__ inline void rotate_pair(float e, float o, float c, float s, float& lo, float& hi) {
    const float os = o * s;
    const float es = e * s;
    lo = __builtin_fmaf(e, c, -os);
    hi = __builtin_fmaf(o, c, es);
}

// q [T, heads, qk_nope + qk_rope]: each head's rotary channels at position
// pos0 + t (src/Attention.cpp:45-48).  One wave per (token, head); the pair
// values are read before any is written (the rotation permutes channels).
__global__ __launch_bounds__(64) void rope_query_kernel(float* q, int32_t heads, int32_t nope, int32_t rope,
                                                        const float* __restrict__ cos_t,
                                                        const float* __restrict__ sin_t, int64_t pos0,
                                                        int64_t max_positions) {
    const int64_t t = blockIdx.x / heads;
    const int h = static_cast<int>(blockIdx.x - t * heads);
    const int64_t pos = pos0 + t;
    if (pos >= max_positions) {
        return;  // RotaryEmbedding::apply leaves positions past its table alone
    }
    const int half = rope / 2;
    float* v = q + (t * heads + h) * static_cast<int64_t>(nope + rope) + nope;
    const float* c = cos_t + pos * half;
    const float* s = sin_t + pos * half;
    float lo[2], hi[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = threadIdx.x + 64 * k;
        if (i < half) {
            rotate_pair(v[2 * i], v[2 * i + 1], c[i], s[i], lo[k], hi[k]);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = threadIdx.x + 64 * k;
        if (i < half) {
            v[i] = lo[k];
            v[i + half] = hi[k];
        }
    }
}

// One token per block (src/Attention.cpp:54-56, :75): kvn[t] = rms_norm of the
// latent's first `rank` channels (gemm::rms_norm: squares summed in double,
// inverse = float(1 / sqrt(mean + eps)), x * inverse * weight), and the rotary
// tail rotated at pos0 + t into the cache's key_rope column slot0 + t.
__global__ __launch_bounds__(256) void kv_prep_kernel(const float* __restrict__ lat, const float* __restrict__ norm_w,
                                                      float* __restrict__ kvn, float* __restrict__ key_rope,
                                                      int32_t rank, int32_t rope, int64_t cap, int64_t slot0,
                                                      const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                      int64_t pos0, int64_t max_positions, float eps) {
    __shared__ double part[4];
    const int64_t t = blockIdx.x;
    const float* row = lat + t * static_cast<int64_t>(rank + rope);
    const float inverse = rms_inverse_256(row, rank, eps, part);
    for (int c = threadIdx.x; c < rank; c += 256) {
        const float scaled = row[c] * inverse;
        kvn[t * rank + c] = scaled * norm_w[c];
    }
    const int half = rope / 2;
    const int64_t pos = pos0 + t;
    const int64_t slot = slot0 + t;
    const float* tail = row + rank;
    for (int i = threadIdx.x; i < half; i += 256) {
        const float e = tail[2 * i];
        const float o = tail[2 * i + 1];
        if (pos < max_positions) {
            float lo, hi;
            rotate_pair(e, o, cos_t[pos * half + i], sin_t[pos * half + i], lo, hi);
            key_rope[static_cast<int64_t>(i) * cap + slot] = lo;
            key_rope[static_cast<int64_t>(i + half) * cap + slot] = hi;
        } else {
            key_rope[static_cast<int64_t>(2 * i) * cap + slot] = e;
            key_rope[static_cast<int64_t>(2 * i + 1) * cap + slot] = o;
        }
    }
}

// kvx [T, heads, qk_nope + v_head] (kv_b_proj's output) into the cache at
// slots slot0 .. slot0 + T - 1 (src/Attention.cpp:66-74).  One thread per
// element, channel fastest.
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ kvx, float* __restrict__ key_nope,
                                                        float* __restrict__ value, int32_t heads, int32_t nope,
                                                        int32_t vh, int64_t cap, int64_t slot0, int64_t total) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= total) {
        return;
    }
    const int width = nope + vh;
    const int64_t th = i / width;  // token * heads + head
    const int j = static_cast<int>(i - th * width);
    const int64_t t = th / heads;
    const int h = static_cast<int>(th - t * heads);
    const int64_t slot = slot0 + t;
    const float v = kvx[i];
    if (j < nope) {
        key_nope[(static_cast<int64_t>(h) * nope + j) * cap + slot] = v;
    } else {
        value[(static_cast<int64_t>(h) * cap + slot) * vh + (j - nope)] = v;
    }
}

// One token (decode): the query projection's rows as matvec_one_kernel forms
// them (two rows per wave, 32 lanes each), then rope_query_kernel's step on
// them before they are stored: rows 2k and 2k + 1 of a wave are a rotary pair
// when nope is even, so each half takes the other's total by one shuffle and
// stores its own output (the even one at nope + i, the odd one at nope + half
// + i).  Positions at or past the table store the rows as they are.
// Rows past the query's (rows2 of them, from w2 into out2) are a second
// projection of the same input with no rotary step: kv_a's, in the same launch.
// With NORM (in_dim <= 2048) x is the raw hidden state: each thread loads its
// rms_norm_kernel elements once, the workgroup forms the inverse from them in
// that kernel's order and writes (x * inverse) * norm_w into LDS, which the
// dot products then read.
template <bool NORM>
__global__ __launch_bounds__(256) void query_rope_one_kernel(const uint16_t* __restrict__ w,
                                                             const float* __restrict__ x, float* __restrict__ q,
                                                             int64_t rows, int32_t in_dim, int32_t nope,
                                                             int32_t rope, const float* __restrict__ cos_t,
                                                             const float* __restrict__ sin_t, int64_t pos,
                                                             int64_t max_positions, const uint16_t* __restrict__ w2,
                                                             float* __restrict__ out2, int64_t rows2,
                                                             const float* __restrict__ norm_w, float eps) {
    const int lane = threadIdx.x & 63;
    const int c = lane & 31;
    const int64_t row_all = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
    const bool second = row_all >= rows;  // uniform over each half wave (rows is even)
    const int64_t row = second ? row_all - rows : row_all;
    const bool live = second ? row < rows2 : true;
    const uint16_t* wr = second ? w2 + (live ? row : rows2 - 1) * in_dim : w + row * in_dim;
    float total;
    if constexpr (NORM) {
        __shared__ __align__(16) float xs[2048];
        __shared__ double part[4];
        float v[8], nw[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = static_cast<int>(threadIdx.x) + 256 * u;
            const int ec = e < in_dim ? e : in_dim - 1;  // unconditional loads
            v[u] = x[ec];
            nw[u] = norm_w[ec];
        }
        const float inverse = rms_inverse_256_regs(v, in_dim, eps, part, xs);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int e = static_cast<int>(threadIdx.x) + 256 * u;
            if (e < in_dim) {
                const float scaled = v[u] * inverse;
                xs[e] = scaled * nw[u];
            }
        }
        lds_barrier();
        total = dot_bf16_lanes32(wr, [&](int e) { return xs[e]; }, in_dim, c);
    } else {
        total = dot_bf16_lanes32(wr, [&](int e) { return x[e]; }, in_dim, c);
    }
    const float other = __shfl_xor(total, 32);  // the pair partner's total
    if (!live || c != 0) {
        return;
    }
    if (second) {
        out2[row] = total;
        return;
    }
    const int qk = nope + rope;
    const int64_t head = row / qk;
    const int d = static_cast<int>(row - head * qk);
    if (d < nope || pos >= max_positions) {
        q[row] = total;
        return;
    }
    const int half = rope / 2;
    const int i = (d - nope) >> 1;
    const bool even = ((d - nope) & 1) == 0;
    float lo, hi;
    rotate_pair(even ? total : other, even ? other : total, cos_t[pos * half + i], sin_t[pos * half + i], lo, hi);
    float* v = q + head * qk + nope;
    if (even) {
        v[i] = lo;
    } else {
        v[i + half] = hi;
    }
}

// One token: kv_prep_kernel, kv_b's projection of the normalised latent and
// kv_append_kernel in one launch.  Every workgroup forms the latent's inverse
// RMS with kv_prep_kernel's thread-strided double sum (the same value in each),
// reads the normalised inputs as (latent * inverse) * weight on the fly, and
// stores its rows straight into the cache; workgroup 0 also stores the rotary
// key.
__global__ __launch_bounds__(256) void kv_one_kernel(const uint16_t* __restrict__ w, const float* __restrict__ lat,
                                                     const float* __restrict__ norm_w, float* __restrict__ key_nope,
                                                     float* __restrict__ value, float* __restrict__ key_rope,
                                                     int32_t heads, int32_t nope, int32_t vh, int32_t rank,
                                                     int32_t rope, int64_t cap, int64_t slot,
                                                     const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                     int64_t pos, int64_t max_positions, float eps) {
    __shared__ double part[4];
    const int lane = threadIdx.x & 63;
    const int c = lane & 31;
    const int width = nope + vh;
    const int64_t rows = static_cast<int64_t>(heads) * width;
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * 2 + (lane >> 5);
    const bool live = row < rows;
    const uint16_t* wr = w + (live ? row : rows - 1) * rank;
    // the lane's first weights, requested before the norm's reduction so they
    // arrive while it runs
    uint32_t pre[kOneAhead];
    const bool use_pre = rank / 32 >= kOneAhead;
    if (use_pre) {
        pre_weights(wr, c, pre);
    }
    const float inverse = rms_inverse_256(lat, rank, eps, part);
    if (blockIdx.x == 0) {
        const int half = rope / 2;
        const float* tail = lat + rank;
        for (int i = threadIdx.x; i < half; i += 256) {
            const float e = tail[2 * i];
            const float o = tail[2 * i + 1];
            if (pos < max_positions) {
                float lo, hi;
                rotate_pair(e, o, cos_t[pos * half + i], sin_t[pos * half + i], lo, hi);
                key_rope[static_cast<int64_t>(i) * cap + slot] = lo;
                key_rope[static_cast<int64_t>(i + half) * cap + slot] = hi;
            } else {
                key_rope[static_cast<int64_t>(2 * i) * cap + slot] = e;
                key_rope[static_cast<int64_t>(2 * i + 1) * cap + slot] = o;
            }
        }
    }
    const auto xn = [&](int e) { return (lat[e] * inverse) * norm_w[e]; };
    const float total = use_pre ? dot_bf16_lanes32(wr, xn, rank, c, pre) : dot_bf16_lanes32(wr, xn, rank, c);
    if (!live || c != 0) {
        return;
    }
    const int h = static_cast<int>(row / width);
    const int j = static_cast<int>(row - static_cast<int64_t>(h) * width);
    if (j < nope) {
        key_nope[(static_cast<int64_t>(h) * nope + j) * cap + slot] = total;
    } else {
        value[(static_cast<int64_t>(h) * cap + slot) * vh + (j - nope)] = total;
    }
}

// gemm::dot's association for one term of a chain: the first count - count % 4
// products are rounded and added in order, the rest fused.
__device__ inline float dot_step(float acc, float a, float b, bool fused) {
    return fused ? __builtin_fmaf(a, b, acc) : acc + a * b;
}

// Scores S[(t * heads + h) * n_stride + key] for token t (cache slot n0 + t,
// seeing keys 0 .. n0 + t) and head h (src/Attention.cpp:83-91): one key per
// lane, KQ tokens per block sharing each key load; q rows staged in LDS.
// grid: x = key tiles, y = heads, z = token blocks of KQ.
template <int KQ>
__global__ __launch_bounds__(kKeyTile) void scores_kernel(const float* __restrict__ q,
                                                          const float* __restrict__ key_nope,
                                                          const float* __restrict__ key_rope, float* __restrict__ S,
                                                          int32_t heads, int32_t nope, int32_t rope, int64_t cap,
                                                          int64_t n0, int64_t T, int64_t n_stride, float scale) {
    extern __shared__ float qs[];  // [KQ][nope + rope]
    const int qk = nope + rope;
    const int h = blockIdx.y;
    const int64_t i0 = static_cast<int64_t>(blockIdx.z) * KQ;
    const int nq = static_cast<int>(std::min<int64_t>(KQ, T - i0));
    const int64_t n_hi = n0 + i0 + nq;  // keys the block's last token sees
    const int64_t key0 = static_cast<int64_t>(blockIdx.x) * kKeyTile;
    if (key0 >= n_hi) {
        return;  // uniform over the block
    }
    for (int j = threadIdx.x; j < KQ * qk; j += kKeyTile) {
        const int iq = j / qk;
        const int d = j - iq * qk;
        qs[j] = iq < nq ? q[((i0 + iq) * heads + h) * qk + d] : 0.0f;
    }
    __syncthreads();
    const int64_t key = key0 + threadIdx.x;
    const int64_t kc = key < n_hi ? key : n_hi - 1;  // lanes past the last key read a valid one
    const float* kn = key_nope + static_cast<int64_t>(h) * nope * cap + kc;
    const float* kr = key_rope + kc;
    float a[KQ], b[KQ];
#pragma unroll
    for (int iq = 0; iq < KQ; ++iq) {
        a[iq] = 0.0f;
        b[iq] = 0.0f;
    }
    const int nope_body = nope - nope % 4;
    for (int d = 0; d < nope; ++d) {
        const float k = kn[static_cast<int64_t>(d) * cap];
        const bool fused = d >= nope_body;
#pragma unroll
        for (int iq = 0; iq < KQ; ++iq) {
            a[iq] = dot_step(a[iq], qs[iq * qk + d], k, fused);
        }
    }
    const int rope_body = rope - rope % 4;
    for (int d = 0; d < rope; ++d) {
        const float k = kr[static_cast<int64_t>(d) * cap];
        const bool fused = d >= rope_body;
#pragma unroll
        for (int iq = 0; iq < KQ; ++iq) {
            b[iq] = dot_step(b[iq], qs[iq * qk + nope + d], k, fused);
        }
    }
#pragma unroll
    for (int iq = 0; iq < KQ; ++iq) {
        if (iq < nq && key <= n0 + i0 + iq) {
            S[((i0 + iq) * heads + h) * n_stride + key] = scale * (a[iq] + b[iq]);
        }
    }
}

// scores_kernel's sums when qk_nope and qk_rope are multiples of 16 (no fused
// tail, and whole groups): one key per lane and KQ query tokens per block, the
// key's channels taken in groups of 16 (the nope groups, then the rope groups)
// with the loads of the next two groups in flight while a group is added, so a
// lane waits for memory once per group of 16 rather than once per loop step.
// The query rows are staged in LDS and read four channels at a time.  Each
// chain keeps scores_kernel's order: products rounded, added from channel 0
// up.  grid: x = key tiles, y = heads, z = token blocks of KQ.
constexpr int kScoreGroup = 16;
// scores_tile_kernel's shape (below), and the query width up to which the
// batched kernel stages its rows in one batch of loads
constexpr int kScoreTile = 64;
constexpr int kScoreTileCh = 192;
constexpr int kScoreTileStride = kScoreTileCh + 4;  // floats per key row (16-byte aligned, banks spread)
constexpr int64_t kScoreTileMaxKeys = 1024;         // longer rows take scores_grouped_kernel<1>

template <int KQ>
__global__ __launch_bounds__(kKeyTile) void scores_grouped_kernel(const float* __restrict__ q,
                                                                  const float* __restrict__ key_nope,
                                                                  const float* __restrict__ key_rope,
                                                                  float* __restrict__ S, int32_t heads, int32_t nope,
                                                                  int32_t rope, int64_t cap, int64_t n0, int64_t T,
                                                                  int64_t n_stride, float scale) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    extern __shared__ __align__(16) float qs[];  // [KQ][nope + rope]
    const int qk = nope + rope;
    const int h = blockIdx.y;
    const int64_t i0 = static_cast<int64_t>(blockIdx.z) * KQ;
    const int nq = static_cast<int>(std::min<int64_t>(KQ, T - i0));
    const int64_t n_hi = n0 + i0 + nq;  // keys the block's last token sees
    const int64_t key0 = static_cast<int64_t>(blockIdx.x) * kKeyTile;
    if (key0 >= n_hi) {
        return;  // uniform over the block
    }
    {
        // the block's query rows, unconditional loads (tokens past the last
        // read the last) so a thread's are in flight together
        constexpr int kPerThread = (KQ * kScoreTileCh + kKeyTile - 1) / kKeyTile;
        float v[kPerThread];
#pragma unroll
        for (int u = 0; u < kPerThread; ++u) {
            const int j = static_cast<int>(threadIdx.x) + kKeyTile * u;
            const int jc = j < KQ * qk ? j : KQ * qk - 1;
            const int iq = jc / qk;
            const int64_t t = i0 + (iq < nq ? iq : nq - 1);
            v[u] = q[(t * heads + h) * qk + (jc - iq * qk)];
        }
#pragma unroll
        for (int u = 0; u < kPerThread; ++u) {
            const int j = static_cast<int>(threadIdx.x) + kKeyTile * u;
            if (j < KQ * qk) {
                qs[j] = j / qk < nq ? v[u] : 0.0f;
            }
        }
        for (int j = static_cast<int>(threadIdx.x) + kKeyTile * kPerThread; j < KQ * qk; j += kKeyTile) {
            const int iq = j / qk;  // rows wider than kScoreTileCh
            qs[j] = iq < nq ? q[((i0 + iq) * heads + h) * qk + (j - iq * qk)] : 0.0f;
        }
    }
    __syncthreads();
    const int64_t key = key0 + threadIdx.x;
    const int64_t kc = key < n_hi ? key : n_hi - 1;  // lanes past the last key read a valid one
    const float* kn = key_nope + static_cast<int64_t>(h) * nope * cap + kc;
    const float* kr = key_rope + kc;
    const int gn = nope / kScoreGroup;
    const int groups = gn + rope / kScoreGroup;
    // group g's 16 keys; groups past the last reload it (every step issues the
    // same loads, so the compiler's waits count exactly)
    auto load = [&](int g, float (&x)[kScoreGroup]) {
        g = g < groups ? g : groups - 1;
        const float* base = g < gn ? kn + static_cast<int64_t>(g) * kScoreGroup * cap
                                   : kr + static_cast<int64_t>(g - gn) * kScoreGroup * cap;
#pragma unroll
        for (int i = 0; i < kScoreGroup; ++i) {
            x[i] = base[static_cast<int64_t>(i) * cap];
        }
    };
    float a[KQ], b[KQ];
#pragma unroll
    for (int iq = 0; iq < KQ; ++iq) {
        a[iq] = 0.0f;
        b[iq] = 0.0f;
    }
    auto add = [&](int g, const float (&x)[kScoreGroup]) {
        if (g >= groups) {
            return;
        }
        const bool nope_part = g < gn;
#pragma unroll
        for (int iq = 0; iq < KQ; ++iq) {
            const f4v* q4 = reinterpret_cast<const f4v*>(qs + iq * qk + g * kScoreGroup);
            float acc = nope_part ? a[iq] : b[iq];
#pragma unroll
            for (int i = 0; i < kScoreGroup / 4; ++i) {
                const f4v w = q4[i];
                acc = acc + w.x * x[4 * i + 0];
                acc = acc + w.y * x[4 * i + 1];
                acc = acc + w.z * x[4 * i + 2];
                acc = acc + w.w * x[4 * i + 3];
            }
            if (nope_part) {
                a[iq] = acc;
            } else {
                b[iq] = acc;
            }
        }
    };
    float x0[kScoreGroup], x1[kScoreGroup], x2[kScoreGroup];
    load(0, x0);
    load(1, x1);
    for (int g = 0; g < groups; g += 3) {
        load(g + 2, x2);
        add(g, x0);
        load(g + 3, x0);
        add(g + 1, x1);
        load(g + 4, x1);
        add(g + 2, x2);
    }
#pragma unroll
    for (int iq = 0; iq < KQ; ++iq) {
        if (iq < nq && key <= n0 + i0 + iq) {
            S[((i0 + iq) * heads + h) * n_stride + key] = scale * (a[iq] + b[iq]);
        }
    }
}

// scores_grouped_kernel's sums for one query token (decode), qk_nope +
// qk_rope <= kScoreTileCh, in tiles of 64 keys: the four waves each load a
// quarter of the tile's key channels (one round trip, ~48 loads in flight per
// lane) into LDS as [key][channel], then wave 0 runs each key's two chains
// (lane = key) in scores_grouped_kernel's order, reading four channels per LDS
// read.  Four times the workgroups of the 256-key tiles, which at a few hundred
// cached tokens leave most lanes waiting on several round trips each; used up
// to kScoreTileMaxKeys keys.

__global__ __launch_bounds__(256) void scores_tile_kernel(const float* __restrict__ q,
                                                          const float* __restrict__ key_nope,
                                                          const float* __restrict__ key_rope, float* __restrict__ S,
                                                          int32_t nope, int32_t rope, int64_t cap, int64_t n,
                                                          float scale) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float ks[kScoreTile * kScoreTileStride];
    __shared__ __align__(16) float qs[kScoreTileCh];
    const int qk = nope + rope;
    const int h = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t key = static_cast<int64_t>(blockIdx.x) * kScoreTile + lane;
    const int64_t kc = key < n ? key : n - 1;  // lanes past the last key read a valid one
    if (threadIdx.x < qk) {
        qs[threadIdx.x] = q[static_cast<int64_t>(h) * qk + threadIdx.x];
    }
    const float* kn = key_nope + static_cast<int64_t>(h) * nope * cap + kc;
    const float* kr = key_rope + kc;
    // channel d of this lane's key (d < nope: the head's key_nope, else the
    // shared rotary key); wave w takes channels w, w + 4, ...
    constexpr int kPer = kScoreTileCh / 4;
    float v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int d = 4 * i + wave;
        const int dc = d < qk ? d : qk - 1;
        v[i] = dc < nope ? kn[static_cast<int64_t>(dc) * cap] : kr[static_cast<int64_t>(dc - nope) * cap];
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        ks[lane * kScoreTileStride + 4 * i + wave] = v[i];
    }
    lds_barrier();
    if (wave != 0) {
        return;
    }
    const f4v* k4 = reinterpret_cast<const f4v*>(ks + lane * kScoreTileStride);
    const f4v* q4 = reinterpret_cast<const f4v*>(qs);
    float a = 0.0f, b = 0.0f;
#pragma unroll 8
    for (int i = 0; i < nope / 4; ++i) {
        const f4v kv = k4[i];
        const f4v w = q4[i];
        a = a + w.x * kv.x;
        a = a + w.y * kv.y;
        a = a + w.z * kv.z;
        a = a + w.w * kv.w;
    }
#pragma unroll 8
    for (int i = nope / 4; i < qk / 4; ++i) {
        const f4v kv = k4[i];
        const f4v w = q4[i];
        b = b + w.x * kv.x;
        b = b + w.y * kv.y;
        b = b + w.z * kv.z;
        b = b + w.w * kv.w;
    }
    if (key < n) {
        S[static_cast<int64_t>(h) * n + key] = scale * (a + b);
    }
}

// gemm::softmax (src/Gemm.cpp:209-223) on each row (token t, head h) of S,
// n0 + t + 1 entries: the maximum, expf(s - max) in place with the total
// accumulated left to right in one chain (each chunk of 64 is added in lane
// order from the lanes' registers), then one reciprocal and a product.  One
// wave per row, four rows per block.
__global__ __launch_bounds__(256) void softmax_rows_kernel(float* S, int64_t rows, int32_t heads, int64_t n0,
                                                           int64_t n_stride) {
    // expf's 2^(i/32) table in LDS: one read in place of a select tree
    __shared__ uint64_t exp_tab[32];
    if (threadIdx.x < 32) {
        exp_tab[threadIdx.x] = exp2_table(threadIdx.x);
    }
    __syncthreads();
    const auto tab = [&](uint32_t i) { return exp_tab[i]; };
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= rows) {
        return;
    }
    const int64_t n = n0 + row / heads + 1;
    float* s = S + row * n_stride;
    // the maximum with eight loads in flight per lane (a duplicate of the last
    // score past the end leaves the maximum unchanged)
    float m = -__builtin_inff();
    for (int64_t cb = lane; cb < n; cb += 8 * 64) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t c = cb + 64 * u;
            v[u] = s[c < n ? c : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            m = fmaxf(m, v[u]);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        m = fmaxf(m, __shfl_xor(m, o));
    }
    float total = 0.0f;
    int64_t c0 = 0;
    // the next chunk's score is requested before this chunk's chain, so the
    // chain never waits for a load
    float next = lane < n ? s[lane] : 0.0f;
    for (; c0 + 64 <= n; c0 += 64) {
        const float cur = next;
        if (c0 + 64 + lane < n) {
            next = s[c0 + 64 + lane];
        }
        const float e = expf_with(cur - m, tab);
        s[c0 + lane] = e;
        const int eb = static_cast<int>(float_bits(e));
#pragma unroll
        for (int k = 0; k < 64; ++k) {
            total = total + bits_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(eb, k)));
        }
    }
    if (c0 < n) {
        const int cnt = static_cast<int>(n - c0);
        float e = 0.0f;
        if (lane < cnt) {
            e = expf_with(s[c0 + lane] - m, tab);
            s[c0 + lane] = e;
        }
        const int eb = static_cast<int>(float_bits(e));
        for (int k = 0; k < cnt; ++k) {
            total = total + bits_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(eb, k)));
        }
    }
    const float inverse = total > 0.0f ? 1.0f / total : 0.0f;
    // each lane rescales the values it wrote, eight loads in flight
    for (int64_t cb = lane; cb < n; cb += 8 * 64) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t c = cb + 64 * u;
            v[u] = s[c < n ? c : n - 1];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int64_t c = cb + 64 * u;
            if (c < n) {
                s[c] = v[u] * inverse;
            }
        }
    }
}

// softmax_rows_kernel's arithmetic for one query token (decode, T = 1), for
// one head's row of n <= kSoftmaxLds scores, by a workgroup of NT threads:
// all threads find the maximum and form expf(s - max) into e (LDS); wave 0 adds
// them left to right in one chain, reading LDS with broadcast loads a batch of
// 64 ahead (a VGPR operand: no lane-to-SGPR hand-off per step).  Returns
// 1 / total to every thread (after a barrier); e then holds the exponentials,
// zero past n up to the next multiple of 128.  red: NT / 64 floats of LDS,
// inverse_lds: one, tab: expf's 2^(i/32) table in LDS.  Its barriers order LDS
// only, so loads the caller has in flight stay in flight; after_max() runs on
// every thread once the scores are in.
constexpr int kSoftmaxLds = 8192;  // a multiple of 128

// (In two parts: softmax_row_load requests the thread's scores, so a caller
// can issue them before other loads, whose results come back after them.)
template <int NT>
constexpr int softmax_per() { return (kSoftmaxLds + NT - 1) / NT; }  // scores per thread

template <int NT>
__device__ inline void softmax_row_load(const float* s, int nn, float (&v)[softmax_per<NT>()]) {
#pragma unroll
    for (int k = 0; k < softmax_per<NT>(); ++k) {
        const int c = static_cast<int>(threadIdx.x) + NT * k;
        v[k] = c < nn ? s[c] : -__builtin_inff();
    }
}

template <int NT, class AfterMax>
__device__ inline float softmax_row_lds(const float (&v)[softmax_per<NT>()], int nn, float* e, float* red,
                                        float* inverse_lds, const uint64_t* tab, AfterMax after_max) {
    constexpr int kPer = softmax_per<NT>();
    constexpr int kW = NT / 64;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        m = fmaxf(m, v[k]);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        m = fmaxf(m, __shfl_xor(m, o));
    }
    if (lane == 0) {
        red[wave] = m;
    }
    lds_barrier();
    m = red[0];
#pragma unroll
    for (int w = 1; w < kW; ++w) {
        m = fmaxf(m, red[w]);
    }
    after_max();  // every thread, once its scores are in
    // e past n is 0 up to the next multiple of 128: adding those exact zeros to
    // the (non-negative) total changes nothing, and the chain below runs in
    // whole pairs of batches without a bounds test
    const int n64 = (nn + 127) / 128 * 128;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
        const int c = tid + NT * k;
        if (c < nn) {
            e[c] = expf_with(v[k] - m, [&](uint32_t i) { return tab[i]; });
        } else if (c < n64) {
            e[c] = 0.0f;
        }
    }
    lds_barrier();
    if (wave == 0) {
        // one batch of 64 values (16 broadcast reads) requested ahead of the
        // batch being added, so the chain does not wait for LDS; a native
        // 4-float vector, so each read stays one 16-byte LDS read (HIP's float4
        // struct is split into four)
        typedef float f4v __attribute__((ext_vector_type(4)));
        const f4v* e4 = reinterpret_cast<const f4v*>(e);
        const int nb = n64 / 64;  // even
        f4v a[16], b[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            a[u] = e4[u];
        }
        float total = 0.0f;
        auto add16 = [&](const f4v (&q)[16]) {
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                total = total + q[u].x;
                total = total + q[u].y;
                total = total + q[u].z;
                total = total + q[u].w;
            }
        };
        for (int bb = 0; bb < nb; bb += 2) {
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                b[u] = e4[(bb + 1) * 16 + u];
            }
            add16(a);
            const int na = (bb + 2 < nb ? bb + 2 : bb) * 16;
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                a[u] = e4[na + u];
            }
            add16(b);
        }
        if (lane == 0) {
            *inverse_lds = total > 0.0f ? 1.0f / total : 0.0f;
        }
    }
    lds_barrier();
    return *inverse_lds;
}

// The decode softmax as its own launch (one workgroup per head), for the
// context kernel's unfused form: P = e * (1 / total) back into S.
__global__ __launch_bounds__(256) void softmax_decode_kernel(float* S, int64_t n, int64_t n_stride) {
    __shared__ __align__(16) float e[kSoftmaxLds];
    __shared__ float red[4];
    __shared__ float inverse_lds;
    __shared__ uint64_t exp_tab[32];  // expf's 2^(i/32) table: one LDS read in place of a select tree
    if (threadIdx.x < 32) {
        exp_tab[threadIdx.x] = exp2_table(threadIdx.x);
    }
    float* s = S + static_cast<int64_t>(blockIdx.x) * n_stride;
    const int nn = static_cast<int>(n);
    float v[softmax_per<256>()];
    softmax_row_load<256>(s, nn, v);
    const float inverse = softmax_row_lds<256>(v, nn, e, red, &inverse_lds, exp_tab, [] {});
    for (int c = threadIdx.x; c < nn; c += 256) {
        s[c] = e[c] * inverse;
    }
}

// ctx[t, h, v] = sum over cached tokens j <= n0 + t, in order, of
// fma(P[t, h, j], value[h, j, v], .) from 0 (gemm::axpy per token,
// src/Attention.cpp:94-97).  One lane per value channel, KQ tokens per block
// sharing each value load; probabilities staged in LDS in chunks of kChunk
// keys and read four at a time.  The keys go in groups of 16 with the loads of
// the next two groups in flight while a group is added; only groups that reach
// the block's first token's own position test which tokens see each key.
// grid: x = heads, y = token blocks of KQ; block = v_head rounded up to 64.
template <int KQ>
__global__ __launch_bounds__(256) void context_kernel(const float* __restrict__ P, const float* __restrict__ value,
                                                      float* __restrict__ ctx, int32_t heads, int32_t vh, int64_t cap,
                                                      int64_t n0, int64_t T, int64_t n_stride) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int kG = 16;  // keys per group
    __shared__ __align__(16) float ps[KQ][kChunk];
    const int h = blockIdx.x;
    const int64_t i0 = static_cast<int64_t>(blockIdx.y) * KQ;
    const int nq = static_cast<int>(std::min<int64_t>(KQ, T - i0));
    const int64_t n_hi = n0 + i0 + nq;  // keys the block's last token sees
    const int64_t n_all = n0 + i0;      // keys every token of the block sees
    const int v = threadIdx.x;
    const bool live = v < vh;
    const float* vp = value + static_cast<int64_t>(h) * cap * vh + (live ? v : 0);
    float acc[KQ];
#pragma unroll
    for (int iq = 0; iq < KQ; ++iq) {
        acc[iq] = 0.0f;
    }
    for (int64_t c0 = 0; c0 < n_hi; c0 += kChunk) {
        const int cend = static_cast<int>(std::min<int64_t>(kChunk, n_hi - c0));
        const int ng = (cend + kG - 1) / kG;
        __syncthreads();
        // the chunk's probabilities of the block's tokens, zero where a token
        // does not see the key, up to the groups' end; the loads are
        // unconditional (keys < n_hi are inside every row; tokens past the
        // last read the last) so each thread's eight are in flight together
        for (int k = threadIdx.x; k < ng * kG; k += blockDim.x) {
            const int64_t key = c0 + k;
            const int64_t kc = key < n_hi ? key : n_hi - 1;
            float v[KQ];
#pragma unroll
            for (int iq = 0; iq < KQ; ++iq) {
                const int64_t t = i0 + (iq < nq ? iq : nq - 1);
                v[iq] = P[(t * heads + h) * n_stride + kc];
            }
#pragma unroll
            for (int iq = 0; iq < KQ; ++iq) {
                ps[iq][k] = iq < nq && key <= n0 + i0 + iq ? v[iq] : 0.0f;
            }
        }
        __syncthreads();
        // group g's 16 values; groups past the last reload it and keys past
        // the last read the last (every step issues the same loads)
        auto load = [&](int g, float (&x)[kG]) {
            g = g < ng ? g : ng - 1;
#pragma unroll
            for (int i = 0; i < kG; ++i) {
                int64_t key = c0 + kG * g + i;
                key = key < n_hi ? key : n_hi - 1;
                x[i] = vp[key * vh];
            }
        };
        auto add = [&](int g, const float (&x)[kG]) {
            if (g >= ng) {
                return;
            }
            const int64_t kfirst = c0 + kG * g;
            if (kfirst + kG <= n_all) {
                // every token of the block sees all 16 keys
#pragma unroll
                for (int u = 0; u < kG / 4; ++u) {
#pragma unroll
                    for (int iq = 0; iq < KQ; ++iq) {
                        const f4v p = *reinterpret_cast<const f4v*>(&ps[iq][kG * g + 4 * u]);
                        acc[iq] = __builtin_fmaf(p.x, x[4 * u + 0], acc[iq]);
                        acc[iq] = __builtin_fmaf(p.y, x[4 * u + 1], acc[iq]);
                        acc[iq] = __builtin_fmaf(p.z, x[4 * u + 2], acc[iq]);
                        acc[iq] = __builtin_fmaf(p.w, x[4 * u + 3], acc[iq]);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < kG; ++i) {
                    const int64_t rel = kfirst + i - n_all;  // token iq sees this key when rel <= iq
#pragma unroll
                    for (int iq = 0; iq < KQ; ++iq) {
                        if (rel <= iq) {
                            acc[iq] = __builtin_fmaf(ps[iq][kG * g + i], x[i], acc[iq]);
                        }
                    }
                }
            }
        };
        float x0[kG], x1[kG], x2[kG];
        load(0, x0);
        load(1, x1);
        for (int g = 0; g < ng; g += 3) {
            load(g + 2, x2);
            add(g, x0);
            load(g + 3, x0);
            add(g + 1, x1);
            load(g + 4, x1);
            add(g + 2, x2);
        }
    }
    if (live) {
#pragma unroll
        for (int iq = 0; iq < KQ; ++iq) {
            if (iq < nq) {
                ctx[((i0 + iq) * heads + h) * vh + v] = acc[iq];
            }
        }
    }
}

// The same sum for one query token (decode), T = 1: ctx[h, v] over cached
// tokens j < n in order.  One workgroup per (head, 16 value channels); lanes
// 0..15 of wave 0 run the 16 chains from LDS.  The channels' values (64 B per
// cached token) and the head's probabilities stream through a ring of
// kCtxDepth LDS slots of kCtxChunk tokens (16 KB of values) by direct-to-LDS
// buffer loads that four loader waves issue: ~119 KB in flight per workgroup, and
// the narrow groups put 128 workgroups (so 128 CUs' worth of loads) on a
// V2-Lite layer, so the stream (~7 us near 4K cached tokens) outruns the
// chains.  The chains cost ~9 cycles per token: a dependent fused multiply-add
// (~4.4 cycles) plus the wave's share of issuing three LDS reads per four
// tokens.  One slot per LDS array and the step loop unrolled over the slots,
// so the compiler knows which slot each load writes and waits only through the
// explicit vmcnt.  vh % 16 == 0.
typedef __attribute__((address_space(3))) void attn_lds_void;
// buffer descriptor word 3 for raw 32-bit buffer access on gfx950
constexpr int kBufferWord3 = 0x00020000;
constexpr int kCtxCh = 16;        // value channels per workgroup
constexpr int kCtxChunk = 256;    // cached tokens per slot
constexpr int kCtxDepth = 8;
constexpr int kCtxLoaders = 4;  // waves 1 .. 4 issue the loads, wave 0 only adds
constexpr int kCtxThreads = (kCtxLoaders + 1) * 64;
constexpr int kCtxTokPerLoad = 64 * 4 / kCtxCh;  // tokens per 1 KB value load
constexpr int kCtxDepthFused = 7;  // slots when the probability row also sits in LDS
constexpr int kCtxValueLoads = kCtxChunk / kCtxTokPerLoad / kCtxLoaders;  // per loader and chunk
static_assert(kCtxChunk % (kCtxTokPerLoad * kCtxLoaders) == 0 && kCtxChunk % (64 * kCtxLoaders) == 0,
              "even shares");
static_assert((kCtxDepth - 1) * (kCtxValueLoads + kCtxChunk / 64 / kCtxLoaders) < 64, "vmcnt immediate");

// FUSED: the softmax of the head's row of scores runs inside the launch
// (softmax_row_lds, every workgroup of the head the same) while the loader
// waves already stream the first value chunks; its probabilities stay in LDS
// (the whole row, n <= kSoftmaxLds) and the ring carries values only, in
// kCtxDepthFused slots.  Otherwise P holds the probabilities (a separate
// softmax launch) and each slot carries its chunk's share of them.
template <bool FUSED>
__global__ __launch_bounds__(kCtxThreads) void context_decode_kernel(const float* __restrict__ P,
                                                                        const float* __restrict__ value,
                                                                        float* __restrict__ ctx, int32_t vh,
                                                                        int64_t cap, int64_t n, int64_t n_stride) {
    constexpr int kDepth = FUSED ? kCtxDepthFused : kCtxDepth;
    constexpr int kLoads = kCtxValueLoads + (FUSED ? 0 : kCtxChunk / 64 / kCtxLoaders);  // per loader and chunk
    // slot = [token][16 channels] values, then (unfused) the chunk's
    // probabilities: one array per slot (separate LDS objects are what the
    // compiler's wait insertion tells apart)
    constexpr int kSlot = kCtxChunk * kCtxCh + (FUSED ? 0 : kCtxChunk);
    __shared__ __align__(16) float s0[kSlot], s1[kSlot], s2[kSlot], s3[kSlot], s4[kSlot], s5[kSlot], s6[kSlot],
        s7[FUSED ? 4 : kSlot];
    __shared__ __align__(16) float prob[FUSED ? kSoftmaxLds : 4];
    float* const ring[8] = {s0, s1, s2, s3, s4, s5, s6, s7};
    const int lane = threadIdx.x & 63;
    // wave-uniform as far as the compiler knows, so the branches on it stay
    // scalar and its wait insertion keeps track of each slot's loads
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    // workgroup b serves head b % heads, channels 16 (b / heads) ..: with the
    // heads a multiple of eight, the groups of one head (which split each
    // token's 128-byte lines between them) share an XCD and so its L2, and
    // every line is fetched from memory once
    const int heads = static_cast<int>(gridDim.x) / (vh / kCtxCh);
    const int h = static_cast<int>(blockIdx.x) % heads;
    const int c0 = (static_cast<int>(blockIdx.x) / heads) * kCtxCh;
    const float* vbase = value + static_cast<int64_t>(h) * cap * vh + c0;
    const float* prow = P + static_cast<int64_t>(h) * n_stride;  // scores (FUSED) or probabilities
    const int64_t nchunks = (n + kCtxChunk - 1) / kCtxChunk;
    // loader wave w = wave - 1's share of chunk c (clamped to the last chunk,
    // so every step issues the same count): value load i (i = w, w + 4, ...)
    // brings tokens kCtxTokPerLoad i .. + kCtxTokPerLoad - 1, lane l token
    // kCtxTokPerLoad i + l / 4 and channels 4 (l % 4) .. + 3, to [token][16];
    // probability load k (k = w, w + 4, ...) tokens 64 k .. 64 k + 63; tokens
    // past n read token n - 1 and are never used.  Wave 0 issues nothing: the
    // address arithmetic and the issue of the loads stay off the chains' wave
    // buffer loads rather than global ones: a global load to LDS counts as a
    // pending flat access, for which the compiler waits for every LDS read at
    // each use (lgkmcnt(0)) and so cannot keep the next block's reads in
    // flight.  Offsets are 32-bit: the host sends here only caches with
    // cap * vh * 4 < 2^31 bytes per head
    const __amdgpu_buffer_rsrc_t vres =
        __builtin_amdgcn_make_buffer_rsrc((void*)vbase, 0, static_cast<int>((cap * vh - c0) * 4), kBufferWord3);
    const __amdgpu_buffer_rsrc_t pres =
        __builtin_amdgcn_make_buffer_rsrc((void*)prow, 0, static_cast<int>(n * 4), kBufferWord3);
    const int lw = wave - 1;
    auto issue = [&](int64_t c, float* slot) {
        c = c < nchunks ? c : nchunks - 1;
#pragma unroll
        for (int k = 0; k < kCtxValueLoads; ++k) {
            const int i = k * kCtxLoaders + lw;
            int64_t tok = c * kCtxChunk + kCtxTokPerLoad * i + (lane >> 2);
            tok = tok < n ? tok : n - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(vres, (attn_lds_void*)(slot + i * 256), 16,
                                                     static_cast<unsigned>((tok * vh + 4 * (lane & 3)) * 4), 0, 0, 0);
        }
#pragma unroll
        for (int k = 0; k < (FUSED ? 0 : kCtxChunk / 64 / kCtxLoaders); ++k) {
            const int i = k * kCtxLoaders + lw;
            int64_t tok = c * kCtxChunk + 64 * i + lane;
            tok = tok < n ? tok : n - 1;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(pres, (attn_lds_void*)(slot + kCtxChunk * kCtxCh + 64 * i), 4,
                                                     static_cast<unsigned>(tok * 4), 0, 0, 0);
        }
    };
    auto first_chunks = [&] {
        if (wave != 0) {
#pragma unroll
            for (int d = 0; d < kDepth - 1; ++d) {
                issue(d, ring[d]);
            }
        }
    };
    if constexpr (FUSED) {
        // the head's probabilities into LDS; the first chunks are requested
        // once the scores are in (results return in issue order), and arrive
        // while the exponentials and the total are formed
        __shared__ float red[kCtxThreads / 64];
        __shared__ float inverse_lds;
        __shared__ uint64_t exp_tab[32];
        if (threadIdx.x < 32) {
            exp_tab[threadIdx.x] = exp2_table(threadIdx.x);
        }
        const int nn = static_cast<int>(n);
        float scores[softmax_per<kCtxThreads>()];
        softmax_row_load<kCtxThreads>(prow, nn, scores);
        const float inverse =
            softmax_row_lds<kCtxThreads>(scores, nn, prob, red, &inverse_lds, exp_tab, first_chunks);
        for (int t = threadIdx.x; t < nn; t += kCtxThreads) {
            prob[t] = prob[t] * inverse;
        }
        lds_barrier();
    } else {
        first_chunks();
    }
    // chunk c is in once at most the kDepth - 2 chunks issued after it are in
    // flight
    constexpr int kVm = (kDepth - 2) * kLoads;
    constexpr int kWait = 0x0070 | 0x0F00 | (kVm & 15) | ((kVm >> 4) << 14);
    const int ch = lane < kCtxCh ? lane : kCtxCh - 1;  // lanes past the group repeat its last channel
    float acc = 0.0f;
    for (int64_t cb = 0; cb < nchunks; cb += kDepth) {
        // no early exit: the loop unrolls over the slots (steps past the last
        // chunk wait and reload as the others and add nothing)
#pragma unroll
        for (int j = 0; j < kDepth; ++j) {
            const int64_t c = cb + j;
            __builtin_amdgcn_s_waitcnt(kWait);
            // every loader's share of chunk c is in; wave 0 has read the slot
            // refilled next (chunk c - 1) and used all of it
            __builtin_amdgcn_s_barrier();
            if (wave != 0) {
                issue(c + kDepth - 1, ring[(j + kDepth - 1) % kDepth]);
                continue;
            }
            const float* vs = ring[j];
            const float* ps = FUSED ? prob + c * kCtxChunk : ring[j] + kCtxChunk * kCtxCh;
            const int64_t rem = n - c * kCtxChunk;
            const int cnt = static_cast<int>(rem < kCtxChunk ? (rem > 0 ? rem : 0) : kCtxChunk);
            if (cnt == kCtxChunk) {
                // blocks of 16 tokens (8 paired value reads + 4 probability
                // reads: few enough that the wait for one block while the
                // next one's reads are in flight fits lgkmcnt's 4 bits), the
                // next block's reads issued before this block's chain
                constexpr int kBlk = 16;
                float xa[kBlk], xb[kBlk];
                float4 pa[kBlk / 4], pb[kBlk / 4];
                auto read = [&](int t0, float (&x)[kBlk], float4 (&p)[kBlk / 4]) {
#pragma unroll
                    for (int t = 0; t < kBlk; ++t) {
                        x[t] = vs[(t0 + t) * kCtxCh + ch];
                    }
#pragma unroll
                    for (int t = 0; t < kBlk / 4; ++t) {
                        p[t] = *reinterpret_cast<const float4*>(ps + t0 + 4 * t);
                    }
                };
                auto chain = [&](const float (&x)[kBlk], const float4 (&p)[kBlk / 4]) {
#pragma unroll
                    for (int t = 0; t < kBlk / 4; ++t) {
                        acc = __builtin_fmaf(p[t].x, x[4 * t + 0], acc);
                        acc = __builtin_fmaf(p[t].y, x[4 * t + 1], acc);
                        acc = __builtin_fmaf(p[t].z, x[4 * t + 2], acc);
                        acc = __builtin_fmaf(p[t].w, x[4 * t + 3], acc);
                    }
                };
                // the scheduling fences keep each block's reads ahead of the
                // previous block's chain (left to itself the scheduler sinks
                // them into it and waits for all of them at once)
                read(0, xa, pa);
#pragma unroll
                for (int t0 = 0; t0 < kCtxChunk; t0 += 2 * kBlk) {
                    read(t0 + kBlk, xb, pb);
                    __builtin_amdgcn_sched_barrier(0);
                    chain(xa, pa);
                    __builtin_amdgcn_sched_barrier(0);
                    if (t0 + 2 * kBlk < kCtxChunk) {
                        read(t0 + 2 * kBlk, xa, pa);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    chain(xb, pb);
                    __builtin_amdgcn_sched_barrier(0);
                }
            } else {
                for (int t = 0; t < cnt; ++t) {
                    acc = __builtin_fmaf(ps[t], vs[t * kCtxCh + ch], acc);
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0F00);  // vmcnt(0): the clamped reloads have landed
    if (wave == 0 && lane < kCtxCh) {
        ctx[static_cast<int64_t>(h) * vh + c0 + lane] = acc;
    }
}

// ---- attention core on MFMA (fp16 operands, fp32 accumulation) ----
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
//
// The projection path's tolerance path for batches of query tokens: per head,
// S = Q K^T and ctx = P V are GEMMs of the grouped MFMA kernel (one group per
// head), over fp16 copies of the cache in panel layout made once per call:
//   keys16    [heads][Kp rows][qk]    row j = [key_nope(h, :, j) | key_rope(:, j)]
//   values16  [heads][vh rows][Kp]    value(h, j, :) transposed, the K of P V
// with Kp = keys rounded up to 32 and zeros past the last key (P is zero
// there too, so no padding value reaches a sum).

// keys16 from the fp32 cache: workgroup (key block of 64, 32-channel panel,
// head) reads 32 channel rows of 64 keys (256 B each, coalesced), transposes
// them in LDS and writes the panel's 64 rows of 64 bytes (contiguous).
__global__ __launch_bounds__(256) void pack_keys16_kernel(const float* __restrict__ key_nope,
                                                          const float* __restrict__ key_rope,
                                                          _Float16* __restrict__ k16, int32_t nope, int32_t qk,
                                                          int64_t cap, int64_t keys, int64_t kp) {
    __shared__ float tile[32][65];
    const int tid = threadIdx.x;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * 64;
    const int p = blockIdx.y;
    const int h = blockIdx.z;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int e = tid + 256 * i;
        const int ch = e >> 6, kk = e & 63;
        const int c = p * 32 + ch;
        const int64_t j = j0 + kk;
        float v = 0.0f;
        if (j < keys) {
            v = c < nope ? key_nope[(static_cast<int64_t>(h) * nope + c) * cap + j]
                         : key_rope[static_cast<int64_t>(c - nope) * cap + j];
        }
        tile[ch][kk] = v;
    }
    __syncthreads();
    const int kk = tid >> 2, part = tid & 3;
    const int64_t j = j0 + kk;
    if (j < kp) {
        half8 out;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            out[e] = static_cast<_Float16>(tile[part * 8 + e][kk]);
        }
        _Float16* const dst = k16 + static_cast<int64_t>(h) * kp * qk + (static_cast<int64_t>(p) * kp + j) * kPanel;
        *reinterpret_cast<half8*>(dst + part * 8) = out;
    }
}

// values16 from the fp32 cache: workgroup (panel of 32 keys, head) reads the
// 32 keys' value rows (coalesced over channels), transposes them in LDS
// (32 x (vh + 1) floats, dynamic) and writes vh rows of 64 bytes (contiguous).
__global__ __launch_bounds__(256) void pack_values16_kernel(const float* __restrict__ value,
                                                            _Float16* __restrict__ v16, int32_t vh, int64_t cap,
                                                            int64_t keys, int64_t kp) {
    extern __shared__ float vtile[];  // [32][vh + 1]
    const int tid = threadIdx.x;
    const int64_t j0 = static_cast<int64_t>(blockIdx.x) * kPanel;
    const int h = blockIdx.y;
    const int stride = vh + 1;
    for (int e = tid; e < 32 * vh; e += 256) {
        const int kk = e / vh, c = e - kk * vh;
        const int64_t j = j0 + kk;
        vtile[kk * stride + c] = j < keys ? value[(static_cast<int64_t>(h) * cap + j) * vh + c] : 0.0f;
    }
    __syncthreads();
    _Float16* const dst = v16 + static_cast<int64_t>(h) * vh * kp + static_cast<int64_t>(blockIdx.x) * vh * kPanel;
    for (int e = tid; e < 4 * vh; e += 256) {
        const int c = e >> 2, part = e & 3;
        half8 out;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            out[i] = static_cast<_Float16>(vtile[(part * 8 + i) * stride + c]);
        }
        *reinterpret_cast<half8*>(dst + c * kPanel + part * 8) = out;
    }
}

// q [T][heads][qk] fp32 -> q16 [heads T rows][qk] panels, row h T + t (the
// query rows of head h are group h).  Thread i converts 8 channels.
__global__ __launch_bounds__(256) void pack_queries16_kernel(const float* __restrict__ q, _Float16* __restrict__ q16,
                                                             int32_t heads, int32_t qk, int64_t T) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int per_row = qk / 8;
    const int64_t rows = heads * T;
    if (i >= rows * per_row) {
        return;
    }
    const int64_t r = i / per_row;
    const int c0 = static_cast<int>(i - r * per_row) * 8;
    const int64_t h = r / T, t = r - h * T;
    const float4* src = reinterpret_cast<const float4*>(q + (t * heads + h) * qk + c0);
    const float4 a = src[0], b = src[1];
    const half8 out = {static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
                       static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
                       static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
    *reinterpret_cast<half8*>(q16 + panel_index(r, c0, rows)) = out;
}

// Causal softmax of the raw scores S [heads T rows][Kp] (row h T + t sees keys
// 0 .. n0 + t) into P [heads T rows][Kp] fp16 panels: p = exp(s scale - max)
// / total, zero past the row's last key.  One wave per row; lane l owns the
// 8 columns 512 k + 8 l .. + 7 of each 512-column step (two 16-byte loads, one
// 16-byte store into the panel of those columns).
__global__ __launch_bounds__(256) void softmax_p16_kernel(const float* __restrict__ S, _Float16* __restrict__ P,
                                                          int64_t rows, int64_t T, int64_t n0, int64_t kp,
                                                          float scale) {
    const int lane = threadIdx.x & 63;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r >= rows) {
        return;
    }
    const int64_t valid = n0 + r % T + 1;
    const float* const row = S + r * kp;
    float m = -INFINITY;
    for (int64_t j = 8 * lane; j < valid; j += 512) {
        const float4 a = *reinterpret_cast<const float4*>(row + j);
        const float4 b = *reinterpret_cast<const float4*>(row + j + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (j + e < valid) {
                m = fmaxf(m, v[e] * scale);
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        m = fmaxf(m, __shfl_xor(m, o));
    }
    float total = 0.0f;
    for (int64_t j = 8 * lane; j < valid; j += 512) {
        const float4 a = *reinterpret_cast<const float4*>(row + j);
        const float4 b = *reinterpret_cast<const float4*>(row + j + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (j + e < valid) {
                total += __expf(v[e] * scale - m);
            }
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        total += __shfl_xor(total, o);
    }
    const float inv = 1.0f / total;
    for (int64_t j = 8 * lane; j < kp; j += 512) {
        half8 out = {};
        if (j < valid) {
            const float4 a = *reinterpret_cast<const float4*>(row + j);
            const float4 b = *reinterpret_cast<const float4*>(row + j + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                out[e] = static_cast<_Float16>(j + e < valid ? __expf(v[e] * scale - m) * inv : 0.0f);
            }
        }
        *reinterpret_cast<half8*>(P + panel_index(r, j, rows)) = out;
    }
}

// c32 [heads T rows][vh] (row h T + t) -> ctx16 [ctx_rows][heads vh] panels at
// row row0 + t, column h vh + c: the output projection's fp16 input.  Thread i
// converts 8 channels.
__global__ __launch_bounds__(256) void unpack_context16_kernel(const float* __restrict__ c32,
                                                               _Float16* __restrict__ ctx16, int32_t heads,
                                                               int32_t vh, int64_t T, int64_t row0,
                                                               int64_t ctx_rows) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int per_row = vh / 8;
    if (i >= heads * T * per_row) {
        return;
    }
    const int64_t r = i / per_row;
    const int c0 = static_cast<int>(i - r * per_row) * 8;
    const int64_t h = r / T, t = r - h * T;
    const float4* src = reinterpret_cast<const float4*>(c32 + r * vh + c0);
    const float4 a = src[0], b = src[1];
    const half8 out = {static_cast<_Float16>(a.x), static_cast<_Float16>(a.y), static_cast<_Float16>(a.z),
                       static_cast<_Float16>(a.w), static_cast<_Float16>(b.x), static_cast<_Float16>(b.y),
                       static_cast<_Float16>(b.z), static_cast<_Float16>(b.w)};
    *reinterpret_cast<half8*>(ctx16 + panel_index(row0 + t, h * vh + c0, ctx_rows)) = out;
}

unsigned blocks_of(int64_t n, int64_t per) { return static_cast<unsigned>((n + per - 1) / per); }

}  // namespace

bool attention_shape_supported(const AttnShape& a) {
    return a.heads > 0 && a.nope >= 0 && a.rope >= 0 && a.rope % 2 == 0 && a.rope <= 256 && a.vh > 0 &&
           a.vh <= 256 && a.rank > 0 && a.cap > 0;
}

hipError_t launch_rope_query(const AttnShape& a, float* q, int64_t T, int64_t pos0, hipStream_t s) {
    if (T <= 0 || a.rope == 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(rope_query_kernel, dim3(static_cast<unsigned>(T * a.heads)), dim3(64), 0, s, q, a.heads, a.nope,
                       a.rope, a.cos_t, a.sin_t, pos0, a.max_positions);
    return hipGetLastError();
}

hipError_t launch_kv_prep(const AttnShape& a, const KvCacheDev& c, const float* lat, const float* norm_w, float* kvn,
                          int64_t T, int64_t slot0, int64_t pos0, float eps, hipStream_t s) {
    if (T <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(kv_prep_kernel, dim3(static_cast<unsigned>(T)), dim3(256), 0, s, lat, norm_w, kvn, c.key_rope,
                       a.rank, a.rope, a.cap, slot0, a.cos_t, a.sin_t, pos0, a.max_positions, eps);
    return hipGetLastError();
}

hipError_t launch_kv_append(const AttnShape& a, const KvCacheDev& c, const float* kvx, int64_t T, int64_t slot0,
                            hipStream_t s) {
    const int64_t total = T * a.heads * static_cast<int64_t>(a.nope + a.vh);
    if (total <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(kv_append_kernel, dim3(blocks_of(total, 256)), dim3(256), 0, s, kvx, c.key_nope, c.value,
                       a.heads, a.nope, a.vh, a.cap, slot0, total);
    return hipGetLastError();
}

bool query_rope_one_supported(const AttnShape& a, int64_t in_dim) {
    return a.nope % 2 == 0 && matvec_rows_supported(static_cast<int64_t>(a.heads) * (a.nope + a.rope), in_dim);
}

hipError_t launch_query_rope_one(const AttnShape& a, const uint16_t* w, const float* x, float* q, int64_t in_dim,
                                 int64_t pos, hipStream_t s, const uint16_t* w2, float* out2, int64_t rows2,
                                 const float* norm_w, float eps) {
    if (!query_rope_one_supported(a, in_dim) || (w2 != nullptr && !matvec_rows_supported(rows2, in_dim)) ||
        (norm_w != nullptr && in_dim > 2048)) {
        return hipErrorInvalidValue;
    }
    const int64_t rows = static_cast<int64_t>(a.heads) * (a.nope + a.rope);
    if (w2 == nullptr) {
        rows2 = 0;
    }
    const dim3 grid(blocks_of(rows + rows2, 8));
    if (norm_w != nullptr) {
        hipLaunchKernelGGL(query_rope_one_kernel<true>, grid, dim3(256), 0, s, w, x, q, rows,
                           static_cast<int32_t>(in_dim), a.nope, a.rope, a.cos_t, a.sin_t, pos, a.max_positions, w2,
                           out2, rows2, norm_w, eps);
    } else {
        hipLaunchKernelGGL(query_rope_one_kernel<false>, grid, dim3(256), 0, s, w, x, q, rows,
                           static_cast<int32_t>(in_dim), a.nope, a.rope, a.cos_t, a.sin_t, pos, a.max_positions, w2,
                           out2, rows2, norm_w, eps);
    }
    return hipGetLastError();
}

bool kv_one_supported(const AttnShape& a) {
    return matvec_rows_supported(static_cast<int64_t>(a.heads) * (a.nope + a.vh), a.rank);
}

hipError_t launch_kv_one(const AttnShape& a, const KvCacheDev& c, const uint16_t* kv_b, const float* lat,
                         const float* norm_w, float eps, int64_t slot, int64_t pos, hipStream_t s) {
    if (!kv_one_supported(a)) {
        return hipErrorInvalidValue;
    }
    const int64_t rows = static_cast<int64_t>(a.heads) * (a.nope + a.vh);
    hipLaunchKernelGGL(kv_one_kernel, dim3(blocks_of(rows, 8)), dim3(256), 0, s, kv_b, lat, norm_w, c.key_nope,
                       c.value, c.key_rope, a.heads, a.nope, a.vh, a.rank, a.rope, a.cap, slot, a.cos_t, a.sin_t,
                       pos, a.max_positions, eps);
    return hipGetLastError();
}

hipError_t launch_attention_core(const AttnShape& a, const KvCacheDev& c, const float* q, float* S, float* ctx,
                                 int64_t T, int64_t n0, float scale, hipStream_t s) {
    if (T <= 0) {
        return hipSuccess;
    }
    const int64_t n_stride = n0 + T;
    const int qk = a.nope + a.rope;
    const unsigned tiles = blocks_of(n_stride, kKeyTile);
    const bool grouped = a.nope % kScoreGroup == 0 && a.rope % kScoreGroup == 0 && qk > 0;
    // the 64-key tiles where the row is short (measured: 0.5 us faster than the
    // 256-key tiles near 512 keys, 2.3 us slower near 4K)
    if (T == 1 && grouped && qk <= kScoreTileCh && n_stride <= kScoreTileMaxKeys) {
        hipLaunchKernelGGL(scores_tile_kernel, dim3(blocks_of(n_stride, kScoreTile), a.heads), dim3(256), 0, s, q,
                           c.key_nope, c.key_rope, S, a.nope, a.rope, a.cap, n_stride, scale);
    } else if (T == 1 && grouped) {
        hipLaunchKernelGGL(scores_grouped_kernel<1>, dim3(tiles, a.heads, 1), dim3(kKeyTile), sizeof(float) * qk, s,
                           q, c.key_nope, c.key_rope, S, a.heads, a.nope, a.rope, a.cap, n0, T, n_stride, scale);
    } else if (grouped) {
        hipLaunchKernelGGL(scores_grouped_kernel<kQueries>, dim3(tiles, a.heads, blocks_of(T, kQueries)),
                           dim3(kKeyTile), sizeof(float) * kQueries * qk, s, q, c.key_nope, c.key_rope, S, a.heads,
                           a.nope, a.rope, a.cap, n0, T, n_stride, scale);
    } else if (T == 1) {
        hipLaunchKernelGGL(scores_kernel<1>, dim3(tiles, a.heads, 1), dim3(kKeyTile), sizeof(float) * qk, s, q,
                           c.key_nope, c.key_rope, S, a.heads, a.nope, a.rope, a.cap, n0, T, n_stride, scale);
    } else {
        hipLaunchKernelGGL(scores_kernel<kQueries>, dim3(tiles, a.heads, blocks_of(T, kQueries)), dim3(kKeyTile),
                           sizeof(float) * kQueries * qk, s, q, c.key_nope, c.key_rope, S, a.heads, a.nope, a.rope,
                           a.cap, n0, T, n_stride, scale);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    const int64_t rows = T * a.heads;
    // one token: the context kernel by channel groups (32-bit buffer offsets),
    // with the softmax inside it while the row fits its LDS
    const bool ctx_decode = T == 1 && a.vh % kCtxCh == 0 && a.cap * a.vh < (int64_t{1} << 29);
    const bool fused = ctx_decode && n0 + 1 <= kSoftmaxLds;
    if (!fused) {
        if (T == 1 && n0 + 1 <= kSoftmaxLds) {
            hipLaunchKernelGGL(softmax_decode_kernel, dim3(static_cast<unsigned>(a.heads)), dim3(256), 0, s, S,
                               n0 + 1, n_stride);
        } else {
            hipLaunchKernelGGL(softmax_rows_kernel, dim3(blocks_of(rows, 4)), dim3(256), 0, s, S, rows, a.heads, n0,
                               n_stride);
        }
        err = hipGetLastError();
        if (err != hipSuccess) {
            return err;
        }
    }
    const unsigned threads = static_cast<unsigned>((a.vh + 63) / 64 * 64);
    const dim3 ctx_grid(static_cast<unsigned>(a.heads * (a.vh / kCtxCh)));
    if (fused) {
        hipLaunchKernelGGL(context_decode_kernel<true>, ctx_grid, dim3(kCtxThreads), 0, s, S, c.value, ctx, a.vh,
                           a.cap, n0 + 1, n_stride);
    } else if (ctx_decode) {
        hipLaunchKernelGGL(context_decode_kernel<false>, ctx_grid, dim3(kCtxThreads), 0, s, S, c.value, ctx, a.vh,
                           a.cap, n0 + 1, n_stride);
    } else if (T == 1) {
        hipLaunchKernelGGL(context_kernel<1>, dim3(a.heads, 1), dim3(threads), 0, s, S, c.value, ctx, a.heads, a.vh,
                           a.cap, n0, T, n_stride);
    } else {
        hipLaunchKernelGGL(context_kernel<kQueries>, dim3(a.heads, blocks_of(T, kQueries)), dim3(threads), 0, s, S,
                           c.value, ctx, a.heads, a.vh, a.cap, n0, T, n_stride);
    }
    return hipGetLastError();
}

bool attention_mfma_supported(const AttnShape& a) {
    // whole panels of channels for the queries and keys and for the context's
    // fp16 copy [T, heads vh] (no padding columns to clear); 8-channel stores
    return a.nope % kPanel == 0 && a.rope % kPanel == 0 && a.nope + a.rope > 0 && a.vh % 8 == 0 && a.vh <= 256 &&
           (a.heads * a.vh) % kPanel == 0;
}

hipError_t launch_pack_kv16(const AttnShape& a, const KvCacheDev& c, int64_t keys, _Float16* k16, _Float16* v16,
                            hipStream_t s) {
    if (keys <= 0) {
        return hipSuccess;
    }
    const int64_t kp = round_up(keys, kPanel);
    const int qk = a.nope + a.rope;
    hipLaunchKernelGGL(pack_keys16_kernel, dim3(blocks_of(kp, 64), static_cast<unsigned>(qk / kPanel), a.heads),
                       dim3(256), 0, s, c.key_nope, c.key_rope, k16, a.nope, qk, a.cap, keys, kp);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    hipLaunchKernelGGL(pack_values16_kernel, dim3(static_cast<unsigned>(kp / kPanel), a.heads), dim3(256),
                       sizeof(float) * kPanel * (a.vh + 1), s, c.value, v16, a.vh, a.cap, keys, kp);
    return hipGetLastError();
}

hipError_t launch_attention_core_mfma(const AttnShape& a, const float* q, const AttnMfmaBufs& b, int64_t T,
                                      int64_t n0, int64_t keys, float scale, _Float16* ctx16, int64_t row0,
                                      int64_t ctx_rows, hipStream_t s) {
    if (T <= 0) {
        return hipSuccess;
    }
    if (n0 + T > keys || row0 + T > ctx_rows) {
        return hipErrorInvalidValue;
    }
    const int qk = a.nope + a.rope;
    const int64_t kp = round_up(keys, kPanel);
    const int64_t rows = a.heads * T;
    hipLaunchKernelGGL(pack_queries16_kernel, dim3(blocks_of(rows * (qk / 8), 256)), dim3(256), 0, s, q, b.q16,
                       a.heads, qk, T);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    // S = Q K^T per head: rows h T + t, Kp columns (keys past the last are zero rows)
    err = launch_mfma_heads(b.q16, b.k16, kp * qk, b.S, a.heads, T, static_cast<int32_t>(kp), qk, b.meta, s);
    if (err != hipSuccess) {
        return err;
    }
    hipLaunchKernelGGL(softmax_p16_kernel, dim3(blocks_of(rows, 4)), dim3(256), 0, s, b.S, b.p16, rows, T, n0, kp,
                       scale);
    err = hipGetLastError();
    if (err != hipSuccess) {
        return err;
    }
    // ctx = P V per head: K = Kp (zero probabilities and zero values past the last key)
    err = launch_mfma_heads(b.p16, b.v16, static_cast<int64_t>(a.vh) * kp, b.c32, a.heads, T, a.vh,
                            static_cast<int32_t>(kp), b.meta, s);
    if (err != hipSuccess) {
        return err;
    }
    hipLaunchKernelGGL(unpack_context16_kernel, dim3(blocks_of(rows * (a.vh / 8), 256)), dim3(256), 0, s, b.c32,
                       ctx16, a.heads, a.vh, T, row0, ctx_rows);
    return hipGetLastError();
}

}  // namespace lm
