// lm_attn.hip -- the C ABI of include/litemind_attention.h: multi-head latent
// attention with its rotary tables and KV caches resident in HBM.
//
// Per layer and call (T tokens, cache slots n0 .. n0 + T - 1), on the context
// stream:
//   q      = q_proj x                 or  q_b_proj rms_norm(q_a_proj x)    (matvec, k_head.hip)
//   q      = rope(q) per head                                             (k_attn.hip)
//   lat    = kv_a_proj x                                                  (matvec)
//   kvn    = rms_norm(lat[:rank]);  cache.key_rope <- rope(lat[rank:])    (k_attn.hip)
//   kvx    = kv_b_proj kvn;         cache.key_nope, cache.value <- kvx    (matvec, k_attn.hip)
//   ctx    = softmax(scale * q . keys) . values, causal                   (k_attn.hip)
//   out    = o_proj ctx   (or out += o_proj ctx)                          (matvec)
// which is Attention::forward (src/Attention.cpp:22-103) for each token in turn.
// Every projection keeps gemm::matvec_bf16's association (bit for bit) unless
// the projection path is MFMA: then, from kAttnMfmaTokens tokens on (LM_PATH_AUTO)
// or for every batch of two or more (LM_PATH_MFMA), each projection is a GEMM on
// the grouped kernel of k_mfma.hip (one group of T rows): the input converted to
// fp16 panels, the weights' fp16 panel copy made at upload, fp32 accumulation;
// results within the tolerance of the MoE block's MFMA path.  With MFMA
// projections the attention core is MFMA as well where the shape allows it
// (k_attn.hip): per head S = Q K^T and ctx = P V on the same grouped kernel,
// over fp16 copies of the cache made once per call.
//
// Query tokens are processed by the core in groups sized from a byte budget
// (lm_attention_set_score_budget, default 1 GiB) for the scores (and the MFMA
// core's fp16 copies), so a long cache takes smaller groups instead of failing
// to allocate.
#include "litemind_attention.h"
#include "lm_error.h"
#include "lm_internal.h"

#include <algorithm>
#include <cmath>
#include <new>
#include <string>
#include <vector>

#define LM_ATT_HIP(call)                                                                                     \
    do {                                                                                                     \
        const hipError_t lm_status_ = (call);                                                                \
        if (lm_status_ != hipSuccess) {                                                                      \
            return lm::set_error(LM_EHIP, std::string(#call) + ": " + hipGetErrorString(lm_status_));        \
        }                                                                                                    \
    } while (0)

namespace lm {

struct AttnLayer {
    void* slab = nullptr;  // the layer's projections (BF16) and norm weights (fp32)
    const uint16_t* q_proj = nullptr;
    const uint16_t* q_a = nullptr;
    const float* q_a_norm = nullptr;
    const uint16_t* q_b = nullptr;
    const uint16_t* kv_a = nullptr;
    const float* kv_a_norm = nullptr;
    const uint16_t* kv_b = nullptr;
    const uint16_t* o = nullptr;
    // fp16 panel copies for the MFMA path (null when a width is not a multiple
    // of 32 or a weight overflows fp16): device table of pointers in the order
    // of Proj, read by the kernel as its group's weights
    void* slab16 = nullptr;
    const _Float16* const* table16 = nullptr;
    float* input_norm = nullptr;  // [H], lm_decoder_forward
    KvCacheDev cache;
    int64_t count = 0;  // KvCache::token_count
};

// Projections in the order of AttnLayer::table16.
enum Proj { kProjQ = 0, kProjQa = 1, kProjQb = 2, kProjKva = 3, kProjKvb = 4, kProjO = 5, kProjCount = 6 };

struct AttnState {
    int32_t path = LM_PATH_AUTO;  // projection path of lm_attention_forward
    // MFMA path: the query projections run on `side` while the key and value
    // projections run on the context stream (fork / join events)
    hipStream_t side = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
    lm_mla_config cfg{};
    AttnShape shape;
    float scale = 0.0f;
    float* tables = nullptr;  // cos [max_positions, rope / 2] then sin
    float* caches = nullptr;  // every layer's cache
    std::vector<AttnLayer> layers;
    float* ws = nullptr;      // per-call scratch (floats)
    size_t ws_floats = 0;
    float* xn = nullptr;      // lm_decoder_forward: normalised rows [T, H]
    size_t xn_floats = 0;
    int64_t score_budget = 0; // bytes of the attention core's scratch (0: the default)
};

void attention_release(AttnState* st) {
    if (st == nullptr) {
        return;
    }
    for (AttnLayer& L : st->layers) {
        (void)hipFree(L.slab);
        (void)hipFree(L.slab16);
        (void)hipFree(L.input_norm);
    }
    if (st->fork != nullptr) {
        (void)hipEventDestroy(st->fork);
    }
    if (st->join != nullptr) {
        (void)hipEventDestroy(st->join);
    }
    if (st->side != nullptr) {
        (void)hipStreamSynchronize(st->side);
        (void)hipStreamDestroy(st->side);
    }
    (void)hipFree(st->tables);
    (void)hipFree(st->caches);
    (void)hipFree(st->ws);
    (void)hipFree(st->xn);
    delete st;
}

}  // namespace lm

namespace {

using lm::AttnLayer;
using lm::AttnState;

// Query tokens per launch of the attention core, at most.
constexpr int64_t kCoreTokens = 512;
// Default byte budget of the attention core's scratch.
constexpr int64_t kScoreBudget = int64_t{1} << 30;
// LM_PATH_AUTO: batches of at least this many tokens take the MFMA projections.
constexpr int64_t kAttnMfmaTokens = 16;

int fail(int code, const std::string& message) { return lm::set_error(code, message); }

// Sizing of the attention core for F tokens after `cached` ones.
struct CorePlan {
    int64_t group = 0;  // query tokens per core launch
    bool mfma = false;  // scores and context on MFMA
    int64_t kp = 0;     // keys rounded up to 32 (MFMA core)
    int64_t bytes = 0;  // the core's scratch
};

// A query group of as many tokens as the budget holds (at least one, at most
// kCoreTokens).  The MFMA core when the projections are MFMA, the shape allows
// it, its fp16 copies of the keys and values fit in half the budget and its
// operands stay within the grouped kernel's 32-bit buffer offsets; its scratch
// per query token is heads (6 Kp + 2 qk) bytes (fp32 scores, fp16
// probabilities and query), the VALU core's heads keys 4 bytes.
CorePlan plan_core(const lm::AttnShape& a, int64_t cached, int64_t F, bool mfma_proj, int64_t budget) {
    CorePlan p;
    if (F <= 0) {
        return p;
    }
    const int64_t keys = cached + F;
    const int64_t heads = a.heads, qk = a.nope + a.rope, vh = a.vh;
    const int64_t limit = 0x7fffffff;
    if (mfma_proj && F >= 2 && lm::attention_mfma_supported(a)) {
        const int64_t kp = lm::round_up(keys, lm::kPanel);
        const int64_t fixed = heads * kp * (qk + vh) * 2;
        const int64_t per = heads * (6 * kp + 2 * qk);
        const int64_t group = std::min({(budget - fixed) / per, kCoreTokens, F, limit / (2 * heads * kp)});
        if (fixed <= budget / 2 && group >= 1 && 4 * kp * std::max(qk, lm::round_up(vh, lm::kPanel)) <= limit) {
            p.group = group;
            p.mfma = true;
            p.kp = kp;
            p.bytes = fixed + group * per;
            return p;
        }
    }
    const int64_t per = heads * keys * 4;
    p.group = std::max<int64_t>(1, std::min({budget / per, kCoreTokens, F}));
    p.bytes = p.group * per;
    return p;
}

bool mfma_projections(int32_t path, int64_t F) {
    return F >= 2 && (path == LM_PATH_MFMA || (path == LM_PATH_AUTO && F >= kAttnMfmaTokens));
}

// yarn_get_mscale (src/Rope.cpp:13-18, src/Config.cpp:12-17):
// 0.1 * mscale * log(scale) + 1, which LiteMind's GCC build fuses into one
// multiply-add of the rounded 0.1 * mscale.
double yarn_mscale(double scale, double mscale) {
    if (scale <= 1.0) {
        return 1.0;
    }
    return std::fma(0.1 * mscale, std::log(scale), 1.0);
}

float softmax_scale(const lm_mla_config& c) {
    // Config::softmax_scale (src/Config.cpp:114-121)
    double scale = 1.0 / std::sqrt(static_cast<double>(c.qk_nope_head_dim + c.qk_rope_head_dim));
    if (c.yarn != 0 && c.mscale_all_dim != 0.0) {
        const double m = yarn_mscale(c.factor, c.mscale_all_dim);
        scale *= m * m;
    }
    return static_cast<float>(scale);
}

// RotaryEmbedding::build (src/Rope.cpp:35-94) into cos / sin [positions, dim / 2]:
// inverse frequencies in double (YaRN: the interpolated and extrapolated
// frequency blended over the correction band, src/Rope.cpp:20-31, 50-81), then
// float(cos(p * f) * magnitude) and float(sin(p * f) * magnitude).
void rope_tables(const lm_mla_config& c, int64_t positions, float* cos_out, float* sin_out) {
    const int32_t dim = c.qk_rope_head_dim;
    const int32_t half = dim / 2;
    const double base = static_cast<double>(static_cast<float>(c.rope_theta));  // Config::rope_theta is a float
    std::vector<double> inv(static_cast<size_t>(half));
    double magnitude = 1.0;
    if (c.yarn == 0) {
        for (int32_t i = 0; i < half; ++i) {
            inv[i] = 1.0 / std::pow(base, 2.0 * static_cast<double>(i) / static_cast<double>(dim));
        }
    } else {
        const double factor = c.factor <= 0.0 ? 1.0 : c.factor;
        const double pi = 3.14159265358979323846;
        auto correction = [&](double rotations) {
            const double num = static_cast<double>(dim) *
                               std::log(static_cast<double>(c.original_max_positions) / (rotations * 2.0 * pi));
            return num / (2.0 * std::log(base));
        };
        double low = std::max(std::floor(correction(c.beta_fast)), 0.0);
        double high = std::min(std::ceil(correction(c.beta_slow)), static_cast<double>(dim) - 1.0);
        if (high - low < 1e-6) {
            high = low + 0.001;
        }
        for (int32_t i = 0; i < half; ++i) {
            const double extrapolated = 1.0 / std::pow(base, 2.0 * static_cast<double>(i) / static_cast<double>(dim));
            const double interpolated = extrapolated / factor;
            const double ramp = std::clamp((static_cast<double>(i) - low) / (high - low), 0.0, 1.0);
            const double keep = 1.0 - ramp;
            const double from_interpolated = interpolated * (1.0 - keep);
            const double from_extrapolated = extrapolated * keep;
            inv[i] = from_interpolated + from_extrapolated;
        }
        magnitude = yarn_mscale(factor, c.mscale) / yarn_mscale(factor, c.mscale_all_dim);
    }
    for (int64_t p = 0; p < positions; ++p) {
        for (int32_t i = 0; i < half; ++i) {
            const double angle = static_cast<double>(p) * inv[i];
            cos_out[p * half + i] = static_cast<float>(std::cos(angle) * magnitude);
            sin_out[p * half + i] = static_cast<float>(std::sin(angle) * magnitude);
        }
    }
}

int check_config(const lm_mla_config* c) {
    if (c == nullptr) {
        return fail(LM_EINVAL, "null attention config");
    }
    if (c->hidden_size <= 0 || c->num_heads <= 0 || c->q_lora_rank < 0 || c->kv_lora_rank <= 0 ||
        c->qk_nope_head_dim < 0 || c->qk_rope_head_dim < 0 || c->v_head_dim <= 0 || c->context_length <= 0) {
        return fail(LM_EINVAL, "attention config: sizes must be positive");
    }
    if (c->qk_rope_head_dim % 2 != 0 || c->qk_rope_head_dim > 256 || c->v_head_dim > 256) {
        return fail(LM_EINVAL, "attention config: qk_rope_head_dim must be even and <= 256, v_head_dim <= 256");
    }
    const int64_t widths[] = {c->hidden_size, c->q_lora_rank, c->kv_lora_rank,
                              static_cast<int64_t>(c->num_heads) * c->v_head_dim};
    for (int64_t w : widths) {
        if (w % 8 != 0 || w > 16384) {
            return fail(LM_EINVAL, "attention config: hidden_size, q_lora_rank, kv_lora_rank and heads * v_head_dim "
                                   "must be multiples of 8 and at most 16384");
        }
    }
    return LM_OK;
}

int get_state(lm_context* ctx, AttnState** out) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    AttnState* st = lm::context_attention(ctx);
    if (st == nullptr) {
        return fail(LM_EINVAL, "attention is not configured (lm_attention_configure)");
    }
    *out = st;
    return LM_OK;
}

int check_attn_layer(AttnState* st, int32_t layer) {
    if (layer < 0 || layer >= static_cast<int32_t>(st->layers.size())) {
        return fail(LM_EINVAL, "layer " + std::to_string(layer) + " out of range");
    }
    return LM_OK;
}

// Grows a scratch buffer (after the stream drains, since queued work may use it).
int ensure_buffer(float** buf, size_t* have, hipStream_t stream, size_t floats) {
    if (*have >= floats) {
        return LM_OK;
    }
    LM_ATT_HIP(hipStreamSynchronize(stream));
    (void)hipFree(*buf);
    *buf = nullptr;
    *have = 0;
    const hipError_t err = hipMalloc(reinterpret_cast<void**>(buf), floats * sizeof(float));
    if (err != hipSuccess) {
        *buf = nullptr;
        return fail(LM_ENOMEM, "attention scratch of " + std::to_string(floats) + " floats: " + hipGetErrorString(err));
    }
    *have = floats;
    return LM_OK;
}

// Scratch of the MFMA projections on one stream: an fp16 panel copy of an
// input that is ready (and which input it is), the buffer for the next
// conversion, and the GEMM's partial sums.
struct ProjScratch {
    const _Float16* ready;
    const float* ready_of;
    _Float16* conv;
    float* partial;
    int64_t partial_floats;
};

// out [F, N] = W x (or out += W x) for x [F, K]: gemm::matvec_bf16 per token
// (bit for bit), or with `mfma` the GEMM on MFMA over W's fp16 panel copy.
int project(const AttnLayer& L, int proj, const uint16_t* w, const float* x, int64_t K, float* out, int64_t N,
            int64_t F, int32_t accumulate, bool mfma, ProjScratch& ps, hipStream_t stream) {
    if (!mfma) {
        LM_ATT_HIP(lm::launch_matvec_tokens(w, x, out, N, K, F, 1.0f, accumulate, stream));
        return LM_OK;
    }
    const int64_t Kp = lm::round_up(K, lm::kPanel);
    if (ps.ready_of != x) {
        LM_ATT_HIP(lm::launch_to_f16_rows(x, ps.conv, F, static_cast<int32_t>(K), static_cast<int32_t>(Kp), stream));
        ps.ready = ps.conv;
        ps.ready_of = x;
    }
    LM_ATT_HIP(lm::launch_mfma_gemm(ps.ready, L.table16 + proj, out, F, static_cast<int32_t>(N),
                                    static_cast<int32_t>(Kp), accumulate, ps.partial, ps.partial_floats, stream));
    return LM_OK;
}

// Attention::forward for F tokens that all fit the cache; out = o_proj ctx or
// out += o_proj ctx.  x [F, H] must not overlap out, except with in_norm: x is
// then the raw hidden state, normalised here by in_norm (into xn_buf [F, H], or
// inside the first projection's launch for one token) before anything else
// reads it, so out may be x itself.
int attention_tokens(AttnState* st, hipStream_t stream, int32_t layer, const float* x, int64_t F, int64_t pos0,
                     float* out, int32_t accumulate, int32_t path, const float* in_norm = nullptr,
                     float* xn_buf = nullptr) {
    const lm_mla_config& c = st->cfg;
    AttnLayer& L = st->layers[static_cast<size_t>(layer)];
    if (L.kv_a == nullptr) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no attention weights (lm_upload_attention)");
    }
    const lm::AttnShape& a = st->shape;
    const int64_t H = c.hidden_size, heads = c.num_heads, qk = c.qk_nope_head_dim + c.qk_rope_head_dim;
    const int64_t rank = c.kv_lora_rank, rope = c.qk_rope_head_dim, vh = c.v_head_dim, ql = c.q_lora_rank;
    const int64_t n0 = L.count;
    const int64_t n_total = n0 + F;
    const bool mfma = L.table16 != nullptr && mfma_projections(path, F);
    const CorePlan plan = plan_core(a, n0, F, mfma, st->score_budget > 0 ? st->score_budget : kScoreBudget);
    const int64_t core = plan.group;
    // Scratch, each region a multiple of 64 floats: q | q latent | kv latent |
    // kv normalised | kv expanded | scores | context; with MFMA projections
    // fp16 copies of x (read by the query and the key / value projections), of
    // the q latent and of the key / value inputs (latent, then context), and
    // partial sums for each stream; with the MFMA core fp16 copies of the keys,
    // values, queries and probabilities and the per-head group table.
    size_t total_f = 0;
    auto region = [&](int64_t floats) {
        const size_t at = total_f;
        total_f += static_cast<size_t>((floats + 63) / 64 * 64);
        return at;
    };
    auto halves = [](int64_t n) { return (n + 1) / 2; };
    const int64_t kp = plan.kp;
    const size_t q_at = region(F * heads * qk);
    const size_t ql_at = region(F * ql);
    const size_t lat_at = region(F * (rank + rope));
    const size_t kvn_at = region(F * rank);
    const size_t kvx_at = region(F * heads * (c.qk_nope_head_dim + vh));
    const size_t s_at = region(plan.mfma ? core * heads * kp : core * heads * n_total);
    const size_t ctx_at = region(F * heads * vh);
    const size_t x16a_at = region(mfma ? halves(F * lm::round_up(H, lm::kPanel)) : 0);
    const size_t x16q_at = region(mfma && ql > 0 ? halves(F * lm::round_up(ql, lm::kPanel)) : 0);
    const size_t x16kv_at = region(mfma ? halves(F * lm::round_up(std::max(rank, heads * vh), lm::kPanel)) : 0);
    const int64_t partq_f = mfma ? 4 * F * std::max(heads * qk, ql) : 0;
    const int64_t partkv_f = mfma ? 4 * F * std::max({rank + rope, heads * (c.qk_nope_head_dim + vh), H}) : 0;
    const size_t partq_at = region(partq_f);
    const size_t partkv_at = region(partkv_f);
    const size_t k16_at = region(plan.mfma ? halves(heads * kp * qk) : 0);
    const size_t v16_at = region(plan.mfma ? halves(heads * vh * kp) : 0);
    const size_t q16_at = region(plan.mfma ? halves(heads * core * qk) : 0);
    const size_t p16_at = region(plan.mfma ? halves(heads * core * kp) : 0);
    const size_t meta_at = region(plan.mfma ? (lm::mfma_heads_meta_bytes(heads) + 3) / 4 : 0);
    int rc = ensure_buffer(&st->ws, &st->ws_floats, stream, total_f);
    if (rc != LM_OK) {
        return rc;
    }
    float* const ws = st->ws;
    auto h16 = [&](size_t at) { return reinterpret_cast<_Float16*>(ws + at); };
    float* q = ws + q_at;
    float* qlat = ws + ql_at;
    float* lat = ws + lat_at;
    float* kvn = ws + kvn_at;
    float* kvx = ws + kvx_at;
    float* S = ws + s_at;
    float* ctxv = ws + ctx_at;
    _Float16* const x16a = h16(x16a_at);
    _Float16* const x16q = h16(x16q_at);
    _Float16* const x16kv = h16(x16kv_at);
    ProjScratch psq{nullptr, nullptr, ql > 0 ? x16q : x16a, ws + partq_at, partq_f};
    ProjScratch pskv{nullptr, nullptr, x16kv, ws + partkv_at, partkv_f};

    // queries (src/Attention.cpp:33-48); for one token the rotary step rides
    // on the projection's launch
    const int64_t q_in = ql == 0 ? H : ql;
    const bool q_fused = F == 1 && lm::query_rope_one_supported(a, q_in);
    // without the q LoRA, kv_a projects the same x: one launch for both
    const bool kv_a_with_q = q_fused && ql == 0 && lm::matvec_rows_supported(rank + rope, H);
    // the input norm inside that launch when it takes the whole row (nothing
    // else reads x then)
    const float* norm_in_launch = kv_a_with_q && H <= 2048 ? in_norm : nullptr;
    if (in_norm != nullptr && norm_in_launch == nullptr) {
        LM_ATT_HIP(lm::launch_rms_norm(x, in_norm, xn_buf, F, static_cast<int32_t>(H), c.rms_norm_eps, stream));
        x = xn_buf;
    }
    // MFMA path: x's fp16 copy, then the query path forks onto the side stream
    hipStream_t qs = stream;
    if (mfma) {
        LM_ATT_HIP(lm::launch_to_f16_rows(x, x16a, F, static_cast<int32_t>(H),
                                          static_cast<int32_t>(lm::round_up(H, lm::kPanel)), stream));
        psq.ready = pskv.ready = x16a;
        psq.ready_of = pskv.ready_of = x;
        LM_ATT_HIP(hipEventRecord(st->fork, stream));
        LM_ATT_HIP(hipStreamWaitEvent(st->side, st->fork, 0));
        qs = st->side;
    }
    const float* q_x = x;
    if (ql != 0) {
        rc = project(L, lm::kProjQa, L.q_a, x, H, qlat, ql, F, 0, mfma, psq, qs);
        if (rc != LM_OK) {
            return rc;
        }
        LM_ATT_HIP(lm::launch_rms_norm(qlat, L.q_a_norm, qlat, F, static_cast<int32_t>(ql), c.rms_norm_eps, qs));
        q_x = qlat;
    }
    const uint16_t* q_w = ql == 0 ? L.q_proj : L.q_b;
    if (kv_a_with_q) {
        LM_ATT_HIP(lm::launch_query_rope_one(a, q_w, q_x, q, q_in, pos0, stream, L.kv_a, lat, rank + rope,
                                             norm_in_launch, c.rms_norm_eps));
    } else if (q_fused) {
        LM_ATT_HIP(lm::launch_query_rope_one(a, q_w, q_x, q, q_in, pos0, stream));
    } else {
        rc = project(L, ql == 0 ? lm::kProjQ : lm::kProjQb, q_w, q_x, q_in, q, heads * qk, F, 0, mfma, psq, qs);
        if (rc != LM_OK) {
            return rc;
        }
        LM_ATT_HIP(lm::launch_rope_query(a, q, F, pos0, qs));
    }
    // compressed keys and values, appended at slots n0 .. n0 + F - 1 (:50-75);
    // for one token the norm, kv_b and the append are one launch
    if (!kv_a_with_q) {
        rc = project(L, lm::kProjKva, L.kv_a, x, H, lat, rank + rope, F, 0, mfma, pskv, stream);
        if (rc != LM_OK) {
            return rc;
        }
    }
    if (F == 1 && lm::kv_one_supported(a)) {
        LM_ATT_HIP(lm::launch_kv_one(a, L.cache, L.kv_b, lat, L.kv_a_norm, c.rms_norm_eps, n0, pos0, stream));
    } else {
        LM_ATT_HIP(lm::launch_kv_prep(a, L.cache, lat, L.kv_a_norm, kvn, F, n0, pos0, c.rms_norm_eps, stream));
        rc = project(L, lm::kProjKvb, L.kv_b, kvn, rank, kvx, heads * (c.qk_nope_head_dim + vh), F, 0, mfma, pskv,
                     stream);
        if (rc != LM_OK) {
            return rc;
        }
        LM_ATT_HIP(lm::launch_kv_append(a, L.cache, kvx, F, n0, stream));
    }
    if (mfma) {  // join: the queries are in
        LM_ATT_HIP(hipEventRecord(st->join, st->side));
        LM_ATT_HIP(hipStreamWaitEvent(stream, st->join, 0));
    }
    // causal attention over the cache (:77-98), in groups of query tokens
    if (plan.mfma) {
        // the context lands in fp16 panels [F, heads vh] in x16kv (free once
        // kv_b has run), the output projection's input; ctxv holds the
        // per-head context of one group
        const lm::AttnMfmaBufs b{h16(k16_at), h16(v16_at), h16(q16_at), S, h16(p16_at), ctxv, ws + meta_at};
        LM_ATT_HIP(lm::launch_pack_kv16(a, L.cache, n_total, b.k16, b.v16, stream));
        for (int64_t t0 = 0; t0 < F; t0 += core) {
            const int64_t n = std::min(core, F - t0);
            LM_ATT_HIP(lm::launch_attention_core_mfma(a, q + t0 * heads * qk, b, n, n0 + t0, n_total, st->scale,
                                                      x16kv, t0, F, stream));
        }
        pskv.ready = x16kv;
        pskv.ready_of = ctxv;
    } else {
        for (int64_t t0 = 0; t0 < F; t0 += core) {
            const int64_t n = std::min(core, F - t0);
            LM_ATT_HIP(lm::launch_attention_core(a, L.cache, q + t0 * heads * qk, S, ctxv + t0 * heads * vh, n,
                                                 n0 + t0, st->scale, stream));
        }
    }
    // output projection (:100-101)
    rc = project(L, lm::kProjO, L.o, ctxv, heads * vh, out, H, F, accumulate, mfma, pskv, stream);
    if (rc != LM_OK) {
        return rc;
    }
    L.count = n_total;
    return LM_OK;
}

int upload(hipStream_t stream, void* dst, const void* src, size_t bytes) {
    LM_ATT_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream));
    return LM_OK;
}

// Copies cached entries [token0, token0 + tokens) of a layer between the
// device cache and host buffers in KvCache's layout (key_nope [tokens, heads,
// qk_nope], key_rope [tokens, qk_rope], value [tokens, heads, v_head]).
// Reading needs token0 + tokens <= the layer's count; writing needs token0 <=
// count (no gap) and token0 + tokens <= capacity, every buffer of a non-empty
// part given, and extends the count to token0 + tokens.  Both wait for the
// context stream first and finish before returning.
int kv_cache_copy(lm_context* ctx, int32_t layer, int64_t token0, int64_t tokens, float* key_nope_host,
                  float* key_rope_host, float* value_host, bool to_device) {
    try {
        AttnState* st = nullptr;
        int rc = get_state(ctx, &st);
        if (rc == LM_OK) {
            rc = check_attn_layer(st, layer);
        }
        if (rc != LM_OK) {
            return rc;
        }
        AttnLayer& L = st->layers[static_cast<size_t>(layer)];
        const int64_t cap = st->cfg.context_length, heads = st->cfg.num_heads, nope = st->cfg.qk_nope_head_dim,
                      rope = st->cfg.qk_rope_head_dim, vh = st->cfg.v_head_dim;
        if (token0 < 0 || tokens < 0) {
            return fail(LM_EINVAL, "negative token range");
        }
        if (!to_device && token0 + tokens > L.count) {
            return fail(LM_EINVAL, "tokens must be within the cache's " + std::to_string(L.count));
        }
        if (to_device) {
            if (token0 > L.count || token0 + tokens > cap) {
                return fail(LM_EINVAL, "write of entries " + std::to_string(token0) + ".." +
                                           std::to_string(token0 + tokens) + " to a cache holding " +
                                           std::to_string(L.count) + " of " + std::to_string(cap));
            }
            if (tokens > 0 && ((nope > 0 && key_nope_host == nullptr) || (rope > 0 && key_rope_host == nullptr) ||
                               value_host == nullptr)) {
                return fail(LM_EINVAL, "a cache write needs the keys, the rotary keys and the values");
            }
        }
        if (tokens == 0) {
            return LM_OK;
        }
        const lm::ContextInfo info = lm::context_info(ctx);
        LM_ATT_HIP(hipSetDevice(info.device));
        LM_ATT_HIP(hipStreamSynchronize(info.stream));
        const hipMemcpyKind kind = to_device ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
        // one 2-D copy per part between the device rows (stride cap) and a
        // staging buffer with the host layout's transpose
        auto copy2d = [&](float* dev, size_t dev_pitch, float* host, size_t width, size_t height) {
            return to_device ? hipMemcpy2DAsync(dev, dev_pitch, host, width, width, height, kind, info.stream)
                             : hipMemcpy2DAsync(host, width, dev, dev_pitch, width, height, kind, info.stream);
        };
        const size_t tb = sizeof(float) * static_cast<size_t>(tokens);
        std::vector<float> kn, kr, v;
        if (key_nope_host != nullptr && nope > 0) {
            kn.resize(static_cast<size_t>(heads * nope * tokens));
            if (to_device) {
                for (int64_t t = 0; t < tokens; ++t) {
                    for (int64_t hd = 0; hd < heads * nope; ++hd) {
                        kn[static_cast<size_t>(hd * tokens + t)] = key_nope_host[t * heads * nope + hd];
                    }
                }
            }
            LM_ATT_HIP(copy2d(L.cache.key_nope + token0, sizeof(float) * cap, kn.data(), tb,
                              static_cast<size_t>(heads * nope)));
        }
        if (key_rope_host != nullptr && rope > 0) {
            kr.resize(static_cast<size_t>(rope * tokens));
            if (to_device) {
                for (int64_t t = 0; t < tokens; ++t) {
                    for (int64_t d = 0; d < rope; ++d) {
                        kr[static_cast<size_t>(d * tokens + t)] = key_rope_host[t * rope + d];
                    }
                }
            }
            LM_ATT_HIP(copy2d(L.cache.key_rope + token0, sizeof(float) * cap, kr.data(), tb, static_cast<size_t>(rope)));
        }
        if (value_host != nullptr) {
            v.resize(static_cast<size_t>(heads * tokens * vh));
            if (to_device) {
                for (int64_t h = 0; h < heads; ++h) {
                    for (int64_t t = 0; t < tokens; ++t) {
                        std::copy_n(value_host + (t * heads + h) * vh, vh, v.data() + (h * tokens + t) * vh);
                    }
                }
            }
            LM_ATT_HIP(copy2d(L.cache.value + token0 * vh, sizeof(float) * cap * vh, v.data(), tb * vh,
                              static_cast<size_t>(heads)));
        }
        LM_ATT_HIP(hipStreamSynchronize(info.stream));
        if (to_device) {
            L.count = std::max(L.count, token0 + tokens);
            return LM_OK;
        }
        if (!kn.empty()) {
            for (int64_t hd = 0; hd < heads * nope; ++hd) {
                for (int64_t t = 0; t < tokens; ++t) {
                    key_nope_host[t * heads * nope + hd] = kn[static_cast<size_t>(hd * tokens + t)];
                }
            }
        }
        if (!kr.empty()) {
            for (int64_t d = 0; d < rope; ++d) {
                for (int64_t t = 0; t < tokens; ++t) {
                    key_rope_host[t * rope + d] = kr[static_cast<size_t>(d * tokens + t)];
                }
            }
        }
        if (!v.empty()) {
            for (int64_t h = 0; h < heads; ++h) {
                for (int64_t t = 0; t < tokens; ++t) {
                    std::copy_n(v.data() + (h * tokens + t) * vh, vh, value_host + (t * heads + h) * vh);
                }
            }
        }
        return LM_OK;
    } catch (const std::bad_alloc&) {
        return fail(LM_ENOMEM, "host allocation failed");
    }
}

}  // namespace

extern "C" {

int lm_mla_softmax_scale(const lm_mla_config* config, float* out) {
    int rc = check_config(config);
    if (rc != LM_OK) {
        return rc;
    }
    if (out == nullptr) {
        return fail(LM_EINVAL, "null output");
    }
    *out = softmax_scale(*config);
    return LM_OK;
}

int lm_rope_tables(const lm_mla_config* config, int64_t positions, float* cos_host, float* sin_host) {
    try {
        int rc = check_config(config);
        if (rc != LM_OK) {
            return rc;
        }
        if (positions < 0 || (positions > 0 && (cos_host == nullptr || sin_host == nullptr))) {
            return fail(LM_EINVAL, "bad position count or null table");
        }
        rope_tables(*config, positions, cos_host, sin_host);
        return LM_OK;
    } catch (const std::bad_alloc&) {
        return fail(LM_ENOMEM, "host allocation failed");
    }
}

int lm_attention_configure(lm_context* ctx, const lm_mla_config* config) {
    try {
        if (ctx == nullptr) {
            return fail(LM_EINVAL, "null context");
        }
        int rc = check_config(config);
        if (rc != LM_OK) {
            return rc;
        }
        const lm::ContextInfo info = lm::context_info(ctx);
        if (config->hidden_size != info.hidden) {
            return fail(LM_EINVAL, "attention hidden_size " + std::to_string(config->hidden_size) +
                                       " differs from the context's " + std::to_string(info.hidden));
        }
        if (lm::context_attention(ctx) != nullptr) {
            return fail(LM_EINVAL, "attention is already configured for this context");
        }
        LM_ATT_HIP(hipSetDevice(info.device));
        auto* st = new AttnState();
        st->cfg = *config;
        st->scale = softmax_scale(*config);
        const int64_t cap = config->context_length;
        const int64_t half = config->qk_rope_head_dim / 2;
        const int64_t heads = config->num_heads, nope = config->qk_nope_head_dim, rope = config->qk_rope_head_dim,
                      vh = config->v_head_dim;
        lm::AttnShape& a = st->shape;
        a.heads = config->num_heads;
        a.nope = config->qk_nope_head_dim;
        a.rope = config->qk_rope_head_dim;
        a.vh = config->v_head_dim;
        a.rank = config->kv_lora_rank;
        a.cap = cap;
        a.max_positions = cap;
        auto cleanup = [&](int code) {
            lm::attention_release(st);
            return code;
        };
        // rotary tables, built on the host in double as RotaryEmbedding::build does
        std::vector<float> tables(static_cast<size_t>(2 * cap * half) + 1);
        rope_tables(*config, cap, tables.data(), tables.data() + cap * half);
        hipError_t err = hipMalloc(reinterpret_cast<void**>(&st->tables), tables.size() * sizeof(float));
        if (err == hipSuccess) {
            err = hipMemcpy(st->tables, tables.data(), tables.size() * sizeof(float), hipMemcpyHostToDevice);
        }
        if (err != hipSuccess) {
            return cleanup(fail(err == hipErrorOutOfMemory ? LM_ENOMEM : LM_EHIP,
                                std::string("rotary tables: ") + hipGetErrorString(err)));
        }
        a.cos_t = st->tables;
        a.sin_t = st->tables + cap * half;
        // every layer's cache: key_nope [heads][nope][cap], key_rope [rope][cap], value [heads][cap][vh]
        const int64_t per_layer = cap * (heads * nope + rope + heads * vh);
        const size_t cache_bytes = static_cast<size_t>(per_layer) * static_cast<size_t>(info.layers) * sizeof(float);
        err = hipMalloc(reinterpret_cast<void**>(&st->caches), cache_bytes);
        if (err != hipSuccess) {
            return cleanup(fail(LM_ENOMEM, "KV caches (" + std::to_string(cache_bytes) + " bytes): " +
                                               hipGetErrorString(err)));
        }
        st->layers.resize(static_cast<size_t>(info.layers));
        for (int32_t l = 0; l < info.layers; ++l) {
            float* base = st->caches + static_cast<int64_t>(l) * per_layer;
            st->layers[l].cache.key_nope = base;
            st->layers[l].cache.key_rope = base + cap * heads * nope;
            st->layers[l].cache.value = base + cap * (heads * nope + rope);
        }
        if (!lm::attention_shape_supported(a)) {
            return cleanup(fail(LM_EINVAL, "attention shape not supported"));
        }
        err = hipStreamCreateWithFlags(&st->side, hipStreamNonBlocking);  // default priority
        if (err == hipSuccess) {
            err = hipEventCreateWithFlags(&st->fork, hipEventDisableTiming);
        }
        if (err == hipSuccess) {
            err = hipEventCreateWithFlags(&st->join, hipEventDisableTiming);
        }
        if (err != hipSuccess) {
            return cleanup(fail(LM_EHIP, std::string("attention stream: ") + hipGetErrorString(err)));
        }
        lm::context_attention(ctx) = st;
        return LM_OK;
    } catch (const std::bad_alloc&) {
        return fail(LM_ENOMEM, "host allocation failed");
    }
}

int lm_upload_attention(lm_context* ctx, int32_t layer, const uint16_t* q_proj_host, const uint16_t* q_a_proj_host,
                        const float* q_a_layernorm_host, const uint16_t* q_b_proj_host,
                        const uint16_t* kv_a_proj_host, const float* kv_a_layernorm_host,
                        const uint16_t* kv_b_proj_host, const uint16_t* o_proj_host) {
    AttnState* st = nullptr;
    int rc = get_state(ctx, &st);
    if (rc == LM_OK) {
        rc = check_attn_layer(st, layer);
    }
    if (rc != LM_OK) {
        return rc;
    }
    const lm_mla_config& c = st->cfg;
    const bool lora = c.q_lora_rank > 0;
    if (lora ? (q_proj_host != nullptr || q_a_proj_host == nullptr || q_a_layernorm_host == nullptr ||
                q_b_proj_host == nullptr)
             : (q_proj_host == nullptr || q_a_proj_host != nullptr || q_a_layernorm_host != nullptr ||
                q_b_proj_host != nullptr)) {
        return fail(LM_EINVAL, lora ? "q_lora_rank > 0: pass q_a_proj, q_a_layernorm and q_b_proj, not q_proj"
                                    : "q_lora_rank == 0: pass q_proj, not q_a_proj / q_a_layernorm / q_b_proj");
    }
    if (kv_a_proj_host == nullptr || kv_a_layernorm_host == nullptr || kv_b_proj_host == nullptr ||
        o_proj_host == nullptr) {
        return fail(LM_EINVAL, "null kv_a_proj, kv_a_layernorm, kv_b_proj or o_proj");
    }
    const lm::ContextInfo info = lm::context_info(ctx);
    LM_ATT_HIP(hipSetDevice(info.device));
    const int64_t H = c.hidden_size, heads = c.num_heads, qk = c.qk_nope_head_dim + c.qk_rope_head_dim;
    const int64_t rank = c.kv_lora_rank, rope = c.qk_rope_head_dim, vh = c.v_head_dim, ql = c.q_lora_rank;
    // element counts, each piece 256-byte aligned in the slab
    const int64_t n_q = lora ? 0 : heads * qk * H;
    const int64_t n_qa = lora ? ql * H : 0;
    const int64_t n_qan = lora ? ql : 0;
    const int64_t n_qb = lora ? heads * qk * ql : 0;
    const int64_t n_kva = (rank + rope) * H;
    const int64_t n_kvb = heads * (c.qk_nope_head_dim + vh) * rank;
    const int64_t n_o = H * heads * vh;
    auto align = [](int64_t bytes) { return (bytes + 255) / 256 * 256; };
    const int64_t off_q = 0;
    const int64_t off_qa = off_q + align(2 * n_q);
    const int64_t off_qan = off_qa + align(2 * n_qa);
    const int64_t off_qb = off_qan + align(4 * n_qan);
    const int64_t off_kva = off_qb + align(2 * n_qb);
    const int64_t off_kvan = off_kva + align(2 * n_kva);
    const int64_t off_kvb = off_kvan + align(4 * rank);
    const int64_t off_o = off_kvb + align(2 * n_kvb);
    const int64_t total = off_o + align(2 * n_o);
    AttnLayer& L = st->layers[static_cast<size_t>(layer)];
    LM_ATT_HIP(hipStreamSynchronize(info.stream));
    (void)hipFree(L.slab);
    L.slab = nullptr;
    L.kv_a = nullptr;
    hipError_t err = hipMalloc(&L.slab, static_cast<size_t>(total));
    if (err != hipSuccess) {
        return fail(LM_ENOMEM, "attention weights of layer " + std::to_string(layer) + ": " + hipGetErrorString(err));
    }
    char* base = static_cast<char*>(L.slab);
    if (lora) {
        rc = upload(info.stream, base + off_qa, q_a_proj_host, static_cast<size_t>(2 * n_qa));
        if (rc == LM_OK) {
            rc = upload(info.stream, base + off_qan, q_a_layernorm_host, static_cast<size_t>(4 * n_qan));
        }
        if (rc == LM_OK) {
            rc = upload(info.stream, base + off_qb, q_b_proj_host, static_cast<size_t>(2 * n_qb));
        }
    } else {
        rc = upload(info.stream, base + off_q, q_proj_host, static_cast<size_t>(2 * n_q));
    }
    if (rc == LM_OK) {
        rc = upload(info.stream, base + off_kva, kv_a_proj_host, static_cast<size_t>(2 * n_kva));
    }
    if (rc == LM_OK) {
        rc = upload(info.stream, base + off_kvan, kv_a_layernorm_host, static_cast<size_t>(4 * rank));
    }
    if (rc == LM_OK) {
        rc = upload(info.stream, base + off_kvb, kv_b_proj_host, static_cast<size_t>(2 * n_kvb));
    }
    if (rc == LM_OK) {
        rc = upload(info.stream, base + off_o, o_proj_host, static_cast<size_t>(2 * n_o));
    }
    if (rc == LM_OK) {
        const hipError_t e = hipStreamSynchronize(info.stream);
        if (e != hipSuccess) {
            rc = fail(LM_EHIP, std::string("upload: ") + hipGetErrorString(e));
        }
    }
    if (rc != LM_OK) {
        (void)hipFree(L.slab);
        L.slab = nullptr;
        return rc;
    }
    // fp16 panel copies of the projections for the MFMA path, when every width
    // a projection reads is a multiple of 32 and no weight overflows fp16
    (void)hipFree(L.slab16);
    L.slab16 = nullptr;
    L.table16 = nullptr;
    const bool panels = H % lm::kPanel == 0 && rank % lm::kPanel == 0 && (heads * vh) % lm::kPanel == 0 &&
                        (!lora || ql % lm::kPanel == 0);
    if (panels) {
        struct Piece {
            int proj;
            int64_t off, rows, cols;
        };
        const Piece pieces[] = {{lm::kProjQ, off_q, lora ? 0 : heads * qk, H},
                                {lm::kProjQa, off_qa, lora ? ql : 0, H},
                                {lm::kProjQb, off_qb, lora ? heads * qk : 0, ql},
                                {lm::kProjKva, off_kva, rank + rope, H},
                                {lm::kProjKvb, off_kvb, heads * (c.qk_nope_head_dim + vh), rank},
                                {lm::kProjO, off_o, H, heads * vh}};
        int64_t bytes16 = align(static_cast<int64_t>(sizeof(void*)) * lm::kProjCount + sizeof(int));
        int64_t offs16[lm::kProjCount] = {};
        for (const Piece& pc : pieces) {
            offs16[pc.proj] = bytes16;
            bytes16 += align(pc.rows * pc.cols * 2);
        }
        err = hipMalloc(&L.slab16, static_cast<size_t>(bytes16));
        if (err != hipSuccess) {
            (void)hipFree(L.slab);
            L.slab = nullptr;
            return fail(LM_ENOMEM, "fp16 attention weights of layer " + std::to_string(layer) + ": " +
                                       hipGetErrorString(err));
        }
        char* b16 = static_cast<char*>(L.slab16);
        int* d_overflow = reinterpret_cast<int*>(b16 + sizeof(void*) * lm::kProjCount);
        const _Float16* table[lm::kProjCount] = {};
        for (const Piece& pc : pieces) {
            table[pc.proj] = pc.rows > 0 ? reinterpret_cast<const _Float16*>(b16 + offs16[pc.proj]) : nullptr;
        }
        rc = LM_OK;
        err = hipMemcpyAsync(b16, table, sizeof table, hipMemcpyHostToDevice, info.stream);
        if (err == hipSuccess) {
            err = hipMemsetAsync(d_overflow, 0, sizeof(int), info.stream);
        }
        for (const Piece& pc : pieces) {
            if (err == hipSuccess && pc.rows > 0) {
                err = lm::launch_bf16_to_f16_panels(reinterpret_cast<const uint16_t*>(base + pc.off),
                                                    reinterpret_cast<_Float16*>(b16 + offs16[pc.proj]), pc.rows,
                                                    pc.cols, d_overflow, nullptr, info.stream);
            }
        }
        int overflow = 0;
        if (err == hipSuccess) {
            err = hipMemcpyAsync(&overflow, d_overflow, sizeof(int), hipMemcpyDeviceToHost, info.stream);
        }
        if (err == hipSuccess) {
            err = hipStreamSynchronize(info.stream);
        }
        if (err != hipSuccess) {
            (void)hipFree(L.slab);
            (void)hipFree(L.slab16);
            L.slab = L.slab16 = nullptr;
            return fail(LM_EHIP, std::string("fp16 attention weights: ") + hipGetErrorString(err));
        }
        if (overflow == 0) {
            L.table16 = reinterpret_cast<const _Float16* const*>(b16);
        } else {
            (void)hipFree(L.slab16);  // a weight outside fp16's range: the layer keeps the BF16 path
            L.slab16 = nullptr;
        }
    }
    L.q_proj = lora ? nullptr : reinterpret_cast<const uint16_t*>(base + off_q);
    L.q_a = lora ? reinterpret_cast<const uint16_t*>(base + off_qa) : nullptr;
    L.q_a_norm = lora ? reinterpret_cast<const float*>(base + off_qan) : nullptr;
    L.q_b = lora ? reinterpret_cast<const uint16_t*>(base + off_qb) : nullptr;
    L.kv_a_norm = reinterpret_cast<const float*>(base + off_kvan);
    L.kv_b = reinterpret_cast<const uint16_t*>(base + off_kvb);
    L.o = reinterpret_cast<const uint16_t*>(base + off_o);
    L.kv_a = reinterpret_cast<const uint16_t*>(base + off_kva);
    return LM_OK;
}

int lm_upload_input_norm(lm_context* ctx, int32_t layer, const float* weight_host) {
    AttnState* st = nullptr;
    int rc = get_state(ctx, &st);
    if (rc == LM_OK) {
        rc = check_attn_layer(st, layer);
    }
    if (rc != LM_OK) {
        return rc;
    }
    if (weight_host == nullptr) {
        return fail(LM_EINVAL, "null input_layernorm weight");
    }
    const lm::ContextInfo info = lm::context_info(ctx);
    LM_ATT_HIP(hipSetDevice(info.device));
    AttnLayer& L = st->layers[static_cast<size_t>(layer)];
    if (L.input_norm == nullptr) {
        LM_ATT_HIP(hipMalloc(reinterpret_cast<void**>(&L.input_norm), sizeof(float) * info.hidden));
    }
    LM_ATT_HIP(hipMemcpyAsync(L.input_norm, weight_host, sizeof(float) * info.hidden, hipMemcpyHostToDevice,
                              info.stream));
    LM_ATT_HIP(hipStreamSynchronize(info.stream));
    return LM_OK;
}

int lm_attention_forward(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, int64_t position0,
                         float* out_dev, int32_t accumulate) {
    try {
        AttnState* st = nullptr;
        int rc = get_state(ctx, &st);
        if (rc == LM_OK) {
            rc = check_attn_layer(st, layer);
        }
        if (rc != LM_OK) {
            return rc;
        }
        if (tokens < 0 || position0 < 0) {
            return fail(LM_EINVAL, "negative token count or position");
        }
        if (tokens == 0) {
            return LM_OK;
        }
        if (x_dev == nullptr || out_dev == nullptr) {
            return fail(LM_EINVAL, "null input or output");
        }
        const lm::ContextInfo info = lm::context_info(ctx);
        const size_t row_bytes = sizeof(float) * static_cast<size_t>(info.hidden) * static_cast<size_t>(tokens);
        const char* xb = reinterpret_cast<const char*>(x_dev);
        const char* ob = reinterpret_cast<const char*>(out_dev);
        if (xb < ob + row_bytes && ob < xb + row_bytes) {
            return fail(LM_EINVAL, "out_dev overlaps x_dev");
        }
        AttnLayer& L = st->layers[static_cast<size_t>(layer)];
        const int64_t room = st->cfg.context_length - L.count;
        const int64_t F = std::min(tokens, room);
        if (F > 0) {
            rc = attention_tokens(st, info.stream, layer, x_dev, F, position0, out_dev, accumulate, st->path);
            if (rc != LM_OK) {
                return rc;
            }
        }
        if (F < tokens) {
            return fail(LM_EFULL, "the KV cache of layer " + std::to_string(layer) + " is full (" +
                                      std::to_string(st->cfg.context_length) + " tokens)");
        }
        return LM_OK;
    } catch (const std::bad_alloc&) {
        return fail(LM_ENOMEM, "host allocation failed");
    }
}

int lm_attention_set_path(lm_context* ctx, int32_t path) {
    AttnState* st = nullptr;
    const int rc = get_state(ctx, &st);
    if (rc != LM_OK) {
        return rc;
    }
    if (path < LM_PATH_AUTO || path > LM_PATH_MFMA) {
        return fail(LM_EINVAL, "unknown path");
    }
    st->path = path;
    return LM_OK;
}

int lm_attention_set_score_budget(lm_context* ctx, int64_t bytes) {
    AttnState* st = nullptr;
    const int rc = get_state(ctx, &st);
    if (rc != LM_OK) {
        return rc;
    }
    if (bytes < 0) {
        return fail(LM_EINVAL, "negative score budget");
    }
    st->score_budget = bytes;
    return LM_OK;
}

int lm_attention_plan_core(const lm_mla_config* config, int64_t cached, int64_t tokens, int32_t path,
                           int64_t budget_bytes, lm_attention_core_plan* out) {
    int rc = check_config(config);
    if (rc != LM_OK) {
        return rc;
    }
    if (out == nullptr || cached < 0 || tokens < 0 || budget_bytes < 0) {
        return fail(LM_EINVAL, "null plan or negative size");
    }
    if (path < LM_PATH_AUTO || path > LM_PATH_MFMA) {
        return fail(LM_EINVAL, "unknown path");
    }
    lm::AttnShape a;
    a.heads = config->num_heads;
    a.nope = config->qk_nope_head_dim;
    a.rope = config->qk_rope_head_dim;
    a.vh = config->v_head_dim;
    const CorePlan p = plan_core(a, cached, tokens, mfma_projections(path, tokens),
                                 budget_bytes > 0 ? budget_bytes : kScoreBudget);
    out->query_group = p.group;
    out->scratch_bytes = p.bytes;
    out->mfma_core = p.mfma ? 1 : 0;
    out->reserved = 0;
    return LM_OK;
}

int lm_kv_cache_clear(lm_context* ctx) {
    AttnState* st = nullptr;
    const int rc = get_state(ctx, &st);
    if (rc != LM_OK) {
        return rc;
    }
    // KvCache::clear only resets the count: slots are overwritten before any
    // score reads them.
    for (AttnLayer& L : st->layers) {
        L.count = 0;
    }
    return LM_OK;
}

int lm_kv_cache_tokens(lm_context* ctx, int32_t layer, int64_t* out_tokens) {
    AttnState* st = nullptr;
    int rc = get_state(ctx, &st);
    if (rc == LM_OK) {
        rc = check_attn_layer(st, layer);
    }
    if (rc != LM_OK) {
        return rc;
    }
    if (out_tokens == nullptr) {
        return fail(LM_EINVAL, "null output");
    }
    *out_tokens = st->layers[static_cast<size_t>(layer)].count;
    return LM_OK;
}

int lm_kv_cache_read(lm_context* ctx, int32_t layer, int64_t tokens, float* key_nope_host, float* key_rope_host,
                     float* value_host) {
    return kv_cache_copy(ctx, layer, 0, tokens, key_nope_host, key_rope_host, value_host, false);
}

int lm_kv_cache_read_range(lm_context* ctx, int32_t layer, int64_t token0, int64_t tokens, float* key_nope_host,
                           float* key_rope_host, float* value_host) {
    return kv_cache_copy(ctx, layer, token0, tokens, key_nope_host, key_rope_host, value_host, false);
}

int lm_kv_cache_write(lm_context* ctx, int32_t layer, int64_t token0, int64_t tokens, const float* key_nope_host,
                      const float* key_rope_host, const float* value_host) {
    return kv_cache_copy(ctx, layer, token0, tokens, const_cast<float*>(key_nope_host),
                         const_cast<float*>(key_rope_host), const_cast<float*>(value_host), true);
}

int lm_kv_cache_truncate(lm_context* ctx, int32_t layer, int64_t tokens) {
    AttnState* st = nullptr;
    int rc = get_state(ctx, &st);
    if (rc == LM_OK) {
        rc = check_attn_layer(st, layer);
    }
    if (rc != LM_OK) {
        return rc;
    }
    AttnLayer& L = st->layers[static_cast<size_t>(layer)];
    if (tokens < 0 || tokens > L.count) {
        return fail(LM_EINVAL, "tokens must be within the cache's " + std::to_string(L.count));
    }
    L.count = tokens;  // later calls append from here; queued work keeps the counts it was given
    return LM_OK;
}

int lm_decoder_forward(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev, int64_t tokens,
                       int64_t position0, int32_t path) {
    try {
        AttnState* st = nullptr;
        int rc = get_state(ctx, &st);
        if (rc == LM_OK) {
            rc = check_attn_layer(st, first_layer);
        }
        if (rc == LM_OK) {
            rc = check_attn_layer(st, last_layer);
        }
        if (rc != LM_OK) {
            return rc;
        }
        if (tokens < 0 || position0 < 0 || first_layer > last_layer) {
            return fail(LM_EINVAL, "negative token count or position, or first_layer > last_layer");
        }
        if (tokens == 0) {
            return LM_OK;
        }
        if (hidden_dev == nullptr) {
            return fail(LM_EINVAL, "null hidden state");
        }
        const lm::ContextInfo info = lm::context_info(ctx);
        int64_t F = tokens;
        for (int32_t l = first_layer; l <= last_layer; ++l) {
            const AttnLayer& L = st->layers[static_cast<size_t>(l)];
            if (L.input_norm == nullptr || L.kv_a == nullptr) {
                return fail(LM_ENOTRES, "layer " + std::to_string(l) + " has no attention weights or input norm");
            }
            F = std::min(F, st->cfg.context_length - L.count);
        }
        if (F > 0) {
            // normalised input rows live in a buffer of their own (the attention
            // scratch is resized inside each layer's call)
            rc = ensure_buffer(&st->xn, &st->xn_floats, info.stream, static_cast<size_t>(info.hidden * F));
            if (rc != LM_OK) {
                return rc;
            }
            float* xn = st->xn;
            for (int32_t l = first_layer; l <= last_layer && rc == LM_OK; ++l) {
                rc = attention_tokens(st, info.stream, l, hidden_dev, F, position0, hidden_dev, 1, path,
                                      st->layers[l].input_norm, xn);
                if (rc == LM_OK) {
                    rc = lm::ffn_sublayer(ctx, l, hidden_dev, F, path);
                }
            }
            if (rc != LM_OK) {
                return rc;
            }
        }
        if (F < tokens) {
            return fail(LM_EFULL, "the KV cache is full (" + std::to_string(st->cfg.context_length) + " tokens)");
        }
        return LM_OK;
    } catch (const std::bad_alloc&) {
        return fail(LM_ENOMEM, "host allocation failed");
    }
}

}  // extern "C"
