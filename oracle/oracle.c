/*
 * oracle.c -- CPU restatement of LiteMind's mixture-of-experts feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the thing measured
 * or shipped.  Compiled with -ffp-contract=off; every fused multiply-add that the
 * reference's GCC build performs is written out as fmaf().  Citations are
 * LiteMind source paths.
 *
 * Pinning (what checks each function against something other than itself):
 *   orc_dot_bf16 / matvec*      KernelTest.cpp:28-79 fixtures + the compiled reference
 *   orc_dot_f32 / matvec_f32    closed form (unfused, left to right) + compiled reference
 *   orc_softmax                 KernelTest.cpp:92-102 + compiled reference
 *   orc_silu_multiply           KernelTest.cpp:104-110 + compiled reference
 *   orc_rms_norm                KernelTest.cpp:81-90 + compiled reference
 *   orc_router_select           MoeRouterSamplerTest.cpp:30-93 + brute-force sort + compiled reference
 *   orc_permute                 brute-force stable sort + invariants (no reference counterpart)
 *   orc_moe_layer               compiled reference (per-token runner composition) + float64 brute force
 *   orc_rope_tables / _apply    compiled reference (tables read back through its apply on unit pairs),
 *                               closed forms (position 0, the rotation's norm), float64 brute force
 *   orc_mla_forward             compiled reference (Attention::forward over token sequences, cache
 *                               contents) + float64 brute force of the attention
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bits_to_float(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* Round-to-nearest-even float -> BF16, as tests/KernelTest.cpp:15-20 writes weights. */
uint16_t orc_bf16_rne(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof bits);
    const uint32_t rounded = bits + 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(rounded >> 16);
}

/* src/Gemm.cpp:18-20 (widen): BF16 bits shifted into the high half of a float. */
static inline float widen(uint16_t bits) { return bits_to_float((uint32_t)bits << 16); }
float orc_widen(uint16_t bits) { return widen(bits); }

/* std::exp(float) resolves to the C library's expf (glibc 2.35 on this image). */
float orc_expf(float x) { return expf(x); }

/*
 * src/Gemm.cpp:46-82 (dot_bf16, AVX2 + FMA branch).  Four 8-lane accumulators
 * take 32 elements per step with a fused multiply-add, a second loop takes 8 at a
 * time into accumulator 0, then (a0+a1)+(a2+a3) lane-wise, then
 * horizontal_sum (:24-31): lanes j and j+4 are added, then (h0+h2) + (h1+h3).
 * The scalar tail `total += widen(w) * x` is contracted to an FMA by GCC.
 */
float orc_dot_bf16(const uint16_t* weights, const float* input, size_t count) {
    float acc[4][8];
    memset(acc, 0, sizeof acc);
    size_t index = 0;
    for (; index + 32 <= count; index += 32) {
        for (int k = 0; k < 4; ++k) {
            for (int lane = 0; lane < 8; ++lane) {
                const size_t at = index + (size_t)k * 8 + (size_t)lane;
                acc[k][lane] = fmaf(widen(weights[at]), input[at], acc[k][lane]);
            }
        }
    }
    for (; index + 8 <= count; index += 8) {
        for (int lane = 0; lane < 8; ++lane) {
            acc[0][lane] = fmaf(widen(weights[index + lane]), input[index + lane], acc[0][lane]);
        }
    }
    float sum[8];
    for (int lane = 0; lane < 8; ++lane) {
        const float low = acc[0][lane] + acc[1][lane];
        const float high = acc[2][lane] + acc[3][lane];
        sum[lane] = low + high;
    }
    const float h0 = sum[0] + sum[4];
    const float h1 = sum[1] + sum[5];
    const float h2 = sum[2] + sum[6];
    const float h3 = sum[3] + sum[7];
    float total = (h0 + h2) + (h1 + h3);
    for (; index < count; ++index) {
        total = fmaf(widen(weights[index]), input[index], total);
    }
    return total;
}

/*
 * src/Gemm.cpp:183-189 (dot).  GCC -O3 vectorises the products and keeps the
 * additions in source order (no reassociation without -ffast-math): each product
 * is rounded, then added strictly left to right, t = fl(t + fl(a*b)).  With AVX2
 * the vector body takes 8 elements and one 4-element epilogue; the last
 * count % 4 elements run through a scalar loop that GCC contracts to an FMA.
 * The MoE path (H = 2048) never reaches that tail.
 */
float orc_dot_f32(const float* left, const float* right, size_t count) {
    const size_t unfused = count - count % 4;
    float total = 0.0f;
    size_t index = 0;
    for (; index < unfused; ++index) {
        const float product = left[index] * right[index];
        total = total + product;
    }
    for (; index < count; ++index) {
        total = fmaf(left[index], right[index], total);
    }
    return total;
}

/* src/Gemm.cpp:125-130 and :139-154: one dot_bf16 per output row (threading does
 * not change any row's arithmetic). */
void orc_matvec_bf16(const uint16_t* weights, const float* input, float* out, size_t out_dim, size_t in_dim) {
    for (size_t row = 0; row < out_dim; ++row) {
        out[row] = orc_dot_bf16(weights + row * in_dim, input, in_dim);
    }
}

/* src/Gemm.cpp:156-175: out[row] += scale * dot, which GCC contracts to
 * fma(scale, dot, out[row]). */
void orc_matvec_bf16_accumulate(const uint16_t* weights, const float* input, float* out, size_t out_dim,
                                size_t in_dim, float scale) {
    for (size_t row = 0; row < out_dim; ++row) {
        out[row] = fmaf(scale, orc_dot_bf16(weights + row * in_dim, input, in_dim), out[row]);
    }
}

/* src/Gemm.cpp:132-137. */
void orc_matvec_f32(const float* weights, const float* input, float* out, size_t out_dim, size_t in_dim) {
    for (size_t row = 0; row < out_dim; ++row) {
        out[row] = orc_dot_f32(weights + row * in_dim, input, in_dim);
    }
}

/* src/Gemm.cpp:209-223: max, exp(v - max) summed left to right, multiply by the
 * correctly rounded reciprocal. */
void orc_softmax(float* values, size_t count) {
    if (count == 0) {
        return;
    }
    float maximum = values[0];
    for (size_t index = 1; index < count; ++index) {
        if (maximum < values[index]) {
            maximum = values[index];
        }
    }
    float total = 0.0f;
    for (size_t index = 0; index < count; ++index) {
        values[index] = orc_expf(values[index] - maximum);
        total = total + values[index];
    }
    const float inverse = total > 0.0f ? 1.0f / total : 0.0f;
    for (size_t index = 0; index < count; ++index) {
        values[index] = values[index] * inverse;
    }
}

/* src/Gemm.cpp:225-231: value / (1 + exp(-value)) * up, two roundings after the exp. */
void orc_silu_multiply(const float* gate, const float* up, float* out, size_t count) {
    for (size_t index = 0; index < count; ++index) {
        const float value = gate[index];
        const float sigmoid_part = value / (1.0f + orc_expf(-value));
        out[index] = sigmoid_part * up[index];
    }
}

/* src/Gemm.cpp:197-207.  The float32 square is exact in double, so whether GCC
 * fuses the double multiply-add does not change the sum. */
void orc_rms_norm(float* values, const float* weight, size_t count, float epsilon) {
    double sum_of_squares = 0.0;
    for (size_t index = 0; index < count; ++index) {
        const double v = (double)values[index];
        sum_of_squares = sum_of_squares + v * v;
    }
    const float inverse = (float)(1.0 / sqrt(sum_of_squares / (double)count + (double)epsilon));
    for (size_t index = 0; index < count; ++index) {
        const float scaled = values[index] * inverse;
        values[index] = scaled * weight[index];
    }
}

/* src/Gemm.cpp:191-195, contracted by GCC to fma(scale, source, destination). */
void orc_axpy(float scale, const float* source, float* destination, size_t count) {
    for (size_t index = 0; index < count; ++index) {
        destination[index] = fmaf(scale, source[index], destination[index]);
    }
}

/* ------------------------------------------------------------------------- */
/* Router: src/MoeRouter.cpp                                                  */
/* ------------------------------------------------------------------------- */

/* The comparator of src/MoeRouter.cpp:21-32: allowed first, then higher score,
 * then lower index.  Returns nonzero when `left` orders before `right`. */
static int router_before(const float* scores, const unsigned char* allowed, int left, int right) {
    const int la = allowed == NULL || allowed[left];
    const int ra = allowed == NULL || allowed[right];
    if (la != ra) {
        return la;
    }
    if (scores[left] != scores[right]) {
        return scores[left] > scores[right];
    }
    return left < right;
}

/* top_k_indices (src/MoeRouter.cpp:14-34): partial_sort leaves the first k
 * entries in comparator order; the comparator is a strict total order over
 * distinct indices, so repeated selection of the minimum reproduces it. */
static int top_k_indices(const float* scores, const unsigned char* allowed, int count, int top_k, int* order) {
    const int take = top_k < count ? top_k : count;
    unsigned char used[1024];
    if (count > 1024) {
        return -1;
    }
    memset(used, 0, (size_t)count);
    for (int slot = 0; slot < take; ++slot) {
        int best = -1;
        for (int candidate = 0; candidate < count; ++candidate) {
            if (used[candidate]) {
                continue;
            }
            if (best < 0 || router_before(scores, allowed, candidate, best)) {
                best = candidate;
            }
        }
        used[best] = 1;
        order[slot] = best;
    }
    return take;
}

/* MoeRouter::select (src/MoeRouter.cpp:54-107) with the constructor's group
 * fallback (:38-52). */
int orc_router_select(const orc_router_cfg* cfg, const float* logits, int32_t logit_count,
                      int32_t* out_index, float* out_weight) {
    int n_group = cfg->n_group > 1 ? cfg->n_group : 1;
    const int topk_group = cfg->topk_group > 1 ? cfg->topk_group : 1;
    int group_limited = cfg->group_limited;
    const int expert_count = cfg->expert_count;
    if (expert_count > 0 && expert_count % n_group != 0) {
        group_limited = 0;
        n_group = 1;
    }
    if (logit_count != expert_count || cfg->top_k == 0 || expert_count == 0 || expert_count > 1024) {
        return 0;
    }

    float scores[1024];
    memcpy(scores, logits, sizeof(float) * (size_t)expert_count);
    orc_softmax(scores, (size_t)expert_count);

    unsigned char allowed_storage[1024];
    const unsigned char* allowed = NULL;
    if (group_limited && n_group > 1) {
        const int per_group = expert_count / n_group;
        float group_scores[1024];
        for (int group = 0; group < n_group; ++group) {
            float best = scores[group * per_group];
            for (int offset = 1; offset < per_group; ++offset) {
                if (best < scores[group * per_group + offset]) {
                    best = scores[group * per_group + offset];
                }
            }
            group_scores[group] = best;
        }
        int group_order[1024];
        const int groups = top_k_indices(group_scores, NULL, n_group, topk_group < n_group ? topk_group : n_group,
                                         group_order);
        memset(allowed_storage, 0, (size_t)expert_count);
        for (int g = 0; g < groups; ++g) {
            for (int offset = 0; offset < per_group; ++offset) {
                allowed_storage[group_order[g] * per_group + offset] = 1;
            }
        }
        allowed = allowed_storage;
    }

    int order[1024];
    const int taken = top_k_indices(scores, allowed, expert_count, cfg->top_k, order);
    float selected_sum = 0.0f;
    for (int slot = 0; slot < taken; ++slot) {
        out_index[slot] = order[slot];
        out_weight[slot] = scores[order[slot]];
        selected_sum = selected_sum + scores[order[slot]];
    }
    if (cfg->top_k > 1 && cfg->normalize) {
        const float denominator = selected_sum + 1e-20f;
        for (int slot = 0; slot < taken; ++slot) {
            out_weight[slot] = out_weight[slot] / denominator;
        }
    } else if (cfg->routed_scaling_factor != 1.0f) {
        for (int slot = 0; slot < taken; ++slot) {
            out_weight[slot] = out_weight[slot] * cfg->routed_scaling_factor;
        }
    }
    return taken;
}

/* ------------------------------------------------------------------------- */
/* Canonical permutation.  The reference visits one token's selections in rank  */
/* order (src/DeepSeekRunner.cpp:277-284) and never groups tokens; the grouped  */
/* GPU path defines the order: expert-major, then token, then rank.            */
/* ------------------------------------------------------------------------- */
void orc_permute(const int32_t* topk_index, int64_t tokens, int32_t top_k, int32_t experts, int32_t* counts,
                 int32_t* offsets, int32_t* perm, int32_t* slot_of) {
    const int64_t total = tokens * (int64_t)top_k;
    for (int e = 0; e < experts; ++e) {
        counts[e] = 0;
    }
    for (int64_t a = 0; a < total; ++a) {
        counts[topk_index[a]] += 1;
    }
    offsets[0] = 0;
    for (int e = 0; e < experts; ++e) {
        offsets[e + 1] = offsets[e] + counts[e];
    }
    int32_t* cursor = (int32_t*)malloc(sizeof(int32_t) * (size_t)(experts > 0 ? experts : 1));
    for (int e = 0; e < experts; ++e) {
        cursor[e] = offsets[e];
    }
    for (int64_t a = 0; a < total; ++a) {
        const int32_t position = cursor[topk_index[a]]++;
        perm[position] = (int32_t)a;
        if (slot_of != NULL) {
            slot_of[a] = position;
        }
    }
    free(cursor);
}

/* ------------------------------------------------------------------------- */
/* MoE block                                                                  */
/* ------------------------------------------------------------------------- */

/* Rows of gate/up, then silu * up, for n tokens of one FFN (src/DeepSeekRunner.cpp:231-235).
 * Row-blocked so a block of weight rows is reused across the tokens; each output
 * element is still exactly one dot_bf16. */
static void ffn_activation(const uint16_t* gate, const uint16_t* up, int hidden, int inter, const float* const* xs,
                           int n, float* act /* [n, inter] */) {
    float* g = (float*)malloc(sizeof(float) * (size_t)n * (size_t)inter);
    float* u = (float*)malloc(sizeof(float) * (size_t)n * (size_t)inter);
    const int block = 16;
    for (int first = 0; first < inter; first += block) {
        const int last = first + block < inter ? first + block : inter;
        for (int j = 0; j < n; ++j) {
            for (int row = first; row < last; ++row) {
                g[(size_t)j * inter + row] = orc_dot_bf16(gate + (size_t)row * hidden, xs[j], (size_t)hidden);
                u[(size_t)j * inter + row] = orc_dot_bf16(up + (size_t)row * hidden, xs[j], (size_t)hidden);
            }
        }
    }
    for (int j = 0; j < n; ++j) {
        orc_silu_multiply(g + (size_t)j * inter, u + (size_t)j * inter, act + (size_t)j * inter, (size_t)inter);
    }
    free(g);
    free(u);
}

/* out[j][row] = dot_bf16(down[row], act[j]) for n activation rows, row-blocked. */
static void ffn_down(const uint16_t* down, int hidden, int inter, const float* act, int n, float* out) {
    const int block = 16;
    for (int first = 0; first < hidden; first += block) {
        const int last = first + block < hidden ? first + block : hidden;
        for (int j = 0; j < n; ++j) {
            for (int row = first; row < last; ++row) {
                out[(size_t)j * hidden + row] =
                    orc_dot_bf16(down + (size_t)row * inter, act + (size_t)j * inter, (size_t)inter);
            }
        }
    }
}

typedef struct ffn_job {
    int expert;    /* -1 = shared */
    int first;     /* first assignment (in permuted order) or first token */
    int count;
} ffn_job;

int orc_moe_layer(const orc_layer_dims* dims, const orc_router_cfg* rcfg, const orc_layer_weights* w,
                  const float* x, int64_t tokens, const float* logit_bias, float* y, float* logits_out,
                  int32_t* topk_index_out, float* topk_weight_out, int32_t threads) {
    const int H = dims->hidden, I = dims->inter, E = dims->experts, K = dims->top_k, S = dims->shared_inter;
    if (tokens <= 0) {
        return 0;
    }
    if (rcfg->top_k != K || rcfg->expert_count != E) {
        return -1;
    }
#ifdef _OPENMP
    if (threads > 0) {
        omp_set_num_threads(threads);
    }
#else
    (void)threads;
#endif
    const int64_t total = tokens * K;
    int32_t* idx = (int32_t*)malloc(sizeof(int32_t) * (size_t)total);
    float* wt = (float*)malloc(sizeof(float) * (size_t)total);
    int bad = 0;

    /* Router: matvec_f32 (src/DeepSeekRunner.cpp:273-274), then select (:275).
     * logit_bias is not part of LiteMind: the skewed-routing workload adds a
     * per-expert bias after the dot, before the softmax. */
#pragma omp parallel for schedule(static) reduction(| : bad)
    for (int64_t t = 0; t < tokens; ++t) {
        float logits[1024];
        orc_matvec_f32(w->router, x + t * H, logits, (size_t)E, (size_t)H);
        if (logit_bias != NULL) {
            for (int e = 0; e < E; ++e) {
                logits[e] = logits[e] + logit_bias[e];
            }
        }
        if (logits_out != NULL) {
            memcpy(logits_out + t * E, logits, sizeof(float) * (size_t)E);
        }
        const int taken = orc_router_select(rcfg, logits, E, idx + t * K, wt + t * K);
        if (taken != K) {
            bad |= 1;
        }
    }
    if (bad) {
        free(idx);
        free(wt);
        return -2;
    }

    int32_t* counts = (int32_t*)malloc(sizeof(int32_t) * (size_t)E);
    int32_t* offsets = (int32_t*)malloc(sizeof(int32_t) * (size_t)(E + 1));
    int32_t* perm = (int32_t*)malloc(sizeof(int32_t) * (size_t)total);
    int32_t* slot_of = (int32_t*)malloc(sizeof(int32_t) * (size_t)total);
    orc_permute(idx, tokens, K, E, counts, offsets, perm, slot_of);

    /* Down-projection results per (token, rank) in permuted order, and per token for the shared expert. */
    float* down_routed = (float*)malloc(sizeof(float) * (size_t)total * (size_t)H);
    float* down_shared = S > 0 ? (float*)malloc(sizeof(float) * (size_t)tokens * (size_t)H) : NULL;

    /* Jobs of up to 16 rows of tokens each so the threads stay busy under skew. */
    const int chunk = 16;
    int job_cap = (int)(total / chunk) + E + (int)(tokens / chunk) + 2;
    ffn_job* jobs = (ffn_job*)malloc(sizeof(ffn_job) * (size_t)job_cap);
    int njobs = 0;
    for (int e = 0; e < E; ++e) {
        for (int first = offsets[e]; first < offsets[e + 1]; first += chunk) {
            const int left = offsets[e + 1] - first;
            jobs[njobs].expert = e;
            jobs[njobs].first = first;
            jobs[njobs].count = left < chunk ? left : chunk;
            ++njobs;
        }
    }
    if (S > 0 && w->shared_gate != NULL) {
        for (int64_t first = 0; first < tokens; first += chunk) {
            const int64_t left = tokens - first;
            jobs[njobs].expert = -1;
            jobs[njobs].first = (int)first;
            jobs[njobs].count = (int)(left < chunk ? left : chunk);
            ++njobs;
        }
    }

#pragma omp parallel for schedule(dynamic, 1)
    for (int j = 0; j < njobs; ++j) {
        const ffn_job job = jobs[j];
        const float* xs[16];
        const uint16_t *gate, *up, *down;
        int inter;
        float* dst;
        if (job.expert >= 0) {
            gate = w->gate[job.expert];
            up = w->up[job.expert];
            down = w->down[job.expert];
            inter = I;
            for (int n = 0; n < job.count; ++n) {
                const int32_t a = perm[job.first + n];
                xs[n] = x + (int64_t)(a / K) * H;
            }
            dst = down_routed + (size_t)job.first * (size_t)H;
        } else {
            gate = w->shared_gate;
            up = w->shared_up;
            down = w->shared_down;
            inter = S;
            for (int n = 0; n < job.count; ++n) {
                xs[n] = x + (int64_t)(job.first + n) * H;
            }
            dst = down_shared + (size_t)job.first * (size_t)H;
        }
        float* act = (float*)malloc(sizeof(float) * (size_t)job.count * (size_t)inter);
        ffn_activation(gate, up, H, inter, xs, job.count, act);
        ffn_down(down, H, inter, act, job.count, dst);
        free(act);
    }

    /* Combine in the runner's order: zeroed output (:268), routed experts in rank
     * order with out += w * dot (:277-284), then the shared expert at scale 1 (:285-288). */
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < tokens; ++t) {
        float* out = y + t * H;
        for (int h = 0; h < H; ++h) {
            out[h] = 0.0f;
        }
        for (int r = 0; r < K; ++r) {
            const int64_t a = t * K + r;
            const float* d = down_routed + (size_t)slot_of[a] * (size_t)H;
            const float scale = wt[a];
            for (int h = 0; h < H; ++h) {
                out[h] = fmaf(scale, d[h], out[h]);
            }
        }
        if (down_shared != NULL) {
            const float* d = down_shared + (size_t)t * (size_t)H;
            for (int h = 0; h < H; ++h) {
                out[h] = fmaf(1.0f, d[h], out[h]);
            }
        }
    }

    if (topk_index_out != NULL) {
        memcpy(topk_index_out, idx, sizeof(int32_t) * (size_t)total);
    }
    if (topk_weight_out != NULL) {
        memcpy(topk_weight_out, wt, sizeof(float) * (size_t)total);
    }
    free(jobs);
    free(down_routed);
    free(down_shared);
    free(counts);
    free(offsets);
    free(perm);
    free(slot_of);
    free(idx);
    free(wt);
    return 0;
}

void orc_dense_ffn(const uint16_t* gate, const uint16_t* up, const uint16_t* down, int32_t hidden, int32_t inter,
                   const float* x, int64_t tokens, float* y, int32_t threads) {
#ifdef _OPENMP
    if (threads > 0) {
        omp_set_num_threads(threads);
    }
#else
    (void)threads;
#endif
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t = 0; t < tokens; ++t) {
        const float* xs[1] = {x + t * hidden};
        float* act = (float*)malloc(sizeof(float) * (size_t)inter);
        ffn_activation(gate, up, hidden, inter, xs, 1, act);
        float* out = y + t * hidden;
        for (int h = 0; h < hidden; ++h) {
            out[h] = 0.0f;
        }
        orc_matvec_bf16_accumulate(down, act, out, (size_t)hidden, (size_t)inter, 1.0f);
        free(act);
    }
}

/* ------------------------------------------------------------------------- */
/* Multi-head latent attention: src/Attention.cpp, src/Rope.cpp, KvCache       */
/* ------------------------------------------------------------------------- */

static const double kPi = 3.14159265358979323846;

/* src/Rope.cpp:13-18; GCC contracts 0.1 * mscale * log(scale) + 1.0 to a fused
 * multiply-add of the rounded 0.1 * mscale. */
static double yarn_mscale(double scale, double mscale) {
    if (scale <= 1.0) {
        return 1.0;
    }
    return fma(0.1 * mscale, log(scale), 1.0);
}

/* Config::softmax_scale (src/Config.cpp:114-121): (qk_nope + qk_rope)^-0.5 in
 * double, times the squared YaRN magnitude when mscale_all_dim is non-zero. */
float orc_softmax_scale(int32_t qk_nope, int32_t qk_rope, int32_t yarn, double factor, double mscale_all_dim) {
    double scale = 1.0 / sqrt((double)(qk_nope + qk_rope));
    if (yarn && mscale_all_dim != 0.0) {
        const double m = yarn_mscale(factor, mscale_all_dim);
        scale *= m * m;
    }
    return (float)scale;
}

/* src/Rope.cpp:24-33. */
static double correction_dimension(double rotations, int32_t dim, double base, int64_t original_max) {
    const double numerator = (double)dim * log((double)original_max / (rotations * 2.0 * kPi));
    return numerator / (2.0 * log(base));
}

/* src/Rope.cpp:36-103: double-precision frequencies (YaRN blend of the
 * extrapolated and interpolated ones), cos and sin in double times the
 * magnitude correction, rounded to float. */
void orc_rope_tables(int32_t dim, int32_t max_positions, double theta, int32_t yarn, double factor,
                     double beta_fast, double beta_slow, double mscale, double mscale_all_dim,
                     int64_t original_max_positions, float* cos_out, float* sin_out) {
    const int32_t half = dim / 2;
    const double base = theta;
    double inverse[512];
    double magnitude = 1.0;
    if (half > 512) {
        return;
    }
    if (!yarn) {
        for (int32_t i = 0; i < half; ++i) {
            const double exponent = 2.0 * (double)i / (double)dim;
            inverse[i] = 1.0 / pow(base, exponent);
        }
    } else {
        const double f = factor <= 0.0 ? 1.0 : factor;
        double low = floor(correction_dimension(beta_fast, dim, base, original_max_positions));
        double high = ceil(correction_dimension(beta_slow, dim, base, original_max_positions));
        low = low > 0.0 ? low : 0.0;
        high = high < (double)dim - 1.0 ? high : (double)dim - 1.0;
        if (high - low < 1e-6) {
            high = low + 0.001;
        }
        for (int32_t i = 0; i < half; ++i) {
            const double exponent = 2.0 * (double)i / (double)dim;
            const double extrapolation = 1.0 / pow(base, exponent);
            const double interpolation = extrapolation / f;
            double ramp = ((double)i - low) / (high - low);
            ramp = ramp < 0.0 ? 0.0 : (ramp > 1.0 ? 1.0 : ramp);
            const double mask = 1.0 - ramp;
            const double a = interpolation * (1.0 - mask);
            const double b = extrapolation * mask;
            inverse[i] = a + b;
        }
        magnitude = yarn_mscale(f, mscale) / yarn_mscale(f, mscale_all_dim);
    }
    for (int64_t p = 0; p < max_positions; ++p) {
        for (int32_t i = 0; i < half; ++i) {
            const double angle = (double)p * inverse[i];
            cos_out[p * half + i] = (float)(cos(angle) * magnitude);
            sin_out[p * half + i] = (float)(sin(angle) * magnitude);
        }
    }
}

/* src/Rope.cpp:105-127: channels (2i, 2i + 1) rotated into (i, i + half); GCC
 * contracts each output to one fused multiply-add whose addend is the other
 * product, rounded: lo = fma(even, cos, -(odd * sin)), hi = fma(odd, cos,
 * even * sin) (checked against the compiled RotaryEmbedding::apply). */
void orc_rope_apply(float* values, int32_t dim, const float* cos_row, const float* sin_row) {
    float source[1024];
    const int32_t half = dim / 2;
    if (dim > 1024) {
        return;
    }
    memcpy(source, values, sizeof(float) * (size_t)dim);
    for (int32_t i = 0; i < half; ++i) {
        const float even = source[2 * i];
        const float odd = source[2 * i + 1];
        /* even*cos - odd*sin and odd*cos + even*sin as LiteMind's build
         * contracts them: the first product of each into the fma */
        const float odd_sin = odd * sin_row[i];
        const float even_sin = even * sin_row[i];
        values[i] = fmaf(even, cos_row[i], -odd_sin);
        values[i + half] = fmaf(odd, cos_row[i], even_sin);
    }
}

/* src/Attention.cpp:22-103 with KvCache::append (src/KvCache.cpp) for one token. */
int orc_mla_forward(const orc_mla_dims* d, const orc_mla_weights* w, const float* cos_table, const float* sin_table,
                    float* key_nope, float* key_rope, float* value, int64_t capacity, int64_t* token_count,
                    const float* x, int64_t position, float* out) {
    const int32_t H = d->hidden, heads = d->heads, nope = d->qk_nope, rope = d->qk_rope, vh = d->v_head;
    const int32_t qk = nope + rope, rank = d->kv_lora_rank, half = rope / 2;
    float* query = (float*)malloc(sizeof(float) * (size_t)heads * (size_t)qk);
    float* q_latent = (float*)malloc(sizeof(float) * (size_t)(d->q_lora_rank > 0 ? d->q_lora_rank : 1));
    float* latent = (float*)malloc(sizeof(float) * (size_t)(rank + rope));
    float* expanded = (float*)malloc(sizeof(float) * (size_t)heads * (size_t)(nope + vh));
    float* context = (float*)malloc(sizeof(float) * (size_t)heads * (size_t)vh);
    float* scores = (float*)malloc(sizeof(float) * (size_t)(capacity > 0 ? capacity : 1));
    int rc = 0;
    /* queries (:34-45) */
    if (d->q_lora_rank == 0) {
        orc_matvec_bf16(w->q_proj, x, query, (size_t)heads * (size_t)qk, (size_t)H);
    } else {
        orc_matvec_bf16(w->q_a_proj, x, q_latent, (size_t)d->q_lora_rank, (size_t)H);
        orc_rms_norm(q_latent, w->q_a_layernorm, (size_t)d->q_lora_rank, d->rms_norm_eps);
        orc_matvec_bf16(w->q_b_proj, q_latent, query, (size_t)heads * (size_t)qk, (size_t)d->q_lora_rank);
    }
    /* rotary channels of each head (:48-50); apply is a no-op past the table (src/Rope.cpp:106-108) */
    const int rotate = position >= 0 && position < d->max_positions;
    for (int32_t h = 0; h < heads && rotate; ++h) {
        orc_rope_apply(query + (size_t)h * (size_t)qk + (size_t)nope, rope, cos_table + position * half,
                       sin_table + position * half);
    }
    /* compressed key and value (:53-61) */
    orc_matvec_bf16(w->kv_a_proj, x, latent, (size_t)(rank + rope), (size_t)H);
    orc_rms_norm(latent, w->kv_a_layernorm, (size_t)rank, d->rms_norm_eps);
    if (rotate) {
        orc_rope_apply(latent + rank, rope, cos_table + position * half, sin_table + position * half);
    }
    orc_matvec_bf16(w->kv_b_proj, latent, expanded, (size_t)heads * (size_t)(nope + vh), (size_t)rank);
    /* append (:63-77, src/KvCache.cpp) */
    if (*token_count >= capacity) {
        rc = -1;
        goto done;
    }
    {
        const int64_t slot = (*token_count)++;
        for (int32_t h = 0; h < heads; ++h) {
            memcpy(key_nope + ((size_t)slot * heads + h) * nope, expanded + (size_t)h * (nope + vh),
                   sizeof(float) * (size_t)nope);
            memcpy(value + ((size_t)slot * heads + h) * vh, expanded + (size_t)h * (nope + vh) + nope,
                   sizeof(float) * (size_t)vh);
        }
        memcpy(key_rope + (size_t)slot * rope, latent + rank, sizeof(float) * (size_t)rope);
    }
    /* attention over every cached position (:79-98) */
    {
        const int64_t length = *token_count;
        memset(context, 0, sizeof(float) * (size_t)heads * (size_t)vh);
        for (int32_t h = 0; h < heads; ++h) {
            const float* qn = query + (size_t)h * qk;
            const float* qr = qn + nope;
            for (int64_t t = 0; t < length; ++t) {
                const float a = orc_dot_f32(qn, key_nope + ((size_t)t * heads + h) * nope, (size_t)nope);
                const float b = orc_dot_f32(qr, key_rope + (size_t)t * rope, (size_t)rope);
                const float sum = a + b;
                scores[t] = d->softmax_scale * sum;
            }
            orc_softmax(scores, (size_t)length);
            for (int64_t t = 0; t < length; ++t) {
                orc_axpy(scores[t], value + ((size_t)t * heads + h) * vh, context + (size_t)h * vh, (size_t)vh);
            }
        }
    }
    /* output projection (:100-101) */
    orc_matvec_bf16(w->o_proj, context, out, (size_t)H, (size_t)heads * (size_t)vh);
done:
    free(query);
    free(q_latent);
    free(latent);
    free(expanded);
    free(context);
    free(scores);
    return rc;
}
