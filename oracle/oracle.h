/*
 * oracle.h -- CPU restatement of LiteMind's mixture-of-experts feed-forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker.  The product
 * path (litemind_amd/) never links or calls it.
 *
 * Every function restates one piece of the reference and cites it (paths are
 * relative to the LiteMind source tree).  Floating-point order follows what the
 * reference's own build (GCC, -O3, AVX2 + FMA, -std=c++20, default
 * -ffp-contract=fast for C++) executes; where GCC fuses a multiply into an add
 * the restatement calls fmaf() explicitly, and this file is compiled with
 * -ffp-contract=off so nothing else is fused behind our back.
 *
 * How each function is pinned (checked against something other than itself) is
 * listed in tests/test_oracle_*.py.
 */
#ifndef LITEMIND_ORACLE_H
#define LITEMIND_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Routing policy, the MoE subset of Config (include/Config.hpp:66-71). */
typedef struct orc_router_cfg {
    int32_t expert_count;        /* n_routed_experts */
    int32_t top_k;               /* num_experts_per_tok */
    int32_t n_group;             /* n_group (>=1) */
    int32_t topk_group;          /* topk_group (>=1) */
    int32_t group_limited;       /* topk_method == "group_limited_greedy" */
    int32_t normalize;           /* norm_topk_prob */
    float routed_scaling_factor; /* routed_scaling_factor */
} orc_router_cfg;

/* Shapes of one MoE layer (include/Config.hpp:58-64, :101-103). */
typedef struct orc_layer_dims {
    int32_t hidden;        /* hidden_size, H */
    int32_t inter;         /* moe_intermediate_size, I */
    int32_t experts;       /* n_routed_experts, E */
    int32_t top_k;         /* num_experts_per_tok, k */
    int32_t shared_inter;  /* moe_intermediate_size * n_shared_experts (0 = none) */
} orc_layer_dims;

/* One MoE layer's weights in host memory, reference layout (row-major, BF16 bits). */
typedef struct orc_layer_weights {
    const float* router;             /* [E, H] fp32 */
    const uint16_t* const* gate;     /* E pointers to [I, H] */
    const uint16_t* const* up;       /* E pointers to [I, H] */
    const uint16_t* const* down;     /* E pointers to [H, I] */
    const uint16_t* shared_gate;     /* [S, H] or NULL */
    const uint16_t* shared_up;       /* [S, H] */
    const uint16_t* shared_down;     /* [H, S] */
} orc_layer_weights;

/* ---- scalar kernels (src/Gemm.cpp) ---- */
uint16_t orc_bf16_rne(float value);
float orc_widen(uint16_t bits);
float orc_expf(float x); /* the C library expf the reference calls through std::exp(float) */
float orc_dot_bf16(const uint16_t* weights, const float* input, size_t count);
float orc_dot_f32(const float* left, const float* right, size_t count);
void orc_matvec_bf16(const uint16_t* weights, const float* input, float* out, size_t out_dim, size_t in_dim);
void orc_matvec_bf16_accumulate(const uint16_t* weights, const float* input, float* out, size_t out_dim,
                                size_t in_dim, float scale);
void orc_matvec_f32(const float* weights, const float* input, float* out, size_t out_dim, size_t in_dim);
void orc_softmax(float* values, size_t count);
void orc_silu_multiply(const float* gate, const float* up, float* out, size_t count);
void orc_rms_norm(float* values, const float* weight, size_t count, float epsilon);
void orc_axpy(float scale, const float* source, float* destination, size_t count);

/* ---- router (src/MoeRouter.cpp) ---- */
/* Returns the number of selected experts (0 on the reference's silent-empty cases). */
int orc_router_select(const orc_router_cfg* cfg, const float* logits, int32_t logit_count,
                      int32_t* out_index, float* out_weight);

/* ---- canonical permutation (no reference counterpart) ---- */
void orc_permute(const int32_t* topk_index, int64_t tokens, int32_t top_k, int32_t experts,
                 int32_t* counts, int32_t* offsets, int32_t* perm, int32_t* slot_of);

/* ---- the MoE block (src/DeepSeekRunner.cpp:228-240, :264-290) ---- */
/* x: [T, H] fp32 (already normalised), y: [T, H] ffn output (no residual).
 * logit_bias: NULL or [E] added after the router dot (a harness extension, see .c).
 * logits/topk_index/topk_weight: optional outputs ([T,E], [T,k], [T,k]). */
int orc_moe_layer(const orc_layer_dims* dims, const orc_router_cfg* rcfg, const orc_layer_weights* w,
                  const float* x, int64_t tokens, const float* logit_bias, float* y, float* logits,
                  int32_t* topk_index, float* topk_weight, int32_t threads);

/* Dense SwiGLU FFN for T tokens: y[t] = down . (silu(gate . x) * (up . x)), the
 * feed_forward() of src/DeepSeekRunner.cpp:228-240 with scale 1 into a zeroed output. */
void orc_dense_ffn(const uint16_t* gate, const uint16_t* up, const uint16_t* down, int32_t hidden,
                   int32_t inter, const float* x, int64_t tokens, float* y, int32_t threads);

/* ---- multi-head latent attention (src/Attention.cpp, src/Rope.cpp, src/KvCache.cpp) ---- */
typedef struct orc_mla_dims {
    int32_t hidden, heads, q_lora_rank, kv_lora_rank, qk_nope, qk_rope, v_head;
    float softmax_scale, rms_norm_eps;
    int32_t max_positions;  /* rows of the rotary tables */
} orc_mla_dims;

typedef struct orc_mla_weights {
    const uint16_t* q_proj;        /* [heads * (qk_nope + qk_rope), hidden] when q_lora_rank == 0 */
    const uint16_t* q_a_proj;      /* [q_lora_rank, hidden] */
    const float* q_a_layernorm;    /* [q_lora_rank] */
    const uint16_t* q_b_proj;      /* [heads * (qk_nope + qk_rope), q_lora_rank] */
    const uint16_t* kv_a_proj;     /* [kv_lora_rank + qk_rope, hidden] */
    const float* kv_a_layernorm;   /* [kv_lora_rank] */
    const uint16_t* kv_b_proj;     /* [heads * (qk_nope + v_head), kv_lora_rank] */
    const uint16_t* o_proj;        /* [hidden, heads * v_head] */
} orc_mla_weights;

/* Config::softmax_scale (src/Config.cpp:114-121). */
float orc_softmax_scale(int32_t qk_nope, int32_t qk_rope, int32_t yarn, double factor, double mscale_all_dim);
/* RotaryEmbedding::build (src/Rope.cpp:36-103): cos / sin [max_positions, dim / 2]. */
void orc_rope_tables(int32_t dim, int32_t max_positions, double theta, int32_t yarn, double factor,
                     double beta_fast, double beta_slow, double mscale, double mscale_all_dim,
                     int64_t original_max_positions, float* cos_out, float* sin_out);
/* RotaryEmbedding::apply (src/Rope.cpp:105-127) on one head's dim rope channels. */
void orc_rope_apply(float* values, int32_t dim, const float* cos_row, const float* sin_row);
/* Attention::forward (src/Attention.cpp:22-103) for one token at `position`,
 * appending to the cache ([capacity, heads, qk_nope], [capacity, qk_rope],
 * [capacity, heads, v_head], *token_count filled slots); out [hidden].
 * Returns 0, or -1 when the cache is full (the reference's `false`). */
int orc_mla_forward(const orc_mla_dims* d, const orc_mla_weights* w, const float* cos_table, const float* sin_table,
                    float* key_nope, float* key_rope, float* value, int64_t capacity, int64_t* token_count,
                    const float* x, int64_t position, float* out);

#ifdef __cplusplus
}
#endif
#endif
