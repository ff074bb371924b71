/*
 * litemind_attention.h -- C ABI of the MI355X (gfx950) multi-head latent
 * attention and its KV cache (DeepSeek-V2 MLA).
 *
 * Replaces LiteMind's Attention (include/Attention.hpp, src/Attention.cpp:10-103),
 * RotaryEmbedding (include/Rope.hpp, src/Rope.cpp:35-118) and KvCache
 * (include/KvCache.hpp, src/KvCache.cpp) for every layer of a context created by
 * lm_context_create (include/litemind_moe.h; same conventions: int status,
 * lm_last_error, *_dev device pointers, work on the context stream).
 *
 * On the bit-exact projection path (LM_PATH_GEMV, and LM_PATH_AUTO below 16
 * tokens per call) results are LiteMind's bit for bit: every projection is
 * gemm::matvec_bf16's association order, the RMS norms gemm::rms_norm's roundings, the rotation
 * RotaryEmbedding::apply's two fused multiply-adds per channel pair, each score
 * scale * (dot(q_nope, k_nope) + dot(q_rope, k_rope)) with gemm::dot's
 * left-to-right sums, the softmax gemm::softmax's (glibc expf, left-to-right
 * total, one reciprocal) and each head's context gemm::axpy's fused chain over
 * the cached tokens in order.  T tokens at once give the same results as T
 * calls of Attention::forward in turn (causal: token i sees the cache up to its
 * own slot), which is how LiteMind's runner prefills (src/DeepSeekRunner.cpp:
 * 468-476).  On the MFMA path (LM_PATH_MFMA for two or more tokens,
 * LM_PATH_AUTO from 16 tokens) each projection of a batch is one GEMM with fp16
 * operands and fp32 accumulation, as the MoE block's MFMA path: the results
 * follow LiteMind's within that path's tolerance, everything after the
 * projections (norms, rotation, scores, softmax, context) unchanged.
 */
#ifndef LITEMIND_ATTENTION_H
#define LITEMIND_ATTENTION_H

#include "litemind_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

#define LM_EFULL (-6)  /* the KV cache has no free slot (Attention::forward returned false) */

/* The attention subset of LiteMind's Config (include/Config.hpp: num_attention_heads,
 * q_lora_rank, kv_lora_rank, qk_nope_head_dim, qk_rope_head_dim, v_head_dim,
 * rope_theta, rope_scaling, rms_norm_eps) and the context length that sizes both
 * RotaryEmbedding::build and KvCache::configure (src/DeepSeekRunner.cpp:359, :416-420). */
typedef struct lm_mla_config {
    int32_t hidden_size;        /* 2048 for DeepSeek-V2-Lite; must equal the context's */
    int32_t num_heads;          /* 16 */
    int32_t q_lora_rank;        /* 0: one q_proj; > 0: q_a_proj -> RMSNorm -> q_b_proj */
    int32_t kv_lora_rank;       /* 512 */
    int32_t qk_nope_head_dim;   /* 128 */
    int32_t qk_rope_head_dim;   /* 64, even, at most 256 */
    int32_t v_head_dim;         /* 128, at most 256 */
    float rms_norm_eps;         /* 1e-6 */
    double rope_theta;          /* 10000 */
    int32_t yarn;               /* rope_scaling.enabled (type "yarn") */
    double factor;              /* 40 */
    double beta_fast;           /* 32 */
    double beta_slow;           /* 1 */
    double mscale;              /* 0.707 */
    double mscale_all_dim;      /* 0.707 */
    int64_t original_max_positions;  /* 4096 */
    int64_t context_length;     /* rotary table rows and KV cache capacity per layer */
} lm_mla_config;

/* Config::softmax_scale (src/Config.cpp:114-121).  Host only. */
int lm_mla_softmax_scale(const lm_mla_config* config, float* out);
/* RotaryEmbedding::build's tables (src/Rope.cpp:35-94): cos and sin
 * [positions, qk_rope_head_dim / 2] fp32.  Host only. */
int lm_rope_tables(const lm_mla_config* config, int64_t positions, float* cos_host, float* sin_host);

/* Attention::configure + RotaryEmbedding::build + KvCache::configure for every
 * layer of the context (src/DeepSeekRunner.cpp:359-362, :416-420): builds the
 * rotary tables, allocates each layer's cache of context_length tokens in HBM
 * (fp32, 4 * (heads * (qk_nope + v_head) + qk_rope) bytes per token and layer)
 * and empties it.  Called once per context. */
int lm_attention_configure(lm_context* ctx, const lm_mla_config* config);
/* Uploads one layer's AttentionWeights (include/Attention.hpp, resolved by
 * src/DeepSeekRunner.cpp:170-190) into HBM, BF16 row-major as WeightView::as_bf16
 * hands them out:
 *   q_lora_rank == 0: q_proj [heads * (qk_nope + qk_rope), hidden]; the q_a / q_b
 *                     arguments must be NULL;
 *   q_lora_rank  > 0: q_a_proj [q_lora_rank, hidden], q_a_layernorm [q_lora_rank] fp32,
 *                     q_b_proj [heads * (qk_nope + qk_rope), q_lora_rank]; q_proj NULL;
 *   kv_a_proj [kv_lora_rank + qk_rope, hidden], kv_a_layernorm [kv_lora_rank] fp32,
 *   kv_b_proj [heads * (qk_nope + v_head), kv_lora_rank], o_proj [hidden, heads * v_head].
 * Every width that a projection reads (hidden, q_lora_rank, kv_lora_rank,
 * heads * v_head) must be a multiple of 8. */
int lm_upload_attention(lm_context* ctx, int32_t layer, const uint16_t* q_proj_host, const uint16_t* q_a_proj_host,
                        const float* q_a_layernorm_host, const uint16_t* q_b_proj_host,
                        const uint16_t* kv_a_proj_host, const float* kv_a_layernorm_host,
                        const uint16_t* kv_b_proj_host, const uint16_t* o_proj_host);
/* input_layernorm weight [H] fp32 of a layer, used by lm_decoder_forward
 * (src/DeepSeekRunner.cpp:255-256). */
int lm_upload_input_norm(lm_context* ctx, int32_t layer, const float* weight_host);

/* Attention::forward (src/Attention.cpp:22-103) for T tokens x_dev [T, hidden]
 * at positions position0 .. position0 + T - 1, appended to the layer's cache in
 * order.  out_dev [T, hidden] receives o_proj . context (accumulate = 0), or
 * out = fma(1, o_proj . context, out) = out + o_proj . context (accumulate = 1:
 * the runner's gemm::axpy(1, block_output, hidden_state), src/DeepSeekRunner.cpp:
 * 257-261, bit for bit).  Positions at or past context_length are not rotated
 * (RotaryEmbedding::apply returns).  When the cache has room for only F < T more
 * tokens, the first F are processed and appended, the other rows of out_dev are
 * not written, and the call returns LM_EFULL, as LiteMind's per-token calls
 * would stop at the first that returns false; F = 0 changes nothing.  out_dev
 * must not overlap x_dev.  Asynchronous. */
int lm_attention_forward(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, int64_t position0,
                         float* out_dev, int32_t accumulate);

/* Projection path of lm_attention_forward (no LiteMind counterpart):
 * LM_PATH_GEMV every projection bit for bit gemm::matvec_bf16; LM_PATH_MFMA
 * batches of two or more tokens on MFMA (fp16 operands, fp32 accumulation;
 * one token keeps the bit-exact single-token launches); LM_PATH_AUTO (the
 * default) MFMA from 16 tokens per call.  Layers whose projection widths are
 * not multiples of 32, or whose weights overflow fp16, always take the
 * bit-exact path. */
int lm_attention_set_path(lm_context* ctx, int32_t path);
/* With MFMA projections the attention core (scores, softmax, context) also
 * runs on MFMA when qk_nope and qk_rope are multiples of 32, v_head_dim of 8
 * and heads * v_head_dim of 32: per head S = Q K^T and ctx = P V with fp16
 * operands over fp16 copies of the cache made once per call, P the causal
 * softmax in fp32 rounded to fp16; within the MFMA path's tolerance.
 *
 * The core takes the call's query tokens in groups sized from a byte budget
 * for its scratch (no LiteMind counterpart): the fp32 scores, and for the MFMA
 * core the fp16 copies of the keys, values, queries and probabilities.  A
 * group holds as many tokens as fit the budget, at least one and at most 512;
 * the MFMA core is used while its key / value copies take at most half of it.
 * bytes = 0 restores the default of 1 GiB. */
int lm_attention_set_score_budget(lm_context* ctx, int64_t bytes);
typedef struct lm_attention_core_plan {
    int64_t query_group;   /* query tokens per core launch */
    int64_t scratch_bytes; /* the core's scratch at that group size */
    int32_t mfma_core;     /* 1: scores and context on MFMA */
    int32_t reserved;
} lm_attention_core_plan;
/* The sizing lm_attention_forward chooses for `tokens` new tokens after
 * `cached` ones on a layer with fp16 weight copies, for a path and a budget
 * (0: the default); host only, no context or GPU. */
int lm_attention_plan_core(const lm_mla_config* config, int64_t cached, int64_t tokens, int32_t path,
                           int64_t budget_bytes, lm_attention_core_plan* out);
/* KvCache::clear for every layer (src/DeepSeekRunner.cpp:432-437, DeepSeekRunner::reset). */
int lm_kv_cache_clear(lm_context* ctx);
/* KvCache::token_count of a layer. */
int lm_kv_cache_tokens(lm_context* ctx, int32_t layer, int64_t* out_tokens);
/* The first `tokens` cached entries of a layer in KvCache's layout
 * (include/KvCache.hpp): key_nope [tokens, heads, qk_nope], key_rope
 * [tokens, qk_rope], value [tokens, heads, v_head], host buffers (any may be
 * NULL).  Synchronous. */
int lm_kv_cache_read(lm_context* ctx, int32_t layer, int64_t tokens, float* key_nope_host, float* key_rope_host,
                     float* value_host);
/* Entries [token0, token0 + tokens) in the same layout (KvCache's read-only
 * accessors, include/KvCache.hpp:60-69).  Synchronous. */
int lm_kv_cache_read_range(lm_context* ctx, int32_t layer, int64_t token0, int64_t tokens, float* key_nope_host,
                           float* key_rope_host, float* value_host);
/* Stores entries [token0, token0 + tokens) from host buffers in KvCache's layout
 * (what LiteMind writes through KvCache's writable accessors,
 * include/KvCache.hpp:49-58): token0 at most the cached count (no gap),
 * token0 + tokens at most the capacity; the count becomes at least
 * token0 + tokens.  Every buffer of a non-empty part is required.
 * Synchronous. */
int lm_kv_cache_write(lm_context* ctx, int32_t layer, int64_t token0, int64_t tokens, const float* key_nope_host,
                      const float* key_rope_host, const float* value_host);
/* Keeps the first `tokens` entries of one layer (at most its count); the next
 * call appends at slot `tokens`.  KvCache::clear (include/KvCache.hpp:31) for
 * one layer is tokens = 0. */
int lm_kv_cache_truncate(lm_context* ctx, int32_t layer, int64_t tokens);

/* DeepSeekRunner::Impl::forward's layer loop (src/DeepSeekRunner.cpp:251-291)
 * for T tokens at positions position0 .. + T - 1, layers first..last, on
 * hidden_dev [T, H] in place: h += Attention(rms_norm(h, input_layernorm)),
 * then h += FFN(rms_norm(h, post_attention_layernorm)) as lm_stack_forward.
 * Every layer needs its attention weights, input norm, norm and FFN resident.
 * `path` selects the FFN's expert path (as lm_moe_forward) and the attention's
 * projection path (as lm_attention_set_path) of every layer.
 * LM_EFULL as lm_attention_forward (hidden_dev is then partly updated). */
int lm_decoder_forward(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev, int64_t tokens,
                       int64_t position0, int32_t path);

#ifdef __cplusplus
}
#endif
#endif
