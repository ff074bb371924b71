/*
 * litemind_moe.h -- C ABI of the MI355X (gfx950) mixture-of-experts feed-forward path.
 *
 * This is the drop-in boundary for LiteMind's MoE block.  Every entry point names
 * the LiteMind interface it replaces (paths relative to the LiteMind source tree).
 * The C++20 wrappers in litemind_amd/host/ restore LiteMind's own class and
 * function signatures (MoeRouter, gemm::, ExpertCache) on top of this ABI.
 *
 * Conventions
 *   - Every function returns an int status: LM_OK (0) or a negative LM_E* code.
 *     No exception ever crosses this boundary.  lm_last_error() returns a
 *     thread-local message for the last failure on the calling thread.
 *   - Pointers named *_dev are device (HBM) pointers; *_host are host pointers.
 *     lm_alloc / lm_copy_* let a caller without its own HIP runtime manage them.
 *   - Work is enqueued on the context's stream and is asynchronous unless the
 *     function says otherwise; lm_synchronize() waits for it.  One context is
 *     driven from one host thread at a time (LiteMind's runner is single-threaded,
 *     and MoeRouter / ExpertCache are not reentrant either).
 *   - Weights are BF16 bit patterns (uint16_t), row-major, exactly as LiteMind's
 *     WeightView::as_bf16() hands them out (include/WeightStore.hpp:38-41).
 */
#ifndef LITEMIND_MOE_H
#define LITEMIND_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LM_OK 0
#define LM_EINVAL (-1)   /* bad argument, shape or state */
#define LM_EHIP (-2)     /* a HIP runtime call failed */
#define LM_ENOMEM (-3)   /* device or host allocation failed */
#define LM_ENOTRES (-4)  /* a weight the call needs is not resident in HBM */
#define LM_EKERNEL (-5)  /* a kernel reported an error through its status word */

typedef struct lm_context lm_context;

/* The MoE subset of LiteMind's Config (include/Config.hpp:48, :58-71, :101-103). */
typedef struct lm_moe_config {
    int32_t hidden_size;            /* 2048 for DeepSeek-V2-Lite */
    int32_t moe_intermediate_size;  /* 1408 */
    int32_t n_routed_experts;       /* 64 (at most 512; the single-token kernel takes at most 64) */
    int32_t num_experts_per_tok;    /* 6 (at most 16) */
    int32_t n_shared_experts;       /* 2 -> one fused shared FFN of width 1408*2 */
    int32_t intermediate_size;      /* dense layers: 10944 */
    int32_t norm_topk_prob;         /* 0 */
    float routed_scaling_factor;    /* 1.0 */
    int32_t group_limited;          /* topk_method == "group_limited_greedy" */
    int32_t n_group;                /* 1 */
    int32_t topk_group;             /* 1 */
    float rms_norm_eps;             /* 1e-6 */
    int32_t num_layers;             /* layers the context can hold (ids 0..num_layers-1) */
} lm_moe_config;

/* Expert-path selection for lm_moe_forward. */
#define LM_PATH_AUTO 0  /* up to LM_DECODE_TOKENS tokens one at a time through the single-token kernel
                            (where the layer's shape has it), else GEMV up to LM_MFMA_CROSSOVER tokens,
                            MFMA above */
#define LM_PATH_GEMV 1  /* fp32-activation weight-streaming kernels */
#define LM_PATH_MFMA 2  /* fp16-operand MFMA grouped GEMM, fp32 accumulate */
#define LM_MFMA_CROSSOVER 2  /* LM_PATH_AUTO: token counts above this take the MFMA path */
#define LM_DECODE_TOKENS 3   /* LM_PATH_AUTO: token counts up to this take the single-token kernel per token */

/* ---- errors, context ---- */
const char* lm_last_error(void);
int lm_version(int32_t* major, int32_t* minor);
/* Replaces DeepSeekRunner::load's MoeRouter(config) / ExpertCache::configure
 * (src/DeepSeekRunner.cpp:361-362): one context per GPU owns the resident weights. */
int lm_context_create(int32_t device, const lm_moe_config* config, lm_context** out);
/* LM_EINVAL (nothing freed) while stack graphs captured on the context are
 * alive: lm_stack_graph_destroy each of them first. */
int lm_context_destroy(lm_context* ctx);
int lm_synchronize(lm_context* ctx);
/* The context's HIP stream (a hipStream_t), so a caller can order its own work
 * with the context's (events, stream waits).  No LiteMind counterpart. */
int lm_context_stream(lm_context* ctx, void** out_stream);
/* The configuration the context was created with. */
int lm_context_config(lm_context* ctx, lm_moe_config* out);

/* ---- device memory plumbing (no LiteMind counterpart: LiteMind has one address space) ---- */
int lm_alloc(lm_context* ctx, size_t bytes, void** out_dev);
int lm_free(lm_context* ctx, void* dev);
int lm_copy_h2d(lm_context* ctx, void* dst_dev, const void* src_host, size_t bytes);  /* synchronous */
int lm_copy_d2h(lm_context* ctx, void* dst_host, const void* src_dev, size_t bytes);  /* synchronous; reports
                                                                                    LM_EKERNEL as lm_synchronize */
int lm_memset(lm_context* ctx, void* dst_dev, int32_t value, size_t bytes);           /* async */

/* ---- HBM residency: replaces ExpertCache + WeightView paging ----
 * (src/ExpertCache.cpp:9-47, src/DeepSeekRunner.cpp:200-222).  Host buffers are
 * copied once into HBM; LiteMind's mmap/madvise paging leaves the hot loop. */
/* Router gate [n_routed_experts, hidden] fp32, as LayerWeights.router holds it
 * after WeightStore::read_float32 (src/DeepSeekRunner.cpp:31, :200-203). */
int lm_upload_router(lm_context* ctx, int32_t layer, const float* gate_host);
/* One routed expert: gate, up [I, H] and down [H, I] (src/DeepSeekRunner.cpp:205-215). */
int lm_upload_expert(lm_context* ctx, int32_t layer, int32_t expert, const uint16_t* gate_host,
                     const uint16_t* up_host, const uint16_t* down_host);
/* The fused shared experts: gate, up [S, H], down [H, S], S = I * n_shared (:217-222). */
int lm_upload_shared(lm_context* ctx, int32_t layer, const uint16_t* gate_host, const uint16_t* up_host,
                     const uint16_t* down_host);
/* A dense SwiGLU layer (layer < first_k_dense_replace): [D, H], [D, H], [H, D] (:192-195). */
int lm_upload_dense(lm_context* ctx, int32_t layer, const uint16_t* gate_host, const uint16_t* up_host,
                    const uint16_t* down_host);
/* post_attention_layernorm weight [H] fp32, used by lm_stack_forward (:265-267). */
int lm_upload_norm(lm_context* ctx, int32_t layer, const float* weight_host);
/* The final norm weight [H] fp32 and the LM head [vocab, H] BF16 that end
 * DeepSeekRunner::Impl::forward (src/DeepSeekRunner.cpp:296-300); needs H % 8 == 0, H <= 16384. */
int lm_upload_head(lm_context* ctx, const float* norm_host, const uint16_t* head_host, int64_t vocab);
/* Per token of hidden_dev [T, H]: logits = head . rms_norm(hidden, norm) with
 * gemm::rms_norm and gemm::matvec_bf16's roundings, bit for bit; then, into
 * token_dev [T], Sampler::select_next's greedy choice (src/Sampler.cpp:117-126):
 * the first maximum (std::max_element), which never picks a NaN after index 0.
 * logits_dev [T, vocab] or token_dev may be null (not both).  Asynchronous. */
int lm_head_forward(lm_context* ctx, const float* hidden_dev, int64_t tokens, float* logits_dev, int32_t* token_dev);
/* Finishes a layer's upload: builds the fp16 shadow copy the MFMA path reads.
 * Must be called after the layer's experts and shared expert are uploaded. */
int lm_finalize_layer(lm_context* ctx, int32_t layer);
/* After lm_finalize_layer: how many of the layer's BF16 weights its fp16 copy
 * does not hold exactly (no counterpart in LiteMind, which has no fp16 copy).
 * The copy is exact for magnitudes in [2^-17, 65504]; larger weights make
 * lm_finalize_layer fail, smaller ones round to fp16 subnormals (absolute
 * error <= 2^-25) in the MFMA path's operands only: the GEMV and single-token
 * paths read the BF16 weights themselves. */
int lm_layer_fp16_inexact(lm_context* ctx, int32_t layer, int64_t* out_count);
/* ---- SafeTensors checkpoints: replaces WeightStore + SafeTensor ----
 * (src/WeightStore.cpp:52-185, src/SafeTensor.cpp:30-160).  lm_checkpoint_open maps
 * every *.safetensors file of a directory read-only (sorted by file name; a tensor
 * name present in two shards resolves to the first shard's) and validates each
 * header as SafeTensor::open does; failures return LM_EINVAL with LiteMind's
 * message in lm_last_error.  Payload pointers stay valid until lm_checkpoint_close.
 * No call of this group except lm_load_layer touches the GPU. */
typedef struct lm_checkpoint lm_checkpoint;
#define LM_DT_BF16 1  /* element types, as SafeTensor::parse_data_type (src/SafeTensor.cpp:15-27) */
#define LM_DT_F16 2
#define LM_DT_F32 3
#define LM_DT_F64 4
#define LM_DT_I8 5
#define LM_DT_I16 6
#define LM_DT_I32 7
#define LM_DT_I64 8
#define LM_DT_U8 9
#define LM_DT_BOOL 10
int lm_checkpoint_open(const char* model_dir, lm_checkpoint** out);
int lm_checkpoint_close(lm_checkpoint* ck);
/* Distinct tensor names and shards. */
int lm_checkpoint_count(const lm_checkpoint* ck, int64_t* tensors, int64_t* shards);
/* WeightStore::find: dtype (LM_DT_*), rank, shape[rank] (rank <= 8), the payload
 * inside the mapping and its bytes; any output may be null. */
int lm_checkpoint_find(const lm_checkpoint* ck, const char* name, int32_t* dtype, int32_t* rank, int64_t* shape,
                       const void** payload, uint64_t* bytes);
/* WeightStore::require (src/WeightStore.cpp:119-140): the tensor must exist with
 * exactly this shape and dtype. */
int lm_checkpoint_require(const lm_checkpoint* ck, const char* name, int32_t rank, const int64_t* shape,
                          int32_t dtype, const void** payload);
/* WeightStore::read_float32 (src/WeightStore.cpp:142-185): F32 copied, BF16 and F16
 * widened exactly; out holds count floats, count the tensor's element count. */
int lm_checkpoint_read_f32(const lm_checkpoint* ck, const char* name, int32_t rank, const int64_t* shape, float* out,
                           uint64_t count);
/* Uploads one layer's FFN from a checkpoint in DeepSeek's tensor names, as
 * DeepSeekRunner::Impl::resolve_layer resolves them (src/DeepSeekRunner.cpp:157-225),
 * prefix model.layers.<layer>.:
 *   post_attention_layernorm.weight [H]                 (any of F32, BF16, F16)
 *   moe = 1: mlp.gate.weight [E, H] (F32, BF16, F16), mlp.experts.<e>.{gate,up}_proj.weight
 *            [I, H] and down_proj.weight [H, I] (BF16), and with n_shared_experts > 0
 *            mlp.shared_experts.* of width I * n_shared_experts;
 *   moe = 0: mlp.{gate,up}_proj.weight [D, H], mlp.down_proj.weight [H, D] (BF16);
 *   moe = -1: MoE when the checkpoint holds the layer's mlp.gate.weight.
 * Every tensor is checked before the first upload; then lm_finalize_layer. */
int lm_load_layer(lm_context* ctx, const lm_checkpoint* ck, int32_t layer, int32_t moe);
/* Uploads model.norm.weight [H] (F32, BF16 or F16) and lm_head.weight [vocab, H] BF16,
 * or model.embed_tokens.weight when the checkpoint has no lm_head.weight (tied
 * embeddings), as DeepSeekRunner::load resolves them (src/DeepSeekRunner.cpp:364-381). */
int lm_load_head(lm_context* ctx, const lm_checkpoint* ck, int64_t vocab);
/* Bytes resident in HBM for weights (all layers). */
int lm_resident_bytes(lm_context* ctx, uint64_t* out);

/* ---- the MoE block: replaces src/DeepSeekRunner.cpp:273-288 for T tokens at once ----
 * matvec_f32 router -> MoeRouter::select -> 6 x feed_forward(expert, weight) ->
 * feed_forward(shared, 1.0), with the routed experts grouped across tokens.
 *   x_dev        [T, H] fp32, the post-attention RMSNorm output ("normalised")
 *   y_dev        [T, H] fp32, the feed-forward output (feed_forward_output; no residual)
 *   logit_bias_dev  NULL or [E] fp32 added to each logit after the router dot product
 *                   (not in LiteMind; used to construct skewed routing)
 *   topk_index_dev  NULL or [T, k] int32: the selected experts in rank order
 *   topk_weight_dev NULL or [T, k] fp32: their weights
 *   logits_dev      NULL or [T, E] fp32: router logits (after the bias)
 *   path            LM_PATH_* */
int lm_moe_forward(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, float* y_dev,
                   const float* logit_bias_dev, int32_t* topk_index_dev, float* topk_weight_dev,
                   float* logits_dev, int32_t path);

/* No counterpart in LiteMind: lm_moe_forward for callers that cannot allocate
 * device memory (tight serving loops, harnesses that forbid hipMalloc).  The
 * same MoE block, each token through the single-token kernel in turn (the
 * LM_PATH_AUTO kernel of one to three tokens), with every scratch word in one
 * fixed device array of 2 MiB per GPU instead of the context's workspace: the
 * call makes no hipMalloc, hipFree or other allocating call.  The array belongs
 * to the GPU, not to the context: every call on one GPU makes its context's
 * stream wait for the previous call's launches (a per-GPU event created at the
 * first lm_context_create on the GPU), so calls from several contexts run one
 * after another on the GPU.  Each call overwrites the array, which holds only
 * scratch (and the selection when topk_index_dev / topk_weight_dev are NULL);
 * outputs go to the caller's buffers.  A wait that gave up
 * is reported by the next lm_synchronize or lm_copy_d2h of any context on that
 * GPU.  Graph capture is not supported: the kernel's hand-off words carry a
 * parity and a tag the host advances per launch, which a replay would repeat;
 * a call while the context's stream is being captured returns LM_EINVAL.
 * LM_EINVAL too for a layer whose shape has no single-token kernel
 * (lm_moe_forward runs those) or whose scratch would not fit the array.
 * topk_index_dev, topk_weight_dev and logits_dev may be NULL.  Asynchronous. */
int lm_moe_forward_noalloc(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, float* y_dev,
                           const float* logit_bias_dev, int32_t* topk_index_dev, float* topk_weight_dev,
                           float* logits_dev);

/* ---- stage entry points (for tests; each is one step of lm_moe_forward) ---- */
/* gemm::matvec_f32 + MoeRouter::select for T tokens (src/Gemm.cpp:132-137,
 * src/MoeRouter.cpp:54-107).  Bit-exact with LiteMind for hidden % 8 == 0. */
int lm_router(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, const float* logit_bias_dev,
              float* logits_dev, int32_t* topk_index_dev, float* topk_weight_dev);
/* MoeRouter::select alone on given logits [T, E] (src/MoeRouter.cpp:54-107). */
int lm_router_select(lm_context* ctx, const float* logits_dev, int64_t tokens, int32_t* topk_index_dev,
                     float* topk_weight_dev);
/* The grouped SwiGLU alone: feed_forward (src/DeepSeekRunner.cpp:228-240) of
 * every (token, expert) assignment of the routing topk_index_dev [T, k], and
 * of the fused shared expert, without routing weights or combine.
 *   out_dev [T*k + T, H] fp32: row t*k + r = W_down(silu(W_gate x_t) * (W_up x_t))
 *           of expert topk_index[t, r]; row T*k + t the shared expert's output
 *           for token t (zero when the layer has no shared expert).
 * The tokens are grouped by lm_permute's canonical permutation; path
 * LM_PATH_GEMV (fp32 activations) or LM_PATH_MFMA (fp16 operands, fp32
 * accumulation); LM_PATH_AUTO picks as lm_moe_forward's batched path does.
 * Every expert id is checked on the host first (a synchronous copy of the T*k
 * ids; LM_EINVAL for one outside [0, E)); the rest is asynchronous. */
int lm_grouped_swiglu(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens,
                      const int32_t* topk_index_dev, float* out_dev, int32_t path);
/* Canonical expert-major permutation of the T*k selections (no LiteMind
 * counterpart: LiteMind visits one token's selections in rank order,
 * src/DeepSeekRunner.cpp:277-284).  counts [E], offsets [E+1], perm [T*k]
 * (assignment t*k+r at each permuted position), slot_of [T*k] (its inverse). */
int lm_permute(lm_context* ctx, const int32_t* topk_index_dev, int64_t tokens, int32_t* counts_dev,
               int32_t* offsets_dev, int32_t* perm_dev, int32_t* slot_of_dev);

/* ---- stack glue for the 27-layer FFN chain (src/DeepSeekRunner.cpp:264-290) ----
 * For each layer l in [first, last]: xn = rms_norm(h, norm[l]); h += FFN_l(xn),
 * FFN_l = dense SwiGLU or the MoE block.  hidden_dev [T, H] fp32 is updated in place. */
int lm_stack_forward(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev, int64_t tokens,
                     int32_t path);
/* The same pass captured once as a HIP graph and replayed (no LiteMind
 * counterpart; the survey's stack glue "run as a graph"): lm_stack_graph_create
 * records lm_stack_forward(ctx, first, last, hidden_dev, tokens, path) without
 * running it, lm_stack_graph_launch replays it on the context's stream (each
 * replay updates hidden_dev in place, like one lm_stack_forward call), and
 * lm_stack_graph_destroy frees it.  Destroy every graph before its context
 * (lm_context_destroy refuses while one is alive).  A replay reads the layers'
 * current weights; lm_stack_graph_launch returns LM_ENOTRES when a layer of its
 * range was uploaded since and not finalized again.  Only for token counts whose layers all take
 * the batched path (T >= 2 beyond the single-token kernel's batches; the
 * single-token kernel tags its hand-offs per launch from the host, which a
 * replay would repeat) and with stage timing off.  While a graph exists the
 * context keeps its workspace: a call needing a larger one fails with LM_EINVAL. */
typedef struct lm_stack_graph lm_stack_graph;
int lm_stack_graph_create(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev,
                          int64_t tokens, int32_t path, lm_stack_graph** graph);
int lm_stack_graph_launch(lm_stack_graph* graph);
int lm_stack_graph_destroy(lm_stack_graph* graph);
/* gemm::rms_norm over T rows (src/Gemm.cpp:197-207), bit for bit; out may
 * equal in.  The kernel the stack and the attention normalise batches of
 * tokens with: squares added in a thread-strided tree, and in LiteMind's order
 * for the rare rows where the two orders could round the inverse differently. */
int lm_rms_norm(lm_context* ctx, const float* in_dev, const float* weight_dev, float* out_dev, int64_t tokens,
                int32_t hidden, float epsilon);
/* Dense SwiGLU FFN of a resident dense layer: y = feed_forward(dense, x, scale 1)
 * into a zeroed output (src/DeepSeekRunner.cpp:228-240, :270-271). */
int lm_dense_forward(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, float* y_dev,
                     int32_t path);

/* ---- per-call gemm compatibility (src/Gemm.cpp:139-175) ----
 * gemm::matvec_bf16 / _serial (accumulate = 0): out = W x, and
 * gemm::matvec_bf16_accumulate (accumulate = 1): out = fma(scale, W x, out), with
 * W [out_dim, in_dim] BF16, each row reduced in dot_bf16's association order
 * (src/Gemm.cpp:46-82), so the result is bit-identical to LiteMind's.  W is read
 * from its HBM copy when lm_weight_prefetch made it resident, otherwise uploaded
 * for this call; x and out are host buffers.  Synchronous. */
int lm_gemm_matvec_bf16(lm_context* ctx, const uint16_t* w_host, const float* x_host, float* out_host,
                        size_t out_dim, size_t in_dim, float scale, int32_t accumulate);

/* out = W x for a row-major fp32 matrix with LiteMind's dot semantics (each
 * product rounded, then added left to right): gemm::matvec_f32
 * (src/Gemm.cpp:132-137, :183-189).  W as for lm_gemm_matvec_bf16.  Synchronous. */
int lm_gemm_matvec_f32(lm_context* ctx, const float* w_host, const float* x_host, float* out_host, size_t out_dim,
                       size_t in_dim);

/* Vector helpers of namespace gemm (src/Gemm.cpp:177-231), computed on the GPU with
 * LiteMind's rounding.  Synchronous; host buffers.
 *   LM_OP_DOT       out[0] = dot(a, b)                         (gemm::dot)
 *   LM_OP_AXPY      out += scalar * a                          (gemm::axpy)
 *   LM_OP_SOFTMAX   out = softmax(a)                           (gemm::softmax)
 *   LM_OP_SILU_MUL  out = silu(a) * b                          (gemm::silu_multiply)
 *   LM_OP_RMS_NORM  out = rms_norm(a, weight b, eps scalar)    (gemm::rms_norm)
 *   LM_OP_WIDEN     out = widen((const uint16_t*)a)            (gemm::widen_bf16) */
#define LM_OP_DOT 0
#define LM_OP_AXPY 1
#define LM_OP_SOFTMAX 2
#define LM_OP_SILU_MUL 3
#define LM_OP_RMS_NORM 4
#define LM_OP_WIDEN 5
int lm_vector_op(lm_context* ctx, int32_t op, const void* a_host, const float* b_host, float* out_host, size_t n,
                 float scalar);

/* Per-pointer HBM residency: replaces WeightView::prefetch / release
 * (src/WeightStore.cpp:40-50), which ExpertCache::touch / evict_oldest call
 * (src/ExpertCache.cpp:33-35, :53-55).  prefetch copies `bytes` from host_ptr
 * into HBM (no-op if resident with the same size); release frees the copy.  The
 * per-call gemm entry points use a resident copy when one exists for their weight
 * pointer, so a prefetched range must not change until it is released. */
int lm_weight_prefetch(lm_context* ctx, const void* host_ptr, size_t bytes);
int lm_weight_release(lm_context* ctx, const void* host_ptr);
int lm_weight_resident(lm_context* ctx, const void* host_ptr, int32_t* out_resident);

/* Testing hook, no counterpart in LiteMind.  The single-token forward starts the
 * routed experts from a speculative selection (a fast, reassociated logit sum)
 * and recomputes any rank where it disagrees with the exact selection.  mode 1
 * makes every speculative rank wrong so that tests exercise the recomputation;
 * outputs must not change.  mode 0 (the default) restores normal operation. */
int lm_decode_speculation_test(lm_context* ctx, int32_t mode);
/* Testing hook, no counterpart in LiteMind.  Every hand-off wait inside the
 * single-token forward is bounded; when one gives up, the kernel still runs to
 * its end, and the next lm_synchronize or lm_copy_d2h returns LM_EKERNEL.
 * mode 1 makes every such wait give up after its second poll, so tests can
 * check that path without a stalled GPU; mode 0 (the default) restores the
 * normal bound. */
int lm_decode_wait_test(lm_context* ctx, int32_t mode);
/* No counterpart in LiteMind.  One token through a layer of more than 64
 * experts (the multi-launch path: DeepSeek-V2's 160) runs the router and the
 * gate/up projections as one launch that streams the experts of a fast,
 * reassociated ranking while the exact logits are summed, and recomputes the
 * activations when the exact set of experts differs.  Outputs are the same
 * bits either way.  mode 1 (the default): that launch; 0: the router, then the
 * gate/up launch; 2 (testing): that launch with the speculated set made wrong,
 * so that the recomputation runs.  Not used under stream capture. */
int lm_router_speculation(lm_context* ctx, int32_t mode);

/* ---- timing: hipEvents on the context stream ---- */
int lm_event_create(lm_context* ctx, void** out_event);
int lm_event_destroy(lm_context* ctx, void* event);
int lm_event_record(lm_context* ctx, void* event);
int lm_event_elapsed_ms(lm_context* ctx, void* start, void* stop, float* out_ms);
/* Per-stage timing of lm_moe_forward: when enabled, each stage is bracketed by
 * events on the context stream and its durations accumulate.  Stage ids:
 * 0 router, 1 permute, 2 gate/up, 3 down, 4 combine. */
int lm_stage_timing(lm_context* ctx, int32_t enable);
int lm_stage_times(lm_context* ctx, double* out_ms, int32_t* out_calls, int32_t stages);
/* The core clock while the context's work runs (no counterpart in LiteMind: a
 * measurement aid).  lm_clock_probe_start launches one wave on a stream of its
 * own that reads the core clock counter and the 100 MHz real-time counter every
 * 20 us for `seconds` (at most 2 s); work enqueued meanwhile on the context
 * stream runs beside it.  lm_clock_probe_finish waits for it and returns the
 * clock of its intervals in MHz: median, minimum, maximum and the count. */
int lm_clock_probe_start(lm_context* ctx, double seconds);
int lm_clock_probe_finish(lm_context* ctx, double* out_median_mhz, double* out_min_mhz, double* out_max_mhz,
                          int32_t* out_intervals);

#ifdef __cplusplus
}
#endif
#endif
