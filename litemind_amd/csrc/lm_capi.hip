// lm_capi.hip -- the C ABI declared in include/litemind_moe.h.
//
// Host orchestration for the gfx950 MoE path: context and stream, HBM residency
// of every layer's weights (replacing LiteMind's SSD-paged ExpertCache,
// src/ExpertCache.cpp:9-47), and the per-layer pipeline
//   router -> permute -> gate/up -> down -> combine
// enqueued asynchronously on the context stream.  No exception crosses the ABI;
// every entry point returns a status and records a thread-local message.
#include "litemind_moe.h"
#include "lm_error.h"
#include "lm_internal.h"

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <exception>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& message) {
    g_error = message;
    return code;
}

#define LM_HIP(call)                                                                                         \
    do {                                                                                                     \
        const hipError_t lm_status_ = (call);                                                                \
        if (lm_status_ != hipSuccess) {                                                                      \
            return fail(LM_EHIP, std::string(#call) + ": " + hipGetErrorString(lm_status_));                 \
        }                                                                                                    \
    } while (0)

#define LM_GUARD_BEGIN try {
#define LM_GUARD_END                                                                                         \
    }                                                                                                        \
    catch (const std::bad_alloc&) {                                                                          \
        return fail(LM_ENOMEM, "host allocation failed");                                                    \
    }                                                                                                        \
    catch (const std::exception& e) {                                                                        \
        return fail(LM_EINVAL, e.what());                                                                    \
    }                                                                                                        \
    catch (...) {                                                                                            \
        return fail(LM_EINVAL, "unknown exception");                                                         \
    }

constexpr int kStages = 5;
constexpr int kEventRing = 256;
// Token count above which LM_PATH_AUTO switches from weight-streaming GEMV to
// the MFMA grouped GEMM.  Both stream every active expert's weights once; the
// MFMA kernel does it through a deep LDS-DMA pipeline and reaches more of the
// HBM bandwidth from three tokens on (T = 3: 130 us against 137 us per V2-Lite
// MoE block, T = 32: 257 against 447 us), while two tokens still favour the
// GEMV's register-held weight rows (114 against 126 us).
constexpr int64_t kMfmaCrossover = LM_MFMA_CROSSOVER;
// LM_PATH_AUTO runs batches of up to this many tokens through the single-token
// kernel, one launch per token, where the layer's shape has that kernel: per
// V2-Lite block 2 x 33.8 us against 103.8 us on the GEMV path at T = 2, and
// 3 x 33.8 against 129.8 us on the MFMA path at T = 3 (about even at T = 4).
constexpr int64_t kDecodeTokens = LM_DECODE_TOKENS;

struct Layer {
    bool allocated = false;
    bool dense = false;
    bool finalized = false;
    int64_t fp16_inexact = 0;          // weights whose fp16 copy rounds (|w| < 2^-17), counted at finalize
    float* router_t = nullptr;         // [H, E], then [ceil(E/4)][H][4], then [ceil(H/4)][E][4]
    float* norm = nullptr;             // [H]
    void* slab = nullptr;              // all FFN matrices of the layer (bf16 then fp16 shadow)
    size_t slab_bytes = 0;
    std::vector<lm::FfnDev> experts;   // E routed
    lm::FfnDev shared;
    lm::FfnDev dense_ffn;
    std::vector<unsigned char> expert_present;
    bool shared_present = false;
    void** table = nullptr;            // device: gu[E+1], down[E+1], gu_h[E+1], down_h[E+1]
};

struct Workspace {
    int64_t tokens = 0;
    int32_t* idx = nullptr;
    float* wts = nullptr;
    int32_t* counts = nullptr;
    int32_t* offsets = nullptr;
    int32_t* active = nullptr;
    int32_t* perm = nullptr;
    int32_t* slot_of = nullptr;
    void* act = nullptr;          // fp32 (GEMV) or fp16 (MFMA) activations
    _Float16* x16 = nullptr;
    float* down_out = nullptr;
    float* xnorm = nullptr;       // stack: normalised input
    float* ffn = nullptr;         // stack / dense: FFN output
    int32_t* zero = nullptr;      // a device int holding 0 (dense layers have no routed experts)
    float* logit_scratch = nullptr;  // [kRouterSplitTokens, E] router hand-off of the few-token launches
    uint32_t* decode_sync = nullptr;  // single-launch decode counters (zeroed once) + error word
    float* decode_part = nullptr;     // single-launch decode: the shared items' partial down projections
    uint32_t* spec_sync = nullptr;   // speculative router + gate/up launches: counters, tags, partial logits (zeroed once)
    uint32_t* ticket = nullptr;      // single-token router arrival counter (kept at 0 between launches)
    int32_t* permute_scratch = nullptr;  // segment counts and arrival ticket of the permutation
};

struct EventSet {
    hipEvent_t ev[kStages + 1];
};

// ---- fixed device scratch of lm_moe_forward_noalloc --------------------------
//
// For callers that cannot allocate device memory, every scratch word of the
// single-token launch lives in one file-scope device array, present on each GPU
// the library runs on from load to process end.  Host code never passes the
// array's name to a kernel or a copy (in host code it is a stand-in, not a
// device address): each device's address is taken once with
// hipGetSymbolAddress, at the first context creation on that device, and only
// that address is used.  Layout, in 32-bit words:
//   [0, kStaticSync)                 hand-off words of the single-token kernel
//   [kStaticLogits, + kMaxExperts)   router logit hand-off
//   [kStaticIdx, + kMaxTopK)         selection when the caller passes none
//   [kStaticWts, + kMaxTopK)         weights when the caller passes none
//   [kStaticAct, kStaticPart)        activations [K Ip + Sp]
//   [kStaticPart, kStaticWords)      the shared items' partial down projections
// 2 MiB: V2-Lite's shape needs 1.4 MiB of partial sums.
constexpr size_t kStaticScratchBytes = 2u << 20;
constexpr int kStaticWords = static_cast<int>(kStaticScratchBytes / 4);
constexpr int kStaticSync = (lm::kDecodeSyncWords + 63) / 64 * 64;
constexpr int kStaticLogits = kStaticSync;
constexpr int kStaticIdx = kStaticLogits + lm::kMaxExperts;
constexpr int kStaticWts = kStaticIdx + lm::kMaxTopK;
constexpr int kStaticAct = (kStaticWts + lm::kMaxTopK + 63) / 64 * 64;
constexpr int kStaticPart = 64 * 1024;
static_assert(kStaticAct < kStaticPart && kStaticPart < kStaticWords, "static scratch layout");

static __device__ __align__(256) uint32_t scratch[kStaticWords];

constexpr int kMaxDevices = 64;
// Per device: the array's address, the state the single-token kernel keeps
// across launches on these words, and an event recorded after the last call's
// launches.  Every call on one GPU shares them: each call makes its context's
// stream wait for that event before its first launch, so calls from different
// contexts (streams) run one after another on the GPU, never interleaved.
struct StaticScratch {
    uint32_t* ptr = nullptr;
    hipEvent_t last = nullptr;
    int32_t parity = 0;
    uint32_t seq = 0;
    bool pending = false;
};
std::mutex g_static_mutex;
StaticScratch g_static[kMaxDevices];

__global__ void fill_words_kernel(uint32_t* p, int64_t n, uint32_t v) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        p[i] = v;
    }
}

}  // namespace

struct lm_context {
    int device = 0;
    hipStream_t stream = nullptr;
    lm_moe_config cfg{};
    int H = 0, Hp = 0, I = 0, Ip = 0, E = 0, K = 0, S = 0, Sp = 0, D = 0, Dp = 0;
    std::vector<Layer> layers;
    Workspace ws;
    uint16_t* staging = nullptr;   // pinned host buffer for repacking uploads
    size_t staging_bytes = 0;
    int* d_overflow = nullptr;
    unsigned long long* d_inexact = nullptr;  // lm_finalize_layer's count of rounded fp16 copies
    uint64_t resident = 0;
    // Per-pointer HBM residency (WeightView::prefetch / release and the per-call
    // gemm entry points), keyed by host pointer.
    struct Cached {
        void* dev;
        size_t bytes;
    };
    std::unordered_map<const void*, Cached> resident_ptrs;
    int32_t decode_parity = 0;   // alternates between single-launch decodes
    uint32_t decode_seq = 0;     // tag of the single-launch decode's hand-off words (never 0 in a launch)
    int32_t decode_perturb = 0;  // testing: force the speculative selection to disagree
    int32_t spec_mode = 1;       // one token over more than 64 experts: 0 router then gate/up, 1 speculative launch, 2 its repair forced
    int32_t spec_parity = 0;     // alternates between speculative launches
    uint32_t spec_seq = 0;       // tag of the last speculative launch
    uint32_t decode_max_spins = 0;  // testing: polls before a wait gives up (0: the kernel's default)
    bool decode_pending = false; // a single-launch decode ran since the last error check
    void* gemm_w = nullptr;      // per-call upload of a matrix that is not resident
    size_t gemm_w_cap = 0;
    float* gemm_x = nullptr;     // per-call scratch: input vector / first operand
    float* gemm_b = nullptr;     // second operand
    float* gemm_out = nullptr;   // output
    size_t gemm_cap = 0;         // floats in each scratch buffer
    // LM head: final norm [H] fp32, head [V, H] BF16, and scratch for one group of
    // lm::kHeadTokens tokens (normalised hidden states, logits when the caller
    // passes none)
    float* head_norm = nullptr;
    uint16_t* head_w = nullptr;
    int64_t vocab = 0;
    float* head_x = nullptr;
    float* head_logits = nullptr;
    lm::HeadBest* head_partial = nullptr;  // per-block candidates of the greedy choice
    lm::AttnState* attention = nullptr;  // lm_attention_configure: MLA weights, rotary tables, KV caches
    int32_t graphs = 0;  // live lm_stack_graph captures (they hold the workspace's pointers)
    // lm_clock_probe_*: its own stream (default priority) and sample buffer
    hipStream_t probe_stream = nullptr;
    uint64_t* probe_buf = nullptr;
    bool probe_running = false;
    // stage timing
    bool timing = false;
    std::vector<EventSet> ring;
    int ring_next = 0;
    int ring_pending = 0;
    double stage_ms[kStages] = {};
    int32_t stage_calls[kStages] = {};
};

namespace {

int set_device(lm_context* ctx) {
    LM_HIP(hipSetDevice(ctx->device));
    return LM_OK;
}

size_t ffn_bytes(int64_t inter_p, int64_t hidden, int64_t hidden_p) {
    // gu [2*inter_p, hidden_p] + down [hidden, inter_p], BF16
    return static_cast<size_t>((2 * inter_p * hidden_p + hidden * inter_p) * 2);
}

// Offsets (floats) of the gate's second and third layouts in Layer::router_t:
// [H, E]; [ceil(E/4)][H][4] (the last slice zero-padded when E % 4 != 0);
// [ceil(H/4)][E][4].
size_t router_quad_expert_offset(const lm_context* ctx) {
    return static_cast<size_t>(ctx->H) * static_cast<size_t>(ctx->E);
}

size_t router_quad_row_offset(const lm_context* ctx) {
    return router_quad_expert_offset(ctx) + static_cast<size_t>(ctx->H) * static_cast<size_t>(lm::round_up(ctx->E, 4));
}

int check_layer(lm_context* ctx, int32_t layer) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    if (layer < 0 || layer >= static_cast<int32_t>(ctx->layers.size())) {
        return fail(LM_EINVAL, "layer " + std::to_string(layer) + " out of range");
    }
    return LM_OK;
}

int ensure_staging(lm_context* ctx, size_t bytes) {
    if (ctx->staging_bytes >= bytes) {
        return LM_OK;
    }
    if (ctx->staging != nullptr) {
        LM_HIP(hipHostFree(ctx->staging));
        ctx->staging = nullptr;
        ctx->staging_bytes = 0;
    }
    LM_HIP(hipHostMalloc(reinterpret_cast<void**>(&ctx->staging), bytes, hipHostMallocDefault));
    ctx->staging_bytes = bytes;
    return LM_OK;
}

// Allocates the layer's slab: E routed experts + shared (MoE layer) or one dense FFN,
// bf16 copies first, then fp16 shadows of the same size.
int allocate_layer(lm_context* ctx, int32_t layer, bool dense) {
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (L.allocated) {
        if (L.dense != dense) {
            return fail(LM_EINVAL, "layer " + std::to_string(layer) + " already holds a different FFN kind");
        }
        return LM_OK;
    }
    const int64_t H = ctx->H, Hp = ctx->Hp;
    std::vector<std::pair<lm::FfnDev*, int64_t>> ffns;  // (ffn, inter)
    if (dense) {
        ffns.push_back({&L.dense_ffn, ctx->D});
    } else {
        L.experts.assign(static_cast<size_t>(ctx->E), lm::FfnDev{});
        L.expert_present.assign(static_cast<size_t>(ctx->E), 0);
        for (int e = 0; e < ctx->E; ++e) {
            ffns.push_back({&L.experts[static_cast<size_t>(e)], ctx->I});
        }
        if (ctx->S > 0) {
            ffns.push_back({&L.shared, ctx->S});
        }
    }
    size_t total = 0;
    for (auto& f : ffns) {
        total += ffn_bytes(lm::round_up(f.second, lm::kPad), H, Hp);
    }
    // The single-token kernel's shared items read the shared expert's down
    // matrix transposed ([Sp, Hp] BF16, 11.5 MB on V2-Lite).
    const bool shared_t = !dense && ctx->S > 0 && lm::decode_supported(ctx->H, ctx->E, ctx->K, ctx->Ip, ctx->Sp);
    const size_t t_bytes = shared_t ? static_cast<size_t>(ctx->Sp) * static_cast<size_t>(Hp) * 2 : 0;
    void* slab = nullptr;
    LM_HIP(hipMalloc(&slab, 2 * total + t_bytes));
    LM_HIP(hipMemsetAsync(slab, 0, 2 * total + t_bytes, ctx->stream));
    char* bf = static_cast<char*>(slab);
    char* fh = bf + total;
    for (auto& f : ffns) {
        const int64_t ip = lm::round_up(f.second, lm::kPad);
        lm::FfnDev& d = *f.first;
        d.inter = static_cast<int32_t>(f.second);
        d.inter_p = static_cast<int32_t>(ip);
        const size_t gu_bytes = static_cast<size_t>(2 * ip * Hp * 2);
        d.gu = reinterpret_cast<uint16_t*>(bf);
        d.down = reinterpret_cast<uint16_t*>(bf + gu_bytes);
        d.gu_h = reinterpret_cast<_Float16*>(fh);
        d.down_h = reinterpret_cast<_Float16*>(fh + gu_bytes);
        const size_t n = ffn_bytes(ip, H, Hp);
        bf += n;
        fh += n;
    }
    if (shared_t) {
        L.shared.down_t = reinterpret_cast<uint16_t*>(static_cast<char*>(slab) + 2 * total);
    }
    L.slab = slab;
    L.slab_bytes = 2 * total + t_bytes;
    L.allocated = true;
    L.dense = dense;
    ctx->resident += 2 * total + t_bytes;
    return LM_OK;
}

// Repacks one FFN into the resident layout (gate/up interleaved in 32-row groups,
// zero padding) in pinned staging memory and copies it to HBM.
int upload_ffn(lm_context* ctx, const lm::FfnDev& d, const uint16_t* gate, const uint16_t* up, const uint16_t* down) {
    const int64_t H = ctx->H, Hp = ctx->Hp, I = d.inter, Ip = d.inter_p;
    const size_t n = ffn_bytes(Ip, H, Hp);
    int rc = ensure_staging(ctx, n);
    if (rc != LM_OK) {
        return rc;
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));  // the previous upload may still read the staging buffer
    uint16_t* gu = ctx->staging;
    std::memset(gu, 0, n);
    for (int64_t j = 0; j < I; ++j) {
        const int64_t gate_row = (j / lm::kGroupRows) * (2 * lm::kGroupRows) + (j % lm::kGroupRows);
        std::memcpy(gu + gate_row * Hp, gate + j * H, static_cast<size_t>(H) * 2);
        std::memcpy(gu + (gate_row + lm::kGroupRows) * Hp, up + j * H, static_cast<size_t>(H) * 2);
    }
    uint16_t* dn = gu + 2 * Ip * Hp;
    for (int64_t h = 0; h < H; ++h) {
        std::memcpy(dn + h * Ip, down + h * I, static_cast<size_t>(I) * 2);
    }
    LM_HIP(hipMemcpyAsync(d.gu, gu, n, hipMemcpyHostToDevice, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
}

int ensure_workspace(lm_context* ctx, int64_t tokens) {
    Workspace& w = ctx->ws;
    if (w.tokens >= tokens && w.idx != nullptr) {
        return LM_OK;
    }
    if (ctx->graphs > 0) {
        return fail(LM_EINVAL, "a captured stack graph holds the workspace (sized for " + std::to_string(w.tokens) +
                                   " tokens); destroy it before a call with " + std::to_string(tokens));
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));
    void** ptrs[] = {reinterpret_cast<void**>(&w.idx),     reinterpret_cast<void**>(&w.wts),
                     reinterpret_cast<void**>(&w.counts),  reinterpret_cast<void**>(&w.offsets),
                     reinterpret_cast<void**>(&w.active),  reinterpret_cast<void**>(&w.perm),
                     reinterpret_cast<void**>(&w.slot_of), reinterpret_cast<void**>(&w.act),
                     reinterpret_cast<void**>(&w.x16),     reinterpret_cast<void**>(&w.down_out),
                     reinterpret_cast<void**>(&w.xnorm),   reinterpret_cast<void**>(&w.ffn),
                     reinterpret_cast<void**>(&w.zero),    reinterpret_cast<void**>(&w.logit_scratch),
                     reinterpret_cast<void**>(&w.ticket),  reinterpret_cast<void**>(&w.permute_scratch)};
    for (void** p : ptrs) {
        if (*p != nullptr) {
            LM_HIP(hipFree(*p));
            *p = nullptr;
        }
    }
    const int64_t T = std::max<int64_t>(tokens, 1);
    const int64_t TK = T * ctx->K;
    const int64_t E = ctx->E;
    const int64_t widest = std::max<int64_t>({ctx->Ip, ctx->Sp, ctx->Dp});
    const size_t act_elems = static_cast<size_t>(TK * ctx->Ip + T * widest);
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.idx), sizeof(int32_t) * static_cast<size_t>(TK)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.wts), sizeof(float) * static_cast<size_t>(TK)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.counts), sizeof(int32_t) * static_cast<size_t>(E + 1)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.offsets), sizeof(int32_t) * static_cast<size_t>(E + 2)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.active), sizeof(int32_t) * static_cast<size_t>(E + 2)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.perm), sizeof(int32_t) * static_cast<size_t>(TK)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.slot_of), sizeof(int32_t) * static_cast<size_t>(TK)));
    LM_HIP(hipMalloc(&w.act, sizeof(float) * act_elems));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.x16), sizeof(_Float16) * static_cast<size_t>(T * ctx->Hp)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.down_out), sizeof(float) * static_cast<size_t>((TK + T) * ctx->H)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.xnorm), sizeof(float) * static_cast<size_t>(T * ctx->H)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.ffn), sizeof(float) * static_cast<size_t>(T * ctx->H)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.zero), sizeof(int32_t) * 4));
    LM_HIP(hipMemsetAsync(w.zero, 0, sizeof(int32_t) * 4, ctx->stream));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.logit_scratch),
                     sizeof(float) * static_cast<size_t>(E) * lm::kRouterSplitTokens));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.ticket), sizeof(uint32_t) * 4));
    LM_HIP(hipMemsetAsync(w.ticket, 0, sizeof(uint32_t) * 4, ctx->stream));
    const size_t permute_bytes = sizeof(int32_t) * static_cast<size_t>(lm::permute_scratch_words(TK));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&w.permute_scratch), permute_bytes));
    LM_HIP(hipMemsetAsync(w.permute_scratch, 0, permute_bytes, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    w.tokens = T;
    return LM_OK;
}

// Stage timing: records event `i` of the current ring slot.
void stage_mark(lm_context* ctx, int i) {
    if (ctx->timing) {
        (void)hipEventRecord(ctx->ring[static_cast<size_t>(ctx->ring_next)].ev[i], ctx->stream);
    }
}

int stage_collect(lm_context* ctx) {
    if (ctx->ring_pending == 0) {
        return LM_OK;
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));
    const int n = ctx->ring_pending;
    for (int k = 0; k < n; ++k) {
        const int slot = (ctx->ring_next - n + k + kEventRing) % kEventRing;
        EventSet& es = ctx->ring[static_cast<size_t>(slot)];
        for (int s = 0; s < kStages; ++s) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, es.ev[s], es.ev[s + 1]) == hipSuccess) {
                ctx->stage_ms[s] += ms;
                ctx->stage_calls[s] += 1;
            }
        }
    }
    ctx->ring_pending = 0;
    return LM_OK;
}

int stage_finish(lm_context* ctx) {
    if (!ctx->timing) {
        return LM_OK;
    }
    ctx->ring_next = (ctx->ring_next + 1) % kEventRing;
    ctx->ring_pending += 1;
    if (ctx->ring_pending >= kEventRing - 1) {
        return stage_collect(ctx);
    }
    return LM_OK;
}

lm::RouteBufs route_bufs(lm_context* ctx, int32_t* idx, float* wts) {
    lm::RouteBufs rb{};
    rb.idx = idx;
    rb.wt = wts;
    rb.counts = ctx->ws.counts;
    rb.offsets = ctx->ws.offsets;
    rb.perm = ctx->ws.perm;
    rb.slot_of = ctx->ws.slot_of;
    rb.active = ctx->ws.active;
    return rb;
}

// The expert kernels' arguments for a layer whose routing is in rb (or a dense FFN).
lm::ExpertArgs expert_args(lm_context* ctx, const Layer& L, const float* x, const _Float16* x16, int64_t T,
                           const lm::RouteBufs& rb) {
    lm::ExpertArgs ea{};
    ea.groups.gu = reinterpret_cast<const uint16_t* const*>(L.table);
    const int ng = L.dense ? 1 : ctx->E + 1;
    ea.groups.down = reinterpret_cast<const uint16_t* const*>(L.table + ng);
    ea.groups.gu_h = reinterpret_cast<const _Float16* const*>(L.table + 2 * ng);
    ea.groups.down_h = reinterpret_cast<const _Float16* const*>(L.table + 3 * ng);
    ea.rb = rb;
    ea.x = x;
    ea.x16 = x16;
    ea.act = static_cast<float*>(ctx->ws.act);
    ea.act16 = static_cast<_Float16*>(ctx->ws.act);
    ea.down_out = ctx->ws.down_out;
    ea.tokens = T;
    ea.hidden = ctx->H;
    ea.hidden_p = ctx->Hp;
    if (L.dense) {
        ea.experts = 0;
        ea.top_k = 0;
        ea.inter_p = 0;
        ea.shared_inter_p = L.dense_ffn.inter_p;
        ea.has_shared = 1;
    } else {
        ea.experts = ctx->E;
        ea.top_k = ctx->K;
        ea.inter_p = ctx->Ip;
        ea.shared_inter_p = L.shared_present ? ctx->Sp : 0;
        ea.has_shared = L.shared_present ? 1 : 0;
    }
    return ea;
}

// Gate/up then down of every group into ws.down_out (one row per slot, then
// the shared rows), with stage marks 2 and 3 before each launch.
// gateup_done: the speculative launch already wrote the activations.
int launch_expert_kernels(lm_context* ctx, const Layer& L, const lm::ExpertArgs& ea, int64_t T, bool mfma,
                          bool gateup_done = false) {
    const int64_t max_active = L.dense ? 0 : std::min<int64_t>(ctx->E, T * ctx->K);
    stage_mark(ctx, 2);
    if (mfma) {
        LM_HIP(lm::launch_mfma_gateup(ea, ctx->stream));
        stage_mark(ctx, 3);
        LM_HIP(lm::launch_mfma_down(ea, ctx->stream));
    } else {
        if (!gateup_done) {
            LM_HIP(lm::launch_gemv_gateup(ea, max_active, ctx->stream));
        }
        stage_mark(ctx, 3);
        LM_HIP(lm::launch_gemv_down(ea, max_active, ctx->stream));
    }
    return LM_OK;
}

// Expert kernels + combine for a layer whose routing is in rb (or a dense FFN).
// next_norm: the next stack layer's RMSNorm weight; the combine then also
// writes that layer's input (ws.xnorm, and ws.x16 when the MFMA path follows).
int run_experts(lm_context* ctx, Layer& L, const float* x, const _Float16* x16, int64_t T, const lm::RouteBufs& rb,
                float* y, const float* residual, bool mfma, const float* next_norm = nullptr,
                bool gateup_done = false) {
    const lm::ExpertArgs ea = expert_args(ctx, L, x, x16, T, rb);
    const int rc = launch_expert_kernels(ctx, L, ea, T, mfma, gateup_done);
    if (rc != LM_OK) {
        return rc;
    }
    stage_mark(ctx, 4);
    lm::CombineArgs ca{};
    ca.down_out = ctx->ws.down_out;
    ca.slot_of = rb.slot_of;
    ca.wts = rb.wt;
    ca.y = y;
    ca.residual = residual;
    ca.tokens = T;
    ca.hidden = ctx->H;
    ca.top_k = ea.top_k;
    ca.has_shared = ea.has_shared;
    ca.next_norm = next_norm;
    ca.xnorm = ctx->ws.xnorm;
    ca.x16 = mfma ? ctx->ws.x16 : nullptr;
    ca.hidden_p = ctx->Hp;
    ca.eps = ctx->cfg.rms_norm_eps;
    LM_HIP(lm::launch_combine(ca, ctx->stream));
    stage_mark(ctx, 5);
    return LM_OK;
}

bool want_mfma(int32_t path, int64_t tokens) {
    return path == LM_PATH_MFMA || (path == LM_PATH_AUTO && tokens > kMfmaCrossover);
}

bool decode_eligible(const lm_context* ctx, const Layer& L) {
    return L.shared_present && lm::decode_supported(ctx->H, ctx->E, ctx->K, ctx->Ip, ctx->Sp);
}

// True when lm_moe_forward runs T tokens of this MoE layer through the
// single-token kernel (one launch per token) rather than the batched path.
bool takes_decode_path(const lm_context* ctx, const Layer& L, int64_t T, int32_t path) {
    return (T == 1 && !want_mfma(path, T) && decode_eligible(ctx, L)) ||
           (path == LM_PATH_AUTO && T <= kDecodeTokens && decode_eligible(ctx, L));
}

// Scratch of single-token launches: the hand-off words (lm::kDecodeSyncWords,
// zero before the first launch; each launch clears the counter set the next
// one uses), the router's logit hand-off [E], the activations [K Ip + Sp], the
// normalised token [H] when the norm is fused, the parity and tag of the last
// launch on these words, and the flag that a launch may have left an error.
struct DecodeScratch {
    uint32_t* sync;
    float* logits;
    float* act;
    float* shared_part;  // lm::decode_shared_part_floats
    float* xnorm;
    int32_t* parity;
    uint32_t* seq;
    bool* pending;
};

// The context's own decode scratch (the workspace; the hand-off words are
// allocated and zeroed on first use).
int ensure_decode_sync(lm_context* ctx) {
    if (ctx->ws.decode_sync == nullptr) {
        const size_t bytes = sizeof(uint32_t) * lm::kDecodeSyncWords;
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->ws.decode_sync), bytes));
        LM_HIP(hipMemsetAsync(ctx->ws.decode_sync, 0, bytes, ctx->stream));
    }
    return LM_OK;
}

int context_decode_scratch(lm_context* ctx, DecodeScratch* out) {
    const int rc = ensure_decode_sync(ctx);
    if (rc != LM_OK) {
        return rc;
    }
    if (ctx->ws.decode_part == nullptr) {
        const size_t floats = static_cast<size_t>(lm::decode_shared_part_floats(ctx->H, ctx->Sp));
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->ws.decode_part), sizeof(float) * floats));
    }
    *out = DecodeScratch{ctx->ws.decode_sync, ctx->ws.logit_scratch,  static_cast<float*>(ctx->ws.act),
                         ctx->ws.decode_part, ctx->ws.xnorm,          &ctx->decode_parity,
                         &ctx->decode_seq,    &ctx->decode_pending};
    return LM_OK;
}

// One token through the single-launch decode kernel (k_decode.hip).  Routed
// experts sit back to back in the layer slab, so expert e's FFN is found by
// offset.  Stage timing sees one launch, attributed to the gate/up stage.
int decode_layer(lm_context* ctx, Layer& L, const DecodeScratch& sc, const float* x, float* y,
                 const float* residual, const float* bias, int32_t* idx, float* wts, float* logits_out,
                 const float* norm) {
    lm::DecodeLaunch d{};
    d.x = x;
    d.norm = norm;
    d.eps = ctx->cfg.rms_norm_eps;
    d.xnorm = sc.xnorm;
    d.wq = L.router_t + router_quad_expert_offset(ctx);
    d.bias = bias;
    d.logits = sc.logits;
    d.logits_out = logits_out;
    d.idx = idx;
    d.wts = wts;
    d.routed = L.experts[0].gu;
    d.routed_stride = static_cast<int64_t>(L.experts[1].gu - L.experts[0].gu);
    d.shared_gu = L.shared.gu;
    d.shared_down = L.shared.down;
    d.shared_t = L.shared.down_t;
    d.shared_part = sc.shared_part;
    d.act = sc.act;
    d.y = y;
    d.residual = residual;
    d.hidden = ctx->H;
    d.hidden_p = ctx->Hp;
    d.inter_p = ctx->Ip;
    d.shared_inter_p = ctx->Sp;
    d.policy = lm::SelectPolicy{ctx->E, ctx->K, ctx->cfg.norm_topk_prob, ctx->cfg.group_limited, ctx->cfg.n_group,
                                ctx->cfg.topk_group, ctx->cfg.routed_scaling_factor};
    d.sync = sc.sync;
    d.parity = *sc.parity;
    d.perturb = ctx->decode_perturb;
    d.max_spins = ctx->decode_max_spins;
    *sc.parity ^= 1;
    *sc.seq = *sc.seq == 0xffffffffu ? 1u : *sc.seq + 1u;
    d.seq = *sc.seq;
    *sc.pending = true;
    stage_mark(ctx, 0);
    stage_mark(ctx, 1);
    stage_mark(ctx, 2);
    LM_HIP(lm::launch_decode(d, ctx->stream));
    stage_mark(ctx, 3);
    stage_mark(ctx, 4);
    stage_mark(ctx, 5);
    return stage_finish(ctx);
}

// One token over more than 64 experts on the GEMV path: the router and the
// gate/up projections in one launch that starts the routed experts from a
// speculative selection (lm::launch_spec_gateup), unless it is off
// (lm_router_speculation), the shape is outside it, or the stream is being
// captured (its hand-off words carry a tag the host advances per launch, which
// a replay would repeat).  Sets *speculated when it launched.
int spec_router_gateup(lm_context* ctx, Layer& L, const lm::RouterArgs& ra, int64_t T, bool mfma, bool* speculated) {
    *speculated = false;
    if (T != 1 || mfma || ctx->spec_mode == 0 || ra.x16 != nullptr || ra.rb.counts == nullptr ||
        !lm::spec_gateup_supported(ctx->E, ctx->H, ctx->K, ctx->cfg.n_group, ctx->cfg.group_limited, ctx->Ip,
                                   L.shared_present ? ctx->Sp : 0)) {
        return LM_OK;
    }
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    LM_HIP(hipStreamIsCapturing(ctx->stream, &capture));
    if (capture != hipStreamCaptureStatusNone) {
        return LM_OK;
    }
    int rc = ensure_decode_sync(ctx);  // its error word
    if (rc != LM_OK) {
        return rc;
    }
    if (ctx->ws.spec_sync == nullptr) {
        const size_t bytes = sizeof(uint32_t) * lm::kSpecSyncWords;
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->ws.spec_sync), bytes));
        LM_HIP(hipMemsetAsync(ctx->ws.spec_sync, 0, bytes, ctx->stream));
    }
    const lm::ExpertArgs ea = expert_args(ctx, L, ra.x, nullptr, 1, ra.rb);
    ctx->spec_seq = ctx->spec_seq == 0xffffffffu ? 1u : ctx->spec_seq + 1u;
    LM_HIP(lm::launch_spec_gateup(ra, ea, ctx->ws.spec_sync, ctx->ws.decode_sync + lm::kDecodeErrorWord,
                                  ctx->spec_parity, ctx->spec_seq, ctx->spec_mode == 2 ? 1 : 0,
                                  ctx->decode_max_spins, ctx->stream));
    ctx->spec_parity ^= 1;
    ctx->decode_pending = true;
    *speculated = true;
    return LM_OK;
}

// norm: when set, x is the hidden state and the block's input is rms_norm(x, norm).
// prenormed (batched path only): the previous layer's combine already wrote
// this layer's normalised input to ws.xnorm (and ws.x16 for the MFMA path).
int moe_layer(lm_context* ctx, int32_t layer, const float* x, int64_t T, float* y, const float* residual,
              const float* bias, int32_t* idx_out, float* w_out, float* logits_out, int32_t path,
              const float* norm = nullptr, const float* next_norm = nullptr, bool prenormed = false) {
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (!L.allocated || L.dense || L.router_t == nullptr) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no resident MoE weights");
    }
    if (!L.finalized) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " is not finalized (lm_finalize_layer)");
    }
    const bool mfma = want_mfma(path, T);
    int rc = ensure_workspace(ctx, T);
    if (rc != LM_OK) {
        return rc;
    }
    int32_t* idx = idx_out != nullptr ? idx_out : ctx->ws.idx;
    float* wts = w_out != nullptr ? w_out : ctx->ws.wts;

    if (takes_decode_path(ctx, L, T, path)) {
        if (prenormed || next_norm != nullptr) {
            return fail(LM_EINVAL, "internal: a fused norm was planned for the single-token path");
        }
        DecodeScratch sc{};
        rc = context_decode_scratch(ctx, &sc);
        if (rc != LM_OK) {
            return rc;
        }
        const int64_t H = ctx->H;
        for (int64_t t = 0; t < T; ++t) {
            rc = decode_layer(ctx, L, sc, x + t * H, y + t * H, residual != nullptr ? residual + t * H : nullptr,
                              bias, idx + t * ctx->K, wts + t * ctx->K,
                              logits_out != nullptr ? logits_out + t * ctx->E : nullptr, norm);
            if (rc != LM_OK) {
                return rc;
            }
        }
        return LM_OK;
    }
    if (prenormed) {
        x = ctx->ws.xnorm;
    } else if (norm != nullptr) {
        LM_HIP(lm::launch_rms_norm(x, norm, ctx->ws.xnorm, T, ctx->H, ctx->cfg.rms_norm_eps, ctx->stream));
        x = ctx->ws.xnorm;
    }

    lm::RouterArgs ra{};
    ra.x = x;
    ra.wt = L.router_t;
    ra.wq4 = L.router_t + router_quad_row_offset(ctx);
    ra.bias = bias;
    ra.logits = logits_out;
    ra.idx = idx;
    ra.wts = wts;
    ra.x16 = mfma && !prenormed ? ctx->ws.x16 : nullptr;
    ra.tokens = T;
    ra.hidden = ctx->H;
    ra.hidden_p = ctx->Hp;
    ra.experts = ctx->E;
    ra.top_k = ctx->K;
    ra.normalize = ctx->cfg.norm_topk_prob;
    ra.group_limited = ctx->cfg.group_limited;
    ra.n_group = ctx->cfg.n_group;
    ra.topk_group = ctx->cfg.topk_group;
    ra.scale = ctx->cfg.routed_scaling_factor;
    ra.do_matvec = 1;
    ra.logits_scratch = ctx->ws.logit_scratch;
    ra.ticket = ctx->ws.ticket;
    ra.rb = route_bufs(ctx, idx, wts);
    stage_mark(ctx, 0);
    bool permuted = false;
    bool speculated = false;
    rc = spec_router_gateup(ctx, L, ra, T, mfma, &speculated);
    if (rc != LM_OK) {
        return rc;
    }
    if (speculated) {
        permuted = true;
    } else {
        LM_HIP(lm::launch_router(ra, ctx->stream, &permuted));
    }
    stage_mark(ctx, 1);

    lm::PermuteArgs pa{};
    pa.idx = idx;
    pa.tokens = T;
    pa.top_k = ctx->K;
    pa.experts = ctx->E;
    pa.rb = ra.rb;
    pa.scratch = ctx->ws.permute_scratch;
    if (!permuted) {
        LM_HIP(lm::launch_permute(pa, ctx->stream));
    }

    rc = run_experts(ctx, L, x, ctx->ws.x16, T, pa.rb, y, residual, mfma, next_norm, speculated);
    if (rc != LM_OK) {
        return rc;
    }
    return stage_finish(ctx);
}

int dense_layer(lm_context* ctx, int32_t layer, const float* x, int64_t T, float* y, const float* residual,
                int32_t path, const float* next_norm = nullptr, bool prenormed = false) {
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (!L.allocated || !L.dense || !L.finalized) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no finalized dense FFN");
    }
    const bool mfma = want_mfma(path, T);
    int rc = ensure_workspace(ctx, T);
    if (rc != LM_OK) {
        return rc;
    }
    if (mfma && !prenormed) {
        LM_HIP(lm::launch_to_f16_rows(x, ctx->ws.x16, T, ctx->H, ctx->Hp, ctx->stream));
    }
    lm::RouteBufs rb{};
    rb.counts = ctx->ws.zero;
    rb.offsets = ctx->ws.zero;
    rb.active = ctx->ws.zero;
    rb.perm = ctx->ws.perm;
    rb.slot_of = ctx->ws.slot_of;
    rb.idx = ctx->ws.idx;
    rb.wt = ctx->ws.wts;
    stage_mark(ctx, 0);
    stage_mark(ctx, 1);
    rc = run_experts(ctx, L, x, ctx->ws.x16, T, rb, y, residual, mfma, next_norm);
    if (rc != LM_OK) {
        return rc;
    }
    return stage_finish(ctx);
}

// Makes host_ptr[0, bytes) resident: uploads it, or replaces a copy of another
// size.  The caller promises the range does not change until it is released.
int resident_copy(lm_context* ctx, const void* host_ptr, size_t bytes, void** dev_out) {
    auto it = ctx->resident_ptrs.find(host_ptr);
    if (it != ctx->resident_ptrs.end() && it->second.bytes != bytes) {
        LM_HIP(hipStreamSynchronize(ctx->stream));
        LM_HIP(hipFree(it->second.dev));
        ctx->resident_ptrs.erase(it);
        it = ctx->resident_ptrs.end();
    }
    if (it == ctx->resident_ptrs.end()) {
        void* dev = nullptr;
        LM_HIP(hipMalloc(&dev, std::max<size_t>(bytes, 1)));
        LM_HIP(hipMemcpyAsync(dev, host_ptr, bytes, hipMemcpyHostToDevice, ctx->stream));
        it = ctx->resident_ptrs.emplace(host_ptr, lm_context::Cached{dev, bytes}).first;
    }
    *dev_out = it->second.dev;
    return LM_OK;
}

// Device view of a matrix for one gemm call: the resident copy when the range was
// prefetched, otherwise this call's own upload into a reused staging buffer (the
// host memory is read on every call, as LiteMind's gemm reads it).
int matrix_for_call(lm_context* ctx, const void* host_ptr, size_t bytes, void** dev_out) {
    auto it = ctx->resident_ptrs.find(host_ptr);
    if (it != ctx->resident_ptrs.end() && it->second.bytes >= bytes) {
        *dev_out = it->second.dev;
        return LM_OK;
    }
    if (ctx->gemm_w_cap < bytes) {
        LM_HIP(hipStreamSynchronize(ctx->stream));
        LM_HIP(hipFree(ctx->gemm_w));
        ctx->gemm_w = nullptr;
        ctx->gemm_w_cap = 0;
        LM_HIP(hipMalloc(&ctx->gemm_w, bytes));
        ctx->gemm_w_cap = bytes;
    }
    if (bytes > 0) {
        LM_HIP(hipMemcpyAsync(ctx->gemm_w, host_ptr, bytes, hipMemcpyHostToDevice, ctx->stream));
    }
    *dev_out = ctx->gemm_w;
    return LM_OK;
}

int ensure_gemm_scratch(lm_context* ctx, size_t floats) {
    if (ctx->gemm_cap >= floats) {
        return LM_OK;
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));
    (void)hipFree(ctx->gemm_x);
    (void)hipFree(ctx->gemm_b);
    (void)hipFree(ctx->gemm_out);
    ctx->gemm_x = ctx->gemm_b = ctx->gemm_out = nullptr;
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->gemm_x), floats * sizeof(float)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->gemm_b), floats * sizeof(float)));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->gemm_out), floats * sizeof(float)));
    ctx->gemm_cap = floats;
    return LM_OK;
}

// Reads a single-token error word after its launches have finished; a set
// word is cleared on the context's stream (a fill kernel, not a memset, so the
// clear is an ordinary kernel on every path).  Sets *failed.
int consume_decode_error(lm_context* ctx, uint32_t* sync, bool* failed) {
    uint32_t error = 0;
    uint32_t* word = sync + lm::kDecodeErrorWord;
    LM_HIP(hipMemcpy(&error, word, sizeof error, hipMemcpyDeviceToHost));
    if (error != 0) {
        hipLaunchKernelGGL(fill_words_kernel, dim3(1), dim3(64), 0, ctx->stream, word, int64_t{1}, 0u);
        LM_HIP(hipGetLastError());
        LM_HIP(hipStreamSynchronize(ctx->stream));
        *failed = true;
    }
    return LM_OK;
}

// After the context's stream has drained: a bounded wait inside a
// single-launch decode that ran out has set the error word; report it once and
// clear it.  The fixed array's word (lm_moe_forward_noalloc, any context on
// this GPU) is read only after the last such call has finished on the GPU
// (its event), with the lock held so that no new call is enqueued meanwhile.
int check_decode_error(lm_context* ctx) {
    bool failed = false;
    if (ctx->decode_pending) {
        ctx->decode_pending = false;
        const int rc = consume_decode_error(ctx, ctx->ws.decode_sync, &failed);
        if (rc != LM_OK) {
            return rc;
        }
    }
    if (ctx->device < kMaxDevices) {
        std::lock_guard<std::mutex> lock(g_static_mutex);
        StaticScratch& st = g_static[ctx->device];
        if (st.pending) {
            st.pending = false;
            LM_HIP(hipEventSynchronize(st.last));
            const int rc = consume_decode_error(ctx, st.ptr, &failed);
            if (rc != LM_OK) {
                return rc;
            }
            LM_HIP(hipEventRecord(st.last, ctx->stream));  // after the clear, if one ran
        }
    }
    if (failed) {
        return fail(LM_EKERNEL, "a single-token decode wait timed out; its outputs are invalid");
    }
    return LM_OK;
}

// Once per device, with the device current: the address of `scratch` on it,
// cleared with a fill kernel on the context's stream.
int static_scratch_setup(lm_context* ctx) {
    if (ctx->device >= kMaxDevices) {
        return LM_OK;  // lm_moe_forward_noalloc reports it
    }
    std::lock_guard<std::mutex> lock(g_static_mutex);
    StaticScratch& st = g_static[ctx->device];
    if (st.ptr != nullptr) {
        return LM_OK;
    }
    void* ptr = nullptr;
    LM_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    hipEvent_t ev = nullptr;
    LM_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    hipLaunchKernelGGL(fill_words_kernel, dim3(64), dim3(256), 0, ctx->stream, static_cast<uint32_t*>(ptr),
                       static_cast<int64_t>(kStaticWords), 0u);
    LM_HIP(hipGetLastError());
    LM_HIP(hipEventRecord(ev, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    st.ptr = static_cast<uint32_t*>(ptr);
    st.last = ev;
    return LM_OK;
}

}  // namespace

int lm::set_error(int code, const std::string& message) { return fail(code, message); }

lm::ContextInfo lm::context_info(const lm_context* ctx) {
    ContextInfo info;
    info.device = ctx->device;
    info.stream = ctx->stream;
    info.hidden = ctx->H;
    info.layers = static_cast<int32_t>(ctx->layers.size());
    return info;
}

lm::AttnState*& lm::context_attention(lm_context* ctx) { return ctx->attention; }

namespace {

// h += FFN(rms_norm(h)) (src/DeepSeekRunner.cpp:265-290) for one layer.  The
// MoE block normalises the hidden state itself (inside the single-token
// launch, or with rms_norm_kernel before the batched path), unless
// `prenormed`: the previous layer's combine already wrote the normalised input.
// With next_norm this layer's combine does the same for the next layer.
int ffn_sublayer_fused(lm_context* ctx, int32_t l, float* hidden, int64_t T, int32_t path, const float* next_norm,
                       bool prenormed) {
    int rc = ensure_workspace(ctx, T);
    if (rc != LM_OK) {
        return rc;
    }
    Layer& L = ctx->layers[static_cast<size_t>(l)];
    if (L.norm == nullptr) {
        return fail(LM_ENOTRES, "layer " + std::to_string(l) + " has no norm weight");
    }
    if (L.dense) {
        if (!prenormed) {
            LM_HIP(lm::launch_rms_norm(hidden, L.norm, ctx->ws.xnorm, T, ctx->H, ctx->cfg.rms_norm_eps, ctx->stream));
        }
        return dense_layer(ctx, l, ctx->ws.xnorm, T, hidden, hidden, path, next_norm, prenormed);
    }
    return moe_layer(ctx, l, hidden, T, hidden, hidden, nullptr, nullptr, nullptr, nullptr, path, L.norm, next_norm,
                     prenormed);
}

// Whether layer l of a stack pass at T tokens takes the batched path (whose
// combine can hand the next layer its normalised input).
bool batched_layer(const lm_context* ctx, int32_t l, int64_t T, int32_t path) {
    const Layer& L = ctx->layers[static_cast<size_t>(l)];
    if (!L.allocated || !L.finalized || L.norm == nullptr) {
        return false;  // the layer reports its own error
    }
    return L.dense || (L.router_t != nullptr && !takes_decode_path(ctx, L, T, path));
}

}  // namespace

int lm::ffn_sublayer(lm_context* ctx, int32_t l, float* hidden, int64_t T, int32_t path) {
    return ffn_sublayer_fused(ctx, l, hidden, T, path, nullptr, false);
}

extern "C" {

const char* lm_last_error(void) { return g_error.c_str(); }

int lm_version(int32_t* major, int32_t* minor) {
    if (major != nullptr) {
        *major = 0;
    }
    if (minor != nullptr) {
        *minor = 1;
    }
    return LM_OK;
}

int lm_context_config(lm_context* ctx, lm_moe_config* out) {
    if (ctx == nullptr || out == nullptr) {
        return fail(LM_EINVAL, "null context or output pointer");
    }
    *out = ctx->cfg;
    return LM_OK;
}

int lm_context_create(int32_t device, const lm_moe_config* config, lm_context** out) {
    LM_GUARD_BEGIN
    if (config == nullptr || out == nullptr) {
        return fail(LM_EINVAL, "null config or output pointer");
    }
    *out = nullptr;
    const lm_moe_config& c = *config;
    if (c.hidden_size <= 0 || c.hidden_size % 8 != 0) {
        return fail(LM_EINVAL, "hidden_size must be a positive multiple of 8");
    }
    if (c.n_routed_experts <= 0 || c.n_routed_experts > lm::kMaxExpertsWide) {
        return fail(LM_EINVAL, "n_routed_experts must be in [1, 512]");
    }
    if (c.num_experts_per_tok <= 0 || c.num_experts_per_tok > lm::kMaxTopK ||
        c.num_experts_per_tok > c.n_routed_experts) {
        return fail(LM_EINVAL, "num_experts_per_tok must be in [1, min(16, n_routed_experts)]");
    }
    if (c.moe_intermediate_size <= 0 || c.n_shared_experts < 0 || c.intermediate_size < 0 || c.num_layers <= 0) {
        return fail(LM_EINVAL, "invalid intermediate sizes or layer count");
    }
    if (c.hidden_size % 16 != 0) {
        return fail(LM_EINVAL, "hidden_size must be a multiple of 16 (GEMV item rows)");
    }
    int count = 0;
    LM_HIP(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) {
        return fail(LM_EINVAL, "device " + std::to_string(device) + " not present");
    }
    auto* ctx = new lm_context();
    ctx->device = device;
    ctx->cfg = c;
    ctx->H = c.hidden_size;
    ctx->Hp = static_cast<int>(lm::round_up(c.hidden_size, lm::kPad));
    ctx->I = c.moe_intermediate_size;
    ctx->Ip = static_cast<int>(lm::round_up(ctx->I, lm::kPad));
    ctx->E = c.n_routed_experts;
    ctx->K = c.num_experts_per_tok;
    ctx->S = c.moe_intermediate_size * c.n_shared_experts;
    ctx->Sp = static_cast<int>(lm::round_up(ctx->S, lm::kPad));
    ctx->D = c.intermediate_size;
    ctx->Dp = static_cast<int>(lm::round_up(ctx->D, lm::kPad));
    ctx->layers.resize(static_cast<size_t>(c.num_layers));
    int rc = set_device(ctx);
    if (rc == LM_OK && hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        rc = fail(LM_EHIP, "hipStreamCreateWithFlags failed");
    }
    if (rc == LM_OK && hipMalloc(reinterpret_cast<void**>(&ctx->d_overflow), sizeof(int)) != hipSuccess) {
        rc = fail(LM_ENOMEM, "hipMalloc failed");
    }
    if (rc == LM_OK && hipMalloc(reinterpret_cast<void**>(&ctx->d_inexact), sizeof(unsigned long long)) != hipSuccess) {
        rc = fail(LM_ENOMEM, "hipMalloc failed");
    }
    if (rc == LM_OK) {
        rc = static_scratch_setup(ctx);
    }
    if (rc != LM_OK) {
        delete ctx;
        return rc;
    }
    *out = ctx;
    return LM_OK;
    LM_GUARD_END
}

int lm_context_destroy(lm_context* ctx) {
    LM_GUARD_BEGIN
    if (ctx == nullptr) {
        return LM_OK;
    }
    if (ctx->graphs > 0) {
        return fail(LM_EINVAL, "lm_context_destroy: " + std::to_string(ctx->graphs) +
                                   " stack graph(s) captured on this context are still alive; "
                                   "lm_stack_graph_destroy them first");
    }
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    for (Layer& L : ctx->layers) {
        (void)hipFree(L.router_t);
        (void)hipFree(L.norm);
        (void)hipFree(L.slab);
        (void)hipFree(L.table);
    }
    Workspace& w = ctx->ws;
    void* ptrs[] = {w.idx, w.wts, w.counts, w.offsets, w.active, w.perm, w.slot_of, w.act, w.x16,
                    w.down_out, w.xnorm, w.ffn, w.zero, w.logit_scratch, w.ticket, w.permute_scratch};
    for (void* p : ptrs) {
        (void)hipFree(p);
    }
    for (auto& kv : ctx->resident_ptrs) {
        (void)hipFree(kv.second.dev);
    }
    (void)hipFree(ctx->gemm_w);
    (void)hipFree(ctx->gemm_x);
    (void)hipFree(ctx->gemm_b);
    (void)hipFree(ctx->gemm_out);
    (void)hipFree(ctx->head_norm);
    (void)hipFree(ctx->head_w);
    (void)hipFree(ctx->head_x);
    (void)hipFree(ctx->head_logits);
    (void)hipFree(ctx->head_partial);
    (void)hipFree(ctx->d_overflow);
    (void)hipFree(ctx->d_inexact);
    (void)hipFree(w.decode_sync);
    (void)hipFree(w.decode_part);
    (void)hipFree(w.spec_sync);
    lm::attention_release(ctx->attention);
    ctx->attention = nullptr;
    if (ctx->staging != nullptr) {
        (void)hipHostFree(ctx->staging);
    }
    for (EventSet& es : ctx->ring) {
        for (hipEvent_t e : es.ev) {
            (void)hipEventDestroy(e);
        }
    }
    if (ctx->probe_stream != nullptr) {
        (void)hipStreamSynchronize(ctx->probe_stream);
        (void)hipStreamDestroy(ctx->probe_stream);
    }
    (void)hipFree(ctx->probe_buf);
    if (ctx->stream != nullptr) {
        (void)hipStreamDestroy(ctx->stream);
    }
    delete ctx;
    return LM_OK;
    LM_GUARD_END
}

int lm_synchronize(lm_context* ctx) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return check_decode_error(ctx);
}

int lm_alloc(lm_context* ctx, size_t bytes, void** out_dev) {
    if (ctx == nullptr || out_dev == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    *out_dev = nullptr;
    if (hipMalloc(out_dev, bytes == 0 ? 1 : bytes) != hipSuccess) {
        return fail(LM_ENOMEM, "hipMalloc of " + std::to_string(bytes) + " bytes failed");
    }
    return LM_OK;
}

int lm_free(lm_context* ctx, void* dev) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));
    LM_HIP(hipFree(dev));
    return LM_OK;
}

int lm_copy_h2d(lm_context* ctx, void* dst_dev, const void* src_host, size_t bytes) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    LM_HIP(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
}

int lm_copy_d2h(lm_context* ctx, void* dst_host, const void* src_dev, size_t bytes) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    LM_HIP(hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    // the copied data may come from a decode whose wait gave up
    return check_decode_error(ctx);
}

int lm_memset(lm_context* ctx, void* dst_dev, int32_t value, size_t bytes) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    LM_HIP(hipMemsetAsync(dst_dev, value, bytes, ctx->stream));
    return LM_OK;
}

int lm_upload_router(lm_context* ctx, int32_t layer, const float* gate_host) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (gate_host == nullptr) {
        return fail(LM_EINVAL, "null router gate");
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    // Three layouts of the gate: [H, E] for the per-wave router; [E/4][H][4]
    // (four experts' weights of one row side by side, each slice contiguous)
    // for the single-token router; [H/4][E][4] (four consecutive rows of one
    // expert side by side) for the ring routers.  E and H are padded to
    // multiples of 4 with zeros in the last slice of the second and third.
    const size_t o2 = router_quad_expert_offset(ctx);
    const size_t o3 = router_quad_row_offset(ctx);
    const size_t total = o3 + static_cast<size_t>(lm::round_up(ctx->H, 4)) * static_cast<size_t>(ctx->E);
    if (L.router_t == nullptr) {
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&L.router_t), total * sizeof(float)));
        ctx->resident += total * sizeof(float);
    }
    std::vector<float> t(total, 0.0f);
    for (int e = 0; e < ctx->E; ++e) {
        for (int i = 0; i < ctx->H; ++i) {
            const float v = gate_host[static_cast<size_t>(e) * ctx->H + i];
            t[static_cast<size_t>(i) * ctx->E + e] = v;
            t[o2 + (static_cast<size_t>(e / 4) * ctx->H + i) * 4 + e % 4] = v;
            t[o3 + (static_cast<size_t>(i / 4) * ctx->E + e) * 4 + i % 4] = v;
        }
    }
    LM_HIP(hipMemcpyAsync(L.router_t, t.data(), total * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_upload_expert(lm_context* ctx, int32_t layer, int32_t expert, const uint16_t* gate_host,
                     const uint16_t* up_host, const uint16_t* down_host) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (expert < 0 || expert >= ctx->E || gate_host == nullptr || up_host == nullptr || down_host == nullptr) {
        return fail(LM_EINVAL, "bad expert index or null weights");
    }
    rc = set_device(ctx);
    if (rc == LM_OK) {
        rc = allocate_layer(ctx, layer, false);
    }
    if (rc != LM_OK) {
        return rc;
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    rc = upload_ffn(ctx, L.experts[static_cast<size_t>(expert)], gate_host, up_host, down_host);
    if (rc == LM_OK) {
        L.expert_present[static_cast<size_t>(expert)] = 1;
        L.finalized = false;
    }
    return rc;
    LM_GUARD_END
}

int lm_upload_shared(lm_context* ctx, int32_t layer, const uint16_t* gate_host, const uint16_t* up_host,
                     const uint16_t* down_host) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (ctx->S == 0) {
        return fail(LM_EINVAL, "the configuration has no shared experts");
    }
    if (gate_host == nullptr || up_host == nullptr || down_host == nullptr) {
        return fail(LM_EINVAL, "null shared-expert weights");
    }
    rc = set_device(ctx);
    if (rc == LM_OK) {
        rc = allocate_layer(ctx, layer, false);
    }
    if (rc != LM_OK) {
        return rc;
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    rc = upload_ffn(ctx, L.shared, gate_host, up_host, down_host);
    if (rc == LM_OK) {
        L.shared_present = true;
        L.finalized = false;
    }
    return rc;
    LM_GUARD_END
}

int lm_upload_dense(lm_context* ctx, int32_t layer, const uint16_t* gate_host, const uint16_t* up_host,
                    const uint16_t* down_host) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (ctx->D == 0) {
        return fail(LM_EINVAL, "the configuration has no dense intermediate size");
    }
    if (gate_host == nullptr || up_host == nullptr || down_host == nullptr) {
        return fail(LM_EINVAL, "null dense weights");
    }
    rc = set_device(ctx);
    if (rc == LM_OK) {
        rc = allocate_layer(ctx, layer, true);
    }
    if (rc != LM_OK) {
        return rc;
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    rc = upload_ffn(ctx, L.dense_ffn, gate_host, up_host, down_host);
    if (rc == LM_OK) {
        L.finalized = false;
    }
    return rc;
    LM_GUARD_END
}

int lm_upload_norm(lm_context* ctx, int32_t layer, const float* weight_host) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (weight_host == nullptr) {
        return fail(LM_EINVAL, "null norm weight");
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (L.norm == nullptr) {
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&L.norm), sizeof(float) * static_cast<size_t>(ctx->H)));
    }
    LM_HIP(hipMemcpyAsync(L.norm, weight_host, sizeof(float) * static_cast<size_t>(ctx->H), hipMemcpyHostToDevice,
                          ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_upload_head(lm_context* ctx, const float* norm_host, const uint16_t* head_host, int64_t vocab) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || norm_host == nullptr || head_host == nullptr || vocab <= 0 || vocab > INT32_MAX) {
        return fail(LM_EINVAL, "bad head arguments");
    }
    if (ctx->H % 8 != 0 || ctx->H > 16384) {
        return fail(LM_EINVAL, "the LM head needs hidden_size % 8 == 0 and hidden_size <= 16384");
    }
    int rc = set_device(ctx);
    if (rc != LM_OK) {
        return rc;
    }
    const size_t H = static_cast<size_t>(ctx->H), V = static_cast<size_t>(vocab);
    LM_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->head_w != nullptr) {
        ctx->resident -= sizeof(uint16_t) * static_cast<size_t>(ctx->vocab) * H + sizeof(float) * H;
    }
    for (void* q : {static_cast<void*>(ctx->head_norm), static_cast<void*>(ctx->head_w),
                    static_cast<void*>(ctx->head_x), static_cast<void*>(ctx->head_logits),
                    static_cast<void*>(ctx->head_partial)}) {
        LM_HIP(hipFree(q));
    }
    ctx->head_norm = nullptr;
    ctx->head_w = nullptr;
    ctx->head_x = nullptr;
    ctx->head_logits = nullptr;
    ctx->head_partial = nullptr;
    ctx->vocab = 0;
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->head_norm), sizeof(float) * H));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->head_w), sizeof(uint16_t) * V * H));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->head_x), sizeof(float) * lm::kHeadTokens * H));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->head_logits), sizeof(float) * lm::kHeadTokens * V));
    LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->head_partial),
                     sizeof(lm::HeadBest) * lm::kHeadTokens * static_cast<size_t>(lm::head_blocks(vocab))));
    LM_HIP(hipMemcpy(ctx->head_norm, norm_host, sizeof(float) * H, hipMemcpyHostToDevice));
    LM_HIP(hipMemcpy(ctx->head_w, head_host, sizeof(uint16_t) * V * H, hipMemcpyHostToDevice));
    ctx->vocab = vocab;
    ctx->resident += sizeof(uint16_t) * V * H + sizeof(float) * H;
    return LM_OK;
    LM_GUARD_END
}

int lm_head_forward(lm_context* ctx, const float* hidden_dev, int64_t tokens, float* logits_dev, int32_t* token_dev) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || hidden_dev == nullptr || tokens < 0 || (logits_dev == nullptr && token_dev == nullptr)) {
        return fail(LM_EINVAL, "bad head forward arguments");
    }
    if (ctx->head_w == nullptr) {
        return fail(LM_ENOTRES, "no LM head uploaded");
    }
    int rc = set_device(ctx);
    if (rc != LM_OK) {
        return rc;
    }
    const int64_t H = ctx->H, V = ctx->vocab;
    // tokens per launch: at most kHeadTokens, and their H floats each within 64 KB of LDS
    const int64_t group = std::max<int64_t>(1, std::min<int64_t>(lm::kHeadTokens, 16384 / H));
    for (int64_t t0 = 0; t0 < tokens; t0 += group) {
        const int32_t n = static_cast<int32_t>(tokens - t0 < group ? tokens - t0 : group);
        float* logits = logits_dev != nullptr ? logits_dev + t0 * V : ctx->head_logits;
        LM_HIP(lm::launch_rms_norm(hidden_dev + t0 * H, ctx->head_norm, ctx->head_x, n, static_cast<int32_t>(H),
                                   ctx->cfg.rms_norm_eps, ctx->stream));
        LM_HIP(lm::launch_head(ctx->head_w, ctx->head_x, logits, ctx->head_partial,
                               token_dev != nullptr ? token_dev + t0 : nullptr, V, static_cast<int32_t>(H), n,
                               ctx->stream));
    }
    return LM_OK;
    LM_GUARD_END
}

int lm_finalize_layer(lm_context* ctx, int32_t layer) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (!L.allocated) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no uploaded FFN weights");
    }
    if (!L.dense) {
        for (int e = 0; e < ctx->E; ++e) {
            if (!L.expert_present[static_cast<size_t>(e)]) {
                return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " expert " + std::to_string(e) +
                                            " was not uploaded");
            }
        }
        if (L.router_t == nullptr) {
            return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no router gate");
        }
    }
    // fp16 shadow of every matrix in panel layout (the MFMA path's operands).
    LM_HIP(hipMemsetAsync(ctx->d_overflow, 0, sizeof(int), ctx->stream));
    LM_HIP(hipMemsetAsync(ctx->d_inexact, 0, sizeof(unsigned long long), ctx->stream));
    std::vector<const lm::FfnDev*> ffns;
    if (L.dense) {
        ffns.push_back(&L.dense_ffn);
    } else {
        for (const lm::FfnDev& f : L.experts) {
            ffns.push_back(&f);
        }
        if (ctx->S > 0) {
            ffns.push_back(&L.shared);
        }
    }
    for (const lm::FfnDev* f : ffns) {
        LM_HIP(lm::launch_bf16_to_f16_panels(f->gu, f->gu_h, 2 * static_cast<int64_t>(f->inter_p), ctx->Hp,
                                             ctx->d_overflow, ctx->d_inexact, ctx->stream));
        LM_HIP(lm::launch_bf16_to_f16_panels(f->down, f->down_h, ctx->H, f->inter_p, ctx->d_overflow, ctx->d_inexact,
                                             ctx->stream));
        if (f->down_t != nullptr) {
            LM_HIP(lm::launch_transpose_u16(f->down, f->down_t, ctx->H, f->inter_p, f->inter_p, ctx->Hp, ctx->stream));
        }
    }
    int overflow = 0;
    unsigned long long inexact = 0;
    LM_HIP(hipMemcpyAsync(&overflow, ctx->d_overflow, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
    LM_HIP(hipMemcpyAsync(&inexact, ctx->d_inexact, sizeof(inexact), hipMemcpyDeviceToHost, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    L.fp16_inexact = static_cast<int64_t>(inexact);
    if (overflow != 0) {
        return fail(LM_EINVAL, "layer " + std::to_string(layer) + ": " + std::to_string(overflow) +
                                   " weights exceed the fp16 range of the MFMA path");
    }
    // Group pointer table: gu, down, gu_h, down_h, each [groups].
    const int ng = L.dense ? 1 : ctx->E + 1;
    std::vector<void*> table(static_cast<size_t>(4 * ng), nullptr);
    for (int g = 0; g < ng; ++g) {
        const lm::FfnDev* f = L.dense ? &L.dense_ffn : (g < ctx->E ? &L.experts[static_cast<size_t>(g)] : &L.shared);
        if (!L.dense && g == ctx->E && !L.shared_present) {
            continue;
        }
        table[static_cast<size_t>(g)] = f->gu;
        table[static_cast<size_t>(ng + g)] = f->down;
        table[static_cast<size_t>(2 * ng + g)] = f->gu_h;
        table[static_cast<size_t>(3 * ng + g)] = f->down_h;
    }
    if (L.table == nullptr) {
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&L.table), sizeof(void*) * table.size()));
    }
    LM_HIP(hipMemcpyAsync(L.table, table.data(), sizeof(void*) * table.size(), hipMemcpyHostToDevice, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    L.finalized = true;
    return LM_OK;
    LM_GUARD_END
}

int lm_layer_fp16_inexact(lm_context* ctx, int32_t layer, int64_t* out_count) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (out_count == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    const Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (!L.finalized) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " is not finalized (lm_finalize_layer)");
    }
    *out_count = L.fp16_inexact;
    return LM_OK;
    LM_GUARD_END
}

int lm_resident_bytes(lm_context* ctx, uint64_t* out) {
    if (ctx == nullptr || out == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    *out = ctx->resident;
    return LM_OK;
}

int lm_moe_forward(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, float* y_dev,
                   const float* logit_bias_dev, int32_t* topk_index_dev, float* topk_weight_dev, float* logits_dev,
                   int32_t path) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (tokens < 0 || (tokens > 0 && (x_dev == nullptr || y_dev == nullptr))) {
        return fail(LM_EINVAL, "bad token count or null x / y");
    }
    if (path < LM_PATH_AUTO || path > LM_PATH_MFMA) {
        return fail(LM_EINVAL, "unknown path");
    }
    if (tokens == 0) {
        return LM_OK;
    }
    return moe_layer(ctx, layer, x_dev, tokens, y_dev, nullptr, logit_bias_dev, topk_index_dev, topk_weight_dev,
                     logits_dev, path);
    LM_GUARD_END
}

int lm_moe_forward_noalloc(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, float* y_dev,
                           const float* logit_bias_dev, int32_t* topk_index_dev, float* topk_weight_dev,
                           float* logits_dev) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (tokens < 0 || (tokens > 0 && (x_dev == nullptr || y_dev == nullptr))) {
        return fail(LM_EINVAL, "bad token count or null x / y");
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (!L.allocated || L.dense || L.router_t == nullptr || !L.finalized) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no finalized MoE weights");
    }
    if (!decode_eligible(ctx, L)) {
        return fail(LM_EINVAL, "lm_moe_forward_noalloc: the layer's shape has no single-token kernel");
    }
    const int64_t act_words = static_cast<int64_t>(ctx->K) * ctx->Ip + ctx->Sp;
    const int64_t part_words = lm::decode_shared_part_floats(ctx->H, ctx->Sp);
    if (act_words > kStaticPart - kStaticAct || part_words > kStaticWords - kStaticPart) {
        return fail(LM_EINVAL, "lm_moe_forward_noalloc: the layer needs " +
                                   std::to_string((kStaticPart + part_words) * 4) +
                                   " bytes of scratch (activations up to " + std::to_string((kStaticAct + act_words) * 4) +
                                   "); the fixed array holds " + std::to_string(kStaticScratchBytes));
    }
    if (ctx->device >= kMaxDevices) {
        return fail(LM_EINVAL, "lm_moe_forward_noalloc: device index beyond the fixed scratch table");
    }
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    LM_HIP(hipStreamIsCapturing(ctx->stream, &capture));
    if (capture != hipStreamCaptureStatusNone) {
        // The single-token kernel's hand-off words carry a parity and a tag that
        // the host advances per launch; a replayed capture would repeat them.
        return fail(LM_EINVAL, "lm_moe_forward_noalloc: the context's stream is being captured; graph capture "
                               "and replay of this entry point are not supported");
    }
    if (tokens == 0) {
        return LM_OK;
    }
    std::lock_guard<std::mutex> lock(g_static_mutex);
    StaticScratch& st = g_static[ctx->device];
    if (st.ptr == nullptr || st.last == nullptr) {
        return fail(LM_EHIP, "lm_moe_forward_noalloc: the fixed scratch was not set up on this device");
    }
    // After the previous call on this GPU, whichever stream it ran on.
    LM_HIP(hipStreamWaitEvent(ctx->stream, st.last, 0));
    float* words = reinterpret_cast<float*>(st.ptr);
    const DecodeScratch sc{st.ptr, words + kStaticLogits, words + kStaticAct, words + kStaticPart, nullptr, &st.parity, &st.seq,
                           &st.pending};
    const int64_t H = ctx->H, K = ctx->K;
    for (int64_t t = 0; t < tokens; ++t) {
        int32_t* idx = topk_index_dev != nullptr ? topk_index_dev + t * K : reinterpret_cast<int32_t*>(st.ptr) + kStaticIdx;
        float* wts = topk_weight_dev != nullptr ? topk_weight_dev + t * K : words + kStaticWts;
        rc = decode_layer(ctx, L, sc, x_dev + t * H, y_dev + t * H, nullptr, logit_bias_dev, idx, wts,
                          logits_dev != nullptr ? logits_dev + t * ctx->E : nullptr, nullptr);
        if (rc != LM_OK) {
            break;
        }
    }
    // The next call on this GPU waits for these launches (also after a failed
    // launch: whatever was enqueued still runs on the array).
    LM_HIP(hipEventRecord(st.last, ctx->stream));
    return rc;
    LM_GUARD_END
}

int lm_router(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, const float* logit_bias_dev,
              float* logits_dev, int32_t* topk_index_dev, float* topk_weight_dev) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (L.router_t == nullptr) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no router gate");
    }
    if (tokens < 0 || (tokens > 0 && (x_dev == nullptr || topk_index_dev == nullptr || topk_weight_dev == nullptr))) {
        return fail(LM_EINVAL, "bad token count or null buffers");
    }
    rc = ensure_workspace(ctx, tokens);
    if (rc != LM_OK) {
        return rc;
    }
    lm::RouterArgs ra{};
    ra.x = x_dev;
    ra.wt = L.router_t;
    ra.wq4 = L.router_t + router_quad_row_offset(ctx);
    ra.logits_scratch = ctx->ws.logit_scratch;
    ra.ticket = ctx->ws.ticket;
    ra.bias = logit_bias_dev;
    ra.logits = logits_dev;
    ra.idx = topk_index_dev;
    ra.wts = topk_weight_dev;
    ra.tokens = tokens;
    ra.hidden = ctx->H;
    ra.hidden_p = ctx->Hp;
    ra.experts = ctx->E;
    ra.top_k = ctx->K;
    ra.normalize = ctx->cfg.norm_topk_prob;
    ra.group_limited = ctx->cfg.group_limited;
    ra.n_group = ctx->cfg.n_group;
    ra.topk_group = ctx->cfg.topk_group;
    ra.scale = ctx->cfg.routed_scaling_factor;
    ra.do_matvec = 1;
    LM_HIP(lm::launch_router(ra, ctx->stream, nullptr));
    return LM_OK;
    LM_GUARD_END
}

int lm_router_select(lm_context* ctx, const float* logits_dev, int64_t tokens, int32_t* topk_index_dev,
                     float* topk_weight_dev) {
    LM_GUARD_BEGIN
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    if (tokens < 0 || (tokens > 0 && (logits_dev == nullptr || topk_index_dev == nullptr || topk_weight_dev == nullptr))) {
        return fail(LM_EINVAL, "bad token count or null buffers");
    }
    lm::RouterArgs ra{};
    ra.x = logits_dev;
    ra.idx = topk_index_dev;
    ra.wts = topk_weight_dev;
    ra.tokens = tokens;
    ra.hidden = ctx->H;
    ra.hidden_p = ctx->Hp;
    ra.experts = ctx->E;
    ra.top_k = ctx->K;
    ra.normalize = ctx->cfg.norm_topk_prob;
    ra.group_limited = ctx->cfg.group_limited;
    ra.n_group = ctx->cfg.n_group;
    ra.topk_group = ctx->cfg.topk_group;
    ra.scale = ctx->cfg.routed_scaling_factor;
    ra.do_matvec = 0;
    LM_HIP(lm::launch_router(ra, ctx->stream, nullptr));
    return LM_OK;
    LM_GUARD_END
}

int lm_permute(lm_context* ctx, const int32_t* topk_index_dev, int64_t tokens, int32_t* counts_dev,
               int32_t* offsets_dev, int32_t* perm_dev, int32_t* slot_of_dev) {
    LM_GUARD_BEGIN
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    if (tokens < 0 || (tokens > 0 && (topk_index_dev == nullptr || counts_dev == nullptr || offsets_dev == nullptr ||
                                      perm_dev == nullptr || slot_of_dev == nullptr))) {
        return fail(LM_EINVAL, "bad token count or null buffers");
    }
    int rc = ensure_workspace(ctx, tokens);
    if (rc != LM_OK) {
        return rc;
    }
    lm::PermuteArgs pa{};
    pa.idx = topk_index_dev;
    pa.tokens = tokens;
    pa.top_k = ctx->K;
    pa.experts = ctx->E;
    pa.rb.idx = const_cast<int32_t*>(topk_index_dev);
    pa.rb.counts = counts_dev;
    pa.rb.offsets = offsets_dev;
    pa.rb.perm = perm_dev;
    pa.rb.slot_of = slot_of_dev;
    pa.rb.active = ctx->ws.active;
    pa.scratch = ctx->ws.permute_scratch;
    LM_HIP(lm::launch_permute(pa, ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_grouped_swiglu(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens,
                      const int32_t* topk_index_dev, float* out_dev, int32_t path) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (tokens < 0 || (tokens > 0 && (x_dev == nullptr || topk_index_dev == nullptr || out_dev == nullptr))) {
        return fail(LM_EINVAL, "bad token count or null x / topk_index / out");
    }
    if (path < LM_PATH_AUTO || path > LM_PATH_MFMA) {
        return fail(LM_EINVAL, "unknown path");
    }
    Layer& L = ctx->layers[static_cast<size_t>(layer)];
    if (!L.allocated || L.dense || L.router_t == nullptr || !L.finalized) {
        return fail(LM_ENOTRES, "layer " + std::to_string(layer) + " has no finalized MoE weights");
    }
    if (tokens == 0) {
        return LM_OK;
    }
    rc = set_device(ctx);
    if (rc == LM_OK) {
        rc = ensure_workspace(ctx, tokens);
    }
    if (rc != LM_OK) {
        return rc;
    }
    // The routing comes from the caller: every expert id must name a routed
    // expert, or the permutation would leave its slot unset.
    const int64_t TK = tokens * ctx->K;
    std::vector<int32_t> host_idx(static_cast<size_t>(TK));
    LM_HIP(hipMemcpyAsync(host_idx.data(), topk_index_dev, sizeof(int32_t) * host_idx.size(), hipMemcpyDeviceToHost,
                          ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    for (int64_t a = 0; a < TK; ++a) {
        if (host_idx[static_cast<size_t>(a)] < 0 || host_idx[static_cast<size_t>(a)] >= ctx->E) {
            return fail(LM_EINVAL, "lm_grouped_swiglu: topk_index[" + std::to_string(a) + "] = " +
                                       std::to_string(host_idx[static_cast<size_t>(a)]) + " is not an expert of [0, " +
                                       std::to_string(ctx->E) + ")");
        }
    }
    // Same path choice as lm_moe_forward's batched path (this entry has no
    // single-token form).
    const bool mfma = path == LM_PATH_MFMA || (path == LM_PATH_AUTO && tokens > kMfmaCrossover);
    lm::RouteBufs rb = route_bufs(ctx, const_cast<int32_t*>(topk_index_dev), ctx->ws.wts);
    lm::PermuteArgs pa{};
    pa.idx = topk_index_dev;
    pa.tokens = tokens;
    pa.top_k = ctx->K;
    pa.experts = ctx->E;
    pa.rb = rb;
    pa.scratch = ctx->ws.permute_scratch;
    // Stage timing: no router; the fp16 copy counts with the permutation, the
    // gather with the combine.
    stage_mark(ctx, 0);
    stage_mark(ctx, 1);
    LM_HIP(lm::launch_permute(pa, ctx->stream));
    if (mfma) {
        LM_HIP(lm::launch_to_f16_rows(x_dev, ctx->ws.x16, tokens, ctx->H, ctx->Hp, ctx->stream));
    }
    const lm::ExpertArgs ea = expert_args(ctx, L, x_dev, ctx->ws.x16, tokens, rb);
    rc = launch_expert_kernels(ctx, L, ea, tokens, mfma);
    if (rc != LM_OK) {
        return rc;
    }
    stage_mark(ctx, 4);
    LM_HIP(lm::launch_gather_slots(ctx->ws.down_out, rb.slot_of, out_dev, TK, tokens, ctx->H, ea.has_shared,
                                   ctx->stream));
    stage_mark(ctx, 5);
    return stage_finish(ctx);
    LM_GUARD_END
}

int lm_context_stream(lm_context* ctx, void** out_stream) {
    if (ctx == nullptr || out_stream == nullptr) {
        return fail(LM_EINVAL, "null context or output pointer");
    }
    *out_stream = static_cast<void*>(ctx->stream);
    return LM_OK;
}

int lm_rms_norm(lm_context* ctx, const float* in_dev, const float* weight_dev, float* out_dev, int64_t tokens,
                int32_t hidden, float epsilon) {
    if (ctx == nullptr || in_dev == nullptr || weight_dev == nullptr || out_dev == nullptr || hidden <= 0) {
        return fail(LM_EINVAL, "null argument or bad hidden size");
    }
    LM_HIP(lm::launch_rms_norm(in_dev, weight_dev, out_dev, tokens, hidden, epsilon, ctx->stream));
    return LM_OK;
}

int lm_dense_forward(lm_context* ctx, int32_t layer, const float* x_dev, int64_t tokens, float* y_dev, int32_t path) {
    LM_GUARD_BEGIN
    int rc = check_layer(ctx, layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (tokens <= 0) {
        return tokens == 0 ? LM_OK : fail(LM_EINVAL, "negative token count");
    }
    return dense_layer(ctx, layer, x_dev, tokens, y_dev, nullptr, path);
    LM_GUARD_END
}

namespace {

// lm_stack_forward's layer loop, the workspace already sized.  Between two
// batched layers the first one's combine also applies the second one's RMSNorm
// (and its fp16 copy): bit for bit the separate kernels' results, one pass over
// the hidden state instead of three.
int stack_pass(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev, int64_t tokens,
               int32_t path) {
    bool prenormed = false;
    for (int32_t l = first_layer; l <= last_layer; ++l) {
        const bool fuse_next = l < last_layer && lm::combine_norm_supported(ctx->H, ctx->Hp) &&
                               batched_layer(ctx, l, tokens, path) && batched_layer(ctx, l + 1, tokens, path);
        const float* next_norm = fuse_next ? ctx->layers[static_cast<size_t>(l + 1)].norm : nullptr;
        const int rc = ffn_sublayer_fused(ctx, l, hidden_dev, tokens, path, next_norm, prenormed);
        if (rc != LM_OK) {
            return rc;
        }
        prenormed = fuse_next;
    }
    return LM_OK;
}

int check_stack_args(lm_context* ctx, int32_t first_layer, int32_t last_layer) {
    int rc = check_layer(ctx, first_layer);
    if (rc == LM_OK) {
        rc = check_layer(ctx, last_layer);
    }
    return rc;
}

}  // namespace

int lm_stack_forward(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev, int64_t tokens,
                     int32_t path) {
    LM_GUARD_BEGIN
    int rc = check_stack_args(ctx, first_layer, last_layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (tokens <= 0 || hidden_dev == nullptr) {
        return tokens == 0 ? LM_OK : fail(LM_EINVAL, "bad token count or null hidden state");
    }
    rc = ensure_workspace(ctx, tokens);
    if (rc != LM_OK) {
        return rc;
    }
    return stack_pass(ctx, first_layer, last_layer, hidden_dev, tokens, path);
    LM_GUARD_END
}

struct lm_stack_graph {
    lm_context* ctx = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    int32_t first = 0, last = -1;
};

int lm_stack_graph_create(lm_context* ctx, int32_t first_layer, int32_t last_layer, float* hidden_dev,
                          int64_t tokens, int32_t path, lm_stack_graph** graph) {
    LM_GUARD_BEGIN
    if (graph == nullptr) {
        return fail(LM_EINVAL, "null graph output");
    }
    *graph = nullptr;
    int rc = check_stack_args(ctx, first_layer, last_layer);
    if (rc != LM_OK) {
        return rc;
    }
    if (first_layer > last_layer || tokens <= 0 || hidden_dev == nullptr) {
        return fail(LM_EINVAL, "empty layer range, bad token count or null hidden state");
    }
    if (ctx->timing) {
        return fail(LM_EINVAL, "lm_stack_graph_create: stage timing is on (its events are host state a replay "
                               "would not update)");
    }
    for (int32_t l = first_layer; l <= last_layer; ++l) {
        const Layer& L = ctx->layers[static_cast<size_t>(l)];
        if (!L.dense && takes_decode_path(ctx, L, tokens, path)) {
            return fail(LM_EINVAL, "lm_stack_graph_create: at " + std::to_string(tokens) + " tokens layer " +
                                       std::to_string(l) +
                                       " runs the single-token kernel, whose hand-off words carry a tag the host "
                                       "advances per launch (a replay would repeat it)");
        }
    }
    rc = ensure_workspace(ctx, tokens);
    if (rc != LM_OK) {
        return rc;
    }
    LM_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    rc = stack_pass(ctx, first_layer, last_layer, hidden_dev, tokens, path);
    hipGraph_t g = nullptr;
    const hipError_t end = hipStreamEndCapture(ctx->stream, &g);
    if (rc != LM_OK || end != hipSuccess) {
        if (g != nullptr) {
            (void)hipGraphDestroy(g);
        }
        return rc != LM_OK ? rc : fail(LM_EHIP, std::string("stack capture: ") + hipGetErrorString(end));
    }
    hipGraphExec_t exec = nullptr;
    const hipError_t inst = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    if (inst != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(LM_EHIP, std::string("stack graph instantiate: ") + hipGetErrorString(inst));
    }
    *graph = new lm_stack_graph{ctx, g, exec, first_layer, last_layer};
    ++ctx->graphs;
    return LM_OK;
    LM_GUARD_END
}

int lm_stack_graph_launch(lm_stack_graph* graph) {
    LM_GUARD_BEGIN
    if (graph == nullptr) {
        return fail(LM_EINVAL, "null graph");
    }
    // The graph reads each layer's slab through the pointers of the capture.  An
    // upload into a layer since then (without lm_finalize_layer) leaves its fp16
    // copy stale, which the eager path refuses too.
    for (int32_t l = graph->first; l <= graph->last; ++l) {
        if (!graph->ctx->layers[static_cast<size_t>(l)].finalized) {
            return fail(LM_ENOTRES, "lm_stack_graph_launch: layer " + std::to_string(l) +
                                        " was uploaded since the capture and is not finalized (lm_finalize_layer)");
        }
    }
    LM_HIP(hipGraphLaunch(graph->exec, graph->ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_stack_graph_destroy(lm_stack_graph* graph) {
    LM_GUARD_BEGIN
    if (graph == nullptr) {
        return LM_OK;
    }
    LM_HIP(hipStreamSynchronize(graph->ctx->stream));  // no replay may still read the workspace
    (void)hipGraphExecDestroy(graph->exec);
    (void)hipGraphDestroy(graph->graph);
    --graph->ctx->graphs;
    delete graph;
    return LM_OK;
    LM_GUARD_END
}

int lm_gemm_matvec_bf16(lm_context* ctx, const uint16_t* w_host, const float* x_host, float* out_host,
                        size_t out_dim, size_t in_dim, float scale, int32_t accumulate) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || w_host == nullptr || x_host == nullptr || out_host == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    if (out_dim == 0) {
        return LM_OK;
    }
    void* w_dev = nullptr;
    int rc = matrix_for_call(ctx, w_host, out_dim * in_dim * 2, &w_dev);
    if (rc == LM_OK) {
        rc = ensure_gemm_scratch(ctx, std::max(out_dim, in_dim));
    }
    if (rc != LM_OK) {
        return rc;
    }
    LM_HIP(hipMemcpyAsync(ctx->gemm_x, x_host, in_dim * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    if (accumulate) {
        LM_HIP(hipMemcpyAsync(ctx->gemm_out, out_host, out_dim * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    }
    LM_HIP(lm::launch_gemv_plain(static_cast<const uint16_t*>(w_dev), ctx->gemm_x, ctx->gemm_out,
                                 static_cast<int64_t>(out_dim), static_cast<int64_t>(in_dim), scale, accumulate,
                                 ctx->stream));
    LM_HIP(hipMemcpyAsync(out_host, ctx->gemm_out, out_dim * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_gemm_matvec_f32(lm_context* ctx, const float* w_host, const float* x_host, float* out_host, size_t out_dim,
                       size_t in_dim) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || w_host == nullptr || x_host == nullptr || out_host == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    if (out_dim == 0) {
        return LM_OK;
    }
    void* w_dev = nullptr;
    int rc = matrix_for_call(ctx, w_host, out_dim * in_dim * sizeof(float), &w_dev);
    if (rc == LM_OK) {
        rc = ensure_gemm_scratch(ctx, std::max(out_dim, in_dim));
    }
    if (rc != LM_OK) {
        return rc;
    }
    LM_HIP(hipMemcpyAsync(ctx->gemm_x, x_host, in_dim * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    LM_HIP(lm::launch_matvec_f32_ref(static_cast<const float*>(w_dev), ctx->gemm_x, ctx->gemm_out,
                                     static_cast<int64_t>(out_dim), static_cast<int64_t>(in_dim), ctx->stream));
    LM_HIP(hipMemcpyAsync(out_host, ctx->gemm_out, out_dim * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_vector_op(lm_context* ctx, int32_t op, const void* a_host, const float* b_host, float* out_host, size_t n,
                 float scalar) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || out_host == nullptr || (n > 0 && a_host == nullptr)) {
        return fail(LM_EINVAL, "null argument");
    }
    if (op < LM_OP_DOT || op > LM_OP_WIDEN) {
        return fail(LM_EINVAL, "unknown vector op");
    }
    const bool needs_b = op == LM_OP_DOT || op == LM_OP_SILU_MUL || op == LM_OP_RMS_NORM;
    if (needs_b && b_host == nullptr) {
        return fail(LM_EINVAL, "the operation needs a second operand");
    }
    if (n == 0) {
        if (op == LM_OP_DOT) {
            out_host[0] = 0.0f;
        }
        return LM_OK;
    }
    int rc = ensure_gemm_scratch(ctx, n);
    if (rc != LM_OK) {
        return rc;
    }
    const size_t a_bytes = op == LM_OP_WIDEN ? n * sizeof(uint16_t) : n * sizeof(float);
    LM_HIP(hipMemcpyAsync(ctx->gemm_x, a_host, a_bytes, hipMemcpyHostToDevice, ctx->stream));
    if (needs_b) {
        LM_HIP(hipMemcpyAsync(ctx->gemm_b, b_host, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    }
    if (op == LM_OP_AXPY) {
        LM_HIP(hipMemcpyAsync(ctx->gemm_out, out_host, n * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
    }
    LM_HIP(lm::launch_vector_op(op, ctx->gemm_x, ctx->gemm_b, ctx->gemm_out, static_cast<int64_t>(n), scalar,
                                ctx->stream));
    const size_t out_n = op == LM_OP_DOT ? 1 : n;
    LM_HIP(hipMemcpyAsync(out_host, ctx->gemm_out, out_n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_weight_prefetch(lm_context* ctx, const void* host_ptr, size_t bytes) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || host_ptr == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    void* dev = nullptr;
    int rc = resident_copy(ctx, host_ptr, bytes, &dev);
    if (rc != LM_OK) {
        return rc;
    }
    LM_HIP(hipStreamSynchronize(ctx->stream));
    return LM_OK;
    LM_GUARD_END
}

int lm_weight_release(lm_context* ctx, const void* host_ptr) {
    LM_GUARD_BEGIN
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    auto it = ctx->resident_ptrs.find(host_ptr);
    if (it != ctx->resident_ptrs.end()) {
        LM_HIP(hipStreamSynchronize(ctx->stream));
        LM_HIP(hipFree(it->second.dev));
        ctx->resident_ptrs.erase(it);
    }
    return LM_OK;
    LM_GUARD_END
}

int lm_weight_resident(lm_context* ctx, const void* host_ptr, int32_t* out_resident) {
    if (ctx == nullptr || out_resident == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    *out_resident = ctx->resident_ptrs.count(host_ptr) != 0 ? 1 : 0;
    return LM_OK;
}

int lm_decode_speculation_test(lm_context* ctx, int32_t mode) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    ctx->decode_perturb = mode != 0 ? 1 : 0;
    return LM_OK;
}

int lm_router_speculation(lm_context* ctx, int32_t mode) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    if (mode < 0 || mode > 2) {
        return fail(LM_EINVAL, "lm_router_speculation: mode must be 0, 1 or 2");
    }
    ctx->spec_mode = mode;
    return LM_OK;
}

int lm_decode_wait_test(lm_context* ctx, int32_t mode) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    ctx->decode_max_spins = mode != 0 ? 1u : 0u;
    return LM_OK;
}

int lm_event_create(lm_context* ctx, void** out_event) {
    if (ctx == nullptr || out_event == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    hipEvent_t e = nullptr;
    LM_HIP(hipEventCreate(&e));
    *out_event = e;
    return LM_OK;
}

int lm_event_destroy(lm_context* ctx, void* event) {
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    LM_HIP(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return LM_OK;
}

int lm_event_record(lm_context* ctx, void* event) {
    if (ctx == nullptr || event == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    LM_HIP(hipEventRecord(static_cast<hipEvent_t>(event), ctx->stream));
    return LM_OK;
}

int lm_event_elapsed_ms(lm_context* ctx, void* start, void* stop, float* out_ms) {
    if (ctx == nullptr || start == nullptr || stop == nullptr || out_ms == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    LM_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
    LM_HIP(hipEventElapsedTime(out_ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    return LM_OK;
}

namespace {
constexpr int32_t kProbePairs = 100000;  // 2 s of 20 us intervals
constexpr int64_t kProbePeriodTicks = 2000;  // 20 us of the 100 MHz counter
}  // namespace

int lm_clock_probe_start(lm_context* ctx, double seconds) {
    LM_GUARD_BEGIN
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    if (!(seconds > 0.0) || seconds > 2.0) {
        return fail(LM_EINVAL, "lm_clock_probe_start: seconds must be in (0, 2]");
    }
    if (ctx->probe_running) {
        return fail(LM_EINVAL, "lm_clock_probe_start: a probe is running (lm_clock_probe_finish first)");
    }
    int rc = set_device(ctx);
    if (rc != LM_OK) {
        return rc;
    }
    if (ctx->probe_stream == nullptr) {
        LM_HIP(hipStreamCreateWithFlags(&ctx->probe_stream, hipStreamNonBlocking));
        LM_HIP(hipMalloc(reinterpret_cast<void**>(&ctx->probe_buf), sizeof(uint64_t) * (2 * kProbePairs + 1)));
    }
    const int64_t total = static_cast<int64_t>(seconds * 1e8);
    LM_HIP(lm::launch_clock_probe(ctx->probe_buf, kProbePairs, kProbePeriodTicks, total, ctx->probe_stream));
    ctx->probe_running = true;
    return LM_OK;
    LM_GUARD_END
}

int lm_clock_probe_finish(lm_context* ctx, double* out_median_mhz, double* out_min_mhz, double* out_max_mhz,
                          int32_t* out_intervals) {
    LM_GUARD_BEGIN
    if (ctx == nullptr || out_median_mhz == nullptr || out_min_mhz == nullptr || out_max_mhz == nullptr ||
        out_intervals == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    if (!ctx->probe_running) {
        return fail(LM_EINVAL, "lm_clock_probe_finish: no probe running");
    }
    ctx->probe_running = false;
    LM_HIP(hipStreamSynchronize(ctx->probe_stream));
    std::vector<uint64_t> h(2 * kProbePairs + 1);
    LM_HIP(hipMemcpy(h.data(), ctx->probe_buf, h.size() * sizeof(uint64_t), hipMemcpyDeviceToHost));
    const int64_t n = std::min<int64_t>(static_cast<int64_t>(h[2 * kProbePairs]), kProbePairs);
    std::vector<double> mhz;
    for (int64_t i = 1; i < n; ++i) {
        const uint64_t dr = h[2 * i] - h[2 * (i - 1)];
        const uint64_t dc = h[2 * i + 1] - h[2 * (i - 1) + 1];
        if (dr > 0) {
            mhz.push_back(static_cast<double>(dc) / static_cast<double>(dr) * 100.0);
        }
    }
    *out_intervals = static_cast<int32_t>(mhz.size());
    if (mhz.empty()) {
        *out_median_mhz = *out_min_mhz = *out_max_mhz = 0.0;
        return LM_OK;
    }
    std::sort(mhz.begin(), mhz.end());
    *out_median_mhz = mhz[mhz.size() / 2];
    *out_min_mhz = mhz.front();
    *out_max_mhz = mhz.back();
    return LM_OK;
    LM_GUARD_END
}

int lm_stage_timing(lm_context* ctx, int32_t enable) {
    LM_GUARD_BEGIN
    if (ctx == nullptr) {
        return fail(LM_EINVAL, "null context");
    }
    if (enable && ctx->ring.empty()) {
        ctx->ring.resize(kEventRing);
        for (EventSet& es : ctx->ring) {
            for (hipEvent_t& e : es.ev) {
                LM_HIP(hipEventCreate(&e));
            }
        }
    }
    int rc = stage_collect(ctx);
    if (rc != LM_OK) {
        return rc;
    }
    ctx->timing = enable != 0;
    for (int s = 0; s < kStages; ++s) {
        ctx->stage_ms[s] = 0.0;
        ctx->stage_calls[s] = 0;
    }
    return LM_OK;
    LM_GUARD_END
}

int lm_stage_times(lm_context* ctx, double* out_ms, int32_t* out_calls, int32_t stages) {
    if (ctx == nullptr || out_ms == nullptr || out_calls == nullptr) {
        return fail(LM_EINVAL, "null argument");
    }
    int rc = stage_collect(ctx);
    if (rc != LM_OK) {
        return rc;
    }
    for (int s = 0; s < stages && s < kStages; ++s) {
        out_ms[s] = ctx->stage_ms[s];
        out_calls[s] = ctx->stage_calls[s];
    }
    return LM_OK;
}

}  // extern "C"
