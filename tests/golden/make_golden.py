"""Writes the golden fixtures under tests/golden/ from LiteMind's own code.

Run in a container that has the LiteMind sources (oracle/_ref/libref.so is built
from them by `make -C oracle ref`):

    python tests/golden/make_golden.py

Every output is computed by the compiled reference (its Gemm, MoeRouter,
ExpertCache and ThreadPool, composed per token as its runner does).  Large
inputs are not stored: they are regenerated from the recorded seeds by
litemind_amd.workload, and their SHA-256 is stored so a changed generator is
detected.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle_lib as ol  # noqa: E402
from litemind_amd import workload as wl  # noqa: E402


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def layer_digest(layer) -> str:
    parts = [layer.router] + layer.gate + layer.up + layer.down
    if layer.shared_gate is not None:
        parts += [layer.shared_gate, layer.shared_up, layer.shared_down]
    return sha(*parts)


def kerneltest():
    """tests/KernelTest.cpp:28-79: 67 x 253 matvec, threaded / serial / accumulate."""
    r = ol.ref()
    out_dim, in_dim = 67, 253
    w = np.zeros((out_dim, in_dim), np.uint16)
    x = np.zeros(in_dim, np.float32)
    r.ref_kerneltest_inputs(ol.p(w), ol.p(x), out_dim, in_dim)
    threaded = np.zeros(out_dim, np.float32)
    serial = np.zeros(out_dim, np.float32)
    acc = np.ones(out_dim, np.float32)
    r.ref_matvec_bf16(4, ol.p(w), ol.p(x), ol.p(threaded), out_dim, in_dim)
    r.ref_matvec_bf16_serial(ol.p(w), ol.p(x), ol.p(serial), out_dim, in_dim)
    r.ref_matvec_bf16_accumulate(4, ol.p(w), ol.p(x), ol.p(acc), out_dim, in_dim, 0.5)
    # closed-form cases of the same test
    rms = np.array([1, 2, 3, 4], np.float32)
    r.ref_rms_norm(ol.p(rms), ol.p(np.full(4, 2.0, np.float32)), 4, 1e-6)
    sm = np.array([1, 2, 3], np.float32)
    r.ref_softmax(ol.p(sm), 3)
    ext = np.array([1000, 1001], np.float32)
    r.ref_softmax(ol.p(ext), 2)
    silu = np.zeros(2, np.float32)
    r.ref_silu_multiply(ol.p(np.array([0, 1], np.float32)), ol.p(np.array([3, 2], np.float32)), ol.p(silu), 2)
    np.savez_compressed(os.path.join(HERE, "kerneltest.npz"), weights=w, input=x, threaded=threaded, serial=serial,
                        accumulate=acc, rms_norm=rms, softmax=sm, softmax_extreme=ext, silu=silu)


ROUTER_VARIANTS = {
    # name: (experts, top_k, normalize, scale, group_limited, n_group, topk_group)
    "greedy": (8, 3, 0, 1.0, 0, 1, 1),
    "normalize": (8, 3, 1, 1.0, 0, 1, 1),
    "scale2": (8, 3, 0, 2.0, 0, 1, 1),
    "both": (8, 3, 1, 2.0, 0, 1, 1),
    "grouped": (8, 2, 0, 1.0, 1, 2, 1),
}
KNOWN_LOGITS = np.array([0.0, 5.0, 1.0, 4.0, 2.0, 3.0, -1.0, -2.0], np.float32)


def router_known():
    """tests/MoeRouterSamplerTest.cpp:30-93 cases through the compiled router."""
    out = {"logits": KNOWN_LOGITS}
    for name, (E, k, norm, scale, grouped, ng, tg) in ROUTER_VARIANTS.items():
        cfg = ol.router_cfg(E, k, bool(norm), scale, bool(grouped), ng, tg)
        idx, w = ol.ref_select(KNOWN_LOGITS, cfg)
        out[f"{name}_index"] = idx
        out[f"{name}_weight"] = w
    idx = np.zeros(3, np.int32)
    w = np.zeros(3, np.float32)
    n = ol.ref().ref_router_select_top_k(ol.p(KNOWN_LOGITS), 8, 8, 3, 1, ol.p(idx), ol.p(w))
    out["legacy_index"], out["legacy_weight"] = idx[:n], w[:n]
    # tie and random cases for E = 64, k = 6
    rng = np.random.default_rng(20240816)
    rand = rng.standard_normal((64, 64)).astype(np.float32)
    rand[:16, 10] = rand[:16, 3]
    rand[16:32] = np.round(rand[16:32])
    rand[32] = 0.0
    cfg = ol.router_cfg(64, 6)
    ri = np.zeros((64, 6), np.int32)
    rw = np.zeros((64, 6), np.float32)
    for t in range(64):
        ri[t], rw[t] = ol.ref_select(rand[t], cfg)
    out["random_logits"], out["random_index"], out["random_weight"] = rand, ri, rw
    np.savez_compressed(os.path.join(HERE, "router_known.npz"), **out)


# More than 64 experts, group-limited greedy routing: DeepSeek-V2's 160 experts
# in 8 groups (3 kept), a 256-expert layer in 8 groups (4 kept, top-8,
# normalised), and 512 experts in 16 groups (4 kept, scaled).
WIDE_VARIANTS = {
    "e160": (160, 6, 0, 1.0, 1, 8, 3),
    "e256": (256, 8, 1, 1.0, 1, 8, 4),
    "e512": (512, 8, 0, 2.5, 1, 16, 4),
    "e160_greedy": (160, 6, 0, 1.0, 0, 1, 1),
}


def router_wide():
    """The compiled router on 48 logit vectors per configuration: random
    N(0, 2), rounded (many exact ties between experts and between groups), and
    one row of equal logits."""
    out = {}
    rng = np.random.default_rng(20260160)
    for name, (E, k, norm, scale, grouped, ng, tg) in WIDE_VARIANTS.items():
        cfg = ol.router_cfg(E, k, bool(norm), scale, bool(grouped), ng, tg)
        logits = (rng.standard_normal((48, E)) * 2).astype(np.float32)
        logits[16:32] = np.round(logits[16:32])
        logits[40] = 0.5
        idx = np.zeros((48, k), np.int32)
        w = np.zeros((48, k), np.float32)
        for t in range(48):
            idx[t], w[t] = ol.ref_select(logits[t], cfg)
        out[f"{name}_logits"], out[f"{name}_index"], out[f"{name}_weight"] = logits, idx, w
    np.savez_compressed(os.path.join(HERE, "router_wide.npz"), **out)


def router_v2lite():
    """Full-width router of DeepSeek-V2-Lite (64 experts, hidden 2048) on 64 seeded tokens."""
    seed, T = wl.MASTER_SEED, 64
    router = wl.normal_f32(seed, wl.stream_id(0, wl.S_ROUTER), 0.02, (64, 2048))
    x = wl.tokens(seed + 1, T, 2048)
    logits = np.zeros((T, 64), np.float32)
    for t in range(T):
        ol.ref().ref_matvec_f32(ol.p(router), ol.p(np.ascontiguousarray(x[t])), ol.p(logits[t]), 64, 2048)
    cfg = ol.router_cfg(64, 6)
    idx = np.zeros((T, 6), np.int32)
    w = np.zeros((T, 6), np.float32)
    for t in range(T):
        idx[t], w[t] = ol.ref_select(logits[t], cfg)
    np.savez_compressed(os.path.join(HERE, "router_v2lite.npz"), seed=np.int64(seed), tokens=np.int64(T),
                        input_sha=np.array(sha(router, x)), logits=logits, index=idx, weight=w)


def layer_tiny():
    """A MoE layer of LiteMind's tiny test checkpoint recipe (tools/make_test_model.py)."""
    dims, layer = wl.tiny_model_layers(1)
    x = wl.tokens(7, 8, dims.hidden)
    y, idx, w = ol.ref_moe_layer(layer, x, workers=4)
    np.savez_compressed(os.path.join(HERE, "layer_tiny.npz"), x=x, y=y, index=idx, weight=w,
                        weights_sha=np.array(layer_digest(layer)))


def layer_v2lite():
    """DeepSeek-V2-Lite MoE layer 0 (seeded) on 4 tokens, plus 4 skewed-bias tokens."""
    seed = wl.MASTER_SEED
    layer = wl.moe_layer(seed, 0)
    x = wl.tokens(seed + 2, 4, 2048)
    y, idx, w = ol.ref_moe_layer(layer, x, workers=0)
    bias = wl.skew_bias()
    yb, idxb, wb = ol.ref_moe_layer(layer, x, bias=bias, workers=0)
    np.savez_compressed(os.path.join(HERE, "layer_v2lite.npz"), seed=np.int64(seed), x=x, y=y, index=idx, weight=w,
                        bias=bias, y_bias=yb, index_bias=idxb, weight_bias=wb,
                        weights_sha=np.array(layer_digest(layer)))


def expert_cache_trace():
    """ExpertCache LRU counters after each touch (src/ExpertCache.cpp:9-68)."""
    r = ol.ref()
    rng = np.random.default_rng(7)
    block = 3 * 1408 * 2048 * 2
    touches = [(int(rng.integers(1, 3)), int(rng.integers(0, 10))) for _ in range(80)]
    out = {"touches": touches, "block_bytes": block, "runs": {}}
    for name, budget in (("budget3", 3 * block), ("storm", 1), ("disabled", 0), ("budget5", 5 * block)):
        h = r.ref_cache_create(budget)
        rows = []
        for layer, expert in touches:
            r.ref_cache_touch(h, r.ref_cache_make_key(layer, expert), 1408, 2048)
            c = np.zeros(7, np.uint64)
            r.ref_cache_counters(h, ol.p(c))
            rows.append([int(v) for v in c])
        r.ref_cache_clear(h)
        c = np.zeros(7, np.uint64)
        r.ref_cache_counters(h, ol.p(c))
        rows.append([int(v) for v in c])
        r.ref_cache_destroy(h)
        out["runs"][name] = {"budget": budget, "counters": rows}
    keys = [[layer, expert, int(r.ref_cache_make_key(layer, expert))] for layer, expert in ((0, 0), (1, 5), (26, 63))]
    out["make_key"] = keys
    with open(os.path.join(HERE, "expert_cache_trace.json"), "w") as f:
        json.dump(out, f)


MLA_SMALL = dict(hidden=256, heads=4, kv_lora_rank=64, qk_nope=32, qk_rope=16, v_head=32, original_max=16,
                 factor=4.0, max_positions=16)
MLA_CASES = {
    # name: (dims overrides, seed, tokens, first position)
    "small_yarn": (dict(MLA_SMALL), 11, 10, 0),
    "small_qlora_plain": (dict(MLA_SMALL, q_lora_rank=96, yarn=False), 12, 10, 3),
    "small_full": (dict(MLA_SMALL, max_positions=4), 13, 6, 0),
    "v2lite": (dict(max_positions=8), 14, 8, 0),
}


def mla_dims(overrides):
    import dataclasses
    return dataclasses.replace(wl.V2_LITE_MLA, **overrides)


def mla_layer_digest(L) -> str:
    return sha(*[a for a in (L.q_proj, L.q_a_proj, L.q_a_layernorm, L.q_b_proj, L.kv_a_proj, L.kv_a_layernorm,
                             L.kv_b_proj, L.o_proj) if a is not None])


def mla():
    """Attention::forward (src/Attention.cpp:22-103) through the compiled
    reference over short token sequences with a fresh KvCache of capacity
    max_positions (as DeepSeekRunner sizes both from the context length), and
    the rotary tables of DeepSeek-V2-Lite read back through RotaryEmbedding::apply."""
    out = {}
    for name, (over, seed, T, pos0) in MLA_CASES.items():
        d = mla_dims(over)
        L = wl.mla_layer(seed, 0, d)
        x = wl.tokens(seed + 1, T, d.hidden)
        y, done, kn, kr, v = ol.ref_mla(L, x, pos0, d.max_positions)
        out[name + "/dims"] = np.array(json.dumps(over))
        out[name + "/meta"] = np.array([seed, T, pos0, done], np.int64)
        out[name + "/weights_sha"] = np.array(mla_layer_digest(L))
        out[name + "/out"] = y
        if name == "v2lite":
            out[name + "/x_sha"] = np.array(sha(x))
            out[name + "/cache_sha"] = np.array(sha(kn[:done], kr[:done], v[:done]))
        else:
            out[name + "/x"] = x
            out[name + "/key_nope"] = kn[:done]
            out[name + "/key_rope"] = kr[:done]
            out[name + "/value"] = v[:done]
    d = wl.V2_LITE_MLA
    cos, sin = ol.ref_rope_tables(d)
    rows = np.array([0, 1, 2, 100, 1000, d.max_positions - 1], np.int64)
    out["rope/rows"] = rows
    out["rope/cos"] = cos[rows]
    out["rope/sin"] = sin[rows]
    out["rope/sha"] = np.array(sha(cos, sin))
    out["rope/softmax_scale"] = np.float32(ol.ref().ref_softmax_scale(d.qk_nope, d.qk_rope, 1, d.factor,
                                                                      d.mscale_all_dim))
    np.savez_compressed(os.path.join(HERE, "mla.npz"), **out)


def main():
    if not ol.have_ref():
        sys.exit("oracle/_ref/libref.so is not built (make -C oracle ref)")
    kerneltest()
    router_known()
    router_wide()
    router_v2lite()
    layer_tiny()
    layer_v2lite()
    expert_cache_trace()
    mla()
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
