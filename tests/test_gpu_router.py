"""Router parity on the GPU: logits, selected experts and weights must equal the
oracle (LiteMind's matvec_f32 + MoeRouter::select restated) bit for bit."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import announce

pytestmark = pytest.mark.gpu


def _gpu_route(ctx, layer, x, bias=None):
    T, E, K = x.shape[0], ctx.config.n_routed_experts, ctx.config.num_experts_per_tok
    dx = ctx.to_device(x)
    db = ctx.to_device(bias) if bias is not None else None
    lg, idx, w = ctx.empty((T, E)), ctx.empty((T, K), np.int32), ctx.empty((T, K))
    ctx.router(layer, dx, T, idx, w, bias=db, logits=lg)
    ctx.synchronize()
    out = lg.download(), idx.download(), w.download()
    for b in (dx, lg, idx, w) + ((db,) if db is not None else ()):
        b.free()
    return out


def _oracle_route(layer, x, bias=None):
    d = layer.dims
    T = x.shape[0]
    logits = np.zeros((T, d.experts), np.float32)
    for t in range(T):
        ol.oracle().orc_matvec_f32(ol.p(layer.router), ol.p(np.ascontiguousarray(x[t])), ol.p(logits[t]),
                                   d.experts, d.hidden)
    if bias is not None:
        logits = (logits + bias.astype(np.float32)).astype(np.float32)
    cfg = ol.router_cfg(d.experts, d.top_k, d.norm_topk_prob, d.routed_scaling_factor)
    idx = np.zeros((T, d.top_k), np.int32)
    w = np.zeros((T, d.top_k), np.float32)
    for t in range(T):
        idx[t], w[t] = ol.oracle_select(logits[t], cfg)
    return logits, idx, w


@pytest.mark.parametrize("case", ["t1", "t5", "t32", "t48_bias", "t64", "t100_ragged", "t512_uniform", "t2048_skewed",
                                  "t4096", "t4100_ragged"])
def test_router_bit_exact_v2lite(v2_ctx, case):
    """Every router kernel of the V2-Lite shape: the single-token split kernel,
    the logits over 8 workgroups per token with a wave per token selecting
    (2 to 64 tokens, with and without a logit bias), and the wide kernel above
    (one partly filled workgroup up to one, two and four tokens per wave,
    including partial last workgroups)."""
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    T = {"t1": 1, "t5": 5, "t32": 32, "t48_bias": 48, "t64": 64, "t100_ragged": 100, "t512_uniform": 512,
         "t2048_skewed": 2048, "t4096": 4096, "t4100_ragged": 4100}[case]
    layer_id = 1 if case == "t512_uniform" else 0
    bias = wl.skew_bias() if case in ("t2048_skewed", "t48_bias") else None
    x = wl.tokens(wl.MASTER_SEED + T, T, 2048)
    announce(f"router {case} T={T} layer={layer_id}")
    g_logits, g_idx, g_w = _gpu_route(ctx, layer_id, x, bias)
    o_logits, o_idx, o_w = _oracle_route(layers[layer_id], x, bias)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32)), "logits differ"
    assert np.array_equal(g_idx, o_idx), "selected experts differ"
    assert np.array_equal(g_w.view(np.uint32), o_w.view(np.uint32)), "weights differ"


@pytest.mark.parametrize("T", [2, 4, 37, 70])
def test_router_bit_exact_32_experts(T):
    """A 32-expert gate (H = 512) is outside the wide kernel's shape: 2 to 64
    tokens take the logits over 4 workgroups per token, more the per-wave
    kernel."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.Dims(hidden=512, inter=128, experts=32, top_k=4, n_shared=1, dense_inter=256, layers=1,
                   norm_topk_prob=True, routed_scaling_factor=2.0)
    layer = wl.moe_layer(wl.MASTER_SEED + 5, 0, dims)
    x = wl.tokens(wl.MASTER_SEED + 100 + T, T, dims.hidden)
    announce(f"router 32 experts H=512 T={T}")
    ctx = Context(dims.moe_config(num_layers=1))
    try:
        wl.upload_moe_layer(ctx, 0, layer)
        g = _gpu_route(ctx, 0, x)
    finally:
        ctx.close()
    o = _oracle_route(layer, x)
    for a, b in zip(g, o):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


@pytest.mark.parametrize("T", [3, 40])
def test_router_bit_exact_60_experts(T):
    """60 experts (not a multiple of 8): no per-token split, so few tokens take
    the 16-wave few-token kernel and more the per-wave kernel; logits, experts
    and weights bit for bit, with a logit bias."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.Dims(hidden=512, inter=128, experts=60, top_k=6, n_shared=1, dense_inter=256, layers=1)
    rng = np.random.default_rng(60 + T)
    gate = (rng.standard_normal((60, 512)) * 0.05).astype(np.float32)
    bias = (rng.standard_normal(60) * 0.01).astype(np.float32)
    x = rng.standard_normal((T, 512)).astype(np.float32)
    layer = wl.MoeLayer(dims, gate, None, None, None, None, None, None)
    announce(f"router 60 experts T={T}")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        ctx.upload_router(0, gate)
        g_logits, g_idx, g_w = _gpu_route(ctx, 0, x, bias)
    o_logits, o_idx, o_w = _oracle_route(layer, x, bias)
    assert np.array_equal(g_logits.view(np.uint32), o_logits.view(np.uint32)), "logits differ"
    assert np.array_equal(g_idx, o_idx), "selected experts differ"
    assert np.array_equal(g_w.view(np.uint32), o_w.view(np.uint32)), "weights differ"


def test_router_tiny_model(tiny_ctx):
    from litemind_amd import workload as wl

    ctx, layer = tiny_ctx
    x = wl.tokens(11, 64, layer.dims.hidden)
    announce("router tiny model T=64")
    g = _gpu_route(ctx, 0, x)
    o = _oracle_route(layer, x)
    for a, b in zip(g, o):
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32))


def _select_ctx(experts, top_k, normalize=False, scale=1.0, group_limited=False, n_group=1, topk_group=1):
    from litemind_amd import Context, MoeConfig

    cfg = MoeConfig(hidden_size=64, moe_intermediate_size=64, n_routed_experts=experts, num_experts_per_tok=top_k,
                    n_shared_experts=0, intermediate_size=0, norm_topk_prob=1 if normalize else 0,
                    routed_scaling_factor=scale, group_limited=1 if group_limited else 0, n_group=n_group,
                    topk_group=topk_group, rms_norm_eps=1e-6, num_layers=1)
    return Context(cfg)


# The known-answer cases of tests/MoeRouterSamplerTest.cpp:30-93.
KNOWN = np.array([0.0, 5.0, 1.0, 4.0, 2.0, 3.0, -1.0, -2.0], np.float32)


@pytest.mark.parametrize("variant", ["greedy", "normalize", "scale2", "both", "grouped"])
def test_router_select_known_answers(variant):
    kw = dict(experts=8, top_k=3)
    if variant == "normalize":
        kw["normalize"] = True
    elif variant == "scale2":
        kw["scale"] = 2.0
    elif variant == "both":
        kw.update(normalize=True, scale=2.0)
    elif variant == "grouped":
        kw.update(group_limited=True, n_group=2, topk_group=1, top_k=2)
    announce(f"router select known answers {variant}")
    with _select_ctx(**kw) as ctx:
        lg = ctx.to_device(KNOWN.reshape(1, 8))
        idx, w = ctx.empty((1, kw["top_k"]), np.int32), ctx.empty((1, kw["top_k"]))
        ctx.router_select(lg, 1, idx, w)
        ctx.synchronize()
        g_idx, g_w = idx.download()[0], w.download()[0]
    cfg = ol.router_cfg(8, kw["top_k"], kw.get("normalize", False), kw.get("scale", 1.0),
                        kw.get("group_limited", False), kw.get("n_group", 1), kw.get("topk_group", 1))
    o_idx, o_w = ol.oracle_select(KNOWN, cfg)
    assert np.array_equal(g_idx, o_idx)
    assert np.array_equal(g_w.view(np.uint32), o_w.view(np.uint32))
    if variant == "greedy":
        assert list(g_idx) == [1, 3, 5]
    if variant == "grouped":
        assert all(e < 4 for e in g_idx)


def test_router_select_ties_and_random():
    """Exact score ties resolve to the lower index; random logits match the oracle."""
    rng = np.random.default_rng(5)
    T = 256
    logits = rng.standard_normal((T, 64)).astype(np.float32)
    logits[:64, 10] = logits[:64, 3]           # exact ties
    logits[64:128] = np.round(logits[64:128])   # many ties
    logits[128] = 0.0                          # all equal
    announce("router select ties/random T=256")
    with _select_ctx(64, 6) as ctx:
        lg = ctx.to_device(logits)
        idx, w = ctx.empty((T, 6), np.int32), ctx.empty((T, 6))
        ctx.router_select(lg, T, idx, w)
        ctx.synchronize()
        g_idx, g_w = idx.download(), w.download()
    cfg = ol.router_cfg(64, 6)
    for t in range(T):
        o_idx, o_w = ol.oracle_select(logits[t], cfg)
        assert np.array_equal(g_idx[t], o_idx), t
        assert np.array_equal(g_w[t].view(np.uint32), o_w.view(np.uint32)), t
    assert list(g_idx[128]) == [0, 1, 2, 3, 4, 5]
