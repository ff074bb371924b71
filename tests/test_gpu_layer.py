"""Full MoE block on the GPU against the oracle: routing bit-exact, outputs within
max-abs 2e-2 and mean-rel (sum|d| / sum|ref|) 1e-3."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu


def _gpu_layer(ctx, layer_id, x, path, bias=None, with_logits=False):
    T = x.shape[0]
    E, K, H = ctx.config.n_routed_experts, ctx.config.num_experts_per_tok, ctx.config.hidden_size
    dx = ctx.to_device(x)
    db = ctx.to_device(bias) if bias is not None else None
    y, idx, w = ctx.empty((T, H)), ctx.empty((T, K), np.int32), ctx.empty((T, K))
    lg = ctx.empty((T, E)) if with_logits else None
    ctx.moe_forward(layer_id, dx, T, y, bias=db, idx=idx, w=w, logits=lg, path=path)
    ctx.synchronize()
    out = (y.download(), idx.download(), w.download()) + ((lg.download(),) if with_logits else ())
    for b in (dx, y, idx, w) + ((db,) if db is not None else ()) + ((lg,) if with_logits else ()):
        b.free()
    return out


@pytest.mark.parametrize("T", [1, 4, 32])
def test_layer_gemv_v2lite(v2_ctx, T):
    from litemind_amd import PATH_GEMV
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 100 + T, T, 2048)
    announce(f"layer GEMV path T={T}")
    y, idx, w = _gpu_layer(ctx, 0, x, PATH_GEMV)
    oy, oidx, ow, _ = ol.oracle_moe_layer(layers[0], x)
    assert np.array_equal(idx, oidx)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
    max_abs, mean_rel = layer_error(y, oy)
    print(f"T={T} max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    # fp32 activations throughout: far inside the tolerance
    assert mean_rel < 1e-5


def test_layer_gemv_tiny(tiny_ctx):
    from litemind_amd import PATH_GEMV
    from litemind_amd import workload as wl

    ctx, layer = tiny_ctx
    x = wl.tokens(17, 9, layer.dims.hidden)
    announce("layer GEMV tiny model T=9")
    y, idx, w = _gpu_layer(ctx, 0, x, PATH_GEMV)
    oy, oidx, ow, _ = ol.oracle_moe_layer(layer, x)
    assert np.array_equal(idx, oidx)
    max_abs, mean_rel = layer_error(y, oy)
    assert max_abs <= 1e-5 and mean_rel <= 1e-5


@pytest.mark.parametrize("case", ["t48_forced", "t512_uniform", "t2048_skewed"])
def test_layer_mfma_v2lite(v2_ctx, case):
    """fp16-operand MFMA path: routing still bit-exact, outputs within tolerance."""
    from litemind_amd import PATH_AUTO, PATH_MFMA
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    T = {"t48_forced": 48, "t512_uniform": 512, "t2048_skewed": 2048}[case]
    layer_id = 1 if case == "t512_uniform" else 0
    bias = wl.skew_bias() if case == "t2048_skewed" else None
    path = PATH_MFMA if case == "t48_forced" else PATH_AUTO
    x = wl.tokens(wl.MASTER_SEED + 200 + T, T, 2048)
    announce(f"layer MFMA {case} T={T}")
    y, idx, w = _gpu_layer(ctx, layer_id, x, path, bias=bias)
    oy, oidx, ow, _ = ol.oracle_moe_layer(layers[layer_id], x, bias=bias)
    assert np.array_equal(idx, oidx)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
    max_abs, mean_rel = layer_error(y, oy)
    print(f"{case} max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL


def test_layer_mfma_tiny(tiny_ctx):
    from litemind_amd import PATH_MFMA
    from litemind_amd import workload as wl

    ctx, layer = tiny_ctx
    x = wl.tokens(23, 300, layer.dims.hidden)
    announce("layer MFMA tiny model T=300")
    y, idx, w = _gpu_layer(ctx, 0, x, PATH_MFMA)
    oy, oidx, ow, _ = ol.oracle_moe_layer(layer, x)
    assert np.array_equal(idx, oidx)
    max_abs, mean_rel = layer_error(y, oy)
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL


def test_gemv_and_mfma_agree(v2_ctx):
    from litemind_amd import PATH_GEMV, PATH_MFMA
    from litemind_amd import workload as wl

    ctx, _ = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 300, 64, 2048)
    announce("layer GEMV vs MFMA T=64")
    yg, ig, wg = _gpu_layer(ctx, 0, x, PATH_GEMV)
    ym, im, wm = _gpu_layer(ctx, 0, x, PATH_MFMA)
    assert np.array_equal(ig, im)
    max_abs, mean_rel = layer_error(ym, yg)
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL


@pytest.mark.parametrize("T", [2, 3])
def test_layer_auto_few_tokens(v2_ctx, T):
    """LM_PATH_AUTO at T = 2 and 3 runs the single-token kernel once per token
    (offset x, y, index, weight and logit pointers): logits, experts and weights
    bit-exact, outputs at the fp32 path's accuracy."""
    from litemind_amd import PATH_AUTO
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 600 + T, T, 2048)
    announce(f"layer AUTO T={T} (single-token kernel per token)")
    y, idx, w, lg = _gpu_layer(ctx, 0, x, PATH_AUTO, with_logits=True)
    oy, oidx, ow, olg = ol.oracle_moe_layer(layers[0], x)
    assert np.array_equal(lg.view(np.uint32), olg.view(np.uint32)), "logits differ"
    assert np.array_equal(idx, oidx)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
    max_abs, mean_rel = layer_error(y, oy)
    print(f"T={T} max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel < 1e-5


def test_layer_auto_t32(v2_ctx):
    """The batched-decode workload's own path: LM_PATH_AUTO at T = 32 takes the
    MFMA kernels with 64-row tiles (T k <= 64 E).  Routing bit-exact, outputs
    within max-abs 2e-2 and mean-rel 1e-3."""
    from litemind_amd import PATH_AUTO
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 7, 32, 2048)  # the tokens the T = 32 benchmark uses
    announce("layer AUTO T=32 (64-row MFMA tiles)")
    y, idx, w, lg = _gpu_layer(ctx, 0, x, PATH_AUTO, with_logits=True)
    oy, oidx, ow, olg = ol.oracle_moe_layer(layers[0], x)
    assert np.array_equal(lg.view(np.uint32), olg.view(np.uint32)), "logits differ"
    assert np.array_equal(idx, oidx)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
    max_abs, mean_rel = layer_error(y, oy)
    print(f"T=32 AUTO max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL


def _oracle_route_all(layer, x):
    """Logits, experts and weights of every token from the oracle's router
    (matvec_f32 + MoeRouter::select), without the experts."""
    d = layer.dims
    T = x.shape[0]
    logits = np.zeros((T, d.experts), np.float32)
    for t in range(T):
        ol.oracle().orc_matvec_f32(ol.p(layer.router), ol.p(np.ascontiguousarray(x[t])), ol.p(logits[t]),
                                   d.experts, d.hidden)
    cfg = ol.router_cfg(d.experts, d.top_k, d.norm_topk_prob, d.routed_scaling_factor)
    idx = np.zeros((T, d.top_k), np.int32)
    w = np.zeros((T, d.top_k), np.float32)
    for t in range(T):
        idx[t], w[t] = ol.oracle_select(logits[t], cfg)
    return logits, idx, w


@pytest.mark.parametrize("T", [4096, 4100])
def test_layer_auto_large_sampled(v2_ctx, T):
    """One MoE layer at the stack's prefill size, T = 4096 (128-row MFMA tiles
    over 24,576 routed slots, the largest workspace; the router at two tokens
    per wave), and at T = 4100 (four tokens per wave, a ragged last workgroup;
    the router also writes the fp16 token copy the MFMA path reads): every
    token's logits, experts and weights bit-exact against the oracle's router;
    the outputs of ~43 tokens spread over the batch (tokens never mix on this
    path, so a sample is a valid check) within the layer tolerance; every
    output finite."""
    from litemind_amd import PATH_AUTO
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + T, T, 2048)
    announce(f"layer AUTO T={T}")
    y, idx, w, lg = _gpu_layer(ctx, 0, x, PATH_AUTO, with_logits=True)
    olg, oidx, ow = _oracle_route_all(layers[0], x)
    assert np.array_equal(lg.view(np.uint32), olg.view(np.uint32)), "logits differ"
    assert np.array_equal(idx, oidx)
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32))
    assert np.all(np.isfinite(y))
    sample = np.unique(np.concatenate([np.arange(0, T, 97), [T - 1]]))
    oy, _, _, _ = ol.oracle_moe_layer(layers[0], x[sample])
    max_abs, mean_rel = layer_error(y[sample], oy)
    print(f"T={T} sample of {sample.size}: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
