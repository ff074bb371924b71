"""Full MoE block on the GPU against the oracle: routing bit-exact, outputs within
max-abs 2e-2 and mean-rel (sum|d| / sum|ref|) 1e-3."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu


def _gpu_layer(ctx, layer_id, x, path, bias=None):
    from litemind_amd import workload as wl  # noqa: F401

    T = x.shape[0]
    E, K, H = ctx.config.n_routed_experts, ctx.config.num_experts_per_tok, ctx.config.hidden_size
    dx = ctx.to_device(x)
    db = ctx.to_device(bias) if bias is not None else None
    y, idx, w = ctx.empty((T, H)), ctx.empty((T, K), np.int32), ctx.empty((T, K))
    ctx.moe_forward(layer_id, dx, T, y, bias=db, idx=idx, w=w, path=path)
    ctx.synchronize()
    out = y.download(), idx.download(), w.download()
    for b in (dx, y, idx, w) + ((db,) if db is not None else ()):
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
