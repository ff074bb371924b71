"""Dense SwiGLU layer (layer 0 of DeepSeek-V2-Lite, width 10944) on both paths."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dense_ctx():
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    gate, up, down = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
    announce("create dense-layer context")
    ctx = Context(dims.moe_config(num_layers=1))
    ctx.upload_dense(0, gate, up, down)
    ctx.finalize_layer(0)
    yield ctx, (gate, up, down)
    ctx.close()


@pytest.mark.parametrize("T,path", [(1, 1), (3, 1), (256, 2)])
def test_dense_layer(dense_ctx, T, path):
    from litemind_amd import workload as wl

    ctx, (gate, up, down) = dense_ctx
    x = wl.tokens(wl.MASTER_SEED + 400 + T, T, 2048)
    announce(f"dense layer T={T} path={path}")
    dx, dy = ctx.to_device(x), ctx.empty((T, 2048))
    ctx.dense_forward(0, dx, T, dy, path=path)
    ctx.synchronize()
    y = dy.download()
    dx.free()
    dy.free()
    oy = ol.oracle_dense(gate, up, down, x)
    max_abs, mean_rel = layer_error(y, oy)
    print(f"dense T={T} max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    if path == 1:
        assert mean_rel < 1e-5
