"""lm_moe_forward_noalloc: the MoE block with every scratch word in the fixed
per-GPU device array (no device allocation in the call), checked through the
C ABI against lm_moe_forward on the same inputs.  Both run the single-token
kernel per token, so logits, experts, weights and outputs must be identical
bit for bit; they are also held to the oracle's routing bit for bit and its
outputs at the fp32 path's accuracy.  Two calls in a row, the second with
fewer tokens, and a third with no selection outputs (the array's own words
hold them)."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, announce, layer_error

pytestmark = pytest.mark.gpu


def _run(ctx, fn, x, **kw):
    T, H = x.shape
    E, K = ctx.config.n_routed_experts, ctx.config.num_experts_per_tok
    dx, y = ctx.to_device(x), ctx.empty((T, H))
    idx, w, lg = ctx.empty((T, K), np.int32), ctx.empty((T, K)), ctx.empty((T, E))
    fn(0, dx, T, y, idx=idx, w=w, logits=lg, **kw)
    ctx.synchronize()
    out = y.download(), idx.download(), w.download(), lg.download()
    for b in (dx, y, idx, w, lg):
        b.free()
    return out


@pytest.mark.parametrize("T", [5, 2])
def test_noalloc_matches_moe_forward(v2_ctx, T):
    from litemind_amd import PATH_AUTO
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 7700 + T, T, 2048)
    announce(f"lm_moe_forward_noalloc T={T}")
    got = _run(ctx, ctx.moe_forward_noalloc, x)
    announce(f"lm_moe_forward (single-token kernel per token) T={T}")
    ref = []
    for t in range(T):  # the same kernel through the existing entry point, one token per call
        ref.append(_run(ctx, ctx.moe_forward, x[t:t + 1], path=PATH_AUTO))
    ref = tuple(np.concatenate([r[i] for r in ref]) for i in range(4))
    for a, b, name in zip(got, ref, ("y", "idx", "weights", "logits")):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name} differ from lm_moe_forward"
    oy, oidx, ow, olg = ol.oracle_moe_layer(layers[0], x)
    assert np.array_equal(got[3].view(np.uint32), olg.view(np.uint32))
    assert np.array_equal(got[1], oidx)
    assert np.array_equal(got[2].view(np.uint32), ow.view(np.uint32))
    max_abs, mean_rel = layer_error(got[0], oy)
    print(f"noalloc T={T} max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel < 1e-5


def test_noalloc_without_selection_outputs(v2_ctx):
    """index / weight / logits omitted: the array's own words hold the selection."""
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 7711, 3, 2048)
    announce("lm_moe_forward_noalloc T=3 without selection outputs")
    dx, y = ctx.to_device(x), ctx.empty((3, 2048))
    ctx.moe_forward_noalloc(0, dx, 3, y)
    ctx.synchronize()
    got = y.download()
    for b in (dx, y):
        b.free()
    oy, _, _, _ = ol.oracle_moe_layer(layers[0], x)
    max_abs, mean_rel = layer_error(got, oy)
    assert max_abs <= MAX_ABS and mean_rel < 1e-5


def test_noalloc_rejects_shapes_without_the_kernel():
    """A layer shape the single-token kernel does not cover returns LM_EINVAL with a message."""
    from litemind_amd import Context, LmError
    from litemind_amd import workload as wl

    dims = wl.Dims(hidden=1024, inter=128, experts=8, top_k=2, n_shared=1)
    announce("lm_moe_forward_noalloc on a shape without the single-token kernel")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        layer = wl.moe_layer(5, 0, dims)
        wl.upload_moe_layer(ctx, 0, layer)
        dx, y = ctx.to_device(wl.tokens(5, 1, 1024)), ctx.empty((1, 1024))
        with pytest.raises(LmError, match="no single-token kernel"):
            ctx.moe_forward_noalloc(0, dx, 1, y)


def test_noalloc_two_contexts_alternate(v2_ctx, v2_layer):
    """Two contexts (two streams) on one GPU share the fixed array.  Calls
    issued alternately from both, with no synchronisation between them, run one
    after another on the GPU (each waits for the previous call's event), so
    every call's outputs equal lm_moe_forward's for its tokens bit for bit."""
    from litemind_amd import PATH_AUTO, Context
    from litemind_amd import workload as wl

    ctx_a, _ = v2_ctx
    announce("second context on the same GPU for alternating noalloc calls")
    with Context(wl.V2_LITE.moe_config(num_layers=1)) as ctx_b:
        wl.upload_moe_layer(ctx_b, 0, v2_layer)
        E, K, H = 64, ctx_a.config.num_experts_per_tok, 2048
        calls = []
        for i in range(6):
            ctx = ctx_a if i % 2 == 0 else ctx_b
            T = 2 if i % 3 else 1
            x = wl.tokens(wl.MASTER_SEED + 7800 + i, T, H)
            bufs = (ctx.to_device(x), ctx.empty((T, H)), ctx.empty((T, K), np.int32), ctx.empty((T, K)),
                    ctx.empty((T, E)))
            calls.append((ctx, x, bufs))
        announce("alternating lm_moe_forward_noalloc calls on two contexts, no synchronisation between them")
        for ctx, x, (dx, y, idx, w, lg) in calls:
            ctx.moe_forward_noalloc(0, dx, x.shape[0], y, idx=idx, w=w, logits=lg)
        ctx_a.synchronize()
        ctx_b.synchronize()
        for n, (ctx, x, (dx, y, idx, w, lg)) in enumerate(calls):
            got = (y.download(), idx.download(), w.download(), lg.download())
            ref = [_run(ctx_a, ctx_a.moe_forward, x[t:t + 1], path=PATH_AUTO) for t in range(x.shape[0])]
            ref = tuple(np.concatenate([r[i] for r in ref]) for i in range(4))
            for a, b, name in zip(got, ref, ("y", "idx", "weights", "logits")):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"call {n}: {name} differ"
            for b in (dx, y, idx, w, lg):
                b.free()


def test_noalloc_refuses_graph_capture(v2_ctx):
    """While the context's stream is being captured the call returns LM_EINVAL
    (its hand-off tags would repeat on replay); nothing is launched, so the
    capture ends with an empty graph."""
    import ctypes as C

    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, _ = v2_ctx
    hip = C.CDLL("libamdhip64.so.7")
    hip.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
    hip.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    hip.hipGraphDestroy.argtypes = [C.c_void_p]
    dx, y = ctx.to_device(wl.tokens(wl.MASTER_SEED + 7900, 1, 2048)), ctx.empty((1, 2048))
    ctx.synchronize()
    stream = C.c_void_p(ctx.stream())
    announce("lm_moe_forward_noalloc while the context stream is captured (refused before any launch)")
    assert hip.hipStreamBeginCapture(stream, 2) == 0  # hipStreamCaptureModeRelaxed
    try:
        with pytest.raises(LmError, match="being captured"):
            ctx.moe_forward_noalloc(0, dx, 1, y)
    finally:
        graph = C.c_void_p()
        assert hip.hipStreamEndCapture(stream, C.byref(graph)) == 0
        if graph.value:
            hip.hipGraphDestroy(graph)
    ctx.moe_forward_noalloc(0, dx, 1, y)  # and works again afterwards
    ctx.synchronize()
    for b in (dx, y):
        b.free()
