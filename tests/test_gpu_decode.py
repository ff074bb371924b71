"""The single-token MoE block (three decode launches) against the oracle.

Every token is a separate lm_moe_forward call with T = 1, the decode case of
LiteMind's runner (src/DeepSeekRunner.cpp:273-290).  Logits, selected experts
and weights must be bit-exact; outputs within the layer tolerance (fp32
activations, so far inside it).
"""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu


def _one_token_calls(ctx, layer_id, x, bias=None, residual=False):
    T, H = x.shape
    E, K = ctx.config.n_routed_experts, ctx.config.num_experts_per_tok
    dx = ctx.to_device(x)
    db = ctx.to_device(bias) if bias is not None else None
    y, idx, w, lg = ctx.empty((T, H)), ctx.empty((T, K), np.int32), ctx.empty((T, K)), ctx.empty((T, E))
    for t in range(T):
        ctx.moe_forward(layer_id, dx.ptr + t * H * 4, 1, y.ptr + t * H * 4, bias=db, idx=idx.ptr + t * K * 4,
                        w=w.ptr + t * K * 4, logits=lg.ptr + t * E * 4)
    ctx.synchronize()
    out = y.download(), idx.download(), w.download(), lg.download()
    for b in (dx, y, idx, w, lg) + ((db,) if db is not None else ()):
        b.free()
    return out


def _check(out, layer, x, bias=None, tol=1e-5):
    y, idx, w, lg = out
    oy, oidx, ow, olg = ol.oracle_moe_layer(layer, x, bias=bias)
    assert np.array_equal(lg.view(np.uint32), olg.view(np.uint32)), "logits differ"
    assert np.array_equal(idx, oidx), "selected experts differ"
    assert np.array_equal(w.view(np.uint32), ow.view(np.uint32)), "weights differ"
    max_abs, mean_rel = layer_error(y, oy)
    print(f"max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    assert mean_rel < tol


@pytest.mark.parametrize("case", ["layer0", "uniform", "skewed"])
def test_decode_v2lite(v2_ctx, case):
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    layer_id = 1 if case == "uniform" else 0
    bias = wl.skew_bias() if case == "skewed" else None
    x = wl.tokens(wl.MASTER_SEED + 500 + layer_id + (7 if bias is not None else 0), 24, 2048)
    announce(f"decode V2-Lite {case}: 24 single-token calls")
    _check(_one_token_calls(ctx, layer_id, x, bias), layers[layer_id], x, bias)


def test_decode_tiny(tiny_ctx):
    from litemind_amd import workload as wl

    ctx, layer = tiny_ctx
    x = wl.tokens(23, 16, layer.dims.hidden)
    announce("decode tiny model: 16 single-token calls")
    _check(_one_token_calls(ctx, 0, x), layer, x)


def test_decode_matches_batched_gemv(v2_ctx):
    """The same tokens one at a time (decode launches) and as one T=8 batch
    (general GEMV path) route identically and agree closely."""
    from litemind_amd import PATH_GEMV
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 909, 8, 2048)
    announce("decode vs batched GEMV, 8 tokens")
    y1, idx1, w1, _ = _one_token_calls(ctx, 0, x)
    dx, y8 = ctx.to_device(x), ctx.empty((8, 2048))
    idx8, w8 = ctx.empty((8, 6), np.int32), ctx.empty((8, 6))
    ctx.moe_forward(0, dx, 8, y8, idx=idx8, w=w8, path=PATH_GEMV)
    ctx.synchronize()
    assert np.array_equal(idx1, idx8.download())
    assert np.array_equal(w1.view(np.uint32), w8.download().view(np.uint32))
    _, mean_rel = layer_error(y1, y8.download())
    assert mean_rel < 1e-5
    for b in (dx, y8, idx8, w8):
        b.free()


def test_decode_speculation_recovery(v2_ctx):
    """Every speculative rank forced wrong: the fix-up path recomputes all ranks
    and the outputs are the exact ones."""
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 4242, 8, 2048)
    announce("decode with every speculative rank forced wrong, 8 tokens")
    ctx._check(ctx.lib.lm_decode_speculation_test(ctx.handle, 1))
    try:
        out = _one_token_calls(ctx, 0, x)
    finally:
        ctx._check(ctx.lib.lm_decode_speculation_test(ctx.handle, 0))
    _check(out, layers[0], x)


def test_decode_wait_timeout_reports_kernel_error(v2_ctx):
    """Every hand-off wait of the single-token kernel made to give up after its
    second poll (a bound the host sets, so every wave still runs to its end):
    the next lm_synchronize returns LM_EKERNEL, the error is reported once, and
    the context then computes exact results again."""
    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    x = wl.tokens(wl.MASTER_SEED + 4343, 1, 2048)
    dx, y = ctx.to_device(x), ctx.empty((1, 2048))
    idx, w = ctx.empty((1, 6), np.int32), ctx.empty((1, 6))
    announce("decode with every hand-off wait giving up at once")
    reported = 0
    ctx._check(ctx.lib.lm_decode_wait_test(ctx.handle, 1))
    try:
        for _ in range(4):
            ctx.moe_forward(0, dx, 1, y, idx=idx, w=w)
            try:
                ctx.synchronize()
            except LmError as error:
                assert "status -5" in str(error) and "timed out" in str(error)
                reported += 1
    finally:
        ctx._check(ctx.lib.lm_decode_wait_test(ctx.handle, 0))
    assert reported >= 1
    ctx.synchronize()  # nothing left to report
    announce("decode after the forced timeouts")
    out = _one_token_calls(ctx, 0, x)
    _check(out, layers[0], x)
    for b in (dx, y, idx, w):
        b.free()


def test_decode_real_misprediction(v2_layer):
    """The single-token kernel's speculation wrong without the testing switch:
    a gate whose expert 6 has products 1e8, 1 and -1e8 in rows 0, 4 and 8.
    LiteMind's left-to-right chain loses the 1 (its logit is 0); the
    approximate logit, each lane adding its row quads and the wave's butterfly
    adding the lanes, keeps it (1).  Expert 5 sits at 0.5 and experts 0-4 lead,
    so rank 5 is speculated as expert 6 and is expert 5 exactly: the down
    workgroups recompute it, and the outputs match the oracle."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    E, H = 64, 2048
    gate = np.zeros((E, H), np.float32)
    gate[:, 12] = -5.0
    for e, v in enumerate((10.0, 9.0, 8.0, 7.0, 6.0)):
        gate[e, 12] = v
    gate[5, 12] = 0.5
    gate[6, 12] = 0.0
    gate[6, 0], gate[6, 4], gate[6, 8] = 1e8, 1.0, -1e8
    layer = wl.MoeLayer(v2_layer.dims, gate, v2_layer.gate, v2_layer.up, v2_layer.down, v2_layer.shared_gate,
                        v2_layer.shared_up, v2_layer.shared_down)
    x = np.zeros((1, H), np.float32)
    x[0, [0, 4, 8, 12]] = 1.0
    announce("decode V2-Lite with a speculation the exact selection overturns")
    with Context(wl.V2_LITE.moe_config(num_layers=1)) as ctx:
        wl.upload_moe_layer(ctx, 0, layer)
        out = _one_token_calls(ctx, 0, x)
    oy, oidx, ow, olg = ol.oracle_moe_layer(layer, x)
    assert olg[0, 6] == 0.0 and oidx[0, 5] == 5
    _check(out, layer, x)
