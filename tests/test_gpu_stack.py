"""The FFN stack (config: dense layer 0, then MoE layers, chained through
RMSNorm with weights 1 and the residual add) against the oracle's chain.

lm_stack_forward runs h += FFN_l(rms_norm(h)) for every layer, the loop of
LiteMind's runner with attention omitted (src/DeepSeekRunner.cpp:264-290).
A short stack (dense + 3 MoE layers) is checked on every token at T = 1 (the
single-launch decode with the residual fused), T = 3 (that kernel once per
token) and T = 300 (the grouped MFMA paths), and at the benchmark's prefill
size T = 4096 on a sample of tokens: tokens never mix along this path, so the
oracle run on a sample of rows checks those rows of the full-size batch.
"""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu

MOE_LAYERS = 3


@pytest.fixture(scope="module")
def stack_ctx():
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    announce(f"create stack context: dense + {MOE_LAYERS} MoE layers")
    ctx = Context(dims.moe_config(num_layers=1 + MOE_LAYERS))
    layers = []
    gate, up, down = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
    ctx.upload_dense(0, gate, up, down)
    ctx.finalize_layer(0)
    layers.append(("dense", (gate, up, down)))
    for l in range(1, 1 + MOE_LAYERS):
        L = wl.moe_layer(wl.MASTER_SEED, l, dims)
        wl.upload_moe_layer(ctx, l, L)
        layers.append(("moe", L))
    ones = np.ones(dims.hidden, np.float32)
    for l in range(1 + MOE_LAYERS):
        ctx.upload_norm(l, ones)
    yield ctx, layers, dims
    ctx.close()


def _run(ctx, h0, first=0, last=MOE_LAYERS):
    T = h0.shape[0]
    dh = ctx.to_device(h0)
    ctx.stack_forward(first, last, dh, T)
    ctx.synchronize()
    out = dh.download()
    dh.free()
    return out


def test_stack_t1_matches_oracle(stack_ctx):
    """One token through the whole chain (the single-launch decode with the
    residual fused, the dense GEMV): fp32 activations and BF16 weights
    throughout, so the chain stays within 1e-5 of the oracle end to end."""
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    for seed in (701, 702):
        h0 = wl.tokens(wl.MASTER_SEED + seed, 1, dims.hidden)
        announce(f"stack T=1 seed {seed}: dense + {MOE_LAYERS} MoE layers")
        h = _run(ctx, h0)
        oh = ol.oracle_stack(layers, h0, dims.rms_norm_eps)
        max_abs, mean_rel = layer_error(h, oh)
        print(f"stack T=1 max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
        assert max_abs <= MAX_ABS and mean_rel < 1e-5


def test_stack_t300_per_layer(stack_ctx):
    """T = 300 (grouped MFMA experts, fp16 operands).  The layer bar (max-abs
    2e-2, mean-rel 1e-3) holds for each layer given the oracle's input to that
    layer; end to end the fp16 differences of successive layers compound, and
    the chain is held to mean-rel 1e-3 on the hidden state."""
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    T = 300
    h0 = wl.tokens(wl.MASTER_SEED + 1000, T, dims.hidden)
    announce(f"stack T={T}: dense + {MOE_LAYERS} MoE layers, per layer")
    states = ol.oracle_stack(layers, h0, dims.rms_norm_eps, every_layer=True)
    inputs = [h0] + states[:-1]
    for l, (h_in, h_out) in enumerate(zip(inputs, states)):
        got = _run(ctx, h_in, l, l)
        # the layer's output: y = h_out - h_in (both sides from the same input)
        max_abs, mean_rel = layer_error(got - h_in, h_out - h_in)
        print(f"layer {l} ({layers[l][0]}) max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
        assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    end = _run(ctx, h0)
    max_abs, mean_rel = layer_error(end, states[-1])
    print(f"stack T={T} end to end max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert np.all(np.isfinite(end)) and mean_rel <= MEAN_REL


def test_stack_tokens_independent(stack_ctx):
    """A token's result does not depend on the batch it runs in: tokens of a
    T = 300 batch and the same tokens alone agree to the fp16 path's accuracy."""
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    h0 = wl.tokens(wl.MASTER_SEED + 1001, 300, dims.hidden)
    announce("stack batch vs single tokens")
    batch = _run(ctx, h0)
    pick = [0, 137, 299]
    single = np.stack([_run(ctx, h0[t:t + 1])[0] for t in pick])
    _, mean_rel = layer_error(batch[pick], single)
    assert mean_rel < MEAN_REL


def test_stack_t1_speculation_recovery(stack_ctx):
    """Every speculative rank forced wrong in every MoE layer of the chain: the
    repair path recomputes the ranks from the normalised token (the hidden
    state itself is updated in place by the same launch) and the chain still
    matches the oracle."""
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    h0 = wl.tokens(wl.MASTER_SEED + 703, 1, dims.hidden)
    announce("stack T=1 with every speculative rank forced wrong")
    ctx._check(ctx.lib.lm_decode_speculation_test(ctx.handle, 1))
    try:
        h = _run(ctx, h0)
    finally:
        ctx._check(ctx.lib.lm_decode_speculation_test(ctx.handle, 0))
    oh = ol.oracle_stack(layers, h0, dims.rms_norm_eps)
    max_abs, mean_rel = layer_error(h, oh)
    print(f"stack T=1 forced repair max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel < 1e-5


def test_stack_t3_matches_oracle(stack_ctx):
    """T = 3: LM_PATH_AUTO runs each MoE layer as three single-token launches
    with the norm fused and the residual written in place (the dense layer takes
    its MFMA path, fp16 operands), checked end to end against the oracle."""
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    h0 = wl.tokens(wl.MASTER_SEED + 333, 3, dims.hidden)
    announce(f"stack T=3: dense + {MOE_LAYERS} MoE layers")
    states = ol.oracle_stack(layers, h0, dims.rms_norm_eps, every_layer=True)
    inputs = [h0] + states[:-1]
    for l, (h_in, h_out) in enumerate(zip(inputs, states)):
        got = _run(ctx, h_in, l, l)
        max_abs, mean_rel = layer_error(got - h_in, h_out - h_in)
        print(f"T=3 layer {l} ({layers[l][0]}) max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
        assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
        if layers[l][0] == "moe":
            assert mean_rel < 1e-5  # fp32 activations in the single-token kernel
    end = _run(ctx, h0)
    max_abs, mean_rel = layer_error(end, states[-1])
    print(f"stack T=3 end to end max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL


def test_stack_t4096_sampled(stack_ctx):
    """The stack at T = 4096 (the benchmark's prefill size: MFMA paths with
    128-row tiles, 24,576 routed slots per MoE layer).  Per layer, the GPU's
    own input to the layer is kept and 48 of its rows are run through the
    oracle's layer: the layer bar holds on those rows.  Then the whole chain in
    one call, 48 sampled tokens against the oracle's chain (mean-rel 1e-3)."""
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    T = 4096
    h0 = wl.tokens(wl.MASTER_SEED + 4097, T, dims.hidden)
    sample = np.unique(np.concatenate([np.arange(0, T, 89), [T - 1]]))
    announce(f"stack T={T}: dense + {MOE_LAYERS} MoE layers, per layer on {sample.size} sampled rows")
    dh = ctx.to_device(h0)
    h_in = h0
    for l in range(1 + MOE_LAYERS):
        ctx.stack_forward(l, l, dh, T)
        ctx.synchronize()
        h_out = dh.download()
        assert np.all(np.isfinite(h_out))
        ref = ol.oracle_stack(layers[l:l + 1], h_in[sample], dims.rms_norm_eps)
        max_abs, mean_rel = layer_error(h_out[sample] - h_in[sample], ref - h_in[sample])
        print(f"T=4096 layer {l} ({layers[l][0]}) max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
        assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
        h_in = h_out
    dh.free()
    announce(f"stack T={T}: whole chain in one call")
    end = _run(ctx, h0)
    oh = ol.oracle_stack(layers, h0[sample], dims.rms_norm_eps)
    max_abs, mean_rel = layer_error(end[sample], oh)
    print(f"stack T=4096 end to end (sample) max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert np.all(np.isfinite(end)) and mean_rel <= MEAN_REL


@pytest.mark.parametrize("T,path_name", [(8, "gemv"), (64, "auto")])
def test_stack_fused_norm_is_bit_exact(stack_ctx, T, path_name):
    """Between two batched layers lm_stack_forward folds the next layer's
    RMSNorm (and its fp16 copy) into the current layer's combine.  A pass over
    the whole stack must give the same bits as the same layers called one at a
    time (a single-layer call never fuses), with norm weights that are not all
    ones so that a wrong weight vector would show."""
    import litemind_amd as lm
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    path = lm.PATH_GEMV if path_name == "gemv" else lm.PATH_AUTO
    rng = np.random.default_rng(31 + T)
    norms = [rng.uniform(0.5, 1.5, dims.hidden).astype(np.float32) for _ in range(1 + MOE_LAYERS)]
    try:
        for l, w in enumerate(norms):
            ctx.upload_norm(l, w)
        h0 = wl.tokens(wl.MASTER_SEED + 77 + T, T, dims.hidden)
        announce(f"stack T={T} ({path_name}): one pass against layer-by-layer calls")
        dh = ctx.to_device(h0)
        ctx.stack_forward(0, MOE_LAYERS, dh, T, path=path)
        ctx.synchronize()
        fused = dh.download()
        dh.free()
        dh = ctx.to_device(h0)
        for l in range(1 + MOE_LAYERS):
            ctx.stack_forward(l, l, dh, T, path=path)
        ctx.synchronize()
        separate = dh.download()
        dh.free()
        assert np.array_equal(fused.view(np.uint32), separate.view(np.uint32))
        # and the chain still follows the oracle with these norm weights
        ref = ol.oracle_stack(layers, h0[:4], dims.rms_norm_eps, norms=norms)
        max_abs, mean_rel = layer_error(fused[:4], ref)
        print(f"max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
        assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    finally:
        ones = np.ones(dims.hidden, np.float32)
        for l in range(1 + MOE_LAYERS):
            ctx.upload_norm(l, ones)


@pytest.mark.parametrize("T", [48, 300])
def test_stack_graph_replays_match_eager(stack_ctx, T):
    """lm_stack_graph_create records a whole stack pass as a HIP graph; three
    replays, with eager uploads, an eager pass and synchronisations between
    them, each give the eager pass's bits.  While the graph exists a call that
    needs a larger workspace fails instead of moving memory the graph uses; a
    token count whose layers take the single-token kernel is refused."""
    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    announce(f"stack graph T={T}: replays against the eager pass")
    h0 = wl.tokens(wl.MASTER_SEED + 91 + T, T, dims.hidden)
    h1 = wl.tokens(wl.MASTER_SEED + 92 + T, T, dims.hidden)
    eager = _run(ctx, h0)
    eager_other = _run(ctx, h1)
    dh = ctx.to_device(h0)
    graph = ctx.stack_graph_create(0, MOE_LAYERS, dh, T)
    try:
        for rep in range(3):
            dh.upload(h0)
            ctx.synchronize()
            ctx.stack_graph_launch(graph)
            ctx.synchronize()
            got = dh.download()
            assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), f"replay {rep}"
            # eager work on the same workspace between the replays
            assert np.array_equal(_run(ctx, h1).view(np.uint32), eager_other.view(np.uint32))
        big = np.zeros((8192, dims.hidden), np.float32)
        dbig = ctx.to_device(big)
        with pytest.raises(LmError):
            ctx.stack_forward(0, MOE_LAYERS, dbig, 8192)
        dbig.free()
    finally:
        ctx.stack_graph_destroy(graph)
        dh.free()
    d1 = ctx.to_device(h0[:1])
    with pytest.raises(LmError):
        ctx.stack_graph_create(0, MOE_LAYERS, d1, 1)
    d1.free()



def test_stack_graph_lifetime(stack_ctx):
    """A live graph holds its context: lm_context_destroy refuses (and frees
    nothing) until the graph is destroyed.  An upload into a layer of the
    graph's range leaves that layer unfinalized, and a replay is refused until
    lm_finalize_layer runs again; then the replay gives the eager bits."""
    import litemind_amd as lm
    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, layers, dims = stack_ctx
    T = 48
    announce(f"stack graph T={T}: context destroy refused, stale layer refused")
    h0 = wl.tokens(wl.MASTER_SEED + 95, T, dims.hidden)
    eager = _run(ctx, h0)
    dh = ctx.to_device(h0)
    graph = ctx.stack_graph_create(0, MOE_LAYERS, dh, T)
    try:
        status = ctx.lib.lm_context_destroy(ctx.handle)
        assert status == -1 and b"still alive" in ctx.lib.lm_last_error()
        moe = layers[1][1]
        ctx.upload_expert(1, 0, moe.gate[0], moe.up[0], moe.down[0])  # same weights, layer left unfinalized
        with pytest.raises(LmError) as err:
            ctx.stack_graph_launch(graph)
        assert err.value.status == -4
        ctx.finalize_layer(1)
        dh.upload(h0)
        ctx.synchronize()
        ctx.stack_graph_launch(graph)
        ctx.synchronize()
        got = dh.download()
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32))
    finally:
        ctx.stack_graph_destroy(graph)
        dh.free()
    assert lm.LM_OK == 0


def test_stack_t1_real_misprediction(stack_ctx):
    """With the norm fused, the single-token kernel speculates from the
    unnormalised products, each thread adding its elements and the wave's
    butterfly adding the threads.  A layer whose expert 6 has products 1e8, 1
    and -1e8 in rows 0, 1 and 2 (threads 0, 1 and 2 of wave 0) keeps the 1
    there (the butterfly adds threads 0 and 2 first) and loses it in LiteMind's
    left-to-right chain over the normalised token (logit 0).  Expert 5 sits at
    0.5 and experts 0-4 lead, so rank 5 is speculated as expert 6 and is expert
    5 exactly; the pass still matches the oracle."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    _, layers, dims = stack_ctx
    base = layers[1][1]
    E, H = dims.experts, dims.hidden
    gate = np.zeros((E, H), np.float32)
    gate[:, 12] = -5.0
    for e, v in enumerate((10.0, 9.0, 8.0, 7.0, 6.0)):
        gate[e, 12] = v
    gate[5, 12] = 0.5
    gate[6, 12] = 0.0
    gate[6, 0], gate[6, 1], gate[6, 2] = 1e8, 1.0, -1e8
    layer = wl.MoeLayer(base.dims, gate, base.gate, base.up, base.down, base.shared_gate, base.shared_up,
                        base.shared_down)
    h0 = np.zeros((1, H), np.float32)
    h0[0, [0, 1, 2, 12]] = 1.0
    # the butterfly's order (threads 0 + 2, then + 1) keeps the 1; the exact
    # logit over the normalised token loses it, and rank 5 is expert 5
    f = np.float32
    assert (f(1e8) + f(-1e8)) + f(1.0) == f(1.0) > f(0.5)
    xn = h0.copy()
    ol.oracle().orc_rms_norm(ol.p(xn[0]), ol.p(np.ones(H, np.float32)), H, dims.rms_norm_eps)
    _, oidx, _, olg = ol.oracle_moe_layer(layer, xn)
    assert olg[0, 6] == 0.0 and oidx[0, 5] == 5
    announce("stack T=1 with a speculation the exact selection overturns")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        wl.upload_moe_layer(ctx, 0, layer)
        ctx.upload_norm(0, np.ones(H, np.float32))
        dh = ctx.to_device(h0)
        ctx.stack_forward(0, 0, dh, 1)
        ctx.synchronize()
        h = dh.download()
        dh.free()
    oh = ol.oracle_stack([("moe", layer)], h0, dims.rms_norm_eps)
    max_abs, mean_rel = layer_error(h, oh)
    print(f"stack T=1 misprediction max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel < 1e-5
