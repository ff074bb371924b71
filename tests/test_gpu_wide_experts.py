"""Layers of more than 64 routed experts on the GPU (LiteMind's MoeRouter takes
any expert count; DeepSeek-V2 routes over 160 experts in 8 groups with
group-limited greedy selection): the general router and selection (a lane owns
experts lane + 64 j), the permutation and both expert paths, against the
oracle.  Logits, experts, weights and the permutation bit-exact; layer outputs
within max-abs 2e-2 and mean-rel 1e-3 (1e-5 on the fp32 GEMV path)."""
import os

import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
WIDE_VARIANTS = {"e160": (160, 6, 0, 1.0, 1, 8, 3), "e256": (256, 8, 1, 1.0, 1, 8, 4),
                 "e512": (512, 8, 0, 2.5, 1, 16, 4), "e160_greedy": (160, 6, 0, 1.0, 0, 1, 1)}


def _dims(E=160, k=6, grouped=True, n_group=8, topk_group=3, hidden=1024, inter=256, norm=False, scale=1.0):
    from litemind_amd import workload as wl

    return wl.Dims(hidden=hidden, inter=inter, experts=E, top_k=k, n_shared=2, dense_inter=0,
                   norm_topk_prob=norm, routed_scaling_factor=scale, group_limited=grouped, n_group=n_group,
                   topk_group=topk_group)


@pytest.fixture(scope="module")
def wide_ctx():
    """DeepSeek-V2's routing (160 experts, 8 groups, 3 kept, top-6) on a reduced
    hidden / intermediate size (1024 / 256) so the oracle stays fast."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = _dims()
    announce("create 160-expert context (8 groups, 3 kept)")
    ctx = Context(dims.moe_config(num_layers=1))
    layer = wl.moe_layer(wl.MASTER_SEED + 160, 0, dims)
    wl.upload_moe_layer(ctx, 0, layer)
    yield ctx, layer
    ctx.close()


def _oracle_route(layer, x):
    d = layer.dims
    T = x.shape[0]
    logits = np.zeros((T, d.experts), np.float32)
    for t in range(T):
        ol.oracle().orc_matvec_f32(ol.p(layer.router), ol.p(np.ascontiguousarray(x[t])), ol.p(logits[t]),
                                   d.experts, d.hidden)
    cfg = ol.router_cfg(d.experts, d.top_k, d.norm_topk_prob, d.routed_scaling_factor, d.group_limited, d.n_group,
                        d.topk_group)
    idx = np.zeros((T, d.top_k), np.int32)
    w = np.zeros((T, d.top_k), np.float32)
    for t in range(T):
        idx[t], w[t] = ol.oracle_select(logits[t], cfg)
    return logits, idx, w


@pytest.mark.parametrize("name", list(WIDE_VARIANTS))
def test_wide_select_golden(name):
    """lm_router_select (MoeRouter::select alone) on the compiled router's
    golden logits, ties included: experts and weights bit for bit."""
    from litemind_amd import Context

    E, k, norm, scale, grouped, ng, tg = WIDE_VARIANTS[name]
    g = np.load(os.path.join(GOLDEN, "router_wide.npz"))
    logits = g[f"{name}_logits"]
    T = logits.shape[0]
    dims = _dims(E, k, bool(grouped), ng, tg, hidden=16, inter=16, norm=bool(norm), scale=scale)
    announce(f"select only, {name}: {T} tokens")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        dl = ctx.to_device(logits)
        idx, w = ctx.empty((T, k), np.int32), ctx.empty((T, k))
        ctx.router_select(dl, T, idx, w)
        ctx.synchronize()
        gi, gw = idx.download(), w.download()
    assert np.array_equal(gi, g[f"{name}_index"])
    assert np.array_equal(gw.view(np.uint32), g[f"{name}_weight"].view(np.uint32))


@pytest.mark.parametrize("T", [1, 7, 300, 1500])
def test_wide_router_bit_exact(wide_ctx, T):
    """Logits (each LiteMind's sequential fp32 chain), experts and weights at
    one and a few tokens (logits over E / 8 workgroups per token) and many
    (the ring router: 8 deep at 300 tokens, 4 deep at 1500)."""
    from litemind_amd import workload as wl

    ctx, layer = wide_ctx
    x = wl.tokens(wl.MASTER_SEED + 1600 + T, T, layer.dims.hidden)
    announce(f"160-expert router T={T}")
    dx = ctx.to_device(x)
    lg, idx, w = ctx.empty((T, 160)), ctx.empty((T, 6), np.int32), ctx.empty((T, 6))
    ctx.router(0, dx, T, idx, w, logits=lg)
    ctx.synchronize()
    glg, gidx, gw = lg.download(), idx.download(), w.download()
    olg, oidx, ow = _oracle_route(layer, x)
    assert np.array_equal(glg.view(np.uint32), olg.view(np.uint32)), "logits differ"
    assert np.array_equal(gidx, oidx), "selected experts differ"
    assert np.array_equal(gw.view(np.uint32), ow.view(np.uint32)), "weights differ"
    per = 160 // 8
    assert all(len({e // per for e in row}) <= 3 for row in gidx)  # at most topk_group groups
    for b in (dx, lg, idx, w):
        b.free()


# experts, top-k, group-limited, groups, kept, hidden, tokens, bias.  Above 256
# tokens (or with E % 8 != 0) the batched ring router: every lane-ownership
# width (two to eight experts per lane), the 8-deep ring (up to 256
# workgroups; above that with one token per wave, workgroups of 8 waves) and
# the 4-deep one, one, two and four tokens per wave, expert
# counts off multiples of 4 and 8, and a hidden size the ring's chunks do not
# divide (the per-token kernel).  Up to 256 tokens with E % 8 == 0: logits
# over E / 8 workgroups per token, then the selection.
RING_CASES = {
    "e100_epl2_deep": (100, 6, False, 1, 1, 512, 700, False),
    "e256_epl4_tpw2": (256, 8, True, 8, 4, 1024, 2100, True),
    "e512_epl8_deep": (512, 8, True, 16, 4, 512, 333, False),
    "e130_epl3_deep": (130, 4, True, 2, 1, 768, 90, True),
    "e130_one_token": (130, 4, True, 2, 1, 768, 1, True),
    "e160_epl3_tpw1": (160, 6, True, 8, 3, 512, 1300, False),
    "e160_epl3_tpw4": (160, 6, True, 8, 3, 256, 4200, True),
    "e100_h1040_fallback": (100, 5, False, 1, 1, 1040, 300, False),
    "e300_epl5_deep": (300, 6, True, 4, 2, 256, 150, False),
    "e384_epl6_tpw2": (384, 8, True, 8, 4, 320, 2060, True),
    "e448_split": (448, 8, False, 1, 1, 256, 77, False),
    "e160_split_256": (160, 6, True, 8, 3, 512, 256, True),
    "e100_epl2_wide8": (100, 6, False, 1, 1, 512, 2048, True),
    "e512_epl8_wide8": (512, 8, True, 16, 4, 256, 1100, False),
}


@pytest.mark.parametrize("name", sorted(RING_CASES))
def test_wide_router_ring_shapes(name):
    """The batched router above 16 tokens over more than 64 experts: logits,
    experts and weights bit for bit against the oracle's chains and selection
    (the logit bias added after the chain, as MoeRouter::route does)."""
    from litemind_amd import Context

    E, k, grouped, ng, tg, H, T, with_bias = RING_CASES[name]
    dims = _dims(E, k, grouped, ng, tg, hidden=H, inter=16)
    rng = np.random.default_rng(E * 7 + H)
    gate = (rng.standard_normal((E, H)) * 0.05).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.01).astype(np.float32) if with_bias else None
    announce(f"ring router {name}: E={E} H={H} T={T}")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        ctx.upload_router(0, gate)
        dx = ctx.to_device(x)
        db = ctx.to_device(bias) if with_bias else None
        lg, idx, w = ctx.empty((T, E)), ctx.empty((T, k), np.int32), ctx.empty((T, k))
        ctx.router(0, dx, T, idx, w, bias=db, logits=lg)
        ctx.synchronize()
        glg, gidx, gw = lg.download(), idx.download(), w.download()
    olg = np.zeros((T, E), np.float32)
    for t in range(T):
        ol.oracle().orc_matvec_f32(ol.p(gate), ol.p(np.ascontiguousarray(x[t])), ol.p(olg[t]), E, H)
    if with_bias:
        olg = olg + bias[None, :]
    cfg = ol.router_cfg(E, k, False, 1.0, grouped, ng, tg)
    assert np.array_equal(glg.view(np.uint32), olg.view(np.uint32)), "logits differ"
    for t in range(T):
        oi, ow = ol.oracle_select(olg[t], cfg)
        assert np.array_equal(gidx[t], oi), f"token {t}: experts differ"
        assert np.array_equal(gw[t].view(np.uint32), ow.view(np.uint32)), f"token {t}: weights differ"


def test_wide_permute(wide_ctx):
    """The canonical permutation of 1500 tokens' selections over 160 experts
    (the counts, offsets, the list of experts with tokens, perm and its inverse)."""
    from litemind_amd import workload as wl

    ctx, layer = wide_ctx
    T = 1500
    _, oidx, _ = _oracle_route(layer, wl.tokens(wl.MASTER_SEED + 1601, T, layer.dims.hidden))
    announce("160-expert permutation T=1500")
    di = ctx.to_device(oidx)
    counts, offsets = ctx.empty((160,), np.int32), ctx.empty((161,), np.int32)
    perm, slot_of = ctx.empty((T * 6,), np.int32), ctx.empty((T * 6,), np.int32)
    ctx.permute(di, T, counts, offsets, perm, slot_of)
    ctx.synchronize()
    oc, oo, op, os_ = ol.oracle_permute(oidx, 160)
    assert np.array_equal(counts.download(), oc)
    assert np.array_equal(offsets.download(), oo)
    assert np.array_equal(perm.download(), op)
    assert np.array_equal(slot_of.download(), os_)


@pytest.mark.parametrize("T,path", [(1, "auto"), (5, "auto"), (33, "gemv"), (300, "auto")])
def test_wide_layer(wide_ctx, T, path):
    """The whole MoE block over 160 experts: at T = 1 and with LM_PATH_GEMV the
    fp32 weight-streaming kernels, from three tokens on the fp16 MFMA kernels."""
    from litemind_amd import PATH_AUTO, PATH_GEMV
    from litemind_amd import workload as wl

    ctx, layer = wide_ctx
    H = layer.dims.hidden
    x = wl.tokens(wl.MASTER_SEED + 1700 + T, T, H)
    announce(f"160-expert layer T={T} path={path}")
    dx, y = ctx.to_device(x), ctx.empty((T, H))
    idx, w = ctx.empty((T, 6), np.int32), ctx.empty((T, 6))
    ctx.moe_forward(0, dx, T, y, idx=idx, w=w, path=PATH_GEMV if path == "gemv" else PATH_AUTO)
    ctx.synchronize()
    gy, gidx, gw = y.download(), idx.download(), w.download()
    oy, oidx, ow, _ = ol.oracle_moe_layer(layer, x)
    assert np.array_equal(gidx, oidx)
    assert np.array_equal(gw.view(np.uint32), ow.view(np.uint32))
    max_abs, mean_rel = layer_error(gy, oy)
    print(f"E=160 T={T} {path} max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    if path == "gemv" or T <= 2:
        assert mean_rel < 1e-5
    for b in (dx, y, idx, w):
        b.free()


# One token over more than 64 experts: the router and gate/up in one
# speculative launch (lm_router_speculation 1, the default), with its repair
# forced (2), and the router then gate/up as separate launches (0).
# (E, k, grouped, n_group, topk_group, hidden, inter, bias)
SPEC_CASES = {
    "e160_g8": (160, 6, True, 8, 3, 1024, 256, False),
    "e160_g8_bias": (160, 6, True, 8, 3, 1024, 256, True),
    "e72_greedy_h2048": (72, 6, False, 1, 1, 2048, 128, False),
    "e256_g8_k8": (256, 8, True, 8, 4, 512, 128, False),
    "e512_greedy_k8": (512, 8, False, 1, 1, 256, 64, False),
    "e100_h1040_ragged": (100, 5, True, 4, 2, 1040, 192, True),
    "e256_h7168_k8": (256, 8, True, 8, 4, 7168, 64, False),
}


@pytest.mark.parametrize("name", sorted(SPEC_CASES))
def test_speculative_router_gateup(name):
    """The three modes give the same bits (logits, experts, weights, layer
    output) on several tokens, and match the oracle: logits, experts and
    weights bit-exact, the output within 1e-5 (the fp32 GEMV path).  The
    ragged case has a last row slice of 16 rows and a logit bias; the widest
    has DeepSeek-V3's routing and hidden size (256 experts, top-8, 7168: seven
    row slices, rows of fourteen 512-column steps)."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    E, k, grouped, ng, tg, hidden, inter, with_bias = SPEC_CASES[name]
    dims = _dims(E, k, grouped, ng, tg, hidden=hidden, inter=inter)
    layer = wl.moe_layer(wl.MASTER_SEED + 2300 + E, 0, dims)
    rng = np.random.default_rng(E + hidden)
    bias = (rng.standard_normal(E) * 0.05).astype(np.float32) if with_bias else None
    announce(f"speculative router + gate/up, {name}")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        wl.upload_moe_layer(ctx, 0, layer)
        db = ctx.to_device(bias) if with_bias else None
        for t in range(3):
            x = wl.tokens(wl.MASTER_SEED + 2400 + t, 1, hidden)
            dx = ctx.to_device(x)
            outs = {}
            for mode in (1, 2, 0, 1):
                ctx.router_speculation(mode)
                y, idx, w, lg = ctx.empty((1, hidden)), ctx.empty((1, k), np.int32), ctx.empty((1, k)), \
                    ctx.empty((1, E))
                ctx.moe_forward(0, dx, 1, y, bias=db, idx=idx, w=w, logits=lg)
                ctx.synchronize()
                got = (y.download(), idx.download(), w.download(), lg.download())
                if mode in outs:
                    ref = outs[mode]
                    assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(got, ref))
                outs[mode] = got
                for bb in (y, idx, w, lg):
                    bb.free()
            for mode in (1, 2):
                assert all(np.array_equal(a.view(np.uint32), b.view(np.uint32)) for a, b in zip(outs[mode], outs[0]))
            ctx.router_speculation(1)
            oy, oidx, ow, ologits = ol.oracle_moe_layer(layer, x, bias)
            gy, gidx, gw, glg = outs[1]
            assert np.array_equal(glg.view(np.uint32), np.asarray(ologits, np.float32).reshape(1, E).view(np.uint32))
            assert np.array_equal(gidx, oidx)
            assert np.array_equal(gw.view(np.uint32), ow.view(np.uint32))
            _, mean_rel = layer_error(gy, oy)
            assert mean_rel < 1e-5
            dx.free()
        with pytest.raises(RuntimeError):
            ctx.router_speculation(3)


def test_speculative_stack_t1_and_graph():
    """Two 160-expert layers as a stack at one token: the eager pass (the
    speculative launch per layer) matches the oracle's chain within 1e-5 and
    gives the same bits as the separate launches (lm_router_speculation 0) and
    as three replays of a captured graph of the pass, which records the
    separate launches (the speculative launch is not used under capture)."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = _dims()
    layers = [("moe", wl.moe_layer(wl.MASTER_SEED + 2500 + l, 0, dims)) for l in range(2)]
    rng = np.random.default_rng(2501)
    norms = [(1.0 + 0.1 * rng.standard_normal(dims.hidden)).astype(np.float32) for _ in range(2)]
    announce("160-expert stack at T=1: eager, separate launches, graph replays")
    with Context(dims.moe_config(num_layers=2)) as ctx:
        for l, (_, layer) in enumerate(layers):
            wl.upload_moe_layer(ctx, l, layer)
            ctx.upload_norm(l, norms[l])
        h0 = wl.tokens(wl.MASTER_SEED + 2502, 1, dims.hidden)

        def run(mode):
            ctx.router_speculation(mode)
            dh = ctx.to_device(h0)
            ctx.stack_forward(0, 1, dh, 1)
            ctx.synchronize()
            out = dh.download()
            dh.free()
            return out

        eager = run(1)
        separate = run(0)
        ctx.router_speculation(1)
        assert np.array_equal(eager.view(np.uint32), separate.view(np.uint32))
        oh = ol.oracle_stack(layers, h0, dims.rms_norm_eps, norms=norms)
        _, mean_rel = layer_error(eager, oh)
        assert mean_rel < 1e-5
        dh = ctx.to_device(h0)
        graph = ctx.stack_graph_create(0, 1, dh, 1)
        try:
            for rep in range(3):
                dh.upload(h0)
                ctx.synchronize()
                ctx.stack_graph_launch(graph)
                ctx.synchronize()
                assert np.array_equal(dh.download().view(np.uint32), eager.view(np.uint32)), f"replay {rep}"
                assert np.array_equal(run(1).view(np.uint32), eager.view(np.uint32))
        finally:
            ctx.stack_graph_destroy(graph)
            dh.free()


def test_speculative_wait_timeout_reports_kernel_error(wide_ctx):
    """Every hand-off wait of the speculative launch made to give up after its
    first poll (a bound the host sets; every wave still runs to its end and
    every index stays clamped): the next lm_synchronize returns LM_EKERNEL,
    and the context then computes exact results again."""
    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, layer = wide_ctx
    H = layer.dims.hidden
    x = wl.tokens(wl.MASTER_SEED + 2600, 1, H)
    dx, y = ctx.to_device(x), ctx.empty((1, H))
    idx, w = ctx.empty((1, 6), np.int32), ctx.empty((1, 6))
    announce("160-expert speculative launch with every wait giving up at once")
    reported = 0
    ctx._check(ctx.lib.lm_decode_wait_test(ctx.handle, 1))
    try:
        for _ in range(4):
            ctx.moe_forward(0, dx, 1, y, idx=idx, w=w)
            try:
                ctx.synchronize()
            except LmError as error:
                assert "status -5" in str(error)
                reported += 1
    finally:
        ctx._check(ctx.lib.lm_decode_wait_test(ctx.handle, 0))
    assert reported >= 1
    ctx.synchronize()
    ctx.moe_forward(0, dx, 1, y, idx=idx, w=w)
    ctx.synchronize()
    oy, oidx, ow, _ = ol.oracle_moe_layer(layer, x)
    assert np.array_equal(idx.download(), oidx)
    assert np.array_equal(w.download().view(np.uint32), ow.view(np.uint32))
    _, mean_rel = layer_error(y.download(), oy)
    assert mean_rel < 1e-5
    for b in (dx, y, idx, w):
        b.free()


@pytest.mark.parametrize("grouped", [True, False])
def test_speculative_router_all_ties(grouped):
    """Every expert's gate row the same: all logits tie exactly, in the exact
    chains and in the reassociated sums alike, so MoeRouter::select's lower
    index rule alone decides (the lowest groups, then the lowest experts).
    The speculative launch and the separate launches give the oracle's
    experts, weights and output."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = _dims(160, 6, grouped, 8 if grouped else 1, 3 if grouped else 1, hidden=1024, inter=128)
    layer = wl.moe_layer(wl.MASTER_SEED + 2700, 0, dims)
    layer.router[:] = layer.router[0]
    announce(f"160-expert layer with tied logits, grouped={grouped}")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        wl.upload_moe_layer(ctx, 0, layer)
        x = wl.tokens(wl.MASTER_SEED + 2701, 1, dims.hidden)
        oy, oidx, ow, _ = ol.oracle_moe_layer(layer, x)
        assert list(oidx[0]) == list(range(6))
        dx = ctx.to_device(x)
        for mode in (1, 0):
            ctx.router_speculation(mode)
            y, idx, w = ctx.empty((1, dims.hidden)), ctx.empty((1, 6), np.int32), ctx.empty((1, 6))
            ctx.moe_forward(0, dx, 1, y, idx=idx, w=w)
            ctx.synchronize()
            assert np.array_equal(idx.download(), oidx)
            assert np.array_equal(w.download().view(np.uint32), ow.view(np.uint32))
            _, mean_rel = layer_error(y.download(), oy)
            assert mean_rel < 1e-5
            for b in (y, idx, w):
                b.free()
        ctx.router_speculation(1)
        dx.free()


@pytest.mark.parametrize("grouped", [True, False])
def test_speculative_router_real_misprediction(grouped):
    """A gate whose exact and reassociated logits order two experts
    differently at the top-k boundary.  Expert 6's products are 1e8, 1 and
    -1e8 in rows 0, 4 and 8: LiteMind's left-to-right sum loses the 1
    (1e8 + 1 rounds to 1e8), so its logit is 0; the partial-sum workgroups add
    the row quads in a tree, (1e8 + -1e8) + 1 = 1.  Expert 5's logit is 0.5
    either way and experts 0-4 lead with 10..6, so the speculation takes
    expert 6 and the exact selection expert 5: the repair runs without the
    testing switch, and the outputs still match the oracle."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    E, H = 160, 1024
    dims = _dims(E, 6, grouped, 8 if grouped else 1, 3 if grouped else 1, hidden=H, inter=128)
    layer = wl.moe_layer(wl.MASTER_SEED + 2800, 0, dims)
    gate = np.zeros((E, H), np.float32)
    gate[:, 12] = -5.0
    for e, v in enumerate((10.0, 9.0, 8.0, 7.0, 6.0)):
        gate[e, 12] = v
    gate[5, 12] = 0.5
    gate[6, 12] = 0.0
    gate[6, 0], gate[6, 4], gate[6, 8] = 1e8, 1.0, -1e8
    layer.router[:] = gate
    x = np.zeros((1, H), np.float32)
    x[0, [0, 4, 8, 12]] = 1.0
    announce(f"160-expert layer whose speculation is wrong, grouped={grouped}")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        wl.upload_moe_layer(ctx, 0, layer)
        oy, oidx, ow, ologits = ol.oracle_moe_layer(layer, x)
        assert ologits[0, 6] == 0.0 and 5 in oidx[0] and 6 not in oidx[0]
        dx = ctx.to_device(x)
        outs = []
        for mode in (1, 0):
            ctx.router_speculation(mode)
            y, idx, w = ctx.empty((1, H)), ctx.empty((1, 6), np.int32), ctx.empty((1, 6))
            ctx.moe_forward(0, dx, 1, y, idx=idx, w=w)
            ctx.synchronize()
            got = (y.download(), idx.download(), w.download())
            assert np.array_equal(got[1], oidx)
            assert np.array_equal(got[2].view(np.uint32), ow.view(np.uint32))
            _, mean_rel = layer_error(got[0], oy)
            assert mean_rel < 1e-5
            outs.append(got)
            for b in (y, idx, w):
                b.free()
        assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32))
        ctx.router_speculation(1)
        dx.free()
