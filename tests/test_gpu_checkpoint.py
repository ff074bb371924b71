"""Layers loaded from a SafeTensors checkpoint (lm_load_layer) against the same
weights uploaded array by array: every output must be the same bits.

The checkpoint holds a dense layer and two MoE layers under DeepSeek's tensor
names (the ones LiteMind's DeepSeekRunner::Impl::resolve_layer requires,
src/DeepSeekRunner.cpp:157-225), one shard per layer, with the router stored as
F32 in one layer and BF16 in the other and the norm weights as F32, BF16 and F16,
so the widening of WeightStore::read_float32 is on the path.
"""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

DIMS = dict(hidden=512, inter=128, experts=32, top_k=4, n_shared=2, dense_inter=384, layers=3,
            norm_topk_prob=True, routed_scaling_factor=2.0)


def _widen_bf16(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    from litemind_amd import workload as wl

    dims = wl.Dims(**DIMS)
    d = tmp_path_factory.mktemp("ckpt")
    rng = np.random.default_rng(17)
    norms = [(1.0 + 0.1 * rng.standard_normal(dims.hidden)).astype(np.float32) for _ in range(3)]
    stored = [norms[0], wl.f32_to_bf16(norms[1]), norms[2].astype(np.float16)]
    widened = [norms[0], _widen_bf16(stored[1]), stored[2].astype(np.float32)]
    dense = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
    moe = [wl.moe_layer(wl.MASTER_SEED + 3, l, dims) for l in (1, 2)]
    wl.save_safetensors(d / "model-00001-of-00003.safetensors", wl.dense_layer_tensors(0, dense, stored[0]))
    wl.save_safetensors(d / "model-00002-of-00003.safetensors", wl.moe_layer_tensors(1, moe[0], stored[1]))
    wl.save_safetensors(d / "model-00003-of-00003.safetensors",
                        wl.moe_layer_tensors(2, moe[1], stored[2], router_dtype=np.uint16))
    routers = [moe[0].router, _widen_bf16(wl.f32_to_bf16(moe[1].router))]
    return dims, d, dense, moe, widened, routers


def _contexts(model):
    from litemind_amd import Checkpoint, Context

    dims, d, dense, moe, norms, routers = model
    cfg = dims.moe_config(num_layers=3)
    a, b = Context(cfg), Context(cfg)
    announce("checkpoint: lm_load_layer for layers 0-2")
    with Checkpoint(d) as ck:
        assert ck.count() == (4 + 2 * (5 + 3 * dims.experts), 3)
        for layer in range(3):
            a.load_layer(ck, layer)
    announce("checkpoint: the same weights through the upload calls")
    b.upload_dense(0, *dense)
    for i, L in enumerate(moe):
        b.upload_router(1 + i, routers[i])
        for e in range(dims.experts):
            b.upload_expert(1 + i, e, L.gate[e], L.up[e], L.down[e])
        b.upload_shared(1 + i, L.shared_gate, L.shared_up, L.shared_down)
    for layer in range(3):
        b.upload_norm(layer, norms[layer])
        b.finalize_layer(layer)
    return a, b


def test_loaded_layers_match_uploaded(model):
    from litemind_amd import workload as wl

    dims = model[0]
    a, b = _contexts(model)
    try:
        assert a.resident_bytes() == b.resident_bytes()
        for T in (1, 3, 37, 300):
            announce(f"checkpoint: stack forward T={T} on both contexts")
            h0 = wl.tokens(wl.MASTER_SEED + 900 + T, T, dims.hidden)
            outs = []
            for ctx in (a, b):
                dh = ctx.to_device(h0)
                ctx.stack_forward(0, 2, dh, T)
                ctx.synchronize()
                outs.append(dh.download())
                dh.free()
            assert np.all(np.isfinite(outs[0]))
            assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32)), T
        for layer in (1, 2):
            T = 16
            announce(f"checkpoint: moe_forward layer {layer} T={T} routing and output")
            x = wl.tokens(wl.MASTER_SEED + 50 + layer, T, dims.hidden)
            res = []
            for ctx in (a, b):
                dx, dy = ctx.to_device(x), ctx.empty((T, dims.hidden))
                di, dw = ctx.empty((T, dims.top_k), np.int32), ctx.empty((T, dims.top_k))
                ctx.moe_forward(layer, dx, T, dy, idx=di, w=dw)
                ctx.synchronize()
                res.append((dy.download(), di.download(), dw.download()))
            for u, v in zip(*res):
                assert np.array_equal(np.asarray(u).view(np.uint32), np.asarray(v).view(np.uint32)), layer
    finally:
        a.close()
        b.close()


def test_load_layer_errors(model, tmp_path):
    from litemind_amd import Checkpoint, Context, LmError
    from litemind_amd import workload as wl

    dims, _, dense, moe, norms, _ = model
    t = wl.moe_layer_tensors(1, moe[0], norms[1])
    del t["model.layers.1.mlp.experts.3.down_proj.weight"]
    t["model.layers.1.mlp.experts.5.up_proj.weight"] = moe[0].up[5][:, :-8].copy()
    wl.save_safetensors(tmp_path / "model.safetensors", t)
    announce("checkpoint: load errors")
    with Checkpoint(tmp_path) as ck, Context(dims.moe_config(num_layers=3)) as ctx:
        with pytest.raises(LmError, match="no tensor named 'model.layers.1.mlp.experts.3.down_proj.weight'"):
            ctx.load_layer(ck, 1)
        with pytest.raises(LmError, match="no tensor named 'model.layers.0.post_attention_layernorm.weight'"):
            ctx.load_layer(ck, 0)
        with pytest.raises(LmError, match="no tensor named 'model.layers.1.mlp.gate_proj.weight'"):
            ctx.load_layer(ck, 1, moe=0)
        assert ctx.resident_bytes() == 0  # nothing was uploaded before the checks failed
