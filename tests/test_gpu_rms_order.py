"""The GPU RMSNorms on rows where the order of the sum of squares matters
(tests/rms_rows.py: a thread-strided tree sum alone rounds their inverse one
ulp away from gemm::rms_norm's in-order sum).  Each kernel must still give
LiteMind's bits (src/Gemm.cpp:197-207):
  * lm_rms_norm (the batched kernel of the stack and the attention) against the
    oracle, row by row, on those rows and on random ones;
  * the single-token kernel's fused norm (lm_stack_forward, T = 1): the layer's
    output equals h + lm_moe_forward(rms_norm(h)) with the norm from the oracle;
  * the decoder's single-token attention, whose input norm runs inside the
    query projection's launch: lm_decoder_forward (T = 1) equals the oracle's
    norm, lm_attention_forward, the residual add and lm_stack_forward called
    one after another."""
import dataclasses

import numpy as np
import pytest

import oracle_lib as ol
import rms_rows as rr
from conftest import announce

pytestmark = pytest.mark.gpu

EPS = np.float32(1e-6)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def oracle_norm(x, w):
    out = np.ascontiguousarray(x, np.float32).copy()
    o = ol.oracle()
    for t in range(out.shape[0]):
        o.orc_rms_norm(ol.p(out[t]), ol.p(w), out.shape[1], EPS)
    return out


def test_rms_norm_kernel_on_order_sensitive_rows(v2_ctx):
    ctx, _ = v2_ctx
    rng = np.random.default_rng(71)
    x = np.concatenate([rr.adversarial_rows(16), rng.standard_normal((16, rr.N)).astype(np.float32)])
    w = rng.uniform(0.5, 1.5, rr.N).astype(np.float32)
    announce("lm_rms_norm on 16 order-sensitive and 16 random rows")
    dx, dw, dy = ctx.to_device(x), ctx.to_device(w), ctx.empty(x.shape)
    ctx.rms_norm(dx, dw, dy, x.shape[0], rr.N, EPS)
    ctx.synchronize()
    got = dy.download()
    ctx.rms_norm(dx, dw, dx, x.shape[0], rr.N, EPS)  # in place
    ctx.synchronize()
    in_place = dx.download()
    for b in (dx, dw, dy):
        b.free()
    want = oracle_norm(x, w)
    assert np.array_equal(bits(got), bits(want))
    assert np.array_equal(bits(in_place), bits(want))


def test_single_token_kernel_fused_norm_on_order_sensitive_rows(v2_ctx):
    from litemind_amd import PATH_AUTO
    ctx, _ = v2_ctx
    w = np.random.default_rng(72).uniform(0.5, 1.5, rr.N).astype(np.float32)
    ctx.upload_norm(0, w)
    rows = rr.adversarial_rows(4, seed=11)
    for i, h in enumerate(rows):
        announce(f"lm_stack_forward T=1 (fused norm) on order-sensitive row {i}")
        dh = ctx.to_device(h[None])
        ctx.stack_forward(0, 0, dh, 1, path=PATH_AUTO)
        ctx.synchronize()
        got = dh.download()
        dh.free()
        xn = ctx.to_device(oracle_norm(h[None], w))
        y = ctx.empty((1, rr.N))
        ctx.moe_forward(0, xn, 1, y, path=PATH_AUTO)
        ctx.synchronize()
        want = h[None] + y.download()
        for b in (xn, y):
            b.free()
        assert np.array_equal(bits(got), bits(want)), f"row {i}"


def test_decoder_fused_input_norm_on_order_sensitive_rows():
    from litemind_amd import PATH_AUTO, Context
    from litemind_amd import workload as wl
    dims = wl.V2_LITE
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=16)
    announce("decoder T=1 with the input norm fused, on order-sensitive rows")
    ctx = Context(dims.moe_config(num_layers=1))
    try:
        ctx.attention_configure(wl.mla_config(d))
        wl.upload_moe_layer(ctx, 0, wl.moe_layer(wl.MASTER_SEED, 0, dims))
        wl.upload_mla_layer(ctx, 0, wl.mla_layer(261, 0, d))
        rng = np.random.default_rng(262)
        in_norm = rng.uniform(0.5, 1.5, rr.N).astype(np.float32)
        ctx.upload_input_norm(0, in_norm)
        ctx.upload_norm(0, rng.uniform(0.5, 1.5, rr.N).astype(np.float32))
        for i, h in enumerate(rr.adversarial_rows(3, seed=13)):
            ctx.kv_cache_clear()
            dh = ctx.to_device(h[None])
            ctx.decoder_forward(0, 0, dh, 1, 0, PATH_AUTO)
            ctx.synchronize()
            got = dh.download()
            dh.free()
            ctx.kv_cache_clear()
            xn = ctx.to_device(oracle_norm(h[None], in_norm))
            a = ctx.empty((1, rr.N))
            ctx.attention_forward(0, xn, 1, 0, a)
            ctx.synchronize()
            dh = ctx.to_device(h[None] + a.download())
            ctx.stack_forward(0, 0, dh, 1, path=PATH_AUTO)
            ctx.synchronize()
            want = dh.download()
            for b in (xn, a, dh):
                b.free()
            assert np.array_equal(bits(got), bits(want)), f"row {i}"
    finally:
        ctx.close()
