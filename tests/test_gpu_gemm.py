"""namespace gemm (src/Gemm.cpp) on the GPU through the C ABI, bit for bit.

The per-call entry points lm_gemm_matvec_bf16 / lm_gemm_matvec_f32 / lm_vector_op
are what the drop-in gemm:: wrappers call.  Each is checked against LiteMind's own
outputs (tests/golden/kerneltest.npz, router_v2lite.npz, written by the compiled
reference) and against the oracle on seeded inputs, including row lengths that
exercise the 8-wide remainder and the scalar tail of dot_bf16.
"""
import os

import numpy as np
import pytest

import oracle_lib as ol
from conftest import announce

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def gctx():
    from litemind_amd import Context
    from litemind_amd import workload as wl

    announce("create context for gemm entry points")
    ctx = Context(wl.V2_LITE.moe_config(num_layers=1))
    yield ctx
    ctx.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def test_kerneltest_matvec_bf16_golden(gctx):
    """tests/KernelTest.cpp:28-79: 67 x 253 matvec, plain and accumulate (scale 0.5 onto ones)."""
    g = np.load(os.path.join(GOLDEN, "kerneltest.npz"))
    w, x = g["weights"], g["input"]
    announce("gemm matvec_bf16 67x253 golden")
    out = np.zeros(67, np.float32)
    gctx.gemm_matvec_bf16(w, x, out)
    assert np.array_equal(bits(out), bits(g["threaded"]))
    assert np.array_equal(bits(out), bits(g["serial"]))
    acc = np.ones(67, np.float32)
    gctx.gemm_matvec_bf16(w, x, acc, scale=0.5, accumulate=True)
    assert np.array_equal(bits(acc), bits(g["accumulate"]))


@pytest.mark.parametrize("out_dim,in_dim", [(1408, 2048), (2048, 1408), (5, 7), (9, 41), (33, 1000), (3, 0)])
def test_matvec_bf16_against_oracle(gctx, out_dim, in_dim):
    from litemind_amd import workload as wl

    w = wl.normal_bf16(out_dim * 7 + in_dim, 3, 0.02, (out_dim, in_dim))
    x = wl.normal_f32(out_dim * 7 + in_dim, 4, 1.0, (in_dim,))
    expect = np.zeros(out_dim, np.float32)
    ol.oracle().orc_matvec_bf16(ol.p(w), ol.p(x), ol.p(expect), out_dim, in_dim)
    announce(f"gemm matvec_bf16 {out_dim}x{in_dim}")
    out = np.full(out_dim, np.nan, np.float32)
    gctx.gemm_matvec_bf16(w, x, out)
    assert np.array_equal(bits(out), bits(expect))
    start = wl.normal_f32(out_dim, 5, 1.0, (out_dim,))
    expect_acc = start.copy()
    ol.oracle().orc_matvec_bf16_accumulate(ol.p(w), ol.p(x), ol.p(expect_acc), out_dim, in_dim, 0.37)
    acc = start.copy()
    gctx.gemm_matvec_bf16(w, x, acc, scale=0.37, accumulate=True)
    assert np.array_equal(bits(acc), bits(expect_acc))


def test_matvec_f32_router_golden(gctx):
    """The router gate of a DeepSeek-V2-Lite layer (64 x 2048) on 64 tokens, against
    the logits LiteMind's matvec_f32 wrote."""
    from litemind_amd import workload as wl

    g = np.load(os.path.join(GOLDEN, "router_v2lite.npz"))
    router = wl.normal_f32(wl.MASTER_SEED, wl.stream_id(0, wl.S_ROUTER), 0.02, (64, 2048))
    x = wl.tokens(wl.MASTER_SEED + 1, 64, 2048)
    announce("gemm matvec_f32 64x2048 golden, 64 tokens")
    for t in range(64):
        out = np.zeros(64, np.float32)
        gctx.gemm_matvec_f32(router, np.ascontiguousarray(x[t]), out)
        assert np.array_equal(bits(out), bits(g["logits"][t])), f"token {t}"


@pytest.mark.parametrize("out_dim,in_dim", [(64, 2048), (7, 13), (3, 3), (130, 515)])
def test_matvec_f32_against_oracle(gctx, out_dim, in_dim):
    from litemind_amd import workload as wl

    w = wl.normal_f32(in_dim, 6, 0.5, (out_dim, in_dim))
    x = wl.normal_f32(in_dim, 7, 1.0, (in_dim,))
    expect = np.zeros(out_dim, np.float32)
    ol.oracle().orc_matvec_f32(ol.p(w), ol.p(x), ol.p(expect), out_dim, in_dim)
    announce(f"gemm matvec_f32 {out_dim}x{in_dim}")
    out = np.zeros(out_dim, np.float32)
    gctx.gemm_matvec_f32(w, x, out)
    assert np.array_equal(bits(out), bits(expect))


def test_vector_ops_golden(gctx):
    """tests/KernelTest.cpp:81-110 closed-form cases, as the compiled reference wrote them."""
    from litemind_amd import OP_RMS_NORM, OP_SILU_MUL, OP_SOFTMAX

    g = np.load(os.path.join(GOLDEN, "kerneltest.npz"))
    announce("gemm vector ops golden")
    out = np.zeros(4, np.float32)
    gctx.vector_op(OP_RMS_NORM, np.array([1, 2, 3, 4], np.float32), np.full(4, 2.0, np.float32), out, 1e-6)
    assert np.array_equal(bits(out), bits(g["rms_norm"]))
    out = np.zeros(3, np.float32)
    gctx.vector_op(OP_SOFTMAX, np.array([1, 2, 3], np.float32), None, out)
    assert np.array_equal(bits(out), bits(g["softmax"]))
    out = np.zeros(2, np.float32)
    gctx.vector_op(OP_SOFTMAX, np.array([1000, 1001], np.float32), None, out)
    assert np.array_equal(bits(out), bits(g["softmax_extreme"]))
    out = np.zeros(2, np.float32)
    gctx.vector_op(OP_SILU_MUL, np.array([0, 1], np.float32), np.array([3, 2], np.float32), out)
    assert np.array_equal(bits(out), bits(g["silu"]))


@pytest.mark.parametrize("n", [1, 5, 64, 2048, 10944])
def test_vector_ops_against_oracle(gctx, n):
    from litemind_amd import OP_AXPY, OP_DOT, OP_RMS_NORM, OP_SILU_MUL, OP_SOFTMAX, OP_WIDEN
    from litemind_amd import workload as wl

    o = ol.oracle()
    a = wl.normal_f32(n, 8, 3.0, (n,))
    b = wl.normal_f32(n, 9, 1.0, (n,))
    announce(f"gemm vector ops n={n}")

    out = np.zeros(1, np.float32)
    gctx.vector_op(OP_DOT, a, b, out)
    assert bits(out)[0] == bits(np.float32(o.orc_dot_f32(ol.p(a), ol.p(b), n)))

    dst = b.copy()
    o.orc_axpy(0.75, ol.p(a), ol.p(dst), n)
    out = b.copy()
    gctx.vector_op(OP_AXPY, a, None, out, 0.75)
    assert np.array_equal(bits(out), bits(dst))

    sm = a.copy()
    o.orc_softmax(ol.p(sm), n)
    out = np.zeros(n, np.float32)
    gctx.vector_op(OP_SOFTMAX, a, None, out)
    assert np.array_equal(bits(out), bits(sm))

    silu = np.zeros(n, np.float32)
    o.orc_silu_multiply(ol.p(a), ol.p(b), ol.p(silu), n)
    out = np.zeros(n, np.float32)
    gctx.vector_op(OP_SILU_MUL, a, b, out)
    assert np.array_equal(bits(out), bits(silu))

    rms = a.copy()
    o.orc_rms_norm(ol.p(rms), ol.p(b), n, 1e-6)
    out = np.zeros(n, np.float32)
    gctx.vector_op(OP_RMS_NORM, a, b, out, 1e-6)
    assert np.array_equal(bits(out), bits(rms))

    raw = wl.normal_bf16(n, 10, 1.0, (n,))
    out = np.zeros(n, np.float32)
    gctx.vector_op(OP_WIDEN, raw, None, out)
    assert np.array_equal(bits(out), (raw.astype(np.uint32) << 16))


def test_weight_residency(gctx):
    """WeightView::prefetch / release on a pointer-keyed HBM copy: a prefetched
    range is read from HBM until it is released; a range that is not resident is
    uploaded again on every call."""
    import ctypes as C

    from litemind_amd import workload as wl

    w = wl.normal_bf16(1, 11, 0.02, (64, 256))
    x = wl.normal_f32(1, 12, 1.0, (256,))
    fresh = wl.normal_bf16(2, 11, 0.02, (64, 256))
    o = ol.oracle()
    expect_w = np.zeros(64, np.float32)
    o.orc_matvec_bf16(ol.p(w), ol.p(x), ol.p(expect_w), 64, 256)
    expect_fresh = np.zeros(64, np.float32)
    o.orc_matvec_bf16(ol.p(fresh), ol.p(x), ol.p(expect_fresh), 64, 256)
    assert not np.array_equal(bits(expect_w), bits(expect_fresh))
    announce("weight residency")
    lib, h = gctx.lib, gctx.handle
    flag = C.c_int32(-1)
    gctx._check(lib.lm_weight_resident(h, ol.p(w), C.byref(flag)))
    assert flag.value == 0
    gctx._check(lib.lm_weight_prefetch(h, ol.p(w), w.nbytes))
    gctx._check(lib.lm_weight_resident(h, ol.p(w), C.byref(flag)))
    assert flag.value == 1
    original = w.copy()
    w[:] = fresh  # the host range changes while resident: the HBM copy is used
    out = np.zeros(64, np.float32)
    gctx.gemm_matvec_bf16(w, x, out)
    assert np.array_equal(bits(out), bits(expect_w))
    gctx._check(lib.lm_weight_release(h, ol.p(w)))
    gctx._check(lib.lm_weight_resident(h, ol.p(w), C.byref(flag)))
    assert flag.value == 0
    gctx.gemm_matvec_bf16(w, x, out)  # not resident: this call reads the host range
    assert np.array_equal(bits(out), bits(expect_fresh))
    w[:] = original
    gctx.gemm_matvec_bf16(w, x, out)
    assert np.array_equal(bits(out), bits(expect_w))
