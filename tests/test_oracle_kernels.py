"""Pins the oracle's kernels (oracle/oracle.c) against LiteMind's own tests,
golden vectors from its compiled sources, closed forms and float64 brute force."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle_lib as ol

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
o = ol.oracle()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_kerneltest_matvec_against_float64():
    """tests/KernelTest.cpp:50-79: 67 x 253 BF16 matvec within 1e-3 of float64."""
    g = np.load(os.path.join(GOLDEN, "kerneltest.npz"))
    w, x = g["weights"], g["input"]
    wf = (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    expected = wf @ x.astype(np.float64)
    out = np.zeros(67, np.float32)
    o.orc_matvec_bf16(ol.p(w), ol.p(x), ol.p(out), 67, 253)
    assert np.max(np.abs(out - expected)) <= 1e-3
    acc = np.ones(67, np.float32)
    o.orc_matvec_bf16_accumulate(ol.p(w), ol.p(x), ol.p(acc), 67, 253, 0.5)
    assert np.max(np.abs(acc - (1.0 + 0.5 * expected))) <= 1e-3


def test_kerneltest_golden_bit_exact():
    """Same case, bit for bit against LiteMind's threaded, serial and accumulate paths."""
    g = np.load(os.path.join(GOLDEN, "kerneltest.npz"))
    w, x = g["weights"], g["input"]
    out = np.zeros(67, np.float32)
    o.orc_matvec_bf16(ol.p(w), ol.p(x), ol.p(out), 67, 253)
    assert np.array_equal(bits(out), bits(g["threaded"]))
    assert np.array_equal(bits(out), bits(g["serial"]))
    acc = np.ones(67, np.float32)
    o.orc_matvec_bf16_accumulate(ol.p(w), ol.p(x), ol.p(acc), 67, 253, 0.5)
    assert np.array_equal(bits(acc), bits(g["accumulate"]))


def test_closed_forms():
    """tests/KernelTest.cpp:81-110."""
    g = np.load(os.path.join(GOLDEN, "kerneltest.npz"))
    v = np.array([1, 2, 3, 4], np.float32)
    o.orc_rms_norm(ol.p(v), ol.p(np.full(4, 2.0, np.float32)), 4, 1e-6)
    scale = 2.0 / np.sqrt(7.5 + 1e-6)
    assert np.allclose(v, np.arange(1, 5) * scale, atol=1e-5, rtol=0)
    assert np.array_equal(bits(v), bits(g["rms_norm"]))
    s = np.array([1, 2, 3], np.float32)
    o.orc_softmax(ol.p(s), 3)
    assert abs(float(s.sum()) - 1.0) <= 1e-6 and s[2] > s[1] > s[0]
    assert np.array_equal(bits(s), bits(g["softmax"]))
    e = np.array([1000, 1001], np.float32)
    o.orc_softmax(ol.p(e), 2)
    assert np.all(np.isfinite(e)) and abs(float(e.sum()) - 1.0) <= 1e-6
    assert np.array_equal(bits(e), bits(g["softmax_extreme"]))
    out = np.zeros(2, np.float32)
    o.orc_silu_multiply(ol.p(np.array([0, 1], np.float32)), ol.p(np.array([3, 2], np.float32)), ol.p(out), 2)
    assert abs(out[0]) <= 1e-6 and abs(out[1] - 2.0 / (1.0 + np.exp(-1.0))) <= 1e-6
    assert np.array_equal(bits(out), bits(g["silu"]))


def test_dot_f32_is_unfused_left_to_right():
    """The router dot: each product rounded, then added in order (float64 restatement),
    and it differs from a fused chain, so a fusing implementation would be caught."""
    rng = np.random.default_rng(3)
    differs = 0
    for n in (16, 64, 2048):
        a = rng.standard_normal(n).astype(np.float32)
        b = rng.standard_normal(n).astype(np.float32)
        t = np.float32(0)
        for i in range(n):
            t = np.float32(t + np.float32(a[i] * b[i]))
        got = np.float32(o.orc_dot_f32(ol.p(a), ol.p(b), n))
        assert bits(got) == bits(t)
        fused = np.float32(0)
        for i in range(n):
            fused = np.float32(np.float64(a[i]) * np.float64(b[i]) + np.float64(fused))
        differs += int(bits(fused) != bits(t))
    assert differs > 0


def test_dot_bf16_association_order():
    """dot_bf16 with 4 x 8-lane FMA accumulators and LiteMind's horizontal sum, restated
    in numpy with explicit float32 rounding."""
    rng = np.random.default_rng(4)
    for n in (32, 40, 253, 2048):
        wbits = (rng.standard_normal(n).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        w = (wbits.astype(np.uint32) << 16).view(np.float32)
        x = rng.standard_normal(n).astype(np.float32)
        fma = lambda a, b, c: np.float32(np.float64(a) * np.float64(b) + np.float64(c))  # exact for fp32 inputs
        acc = np.zeros((4, 8), np.float32)
        i = 0
        while i + 32 <= n:
            for k in range(4):
                for l in range(8):
                    acc[k, l] = fma(w[i + 8 * k + l], x[i + 8 * k + l], acc[k, l])
            i += 32
        while i + 8 <= n:
            for l in range(8):
                acc[0, l] = fma(w[i + l], x[i + l], acc[0, l])
            i += 8
        s = (acc[0] + acc[1]) + (acc[2] + acc[3])
        h = [np.float32(s[j] + s[j + 4]) for j in range(4)]
        total = np.float32(np.float32(h[0] + h[2]) + np.float32(h[1] + h[3]))
        while i < n:
            total = fma(w[i], x[i], total)
            i += 1
        got = np.float32(o.orc_dot_bf16(ol.p(wbits), ol.p(x), n))
        assert bits(got) == bits(total), n


@pytest.mark.skipif(not ol.have_ref(), reason="LiteMind sources not compiled (oracle/_ref)")
def test_oracle_matches_compiled_reference():
    r = ol.ref()
    rng = np.random.default_rng(5)
    for od, idim in ((67, 253), (64, 2048), (2048, 1408), (5, 7), (3, 33)):
        w = (rng.standard_normal((od, idim)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        x = rng.standard_normal(idim).astype(np.float32)
        a, b = np.zeros(od, np.float32), np.zeros(od, np.float32)
        o.orc_matvec_bf16(ol.p(w), ol.p(x), ol.p(a), od, idim)
        r.ref_matvec_bf16(4, ol.p(w), ol.p(x), ol.p(b), od, idim)
        assert np.array_equal(bits(a), bits(b))
        wf = rng.standard_normal((od, idim)).astype(np.float32)
        o.orc_matvec_f32(ol.p(wf), ol.p(x), ol.p(a), od, idim)
        r.ref_matvec_f32(ol.p(wf), ol.p(x), ol.p(b), od, idim)
        assert np.array_equal(bits(a), bits(b))
    for n in (3, 64, 100, 2048):
        v = (rng.standard_normal(n) * 3).astype(np.float32)
        v1, v2 = v.copy(), v.copy()
        o.orc_softmax(ol.p(v1), n)
        r.ref_softmax(ol.p(v2), n)
        assert np.array_equal(bits(v1), bits(v2))
        g, u = (rng.standard_normal(n) * 4).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        s1, s2 = np.zeros(n, np.float32), np.zeros(n, np.float32)
        o.orc_silu_multiply(ol.p(g), ol.p(u), ol.p(s1), n)
        r.ref_silu_multiply(ol.p(g), ol.p(u), ol.p(s2), n)
        assert np.array_equal(bits(s1), bits(s2))
        wn = rng.uniform(0.5, 2, n).astype(np.float32)
        n1, n2 = v.copy(), v.copy()
        o.orc_rms_norm(ol.p(n1), ol.p(wn), n, 1e-6)
        r.ref_rms_norm(ol.p(n2), ol.p(wn), n, 1e-6)
        assert np.array_equal(bits(n1), bits(n2))


@pytest.mark.skipif(not ol.have_ref(), reason="LiteMind sources not compiled (oracle/_ref)")
def test_reference_thread_pool_visits_each_index_once():
    """tests/KernelTest.cpp:112-121 against the compiled ThreadPool the CPU baseline uses."""
    for workers in (1, 2, 8):
        visits = np.zeros(1000, np.int32)
        ol.ref().ref_parallel_for_visit(workers, 1000, ol.p(visits))
        assert np.all(visits == 1)
