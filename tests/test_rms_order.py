"""The order of gemm::rms_norm's sum of squares (CPU, no GPU): on the rows of
tests/rms_rows.py a thread-strided tree sum (the GPU kernels' first pass)
rounds the inverse differently from LiteMind's in-order sum, so a kernel that
stopped at the tree would not be bit-exact; the oracle's rms_norm follows the
in-order sum there, and so does LiteMind's compiled gemm::rms_norm.  The GPU
kernels' outputs on the same rows are checked in tests/test_gpu_rms_order.py."""
import numpy as np

import oracle_lib as ol
import rms_rows as rr


def test_tree_order_alone_rounds_differently():
    rows = rr.adversarial_rows(12)
    eps = np.float32(1e-6)
    for x in rows:
        t, s = rr.inverse(rr.tree_sum(x), rr.N, eps), rr.inverse(rr.seq_sum(x), rr.N, eps)
        assert abs(int(t.view(np.uint32)) - int(s.view(np.uint32))) == 1


def test_oracle_and_litemind_follow_the_element_order():
    rows = rr.adversarial_rows(12)
    eps = np.float32(1e-6)
    w = np.ones(rr.N, np.float32)
    o = ol.oracle()
    for x in rows:
        got = x.copy()
        o.orc_rms_norm(ol.p(got), ol.p(w), rr.N, eps)
        inv = rr.inverse(rr.seq_sum(x), rr.N, eps)
        want = (x * inv) * w
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        if ol.have_ref():
            ref = x.copy()
            ol.ref().ref_rms_norm(ol.p(ref), ol.p(w), rr.N, eps)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_random_rows_rarely_differ():
    """On N(0, 1) rows the two orders agree: the differences are a few ulps of
    a double, far below a float's rounding step (none in 2,000 rows)."""
    rng = np.random.default_rng(9)
    eps = np.float32(1e-6)
    x = rng.standard_normal((2000, rr.N)).astype(np.float32)
    d = x.astype(np.float64)
    seq = np.zeros(len(x))
    for i in range(rr.N):
        seq = seq + d[:, i] ** 2
    sq = np.zeros((len(x), 256))
    for u in range(8):
        sq = sq + d[:, u * 256:(u + 1) * 256] ** 2
    w = sq.reshape(-1, 4, 64)
    for o in (32, 16, 8, 4, 2, 1):
        w = w + w[:, :, np.arange(64) ^ o]
    tree = (w[:, 0, 0] + w[:, 1, 0]) + (w[:, 2, 0] + w[:, 3, 0])
    inv = lambda s: (1.0 / np.sqrt(s / rr.N + np.float64(eps))).astype(np.float32)
    assert np.array_equal(inv(seq), inv(tree))
