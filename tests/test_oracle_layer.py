"""Pins the oracle MoE block and the canonical permutation."""
import hashlib
import os

import numpy as np
import pytest

import oracle_lib as ol
from conftest import layer_error

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def layer_sha(layer):
    h = hashlib.sha256()
    for a in [layer.router] + layer.gate + layer.up + layer.down + [layer.shared_gate, layer.shared_up,
                                                                     layer.shared_down]:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def test_tiny_layer_golden(tiny_layer):
    dims, layer = tiny_layer
    g = np.load(os.path.join(GOLDEN, "layer_tiny.npz"))
    assert layer_sha(layer) == str(g["weights_sha"])
    y, idx, w, _ = ol.oracle_moe_layer(layer, g["x"])
    assert np.array_equal(idx, g["index"])
    assert np.array_equal(bits(w), bits(g["weight"]))
    assert np.array_equal(bits(y), bits(g["y"]))


def test_v2lite_layer_golden(v2_layer):
    g = np.load(os.path.join(GOLDEN, "layer_v2lite.npz"))
    assert layer_sha(v2_layer) == str(g["weights_sha"])
    y, idx, w, _ = ol.oracle_moe_layer(v2_layer, g["x"])
    assert np.array_equal(idx, g["index"]) and np.array_equal(bits(w), bits(g["weight"]))
    assert np.array_equal(bits(y), bits(g["y"]))
    y, idx, w, _ = ol.oracle_moe_layer(v2_layer, g["x"], bias=g["bias"])
    assert np.array_equal(idx, g["index_bias"]) and np.array_equal(bits(y), bits(g["y_bias"]))


def _silu(v):
    return v / (1.0 + np.exp(-v))


def test_tiny_layer_float64_brute_force(tiny_layer):
    """y = sum_r w_r FFN_{e_r}(x) + FFN_shared(x), evaluated in float64."""
    dims, layer = tiny_layer
    x = np.random.default_rng(1).standard_normal((16, dims.hidden)).astype(np.float32)
    y, idx, w, _ = ol.oracle_moe_layer(layer, x)
    f = lambda m: (m.astype(np.uint32) << 16).view(np.float32).astype(np.float64)

    def ffn(g, u, d, v):
        return f(d) @ (_silu(f(g) @ v) * (f(u) @ v))

    for t in range(16):
        v = x[t].astype(np.float64)
        ref = sum(float(w[t, r]) * ffn(layer.gate[idx[t, r]], layer.up[idx[t, r]], layer.down[idx[t, r]], v)
                  for r in range(dims.top_k))
        ref = ref + ffn(layer.shared_gate, layer.shared_up, layer.shared_down, v)
        assert np.max(np.abs(y[t] - ref)) <= 1e-5 * max(1.0, np.max(np.abs(ref)))


@pytest.mark.skipif(not ol.have_ref(), reason="LiteMind sources not compiled (oracle/_ref)")
def test_layer_matches_compiled_reference(tiny_layer):
    """The expert-major oracle equals LiteMind's per-token composition bit for bit."""
    dims, layer = tiny_layer
    x = np.random.default_rng(2).standard_normal((40, dims.hidden)).astype(np.float32)
    y, idx, w, _ = ol.oracle_moe_layer(layer, x)
    yr, idxr, wr = ol.ref_moe_layer(layer, x, workers=3)
    assert np.array_equal(idx, idxr) and np.array_equal(bits(w), bits(wr)) and np.array_equal(bits(y), bits(yr))


def test_dense_ffn_float64():
    rng = np.random.default_rng(6)
    H, D = 64, 96
    mk = lambda *s: (rng.standard_normal(s).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    gate, up, down = mk(D, H), mk(D, H), mk(H, D)
    x = rng.standard_normal((5, H)).astype(np.float32)
    y = ol.oracle_dense(gate, up, down, x)
    f = lambda m: (m.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    ref = (_silu(x.astype(np.float64) @ f(gate).T) * (x.astype(np.float64) @ f(up).T)) @ f(down).T
    assert layer_error(y, ref)[1] < 1e-6


@pytest.mark.parametrize("T,E,K", [(1, 64, 6), (37, 64, 6), (2048, 64, 6), (5, 8, 8), (0, 64, 6)])
def test_permutation_brute_force(T, E, K):
    rng = np.random.default_rng(T + E)
    rows = [rng.choice(E, size=K, replace=False) for _ in range(T)]
    idx = (np.stack(rows) if rows else np.zeros((0, K))).astype(np.int32).reshape(T, K)
    counts, offsets, perm, slot_of = ol.oracle_permute(idx, E)
    flat = idx.reshape(-1)
    order = sorted(range(T * K), key=lambda a: (flat[a], a))  # stable by expert
    assert list(perm) == order
    assert np.array_equal(counts, np.bincount(flat, minlength=E))
    assert offsets[0] == 0 and np.array_equal(np.diff(offsets), counts)
    assert np.array_equal(slot_of[perm], np.arange(T * K))
