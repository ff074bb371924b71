"""Pins the oracle's multi-head latent attention (Attention::forward,
src/Attention.cpp:22-103), rotary embedding (src/Rope.cpp:35-118) and KV cache
append (src/KvCache.cpp) against the compiled reference, its golden fixture,
closed forms and a float64 brute force."""
import dataclasses
import json
import os

import numpy as np
import pytest

import oracle_lib as ol
from litemind_amd import workload as wl

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
SMALL = dataclasses.replace(wl.V2_LITE_MLA, hidden=256, heads=4, kv_lora_rank=64, qk_nope=32, qk_rope=16, v_head=32,
                            original_max=16, factor=4.0, max_positions=16)
needs_ref = pytest.mark.skipif(not ol.have_ref(), reason="oracle/_ref/libref.so not built")


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def golden():
    return np.load(os.path.join(GOLDEN, "mla.npz"))


def widen(w):
    return (w.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def brute_mla(L, x, position0):
    """Attention in float64 from the definitions (no reference code): the
    projections, RMS norms, rotation of the (even, odd) channel pairs into
    (first half, second half), causal softmax attention and the output
    projection."""
    d = L.dims
    cos, sin = ol.oracle_rope_tables(d)
    nope, rope, vh, qk, half = d.qk_nope, d.qk_rope, d.v_head, d.qk_head, d.qk_rope // 2

    def rms(v, w):
        return v / np.sqrt(np.mean(v * v) + d.rms_norm_eps) * w.astype(np.float64)

    def rotate(v, pos):
        if pos >= d.max_positions:
            return v
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        e, o = v[0::2], v[1::2]
        return np.concatenate([e * c - o * s, o * c + e * s])

    keys, values, out = [], [], []
    scale = ol.softmax_scale(d)
    for t in range(x.shape[0]):
        pos = position0 + t
        xt = x[t].astype(np.float64)
        if d.q_lora_rank == 0:
            q = widen(L.q_proj) @ xt
        else:
            q = widen(L.q_b_proj) @ rms(widen(L.q_a_proj) @ xt, L.q_a_layernorm)
        q = q.reshape(d.heads, qk)
        q = np.concatenate([q[:, :nope], np.stack([rotate(q[h, nope:], pos) for h in range(d.heads)])], axis=1)
        lat = widen(L.kv_a_proj) @ xt
        c = rms(lat[:d.kv_lora_rank], L.kv_a_layernorm)
        kr = rotate(lat[d.kv_lora_rank:], pos)
        kv = (widen(L.kv_b_proj) @ c).reshape(d.heads, nope + vh)
        keys.append(np.concatenate([kv[:, :nope], np.broadcast_to(kr, (d.heads, rope))], axis=1))
        values.append(kv[:, nope:])
        K, V = np.stack(keys, 1), np.stack(values, 1)  # [heads, tokens, dim]
        s = np.einsum("hd,htd->ht", q, K) * scale
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ctx = np.einsum("ht,htd->hd", p, V).reshape(-1)
        out.append(widen(L.o_proj) @ ctx)
    return np.stack(out)


# ---- rotary embedding ----

@pytest.mark.parametrize("yarn", [False, True])
def test_rope_closed_forms(yarn):
    """Position 0 is the magnitude on cos and zero on sin; with mscale ==
    mscale_all_dim the rotation keeps each pair's norm; the first channel's
    inverse frequency is 1 without YaRN, so cos[p, 0] = cos(p)."""
    d = dataclasses.replace(wl.V2_LITE_MLA, yarn=yarn, max_positions=512)
    cos, sin = ol.oracle_rope_tables(d)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    np.testing.assert_allclose(cos.astype(np.float64) ** 2 + sin.astype(np.float64) ** 2, 1.0, atol=2e-7)
    if not yarn:
        np.testing.assert_array_equal(cos[:, 0], np.cos(np.arange(512, dtype=np.float64)).astype(np.float32))
        inv = 1.0 / 10000.0 ** (np.arange(32) * 2.0 / 64.0)
        np.testing.assert_allclose(sin, np.sin(np.arange(512)[:, None] * inv[None, :]), atol=6e-8)
    # position 0 de-interleaves: (e0, o0, e1, o1, ...) -> (e0, e1, ..., o0, o1, ...)
    v = np.arange(64, dtype=np.float32)
    ol.oracle().orc_rope_apply(ol.p(v), 64, ol.p(cos[0]), ol.p(sin[0]))
    np.testing.assert_array_equal(v, np.concatenate([np.arange(0, 64, 2), np.arange(1, 64, 2)]).astype(np.float32))


def test_rope_yarn_magnitude():
    """mscale != mscale_all_dim scales every table entry by the ratio of the two
    YaRN magnitudes 0.1 m ln(factor) + 1."""
    d = dataclasses.replace(wl.V2_LITE_MLA, factor=40.0, mscale=1.0, mscale_all_dim=0.5, max_positions=64)
    cos, sin = ol.oracle_rope_tables(d)
    ratio = (0.1 * np.log(40.0) + 1.0) / (0.05 * np.log(40.0) + 1.0)
    np.testing.assert_allclose(cos[0], ratio, rtol=1e-7)
    np.testing.assert_allclose(np.hypot(cos, sin), ratio, rtol=3e-7)
    # softmax scale: (nope + rope)^-1/2 times the squared all-dim magnitude
    want = (192 ** -0.5) * (0.05 * np.log(40.0) + 1.0) ** 2
    assert abs(ol.softmax_scale(d) - want) <= 1e-8


@needs_ref
@pytest.mark.parametrize("yarn,factor,mscale,mscale_all", [(False, 1.0, 1.0, 1.0), (True, 40.0, 0.707, 0.707),
                                                           (True, 40.0, 0.5, 1.0), (True, 8.0, 1.0, 0.0)])
def test_rope_tables_match_reference(yarn, factor, mscale, mscale_all):
    d = dataclasses.replace(wl.V2_LITE_MLA, yarn=yarn, factor=factor, mscale=mscale, mscale_all_dim=mscale_all,
                            max_positions=1024)
    oc, osn = ol.oracle_rope_tables(d)
    rc, rs = ol.ref_rope_tables(d)
    np.testing.assert_array_equal(bits(oc), bits(rc))
    np.testing.assert_array_equal(bits(osn), bits(rs))
    assert ol.softmax_scale(d) == ol.ref().ref_softmax_scale(d.qk_nope, d.qk_rope, 1 if yarn else 0, factor,
                                                            mscale_all)


@needs_ref
def test_rope_apply_matches_reference():
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=256)
    cos, sin = ol.oracle_rope_tables(d)
    rng = np.random.default_rng(5)
    for pos in list(range(0, 256, 7)) + [255, 256, 300]:
        v = (rng.standard_normal(64) * 3).astype(np.float32)
        r = v.copy()
        ol.ref().ref_rope_apply(*ol._rope_args(d), ol.p(r), pos)
        if pos < d.max_positions:
            ol.oracle().orc_rope_apply(ol.p(v), 64, ol.p(cos[pos]), ol.p(sin[pos]))
        # past the table the reference leaves the values unrotated
        np.testing.assert_array_equal(bits(v), bits(r))


def test_rope_golden():
    g = golden()
    d = wl.V2_LITE_MLA
    cos, sin = ol.oracle_rope_tables(d)
    rows = g["rope/rows"]
    np.testing.assert_array_equal(bits(cos[rows]), bits(g["rope/cos"]))
    np.testing.assert_array_equal(bits(sin[rows]), bits(g["rope/sin"]))
    import hashlib
    h = hashlib.sha256()
    h.update(cos.tobytes())
    h.update(sin.tobytes())
    assert h.hexdigest() == str(g["rope/sha"])
    assert np.float32(ol.softmax_scale(d)) == g["rope/softmax_scale"]


# ---- attention ----

def run_golden_case(g, name):
    over = json.loads(str(g[name + "/dims"]))
    d = dataclasses.replace(wl.V2_LITE_MLA, **over)
    seed, T, pos0, done = (int(v) for v in g[name + "/meta"])
    L = wl.mla_layer(seed, 0, d)
    x = wl.tokens(seed + 1, T, d.hidden)
    cache = ol.OracleKvCache(d, d.max_positions)
    y, n = ol.oracle_mla(L, x, pos0, cache)
    return d, L, x, y, n, cache, done


@pytest.mark.parametrize("name", ["small_yarn", "small_qlora_plain", "small_full", "v2lite"])
def test_mla_golden(name):
    import hashlib
    g = golden()
    d, L, x, y, n, cache, done = run_golden_case(g, name)
    assert n == done
    if name + "/x" in g:
        np.testing.assert_array_equal(bits(x), bits(g[name + "/x"]))
        np.testing.assert_array_equal(bits(cache.key_nope[:n]), bits(g[name + "/key_nope"]))
        np.testing.assert_array_equal(bits(cache.key_rope[:n]), bits(g[name + "/key_rope"]))
        np.testing.assert_array_equal(bits(cache.value[:n]), bits(g[name + "/value"]))
    else:
        h = hashlib.sha256()
        h.update(cache.key_nope[:n].tobytes())
        h.update(cache.key_rope[:n].tobytes())
        h.update(cache.value[:n].tobytes())
        assert h.hexdigest() == str(g[name + "/cache_sha"])
    # tokens that found the cache full leave their output rows untouched
    np.testing.assert_array_equal(bits(y[:n]), bits(g[name + "/out"][:n]))


@needs_ref
@pytest.mark.parametrize("over,T,pos0", [
    (dict(), 9, 0),
    (dict(yarn=False), 7, 2),
    (dict(q_lora_rank=48), 9, 0),
    (dict(max_positions=5), 8, 0),
    (dict(max_positions=12), 4, 10),  # positions past the rotary table
    (dict(qk_rope=6, qk_nope=22, v_head=24, heads=3), 6, 0),  # dot tails past the 4-element body
])
def test_mla_matches_reference(over, T, pos0):
    d = dataclasses.replace(SMALL, **over)
    L = wl.mla_layer(21, 0, d)
    x = wl.tokens(22, T, d.hidden)
    cache = ol.OracleKvCache(d, d.max_positions)
    y, n = ol.oracle_mla(L, x, pos0, cache)
    r, rn, kn, kr, v = ol.ref_mla(L, x, pos0, d.max_positions)
    assert n == rn == min(T, d.max_positions)
    np.testing.assert_array_equal(bits(y[:n]), bits(r[:n]))
    np.testing.assert_array_equal(bits(cache.key_nope), bits(kn))
    np.testing.assert_array_equal(bits(cache.key_rope), bits(kr))
    np.testing.assert_array_equal(bits(cache.value), bits(v))


@pytest.mark.parametrize("over", [dict(), dict(q_lora_rank=48, yarn=False)])
def test_mla_float64_brute_force(over):
    d = dataclasses.replace(SMALL, **over)
    L = wl.mla_layer(31, 0, d)
    x = wl.tokens(32, 10, d.hidden)
    cache = ol.OracleKvCache(d, d.max_positions)
    y, n = ol.oracle_mla(L, x, 1, cache)
    want = brute_mla(L, x, 1)
    err = np.abs(y.astype(np.float64) - want)
    assert err.max() <= 1e-5 * max(1.0, np.abs(want).max()), err.max()


def test_mla_cache_full_returns_and_keeps_cache():
    d = dataclasses.replace(SMALL, max_positions=3)
    L = wl.mla_layer(41, 0, d)
    x = wl.tokens(42, 5, d.hidden)
    cache = ol.OracleKvCache(d, 3)
    y, n = ol.oracle_mla(L, x, 0, cache)
    assert n == 3 and cache.count.value == 3
    before = cache.value.copy()
    y2, n2 = ol.oracle_mla(L, x[3:], 3, cache)
    assert n2 == 0 and cache.count.value == 3
    np.testing.assert_array_equal(cache.value, before)


# ---- the library's host-side table builder (no GPU) ----

@pytest.mark.parametrize("over", [dict(), dict(yarn=False), dict(mscale=0.5, mscale_all_dim=1.0),
                                  dict(factor=8.0, mscale_all_dim=0.0, original_max=2048)])
def test_library_rope_tables_match_oracle(over):
    """lm_rope_tables / lm_mla_softmax_scale (the product's RotaryEmbedding::build
    and Config::softmax_scale, run on the host) against the oracle, bit for bit."""
    import litemind_amd
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=2048, **over)
    cos, sin = litemind_amd.rope_tables(wl.mla_config(d), d.max_positions)
    oc, osn = ol.oracle_rope_tables(d)
    np.testing.assert_array_equal(bits(cos), bits(oc))
    np.testing.assert_array_equal(bits(sin), bits(osn))
    assert litemind_amd.mla_softmax_scale(wl.mla_config(d)) == ol.softmax_scale(d)
