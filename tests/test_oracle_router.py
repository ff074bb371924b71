"""Pins the oracle router (MoeRouter::select restated) against LiteMind's
known-answer tests, golden vectors from the compiled router, and brute force."""
import os

import numpy as np
import pytest

import oracle_lib as ol

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
KNOWN = np.array([0.0, 5.0, 1.0, 4.0, 2.0, 3.0, -1.0, -2.0], np.float32)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_known_answers():
    """tests/MoeRouterSamplerTest.cpp:30-93."""
    idx, w = ol.oracle_select(KNOWN, ol.router_cfg(8, 3))
    assert list(idx) == [1, 3, 5] and w[0] > w[1]
    assert 0.5 < float(w.astype(np.float64).sum()) < 1.0
    denom = np.exp(KNOWN.astype(np.float64) - 5.0).sum()
    assert abs(w[0] - 1.0 / denom) <= 1e-6
    _, wn = ol.oracle_select(KNOWN, ol.router_cfg(8, 3, normalize=True))
    assert abs(float(wn.astype(np.float64).sum()) - 1.0) <= 1e-5
    _, ws = ol.oracle_select(KNOWN, ol.router_cfg(8, 3, scale=2.0))
    assert abs(ws[0] - 2.0 * w[0]) <= 1e-6
    _, wb = ol.oracle_select(KNOWN, ol.router_cfg(8, 3, normalize=True, scale=2.0))
    assert abs(float(wb.astype(np.float64).sum()) - 1.0) <= 1e-5
    ig, _ = ol.oracle_select(KNOWN, ol.router_cfg(8, 2, group_limited=True, n_group=2, topk_group=1))
    assert len(ig) == 2 and all(e < 4 for e in ig)


def test_known_answers_golden():
    g = np.load(os.path.join(GOLDEN, "router_known.npz"))
    variants = {"greedy": ol.router_cfg(8, 3), "normalize": ol.router_cfg(8, 3, normalize=True),
                "scale2": ol.router_cfg(8, 3, scale=2.0), "both": ol.router_cfg(8, 3, normalize=True, scale=2.0),
                "grouped": ol.router_cfg(8, 2, group_limited=True, n_group=2, topk_group=1)}
    for name, cfg in variants.items():
        idx, w = ol.oracle_select(g["logits"], cfg)
        assert np.array_equal(idx, g[f"{name}_index"]), name
        assert np.array_equal(bits(w), bits(g[f"{name}_weight"])), name
    idx, w = ol.oracle_select(g["logits"], ol.router_cfg(8, 3, normalize=True))
    assert np.array_equal(idx, g["legacy_index"]) and np.array_equal(bits(w), bits(g["legacy_weight"]))
    cfg = ol.router_cfg(64, 6)
    for t in range(g["random_logits"].shape[0]):
        idx, w = ol.oracle_select(g["random_logits"][t], cfg)
        assert np.array_equal(idx, g["random_index"][t]), t
        assert np.array_equal(bits(w), bits(g["random_weight"][t])), t


def test_brute_force_order():
    """Selection = full sort by (score desc, index asc) of the oracle softmax."""
    rng = np.random.default_rng(11)
    cfg = ol.router_cfg(64, 6)
    for t in range(300):
        logits = rng.standard_normal(64).astype(np.float32)
        if t % 3 == 0:
            logits = np.round(logits * 2).astype(np.float32)  # many exact ties
        scores = logits.copy()
        ol.oracle().orc_softmax(ol.p(scores), 64)
        order = sorted(range(64), key=lambda e: (-float(scores[e]), e))[:6]
        idx, w = ol.oracle_select(logits, cfg)
        assert list(idx) == order
        assert np.array_equal(bits(w), bits(scores[order]))


def test_v2lite_router_golden():
    """Full-width router (64 x 2048) on 64 seeded tokens: logits, experts and weights."""
    from litemind_amd import workload as wl

    g = np.load(os.path.join(GOLDEN, "router_v2lite.npz"))
    seed, T = int(g["seed"]), int(g["tokens"])
    router = wl.normal_f32(seed, wl.stream_id(0, wl.S_ROUTER), 0.02, (64, 2048))
    x = wl.tokens(seed + 1, T, 2048)
    import hashlib

    assert hashlib.sha256(router.tobytes() + x.tobytes()).hexdigest() == str(g["input_sha"])
    logits = np.zeros((T, 64), np.float32)
    for t in range(T):
        ol.oracle().orc_matvec_f32(ol.p(router), ol.p(np.ascontiguousarray(x[t])), ol.p(logits[t]), 64, 2048)
    assert np.array_equal(bits(logits), bits(g["logits"]))
    cfg = ol.router_cfg(64, 6)
    for t in range(T):
        idx, w = ol.oracle_select(logits[t], cfg)
        assert np.array_equal(idx, g["index"][t]) and np.array_equal(bits(w), bits(g["weight"][t]))


@pytest.mark.skipif(not ol.have_ref(), reason="LiteMind sources not compiled (oracle/_ref)")
def test_router_matches_compiled_reference_random():
    rng = np.random.default_rng(12)
    configs = [ol.router_cfg(64, 6), ol.router_cfg(64, 6, normalize=True), ol.router_cfg(16, 4, scale=2.5),
               ol.router_cfg(64, 6, group_limited=True, n_group=8, topk_group=3),
               ol.router_cfg(12, 3, group_limited=True, n_group=5, topk_group=2),  # 12 % 5 != 0: greedy fallback
               ol.router_cfg(160, 6, group_limited=True, n_group=8, topk_group=3),
               ol.router_cfg(256, 8, normalize=True, group_limited=True, n_group=8, topk_group=4)]
    for cfg in configs:
        for _ in range(100):
            logits = (rng.standard_normal(cfg.expert_count) * 2).astype(np.float32)
            a = ol.oracle_select(logits, cfg)
            b = ol.ref_select(logits, cfg)
            assert np.array_equal(a[0], b[0]) and np.array_equal(bits(a[1]), bits(b[1]))


def test_select_rejects_like_reference():
    """Size mismatch and k = 0 give an empty selection (src/MoeRouter.cpp:56-59)."""
    idx, _ = ol.oracle_select(np.zeros(7, np.float32), ol.router_cfg(8, 3))
    assert len(idx) == 0
    idx, _ = ol.oracle_select(np.zeros(8, np.float32), ol.router_cfg(8, 0))
    assert len(idx) == 0


WIDE_VARIANTS = {"e160": (160, 6, 0, 1.0, 1, 8, 3), "e256": (256, 8, 1, 1.0, 1, 8, 4),
                 "e512": (512, 8, 0, 2.5, 1, 16, 4), "e160_greedy": (160, 6, 0, 1.0, 0, 1, 1)}


def wide_cfg(name):
    E, k, norm, scale, grouped, ng, tg = WIDE_VARIANTS[name]
    return ol.router_cfg(E, k, bool(norm), scale, bool(grouped), ng, tg)


@pytest.mark.parametrize("name", list(WIDE_VARIANTS))
def test_wide_router_golden(name):
    """More than 64 experts with group-limited greedy routing (DeepSeek-V2's 160
    experts in 8 groups, 3 kept; 256 and 512 experts): the oracle against the
    compiled router's outputs (tests/golden/router_wide.npz), ties included."""
    g = np.load(os.path.join(GOLDEN, "router_wide.npz"))
    cfg = wide_cfg(name)
    for t in range(g[f"{name}_logits"].shape[0]):
        idx, w = ol.oracle_select(g[f"{name}_logits"][t], cfg)
        assert np.array_equal(idx, g[f"{name}_index"][t]), (name, t)
        assert np.array_equal(bits(w), bits(g[f"{name}_weight"][t])), (name, t)


def test_wide_router_brute_force_groups():
    """Group-limited selection by its definition (src/MoeRouter.cpp:67-84): each
    group scored by its maximum softmax score, the topk_group best groups (lower
    index on ties) kept, then the best experts of the kept groups, ties to the
    lower index; computed here in float64 order from the oracle's own scores."""
    rng = np.random.default_rng(13)
    E, k, ng, tg = 160, 6, 8, 3
    cfg = ol.router_cfg(E, k, group_limited=True, n_group=ng, topk_group=tg)
    per = E // ng
    for t in range(200):
        logits = (rng.standard_normal(E) * 2).astype(np.float32)
        if t % 2 == 0:
            logits = np.round(logits).astype(np.float32)
        scores = logits.copy()
        ol.oracle().orc_softmax(ol.p(scores), E)
        gmax = [float(scores[g * per:(g + 1) * per].max()) for g in range(ng)]
        kept = sorted(range(ng), key=lambda g: (-gmax[g], g))[:tg]
        allowed = [e for e in range(E) if e // per in kept]
        order = sorted(allowed, key=lambda e: (-float(scores[e]), e))[:k]
        idx, w = ol.oracle_select(logits, cfg)
        assert list(idx) == order
        assert np.array_equal(bits(w), bits(scores[order]))
