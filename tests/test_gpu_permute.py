"""The GPU permutation must equal the canonical one (expert-major, then token,
then rank) exactly, including empty and overloaded experts."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import announce

pytestmark = pytest.mark.gpu


def _gpu_permute(ctx, idx, experts):
    T, K = idx.shape
    d_idx = ctx.to_device(idx)
    counts, offsets = ctx.empty(experts, np.int32), ctx.empty(experts + 1, np.int32)
    perm, slot_of = ctx.empty(T * K, np.int32), ctx.empty(T * K, np.int32)
    ctx.permute(d_idx, T, counts, offsets, perm, slot_of)
    ctx.synchronize()
    out = counts.download(), offsets.download(), perm.download(), slot_of.download()
    for b in (d_idx, counts, offsets, perm, slot_of):
        b.free()
    return out


def _distinct_topk(rng, T, E, K, p=None):
    return np.stack([rng.choice(E, size=K, replace=False, p=p) for _ in range(T)]).astype(np.int32)


# Segments of 1,024 assignments: one partial (1, 7, 32: the single-launch
# kernel; 170: 1,020 assignments), several with a ragged last one (171: 1,026
# assignments; 1000), whole ones (2048, 4096).
@pytest.mark.parametrize("T", [1, 7, 32, 170, 171, 1000, 2048, 4096])
def test_permute_matches_canonical(v2_ctx, T):
    ctx, _ = v2_ctx
    rng = np.random.default_rng(T)
    idx = _distinct_topk(rng, T, 64, 6)
    announce(f"permute random T={T}")
    g = _gpu_permute(ctx, idx, 64)
    o = ol.oracle_permute(idx, 64)
    for a, b in zip(g, o):
        assert np.array_equal(a, b)


def test_permute_skewed_and_empty(v2_ctx):
    ctx, _ = v2_ctx
    rng = np.random.default_rng(3)
    p = np.zeros(64)
    p[:8] = 0.9 / 8
    p[8:12] = 0.1 / 4          # experts 12..63 never chosen
    idx = _distinct_topk(rng, 2048, 64, 6, p)
    announce("permute skewed with empty experts T=2048")
    g = _gpu_permute(ctx, idx, 64)
    o = ol.oracle_permute(idx, 64)
    for a, b in zip(g, o):
        assert np.array_equal(a, b)
    counts, offsets, perm, slot_of = g
    assert counts[12:].sum() == 0
    # bijection and stability inside each bucket
    assert np.array_equal(np.sort(perm), np.arange(2048 * 6))
    assert np.array_equal(slot_of[perm], np.arange(2048 * 6))
    for e in range(12):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(seg) > 0)


@pytest.mark.parametrize("E,T", [(64, 150), (160, 100)])
def test_permute_single_segment_skewed(v2_ctx, E, T):
    """One segment (the single-launch kernel) with empty experts, over 64 and
    160 experts."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    rng = np.random.default_rng(E + T)
    p = np.zeros(E)
    p[:6] = 0.8 / 6
    p[6:10] = 0.2 / 4          # experts 10.. never chosen
    idx = _distinct_topk(rng, T, E, 6, p)
    announce(f"permute single segment skewed E={E} T={T}")
    if E == 64:
        ctx, _ = v2_ctx
        g = _gpu_permute(ctx, idx, E)
    else:
        dims = wl.Dims(hidden=16, inter=16, experts=E, top_k=6, n_shared=0, dense_inter=0)
        with Context(dims.moe_config(num_layers=1)) as c:
            g = _gpu_permute(c, idx, E)
    o = ol.oracle_permute(idx, E)
    for a, b in zip(g, o):
        assert np.array_equal(a, b)
    assert g[0][10:].sum() == 0
