"""lm_grouped_swiglu, the grouped SwiGLU stage alone: for a routing [T, k], the
down projection of every (token, expert) assignment and of the shared expert,
before routing weights and combine.  Each row is checked against LiteMind's
feed_forward for that one token and expert (src/DeepSeekRunner.cpp:228-240:
matvec_bf16 gate and up, silu_multiply, matvec_bf16 down), composed from the
oracle's restatement of those kernels (orc_dense_ffn runs exactly that
sequence into a zeroed output, i.e. scale 1).

GEMV path (fp32 activations): within 1e-5 relative of the oracle (its dot
products keep LiteMind's association only per lane group).  MFMA path (fp16
operands, fp32 accumulation): the layer bar, max-abs 2e-2 and mean-rel 1e-3.
At T = 2048 (skewed routing) a sample of 48 tokens is checked, all their
assignments and shared rows."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu


def _reference_rows(layer, x, idx, tokens):
    """FFN output of every (t, r) assignment of `tokens`, and their shared rows."""
    K = idx.shape[1]
    routed = np.zeros((len(tokens), K, x.shape[1]), np.float32)
    by_expert = {}
    for i, t in enumerate(tokens):
        for r in range(K):
            by_expert.setdefault(int(idx[t, r]), []).append((i, r, t))
    for e, items in by_expert.items():
        rows = np.stack([x[t] for _, _, t in items])
        y = ol.oracle_dense(layer.gate[e], layer.up[e], layer.down[e], rows)
        for (i, r, _), v in zip(items, y):
            routed[i, r] = v
    shared = ol.oracle_dense(layer.shared_gate, layer.shared_up, layer.shared_down, x[tokens])
    return routed, shared


@pytest.mark.parametrize("case", ["t32_gemv", "t32_mfma", "t512_uniform", "t2048_skewed"])
def test_grouped_swiglu_rows(v2_ctx, case):
    from litemind_amd import PATH_AUTO, PATH_GEMV, PATH_MFMA
    from litemind_amd import workload as wl

    ctx, layers = v2_ctx
    T = {"t32_gemv": 32, "t32_mfma": 32, "t512_uniform": 512, "t2048_skewed": 2048}[case]
    path = {"t32_gemv": PATH_GEMV, "t32_mfma": PATH_MFMA}.get(case, PATH_AUTO)
    layer_id = 1 if case == "t512_uniform" else 0
    layer = layers[layer_id]
    bias = wl.skew_bias() if case == "t2048_skewed" else None
    H, K = 2048, ctx.config.num_experts_per_tok
    x = wl.tokens(wl.MASTER_SEED + 900 + T, T, H)
    announce(f"grouped SwiGLU {case}: routing")
    dx = ctx.to_device(x)
    db = ctx.to_device(bias) if bias is not None else None
    didx, dw = ctx.empty((T, K), np.int32), ctx.empty((T, K))
    ctx.router(layer_id, dx, T, didx, dw, bias=db)
    ctx.synchronize()
    idx = didx.download()
    announce(f"grouped SwiGLU {case}: lm_grouped_swiglu")
    dout = ctx.empty((T * K + T, H))
    ctx.grouped_swiglu(layer_id, dx, T, didx, dout, path=path)
    ctx.synchronize()
    out = dout.download()
    for b in (dx, didx, dw, dout) + ((db,) if db is not None else ()):
        b.free()
    assert np.all(np.isfinite(out))
    tokens = np.arange(T) if T <= 512 else np.unique(np.concatenate([np.arange(0, T, 43), [T - 1]]))
    routed, shared = _reference_rows(layer, x, idx, tokens)
    got_routed = out[:T * K].reshape(T, K, H)[tokens]
    got_shared = out[T * K:][tokens]
    if T == 2048:
        counts = np.bincount(idx.ravel(), minlength=64)
        print(f"hottest expert {counts.max()} rows, coldest {counts.min()}")
    for name, got, ref in (("routed", got_routed, routed), ("shared", got_shared, shared)):
        max_abs, mean_rel = layer_error(got, ref)
        exact = float(np.mean(got.view(np.uint32) == ref.view(np.uint32)))
        print(f"{case} {name}: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e} bit-identical {exact:.4f}")
        if path == PATH_GEMV:
            assert mean_rel < 1e-5
        else:
            assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL


def test_grouped_swiglu_matches_moe_forward(v2_ctx):
    """Weighting the stage's rows by the router's weights in rank order and
    adding the shared row (the combine, done here in float64) reproduces
    lm_moe_forward's output on the same path to float rounding."""
    from litemind_amd import PATH_MFMA
    from litemind_amd import workload as wl

    ctx, _ = v2_ctx
    T, H, K = 64, 2048, ctx.config.num_experts_per_tok
    x = wl.tokens(wl.MASTER_SEED + 977, T, H)
    announce("grouped SwiGLU T=64 against lm_moe_forward")
    dx = ctx.to_device(x)
    didx, dw, dy = ctx.empty((T, K), np.int32), ctx.empty((T, K)), ctx.empty((T, H))
    ctx.moe_forward(0, dx, T, dy, idx=didx, w=dw, path=PATH_MFMA)
    dout = ctx.empty((T * K + T, H))
    ctx.grouped_swiglu(0, dx, T, didx, dout, path=PATH_MFMA)
    ctx.synchronize()
    y, w, out = dy.download(), dw.download(), dout.download()
    for b in (dx, didx, dw, dy, dout):
        b.free()
    routed = out[:T * K].reshape(T, K, H).astype(np.float64)
    combined = (routed * w[:, :, None].astype(np.float64)).sum(axis=1) + out[T * K:]
    d = np.abs(combined - y)
    assert d.max() <= 1e-5 * max(1.0, np.abs(y).max())


def test_grouped_swiglu_rejects_bad_expert_ids(v2_ctx):
    """An expert id outside [0, E) is refused before any launch (the
    permutation would leave its slot unset)."""
    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, _ = v2_ctx
    T, H, K = 4, 2048, ctx.config.num_experts_per_tok
    announce("grouped SwiGLU with an expert id of 64 (refused on the host)")
    idx = np.tile(np.arange(K, dtype=np.int32), (T, 1))
    idx[2, 3] = 64
    dx, didx, dout = ctx.to_device(wl.tokens(5, T, H)), ctx.to_device(idx), ctx.empty((T * K + T, H))
    with pytest.raises(LmError, match="not an expert"):
        ctx.grouped_swiglu(0, dx, T, didx, dout)
    for b in (dx, didx, dout):
        b.free()
