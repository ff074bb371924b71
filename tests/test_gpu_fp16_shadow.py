"""The fp16 copy of a layer's BF16 weights (the MFMA path's operands):
lm_finalize_layer counts the weights it cannot hold exactly (BF16 magnitudes
below 2^-17 round to fp16 subnormals) and lm_layer_fp16_inexact reports them;
weights beyond the fp16 range make the finalize fail.  The expected count is
numpy's round-to-nearest-even fp16 conversion of every uploaded weight."""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def _f32(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def _bf16(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


def _lossy(bits):
    v = _f32(bits)
    return int(np.count_nonzero(v.astype(np.float16).astype(np.float32) != v))


def _layer(seed):
    from litemind_amd import workload as wl

    dims = wl.Dims(hidden=128, inter=64, experts=8, top_k=2, n_shared=1, dense_inter=0)
    return dims, wl.moe_layer(seed, 0, dims)


def test_fp16_inexact_count():
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims, L = _layer(5)
    rng = np.random.default_rng(9)
    # plant small weights: below 2^-17 (rounded), at 2^-17 and 2^-15 (exact)
    planted = [3e-6, -1e-7, 7.4e-6, 2.0 ** -17, -(2.0 ** -15), 1e-30]
    for mats in (L.gate, L.down):
        for e in (1, 6):
            flat = mats[e].reshape(-1)
            pos = rng.choice(flat.size, len(planted), replace=False)
            flat[pos] = _bf16(planted)
    L.shared_up.reshape(-1)[:3] = _bf16([1e-6, 2e-6, 5e-6])
    want = sum(_lossy(m) for mats in (L.gate, L.up, L.down) for m in mats)
    want += sum(_lossy(m) for m in (L.shared_gate, L.shared_up, L.shared_down))
    announce(f"fp16 copy: {want} rounded weights expected")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        wl.upload_moe_layer(ctx, 0, L)
        got = ctx.layer_fp16_inexact(0)
    assert want >= 2 * 2 * 4 + 3  # the planted ones below 2^-17 at least
    assert got == want


def test_fp16_overflow_refused():
    from litemind_amd import Context, LmError

    dims, L = _layer(6)
    L.up[3].reshape(-1)[17] = _bf16([70000.0])[0]
    announce("fp16 copy: a weight beyond the fp16 range")
    with Context(dims.moe_config(num_layers=1)) as ctx:
        ctx.upload_router(0, L.router)
        for e in range(dims.experts):
            ctx.upload_expert(0, e, L.gate[e], L.up[e], L.down[e])
        ctx.upload_shared(0, L.shared_gate, L.shared_up, L.shared_down)
        with pytest.raises(LmError, match="fp16 range"):
            ctx.finalize_layer(0)
        with pytest.raises(LmError):
            ctx.layer_fp16_inexact(0)  # not finalized
