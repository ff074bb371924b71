"""The whole FFN stack of DeepSeek-V2-Lite at its real depth: the dense layer
0 (intermediate 10944) and 26 MoE layers with independent seeds, all resident
in HBM (59.7 GB with the fp16 copies), chained through RMSNorm (weights 1)
and the residual add by lm_stack_forward, as LiteMind's runner chains the
FFN sublayers (src/DeepSeekRunner.cpp:264-290, attention omitted).

Tokens never mix along this path, so 16 sampled tokens of the 4096-token
batch are run through the oracle's chain, one layer at a time as each layer is
generated (the host copy of a layer is dropped once it is uploaded and the
oracle has advanced the sample through it).  Checks:
  * T = 4096 (grouped MFMA paths, fp16 operands, fp32 accumulation): every
    output finite, and the sampled rows within mean-rel 1e-3 of the oracle's
    chain.  Each layer adds its fp16 rounding differences (~3.6e-4 of the
    layer's output); they pass into the next layer's input and compound over
    27 layers, against a hidden state that grows as the layers' outputs add up.
  * T = 1 (the single-token kernel with the norm and residual fused; fp32
    activations): mean-rel below 1e-5 of the oracle's chain."""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu

MOE_LAYERS = 26
T_BIG = 4096


@pytest.mark.timeout(900)
def test_full_stack_t4096_and_t1():
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims = wl.V2_LITE
    n = 1 + MOE_LAYERS
    h0 = wl.tokens(wl.MASTER_SEED + 11, T_BIG, dims.hidden)
    sample = np.unique(np.concatenate([np.arange(0, T_BIG, 273), [T_BIG - 1]]))
    assert sample.size == 16
    ref = h0[sample].copy()
    ones = np.ones(dims.hidden, np.float32)
    announce(f"full stack: create context for dense + {MOE_LAYERS} MoE layers")
    with Context(dims.moe_config(num_layers=n)) as ctx:
        gate, up, down = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
        ctx.upload_dense(0, gate, up, down)
        ctx.finalize_layer(0)
        ctx.upload_norm(0, ones)
        ref = ol.oracle_stack([("dense", (gate, up, down))], ref, dims.rms_norm_eps)
        del gate, up, down
        for l in range(1, n):
            L = wl.moe_layer(wl.MASTER_SEED, l, dims)
            wl.upload_moe_layer(ctx, l, L)
            ctx.upload_norm(l, ones)
            ref = ol.oracle_stack([("moe", L)], ref, dims.rms_norm_eps)
            del L
            print(f"[full-stack] layer {l} uploaded, oracle sample advanced", flush=True)
        resident = ctx.resident_bytes()
        print(f"[full-stack] resident {resident / 1e9:.2f} GB", flush=True)
        assert resident > 55e9

        announce(f"full stack: lm_stack_forward T={T_BIG} over {n} layers")
        dh = ctx.to_device(h0)
        ctx.stack_forward(0, n - 1, dh, T_BIG)
        ctx.synchronize()
        out = dh.download()
        dh.free()
        assert np.all(np.isfinite(out))
        max_abs, mean_rel = layer_error(out[sample], ref)
        print(f"[full-stack] T={T_BIG} sampled rows: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e} "
              f"(|h| mean {np.abs(ref).mean():.3f})", flush=True)
        assert mean_rel <= MEAN_REL

        t0 = int(sample[0])
        announce(f"full stack: lm_stack_forward T=1 (token {t0}) over {n} layers")
        d1 = ctx.to_device(h0[t0:t0 + 1])
        ctx.stack_forward(0, n - 1, d1, 1)
        ctx.synchronize()
        one = d1.download()
        d1.free()
        assert np.all(np.isfinite(one))
        max_abs, mean_rel = layer_error(one, ref[:1])
        print(f"[full-stack] T=1: max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}", flush=True)
        assert mean_rel < 1e-5
