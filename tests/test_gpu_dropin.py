"""The drop-in layer on the GPU: LiteMind's MoE block composed from the drop-in
gemm::, MoeRouter and ExpertCache (litemind_amd/host/dropin_demo.cpp), token by
token as src/DeepSeekRunner.cpp:273-290 does, must reproduce LiteMind's result bit
for bit (the oracle restates that composition and is itself pinned to LiteMind's
compiled sources); the batched MoeBlockGpu path on the same tokens routes
identically and stays within the layer tolerance."""
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEMO = os.path.join(ROOT, "litemind_amd", "bin", "dropin_demo")


def write_case(d, layer, x, budget_experts):
    dims = layer.dims
    S = dims.shared_inter if layer.shared_gate is not None else 0
    with open(os.path.join(d, "case.txt"), "w") as f:
        f.write(f"{dims.hidden} {dims.inter} {dims.experts} {dims.top_k} {S} {x.shape[0]} "
                f"{1 if dims.norm_topk_prob else 0} {dims.routed_scaling_factor!r} {budget_experts}\n")
    layer.router.astype(np.float32).tofile(os.path.join(d, "router.f32"))
    np.stack(layer.gate).tofile(os.path.join(d, "gate.bf16"))
    np.stack(layer.up).tofile(os.path.join(d, "up.bf16"))
    np.stack(layer.down).tofile(os.path.join(d, "down.bf16"))
    if S:
        layer.shared_gate.tofile(os.path.join(d, "shared_gate.bf16"))
        layer.shared_up.tofile(os.path.join(d, "shared_up.bf16"))
        layer.shared_down.tofile(os.path.join(d, "shared_down.bf16"))
    np.ascontiguousarray(x, dtype=np.float32).tofile(os.path.join(d, "x.f32"))


def run_case(d, name, layer, x, budget_experts):
    write_case(d, layer, x, budget_experts)
    announce(f"dropin_demo moe {name} T={x.shape[0]} budget={budget_experts} experts")
    subprocess.run([DEMO, "moe", str(d)], check=True, timeout=240)
    T, K, H = x.shape[0], layer.dims.top_k, layer.dims.hidden

    def load(n, dt, shape):
        return np.fromfile(os.path.join(d, n), dtype=dt).reshape(shape)

    out = {k: load(f"{k}.f32", np.float32, (T, H)) for k in ("y_token", "y_batch")}
    for k in ("index_token", "index_batch"):
        out[k] = load(f"{k}.i32", np.int32, (T, K))
    for k in ("weight_token", "weight_batch"):
        out[k] = load(f"{k}.f32", np.float32, (T, K))
    out["cache"] = [int(v) for v in open(os.path.join(d, "cache.txt")).read().split()]
    return out


def check(out, layer, x, budget_experts):
    oy, oidx, ow, _ = ol.oracle_moe_layer(layer, x)
    T, K = oidx.shape
    for path in ("token", "batch"):
        assert np.array_equal(out[f"index_{path}"], oidx), path
        assert np.array_equal(out[f"weight_{path}"].view(np.uint32), ow.view(np.uint32)), path
    # per-token drop-in: LiteMind's own arithmetic, bit for bit
    assert np.array_equal(out["y_token"].view(np.uint32), oy.view(np.uint32))
    max_abs, mean_rel = layer_error(out["y_batch"], oy)
    print(f"batched max_abs={max_abs:.3e} mean_rel={mean_rel:.3e}")
    assert max_abs <= MAX_ABS and mean_rel <= MEAN_REL
    resident, n_res, loads, hits, evictions, streamed, enabled = out["cache"]
    if budget_experts:
        assert enabled == 1 and loads + hits == T * K
        assert n_res <= budget_experts and evictions == loads - n_res
    else:
        assert enabled == 0 and loads == hits == 0


@pytest.mark.skipif(not os.path.exists(DEMO), reason="dropin_demo not built")
def test_dropin_tiny_layer(tmp_path, tiny_layer):
    from litemind_amd import workload as wl

    dims, layer = tiny_layer
    x = wl.tokens(31, 9, dims.hidden)
    for budget in (0, 2):
        d = tmp_path / f"tiny{budget}"
        d.mkdir()
        check(run_case(d, "tiny", layer, x, budget), layer, x, budget)


@pytest.mark.skipif(not os.path.exists(DEMO), reason="dropin_demo not built")
def test_dropin_v2lite_layer(tmp_path, v2_layer):
    from litemind_amd import workload as wl

    x = wl.tokens(wl.MASTER_SEED + 77, 2, 2048)
    check(run_case(tmp_path, "v2lite", v2_layer, x, 4), v2_layer, x, 4)


@pytest.mark.skipif(not os.path.exists(DEMO), reason="dropin_demo not built")
def test_dropin_reports_kernel_timeout(tmp_path, tiny_layer):
    """gpu::MoeBlockGpu::forward throws with the library's LM_EKERNEL message
    when the single-token kernel's waits give up (forced from the host with
    lm_decode_wait_test), and works again once they no longer do."""
    from litemind_amd import workload as wl

    dims, layer = tiny_layer
    x = wl.tokens(37, 1, dims.hidden)
    write_case(tmp_path, layer, x, 0)
    announce("dropin_demo moe-timeout tiny T=1")
    proc = subprocess.run([DEMO, "moe-timeout", str(tmp_path)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                          text=True, timeout=240)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout
    assert "LM_EKERNEL reported" in proc.stdout
