import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running CPU test")


def pytest_collection_modifyitems(config, items):
    # GPU tests print the case before each GPU step; keep their order stable.
    pass


# MoE layer tolerance of the north star: max-abs 2e-2 and mean-rel 1e-3, with
# mean-rel defined as the aggregate relative L1 error sum|d| / sum|ref|.
MAX_ABS = 2e-2
MEAN_REL = 1e-3


def layer_error(y: np.ndarray, ref: np.ndarray):
    d = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    return float(d.max()), float(d.sum() / max(np.abs(ref.astype(np.float64)).sum(), 1e-30))


@pytest.fixture(scope="session")
def v2_layer():
    from litemind_amd import workload as wl

    return wl.moe_layer(wl.MASTER_SEED, 0)


@pytest.fixture(scope="session")
def tiny_layer():
    from litemind_amd import workload as wl

    return wl.tiny_model_layers(1)


def announce(msg: str) -> None:
    """Names the GPU case before its GPU step runs (flushed, so a fault still shows it)."""
    print(f"[gpu-case] {msg}", flush=True)


@pytest.fixture(scope="session")
def v2_ctx(v2_layer):
    """A context holding layer 0 (id 0) and layer 0 with its router gate scaled by
    1e-2 (id 1, the near-uniform routing of the T=512 workload)."""
    from litemind_amd import Context
    from litemind_amd import workload as wl

    announce("create V2-Lite context and upload 2 layers")
    ctx = Context(wl.V2_LITE.moe_config(num_layers=2))
    wl.upload_moe_layer(ctx, 0, v2_layer)
    scaled = wl.MoeLayer(v2_layer.dims, (v2_layer.router.astype(np.float64) * 1e-2).astype(np.float32),
                         v2_layer.gate, v2_layer.up, v2_layer.down, v2_layer.shared_gate, v2_layer.shared_up,
                         v2_layer.shared_down)
    wl.upload_moe_layer(ctx, 1, scaled)
    yield ctx, {0: v2_layer, 1: scaled}
    ctx.close()


@pytest.fixture(scope="session")
def tiny_ctx(tiny_layer):
    from litemind_amd import Context
    from litemind_amd import workload as wl

    dims, layer = tiny_layer
    announce("create tiny-model context")
    ctx = Context(dims.moe_config(num_layers=1))
    wl.upload_moe_layer(ctx, 0, layer)
    yield ctx, layer
    ctx.close()
