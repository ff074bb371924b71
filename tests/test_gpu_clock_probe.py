"""lm_clock_probe_*: the core clock sampled by one wave on a stream of its own
while layers run on the context stream (the bench's clock reading).  The
reading must be a plausible engine clock (MI355X runs up to 2400 MHz), cover
the run with intervals, and the entry points must refuse misuse."""
import numpy as np
import pytest

from conftest import announce

pytestmark = pytest.mark.gpu


def test_clock_probe_reads_a_plausible_clock(v2_ctx):
    from litemind_amd import LmError
    from litemind_amd import workload as wl

    ctx, _ = v2_ctx
    announce("clock probe over 40 single-token layers")
    x = wl.tokens(wl.MASTER_SEED + 91, 1, 2048)
    dx, dy = ctx.to_device(x), ctx.empty((1, 2048))
    ctx.clock_probe_start(0.02)
    for _ in range(40):
        ctx.moe_forward(0, dx, 1, dy)
    ctx.synchronize()
    r = ctx.clock_probe_finish()
    dx.free()
    dy.free()
    print(r)
    assert r["intervals"] >= 500  # 20 ms of 20 us intervals
    assert 300.0 <= r["min_mhz"] <= r["mhz"] <= r["max_mhz"] <= 3000.0
    with pytest.raises(LmError):
        ctx.clock_probe_finish()  # none running
    with pytest.raises(LmError):
        ctx.clock_probe_start(3.0)  # longer than 2 s
    ctx.clock_probe_start(0.001)
    with pytest.raises(LmError):
        ctx.clock_probe_start(0.001)  # one at a time
    assert ctx.clock_probe_finish()["intervals"] >= 1
