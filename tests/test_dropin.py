"""The C++20 drop-in layer (litemind_amd/host): ExpertCache bookkeeping on the CPU.

ExpertCache keeps LiteMind's LRU policy and counters (src/ExpertCache.cpp:5-76);
only what residency means changes (HBM instead of the page cache).  The demo's
cache-trace mode replays the touch sequence of tests/golden/expert_cache_trace.json
with byte-less views, which never reach the GPU, and every counter after every
touch must equal what LiteMind's own ExpertCache reported.
"""
import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEMO = os.path.join(ROOT, "litemind_amd", "bin", "dropin_demo")
GOLDEN = os.path.join(ROOT, "tests", "golden", "expert_cache_trace.json")


def _trace(budget, block, touches):
    args = [DEMO, "cache-trace", str(budget), str(block)]
    for layer, expert in touches:
        args += [str(layer), str(expert)]
    out = subprocess.run(args, check=True, capture_output=True, text=True, timeout=60).stdout
    return [[int(v) for v in line.split()] for line in out.strip().splitlines()]


@pytest.mark.skipif(not os.path.exists(DEMO), reason="dropin_demo not built")
@pytest.mark.parametrize("run", ["budget3", "storm", "disabled", "budget5"])
def test_expert_cache_counters_match_litemind(run):
    g = json.load(open(GOLDEN))
    r = g["runs"][run]
    rows = _trace(r["budget"], g["block_bytes"], g["touches"])
    assert rows == r["counters"]


@pytest.mark.skipif(not os.path.exists(DEMO), reason="dropin_demo not built")
def test_expert_cache_invariants():
    """Budget never exceeded after a touch (unless one block alone exceeds it),
    loads + hits = touches, evictions = loads - resident."""
    block = 3 * 1408 * 2048 * 2
    touches = [(l, e) for l in range(3) for e in (0, 1, 2, 0, 5, 1)]
    for budget_blocks in (1, 2, 4, 100):
        rows = _trace(budget_blocks * block, block, touches)
        for i, (resident, n_res, loads, hits, evictions, streamed, enabled) in enumerate(rows[:-1]):
            assert resident <= budget_blocks * block
            assert loads + hits == i + 1
            assert evictions == loads - n_res
            assert streamed == loads * block and enabled == 1
        assert rows[-1][:2] == [0, 0]
