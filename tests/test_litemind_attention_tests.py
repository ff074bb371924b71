"""LiteMind's own AttentionTest and RopeTest against the attention drop-in.

oracle/_ref/AttentionTest_gpu and RopeTest_gpu are LiteMind's
tests/AttentionTest.cpp and tests/RopeTest.cpp compiled unchanged from its
sources (`make -C oracle ref-tests`) with this library's Attention, KvCache and
Rope sources and liblitemind_moe.so in place of LiteMind's: the KvCache checks
run on the drop-in's cache, the RotaryEmbedding checks on tables built by the
library (lm_rope_tables).  Neither reaches the GPU (the drop-in touches it only
in Attention::forward), so both run on the CPU; every check they contain must
pass.
"""
import os
import subprocess

import pytest

REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref")


@pytest.mark.parametrize("name", ["AttentionTest_gpu", "RopeTest_gpu"])
def test_litemind_attention_unit_test_passes(name):
    exe = os.path.join(REF, name)
    if not os.path.exists(exe):
        pytest.skip(f"{name} not built (needs the LiteMind sources: make -C oracle ref-tests)")
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stderr
    assert "all checks passed" in proc.stdout
