"""LiteMind's own unit tests, run against the GPU drop-in.

oracle/_ref/KernelTest_gpu and MoeRouterSamplerTest_gpu are LiteMind's
tests/KernelTest.cpp and tests/MoeRouterSamplerTest.cpp compiled unchanged from
its sources (`make -C oracle ref-tests`), linked with this library's Gemm,
MoeRouter and ExpertCache sources and liblitemind_moe.so in place of LiteMind's
CPU kernels.  Every gemm:: and MoeRouter call they make runs on the GPU, and
every check they contain must pass.
"""
import os
import subprocess

import pytest

from conftest import announce

pytestmark = pytest.mark.gpu

REF = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "_ref")


@pytest.mark.parametrize("name", ["KernelTest_gpu", "MoeRouterSamplerTest_gpu"])
def test_litemind_unit_test_passes_on_gpu(name):
    exe = os.path.join(REF, name)
    if not os.path.exists(exe):
        pytest.skip(f"{name} not built (needs the LiteMind sources: make -C oracle ref-tests)")
    announce(f"LiteMind {name}")
    proc = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    print(proc.stderr)
    assert proc.returncode == 0, proc.stderr
    assert "all checks passed" in proc.stdout
    if name == "KernelTest_gpu":
        assert "gfx950" in proc.stdout  # gemm::kernel_description() comes from the drop-in
