"""Builds the native parts of litemind_amd in-tree.

  litemind_amd/liblitemind_moe.so   gfx950 HIP kernels + the C ABI (include/litemind_moe.h)
  litemind_amd/libsynth.so          host generator of the seeded synthetic workloads
  litemind_amd/bin/dropin_demo      C++20 drop-in wrappers exercised like LiteMind's runner
  oracle/liboracle.so               CPU oracle (test infrastructure)
  oracle/_ref/libref.so             LiteMind's own sources, where the source tree is present
  oracle/_ref/*_gpu                 LiteMind's own unit tests linked against the GPU drop-in

Every call recompiles.  Run:  python -m litemind_amd.build
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
HOST = os.path.join(HERE, "host")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
REFERENCE = os.environ.get("LITEMIND_REFERENCE", "/root/reference")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_SOURCES = ["k_router.hip", "k_permute.hip", "k_gemv.hip", "k_decode.hip", "k_mfma.hip",
               "k_misc.hip", "k_head.hip", "k_attn.hip", "k_spec.hip", "lm_capi.hip", "lm_attn.hip"]
# Host-only parts of the same library (no device code), compiled by g++.
HOST_SOURCES = ["lm_checkpoint.cpp"]
# -ffp-contract=off: every fused multiply-add in the kernels is written out
# explicitly; the router must not fuse at all to match LiteMind bit for bit.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 generated from float code.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", INCLUDE, "-I", CSRC, "-Wall", "-Wno-unused-command-line-argument",
]
HOST_FLAGS = ["-O3", "-march=x86-64-v3", "-std=c++20", "-fPIC", "-pthread", "-Wall", "-Wextra"]


def _run(cmd: list[str], cwd: str | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; that warning is harmless.
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        sys.stderr.write(out + "\n")


def build_hip(jobs: int = 6) -> str:
    os.makedirs(BUILD, exist_ok=True)
    objects = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD, src.replace(".hip", ".o"))
        objects.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    for src in HOST_SOURCES:
        obj = os.path.join(BUILD, src.replace(".cpp", ".o"))
        objects.append(obj)
        cmds.append(["g++", *HOST_FLAGS, "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj])
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, c) for c in cmds]:
            fut.result()
    lib = os.path.join(HERE, "liblitemind_moe.so")
    tmp = lib + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objects])
    os.replace(tmp, lib)
    return lib


def build_synth() -> str:
    lib = os.path.join(HERE, "libsynth.so")
    tmp = lib + ".tmp"
    _run(["g++", *HOST_FLAGS, "-fopenmp", "-shared", "-I", CSRC, "-o", tmp, os.path.join(CSRC, "synth.cpp")])
    os.replace(tmp, lib)
    return lib


def build_dropin() -> str | None:
    """C++20 drop-in wrappers (MoeRouter / gemm / ExpertCache / MoeBlockGpu) and their demo program."""
    demo_src = os.path.join(HOST, "dropin_demo.cpp")
    if not os.path.exists(demo_src):
        return None
    src_dir = os.path.join(HOST, "src")
    srcs = [os.path.join(src_dir, f) for f in sorted(os.listdir(src_dir)) if f.endswith(".cpp")]
    bindir = os.path.join(HERE, "bin")
    os.makedirs(bindir, exist_ok=True)
    exe = os.path.join(bindir, "dropin_demo")
    # host/include: what the drop-in adds; host/litemind_api: LiteMind's interfaces
    # (inside LiteMind its own include/ takes this place)
    _run(["g++", *HOST_FLAGS, "-I", os.path.join(HOST, "include"), "-I", os.path.join(HOST, "litemind_api"),
          "-I", INCLUDE, "-o", exe + ".tmp", demo_src,
          *srcs, "-L", HERE, "-llitemind_moe", "-Wl,-rpath,$ORIGIN/..", "-pthread"])
    os.replace(exe + ".tmp", exe)
    return exe


def build_oracle() -> None:
    _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "-B", "liboracle.so"])
    if os.path.isdir(os.path.join(REFERENCE, "src")):
        _run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "-B", "ref", f"REF={REFERENCE}"])


def build_ref_tests() -> None:
    """LiteMind's own KernelTest / MoeRouterSamplerTest / AttentionTest / RopeTest and its whole runner
    (DeepSeekRunner through oracle/runner_driver.cpp) linked against the GPU drop-in, and the runner over
    LiteMind's own sources as the CPU reference."""
    if os.path.isdir(os.path.join(REFERENCE, "tests")):
        _run(["make", "-s", "-j4", "-C", os.path.join(ROOT, "oracle"), "-B", "ref-tests", f"REF={REFERENCE}"])


def build_all() -> None:
    build_oracle()
    build_synth()
    build_hip()
    build_dropin()
    build_ref_tests()


if __name__ == "__main__":
    build_all()
    print("built:", os.path.join(HERE, "liblitemind_moe.so"))
