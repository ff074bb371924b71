"""The C ABI library loads and exports every entry point include/*.h declares
(no GPU calls)."""
import glob
import os
import re
import subprocess

import litemind_amd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def declared():
    names = set()
    for h in HEADERS:
        names.update(re.findall(r"^(?:int|const char\*)\s+(lm_[a-z0-9_]+)\(", open(h).read(), re.M))
    return sorted(names)


def test_header_declares_the_abi():
    names = declared()
    assert "lm_moe_forward" in names and "lm_last_error" in names and len(names) >= 30
    assert "lm_attention_forward" in names and "lm_kv_cache_read" in names


def test_library_exports_every_declared_symbol():
    lib = litemind_amd.load_library()
    out = subprocess.run(["nm", "-D", "--defined-only", litemind_amd.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = set(line.split()[-1] for line in out.splitlines() if line.strip())
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing
    for n in declared():
        getattr(lib, n)


def test_python_binding_covers_the_abi():
    assert set(declared()) == set(litemind_amd.PROTOTYPES)


def test_last_error_is_callable_without_gpu():
    lib = litemind_amd.load_library()
    assert isinstance(lib.lm_last_error(), bytes)
    assert lib.lm_version(None, None) == 0
