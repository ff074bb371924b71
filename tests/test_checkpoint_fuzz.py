"""The SafeTensors reader (litemind_amd/csrc/lm_checkpoint.cpp) under
AddressSanitizer and UndefinedBehaviorSanitizer: a CPU build of the reader
and a mutation fuzzer (litemind_amd/csrc/fuzz_checkpoint.cpp) run over
malformed headers derived from the validation cases of test_checkpoint.py
and from valid files (bit flips, truncation, JSON fragments, rewritten
header lengths).  Every case must return a status; any out-of-bounds access,
use after free or undefined behaviour fails the run."""
import json
import os
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "litemind_amd", "csrc")


def _st(header, payload=b""):
    h = header if isinstance(header, bytes) else header.encode()
    return struct.pack("<Q", len(h)) + h + payload


SEEDS = {
    "valid_bf16": _st(json.dumps({"test.weight": {"dtype": "BF16", "shape": [3], "data_offsets": [0, 6]}}),
                      np.array([0x3F80, 0xC020, 0x3F00], np.uint16).tobytes()),
    "valid_multi": _st(json.dumps({"__metadata__": {"k": "v"},
                                   "a": {"dtype": "F32", "shape": [2, 2], "data_offsets": [0, 16]},
                                   "b": {"dtype": "F16", "shape": [4], "data_offsets": [16, 24]},
                                   "x": {"dtype": "I64", "shape": [1], "data_offsets": [24, 32]}}),
                       np.arange(8, dtype=np.float32).tobytes()),
    "escapes": _st('{"a\\u00e9\\n":{"dtype":"U8","shape":[0],"data_offsets":[0,0]},'
                   '"b":{"dtype":"BOOL","shape":[2],"data_offsets":[0,2]}}', b"\x01\x00"),
    "deep": _st("[" * 100 + "]" * 100),
    "size_mismatch": _st('{"a":{"dtype":"F32","shape":[2],"data_offsets":[0,4]}}', b"\0" * 8),
    "descending": _st('{"a":{"dtype":"U8","shape":[1],"data_offsets":[1,0]}}', b"\0"),
    "past_end": _st('{"a":{"dtype":"BF16","shape":[9999],"data_offsets":[0,19998]}}'),
}


def _have(tool):
    return subprocess.run(["which", tool], stdout=subprocess.DEVNULL).returncode == 0


@pytest.mark.skipif(not _have("g++"), reason="no g++")
def test_reader_under_sanitizers(tmp_path):
    exe = tmp_path / "fuzz_checkpoint"
    # a host-only build (no GPU code): the reader and the fuzzer with ASan + UBSan
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
                    "-I", os.path.join(ROOT, "include"), "-I", CSRC,
                    os.path.join(CSRC, "lm_checkpoint.cpp"), os.path.join(CSRC, "fuzz_checkpoint.cpp"),
                    "-o", str(exe)], check=True, timeout=300)
    seeds = []
    for name, data in SEEDS.items():
        p = tmp_path / f"seed_{name}.bin"
        p.write_bytes(data)
        seeds.append(str(p))
    work = tmp_path / "work"
    work.mkdir()
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    for seed in (1, 2):
        proc = subprocess.run([str(exe), str(work), "15000", str(seed), *seeds], stdout=subprocess.PIPE,
                              stderr=subprocess.STDOUT, text=True, env=env, timeout=300)
        print(proc.stdout[-2000:])
        assert proc.returncode == 0, proc.stdout[-4000:]
        assert "no fault" in proc.stdout
        assert "ERROR: AddressSanitizer" not in proc.stdout and "runtime error" not in proc.stdout
