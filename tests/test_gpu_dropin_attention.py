"""The attention drop-in on the GPU: LiteMind's Attention / KvCache /
RotaryEmbedding interfaces (litemind_amd/host/src/Attention.cpp, KvCache.cpp,
Rope.cpp) driven by litemind_amd/bin/dropin_demo as DeepSeekRunner drives them
(src/DeepSeekRunner.cpp:251-262, :358-360, :416-437): one Attention over
several layers' caches and weights, token by token.  Every output row and
every cached entry must equal LiteMind's compiled Attention::forward
(oracle/_ref/libref.so) bit for bit, or the oracle's restatement of it (itself
pinned to the compiled one) where libref.so is absent.  The script also covers
what the device copy of a cache must follow: KvCache::clear (host only, inline)
then a restart at position 0, a cache filled by hand through the writable
accessors then continued on the GPU, a full cache (forward returns false and
writes nothing), and positions past the rotary table."""
import dataclasses
import os
import subprocess

import numpy as np
import pytest

import oracle_lib as ol
from conftest import announce

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEMO = os.path.join(ROOT, "litemind_amd", "bin", "dropin_demo")
CAP = 12  # KvCache capacity and rotary table positions


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def dims(q_lora):
    from litemind_amd import workload as wl
    return dataclasses.replace(wl.V2_LITE_MLA, hidden=256, heads=4, kv_lora_rank=64, qk_nope=32, qk_rope=16,
                               v_head=32, original_max=16, factor=4.0, max_positions=CAP, q_lora_rank=q_lora)


def write_case(d, D, sets, x, script):
    with open(os.path.join(d, "case.txt"), "w") as f:
        f.write(f"{D.hidden} {D.heads} {D.q_lora_rank} {D.kv_lora_rank} {D.qk_nope} {D.qk_rope} {D.v_head} 4 {CAP} "
                f"{D.rms_norm_eps!r} {float(D.rope_theta)!r} {1 if D.yarn else 0} {float(D.factor)!r} "
                f"{float(D.beta_fast)!r} {float(D.beta_slow)!r} {float(D.mscale)!r} {float(D.mscale_all_dim)!r} "
                f"{int(D.original_max)} {len(sets)} 4 {x.shape[0]}\n")
    for i, L in enumerate(sets):
        w = os.path.join(d, f"w{i}_")
        if D.q_lora_rank == 0:
            L.q_proj.tofile(w + "q.bf16")
        else:
            L.q_a_proj.tofile(w + "qa.bf16")
            L.q_a_layernorm.astype(np.float32).tofile(w + "qan.f32")
            L.q_b_proj.tofile(w + "qb.bf16")
        L.kv_a_proj.tofile(w + "kva.bf16")
        L.kv_a_layernorm.astype(np.float32).tofile(w + "kvan.f32")
        L.kv_b_proj.tofile(w + "kvb.bf16")
        L.o_proj.tofile(w + "o.bf16")
    np.ascontiguousarray(x, np.float32).tofile(os.path.join(d, "x.f32"))
    with open(os.path.join(d, "script.txt"), "w") as f:
        f.write("\n".join(script) + "\n")


def expected(layer, x, pos0):
    """LiteMind's Attention::forward over the rows of x from an empty cache of
    CAP positions (rotary table CAP rows): (out, done, key_nope, key_rope, value)."""
    if os.path.exists(ol.REF_PATH):
        return ol.ref_mla(layer, x, pos0, CAP)
    cache = ol.OracleKvCache(layer.dims, CAP)
    out, done = ol.oracle_mla(layer, x, pos0, cache, tables=ol.oracle_rope_tables(layer.dims))
    return out, done, cache.key_nope, cache.key_rope, cache.value


@pytest.mark.parametrize("q_lora", [0, 48])
def test_dropin_attention_matches_litemind(tmp_path, q_lora):
    from litemind_amd import workload as wl
    D = dims(q_lora)
    sets = [wl.mla_layer(400 + q_lora, 0, D), wl.mla_layer(401 + q_lora, 1, D)]
    x = wl.tokens(402 + q_lora, 21, D.hidden)
    script = []
    for t in range(6):  # two layers interleaved, as the runner's layer loop does
        script += [f"fwd 0 0 {t} {t}", f"fwd 1 1 {t} {6 + t}"]
    script += ["dump 0", "dump 1"]
    script += ["clear 0"] + [f"fwd 0 0 {t} {12 + t}" for t in range(3)] + ["dump 0"]
    script += ["copy 2 1", "fwd 2 1 6 18", "fwd 1 1 6 18", "dump 2"]
    script += [f"fwd 3 0 {t} {t}" for t in range(CAP + 1)] + ["dump 3"]
    script += ["clear 3", "fwd 3 0 15 19", "fwd 3 0 16 20"]
    write_case(str(tmp_path), D, sets, x, script)
    announce(f"dropin_demo attention q_lora={q_lora}: {len(script)} commands")
    proc = subprocess.run([DEMO, "attention", str(tmp_path)], capture_output=True, text=True, timeout=240)
    print(proc.stdout, proc.stderr)
    assert proc.returncode == 0, proc.stderr
    H = D.hidden
    fwd = [c for c in script if c.startswith("fwd")]
    out = np.fromfile(tmp_path / "out.f32", np.float32).reshape(len(fwd), H)
    ok = [int(v) for v in open(tmp_path / "results.txt").read().split()]
    rows = {}  # (cache, index of the call on that cache) -> output row
    for i, c in enumerate(fwd):
        rows.setdefault(c.split()[1], []).append(i)

    def dump(c):
        n = int(open(tmp_path / f"cache{c}.txt").read())
        kn = np.fromfile(tmp_path / f"cache{c}_kn.f32", np.float32).reshape(n, D.heads, D.qk_nope)
        kr = np.fromfile(tmp_path / f"cache{c}_kr.f32", np.float32).reshape(n, D.qk_rope)
        v = np.fromfile(tmp_path / f"cache{c}_v.f32", np.float32).reshape(n, D.heads, D.v_head)
        return n, kn, kr, v

    def same(got, want, what):
        assert np.array_equal(bits(got), bits(want)), what

    # cache 0: six tokens of set 0, then after clear() three more from position 0
    a = expected(sets[0], x[0:6], 0)
    c = expected(sets[0], x[12:15], 0)
    got0 = out[rows["0"]]
    same(got0[:6], a[0], "cache 0 first run")
    same(got0[6:], c[0], "cache 0 after clear")
    n, kn, kr, v = dump(0)
    assert n == 3
    same(kn, c[2][:3], "cache 0 keys after clear")
    same(kr, c[3][:3], "cache 0 rotary keys after clear")
    same(v, c[4][:3], "cache 0 values after clear")
    # cache 1: six tokens of set 1, then position 6; cache 2 holds cache 1's
    # entries written by hand and continues with the same token
    b = expected(sets[1], np.concatenate([x[6:12], x[18:19]]), 0)
    got1 = out[rows["1"]]
    same(got1[:6], b[0][:6], "cache 1")
    same(got1[6], b[0][6], "cache 1 continued")
    same(out[rows["2"]][0], b[0][6], "cache 2 (filled by hand) continued")
    n, kn, kr, v = dump(2)
    assert n == 7
    same(kn, b[2][:7], "cache 2 keys")
    same(kr, b[3][:7], "cache 2 rotary keys")
    same(v, b[4][:7], "cache 2 values")
    # cache 3: filled to capacity, the next call refused with its row untouched
    e = expected(sets[0], x[0:CAP + 1], 0)
    assert e[1] == CAP
    got3 = out[rows["3"]]
    same(got3[:CAP], e[0][:CAP], "cache 3 up to capacity")
    assert [ok[i] for i in rows["3"][:CAP + 1]] == [1] * CAP + [0]
    assert np.all(np.isnan(got3[CAP]))
    n, kn, kr, v = dump(3)
    assert n == CAP
    same(kn, e[2], "cache 3 keys")
    same(v, e[4], "cache 3 values")
    # positions 15 and 16 are past the 12-row rotary table: no rotation
    f = expected(sets[0], x[19:21], 15)
    same(got3[CAP + 1:], f[0], "positions past the rotary table")
    assert sum(ok) == len(fwd) - 1
