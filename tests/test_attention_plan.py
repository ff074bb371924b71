"""Sizing of the attention core (lm_attention_plan_core, host only): the query
tokens of one core launch are chosen from a byte budget, so a long cache takes
smaller groups instead of one 512-token group whose scores would not fit.  The
expected groups are worked out here from the rule the header states (as many
tokens as the budget holds, at least one, at most 512 and the call's tokens;
the MFMA core while its fp16 key / value copies take at most half the budget),
with the byte counts of the buffers written out per case."""
import dataclasses

import pytest

from litemind_amd import PATH_AUTO, PATH_GEMV, PATH_MFMA, LmError, attention_plan_core
from litemind_amd import workload as wl

GIB = 1 << 30


def cfg(**over):
    return wl.mla_config(dataclasses.replace(wl.V2_LITE_MLA, **over))


def fits(per_token, budget, tokens):
    """Largest g in [1, min(512, tokens)] with g * per_token <= budget (1 if none)."""
    g = 1
    while g < min(512, tokens) and (g + 1) * per_token <= budget:
        g += 1
    return g


@pytest.mark.parametrize("heads,cached,tokens,budget", [
    (16, 0, 512, 0),             # V2-Lite prefill: one group of 512
    (16, 160_000, 512, 0),       # a late chunk: 16 x 160512 x 4 B per query token
    (128, 160_000, 512, 0),      # V2's 128 heads
    (16, 0, 512, 1 << 20),       # a 1 MiB budget: 32 tokens of 16 x 512 x 4 B
    (16, 10_000_000, 4, 0),      # one token's scores exceed the budget: still one
    (16, 100, 7, 0),             # fewer tokens than the budget holds
])
def test_valu_core_groups(heads, cached, tokens, budget):
    c = cfg(heads=heads)
    p = attention_plan_core(c, cached, tokens, PATH_GEMV, budget)
    per = heads * (cached + tokens) * 4
    want = fits(per, budget or GIB, tokens)
    assert p.mfma_core == 0
    assert p.query_group == want
    assert p.scratch_bytes == want * per
    if want > 1:
        assert p.scratch_bytes <= (budget or GIB)


def test_valu_core_late_chunk_numbers():
    """The figures of a 512-token chunk after 160000 cached tokens, spelled out:
    V2-Lite 1 GiB / (16 * 160512 * 4 B) = 104 tokens (5.4 GB for all 512), full
    V2 (128 heads) 13 tokens."""
    assert attention_plan_core(cfg(), 160_000, 512, PATH_GEMV).query_group == 104
    assert attention_plan_core(cfg(heads=128), 160_000, 512, PATH_GEMV).query_group == 13


def mfma_bytes(heads, qk, vh, keys):
    kp = (keys + 31) // 32 * 32
    fixed = heads * kp * (qk + vh) * 2          # fp16 keys [Kp][qk] and values [vh][Kp] per head
    per = heads * (kp * 4 + kp * 2 + qk * 2)    # fp32 scores, fp16 probabilities, fp16 query
    return fixed, per


@pytest.mark.parametrize("cached,tokens,budget,path", [
    (0, 512, 0, PATH_AUTO),
    (0, 512, 0, PATH_MFMA),
    (3000, 512, 0, PATH_AUTO),
    (0, 96, 0, PATH_AUTO),
    (40, 96, 3_300_000, PATH_AUTO),  # (3300000 - 1638400) // 21504 = 77 tokens: two launches
    (160_000, 512, 4 * GIB, PATH_AUTO),
])
def test_mfma_core_groups(cached, tokens, budget, path):
    c = cfg()
    p = attention_plan_core(c, cached, tokens, path, budget)
    fixed, per = mfma_bytes(16, 192, 128, cached + tokens)
    b = budget or GIB
    assert fixed <= b // 2
    want = min(512, tokens, (b - fixed) // per)
    assert p.mfma_core == 1
    assert p.query_group == want
    assert p.scratch_bytes == fixed + want * per <= b


def test_mfma_core_falls_back():
    c = cfg()
    # copies of 160512 keys: 16 x 160512 x 320 x 2 B = 1.64 GB > half of 1 GiB -> VALU core
    p = attention_plan_core(c, 160_000, 512, PATH_AUTO)
    assert p.mfma_core == 0 and p.query_group == 104
    # the projections are not MFMA: AUTO below 16 tokens, or one token, or GEMV
    assert attention_plan_core(c, 0, 8, PATH_AUTO).mfma_core == 0
    assert attention_plan_core(c, 0, 1, PATH_MFMA).mfma_core == 0
    assert attention_plan_core(c, 0, 512, PATH_GEMV).mfma_core == 0
    assert attention_plan_core(c, 0, 8, PATH_MFMA).mfma_core == 1
    # channel counts that are not whole 32-channel panels
    assert attention_plan_core(cfg(qk_rope=16), 0, 512, PATH_AUTO).mfma_core == 0
    assert attention_plan_core(cfg(qk_nope=48), 0, 512, PATH_AUTO).mfma_core == 0
    assert attention_plan_core(cfg(heads=1, v_head=8, kv_lora_rank=64), 0, 512, PATH_AUTO).mfma_core == 0


def test_plan_rejects_bad_arguments():
    c = cfg()
    with pytest.raises(LmError):
        attention_plan_core(c, -1, 4)
    with pytest.raises(LmError):
        attention_plan_core(c, 0, 4, PATH_AUTO, -5)
    with pytest.raises(LmError):
        attention_plan_core(c, 0, 4, 9)
    p = attention_plan_core(c, 10, 0)
    assert p.query_group == 0 and p.scratch_bytes == 0
