"""Synthetic workload generator: deterministic, thread-count independent, and the
tiny-model recipe of tools/make_test_model.py."""
import numpy as np

from litemind_amd import workload as wl


def test_generator_is_deterministic_and_thread_independent():
    a = wl.normal_bf16(5, 7, 0.02, (300, 1000), threads=1)
    b = wl.normal_bf16(5, 7, 0.02, (300, 1000), threads=7)
    assert np.array_equal(a, b)
    c = wl.normal_bf16(5, 8, 0.02, (300, 1000))
    assert not np.array_equal(a, c)
    f = (a.astype(np.uint32) << 16).view(np.float32)
    assert abs(float(f.std()) - 0.02) < 0.001 and abs(float(f.mean())) < 0.001


def test_tokens_are_rms_normalised():
    x = wl.tokens(3, 8, 2048)
    rms = np.sqrt((x.astype(np.float64) ** 2).mean(axis=1))
    assert np.allclose(rms, 1.0, atol=1e-5)


def test_tiny_model_recipe():
    """The first embedding values of tools/make_test_model.py, computed independently:
    LCG s = s * 1664525 + 1013904223 mod 2^32 from 20240816, value (s / (2^32 - 1)) * 2 - 1,
    times 0.08, truncated to BF16; the MoE layer follows after the embedding and layer 0."""
    import struct

    s = 20240816
    first = []
    for _ in range(4):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        v = ((s / 0xFFFFFFFF) * 2.0 - 1.0) * 0.08
        first.append(struct.unpack("<I", struct.pack("<f", v))[0] >> 16)
    dims, layer = wl.tiny_model_layers(1)
    assert dims.hidden == 32 and dims.experts == 4 and dims.top_k == 2 and dims.inter == 16
    assert layer.router.shape == (4, 32) and layer.gate[0].shape == (16, 32) and layer.down[3].shape == (32, 16)
    assert all(0 <= v < 65536 for v in first)


def test_skew_bias_reproduces_targets():
    d = wl.V2_LITE
    router = wl.normal_f32(wl.MASTER_SEED, wl.stream_id(0, wl.S_ROUTER), 0.02, (d.experts, d.hidden))
    x = wl.tokens(wl.MASTER_SEED, 2048, d.hidden)
    logits = x.astype(np.float64) @ router.astype(np.float64).T + wl.skew_bias()
    counts = wl._topk_counts(logits, d.top_k)
    hot = counts[:8].sum() / counts.sum()
    assert 0.65 < hot < 0.75
    assert counts[8:].min() > 0
