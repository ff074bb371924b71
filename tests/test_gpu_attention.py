"""Multi-head latent attention on the GPU (include/litemind_attention.h) against
the oracle's Attention::forward (src/Attention.cpp:22-103), bit for bit on the
bit-exact projection path (LM_PATH_GEMV, which these tests select): the
outputs and the KV cache contents, for decode (one token per call), batched
prefill (T tokens per call, causal) and their mix, with and without the
q_lora path and YaRN, positions past the rotary table, a cache that fills, the
residual accumulate and DeepSeek-V2-Lite's full shapes.  The decoder layer
(attention + FFN, src/DeepSeekRunner.cpp:251-291) is checked against the oracle
chain within the FFN's tolerance."""
import dataclasses

import numpy as np
import pytest

import oracle_lib as ol
from conftest import MAX_ABS, MEAN_REL, announce, layer_error

pytestmark = pytest.mark.gpu

SMALL_OVER = dict(hidden=256, heads=4, kv_lora_rank=64, qk_nope=32, qk_rope=16, v_head=32, original_max=16,
                  factor=4.0, max_positions=24)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def small_dims(**over):
    from litemind_amd import workload as wl
    return dataclasses.replace(wl.V2_LITE_MLA, **dict(SMALL_OVER, **over))


def moe_dims_for(hidden):
    from litemind_amd import workload as wl
    return wl.Dims(hidden=hidden, inter=128, experts=8, top_k=2, n_shared=1, dense_inter=256, layers=2)


class Mla:
    """A context holding one attention layer (id 0) and the oracle's mirror of it."""

    def __init__(self, d, seed, layers=1, path=None):
        from litemind_amd import PATH_GEMV
        path = PATH_GEMV if path is None else path
        from litemind_amd import Context
        from litemind_amd import workload as wl
        self.d = d
        self.ctx = Context(moe_dims_for(d.hidden).moe_config(num_layers=layers))
        self.ctx.attention_configure(wl.mla_config(d))
        self.ctx.attention_set_path(path)
        self.L = wl.mla_layer(seed, 0, d)
        wl.upload_mla_layer(self.ctx, 0, self.L)
        self.cache = ol.OracleKvCache(d, d.max_positions)

    def forward(self, x, pos0, accumulate_into=None):
        T = x.shape[0]
        dx = self.ctx.to_device(x)
        init = accumulate_into if accumulate_into is not None else np.full_like(x, np.nan)
        dout = self.ctx.to_device(init)
        try:
            self.ctx.attention_forward(0, dx, T, pos0, dout, accumulate=accumulate_into is not None)
        finally:
            self.ctx.synchronize()
            out = dout.download()
            dx.free()
            dout.free()
        return out

    def oracle(self, x, pos0):
        return ol.oracle_mla(self.L, x, pos0, self.cache)

    def check_cache(self):
        n = int(self.cache.count.value)
        assert self.ctx.kv_cache_tokens(0) == n
        kn, kr, v = self.ctx.kv_cache_read(0, n)
        np.testing.assert_array_equal(bits(kn), bits(self.cache.key_nope[:n]))
        np.testing.assert_array_equal(bits(kr), bits(self.cache.key_rope[:n]))
        np.testing.assert_array_equal(bits(v), bits(self.cache.value[:n]))

    def close(self):
        self.ctx.close()


def tokens(seed, T, hidden):
    from litemind_amd import workload as wl
    return wl.tokens(seed, T, hidden)


@pytest.mark.parametrize("over", [dict(), dict(yarn=False), dict(q_lora_rank=48)])
def test_decode_sequence_bit_exact(over):
    """Twelve single-token calls in a row (decode), each output and the cache
    against the oracle's per-token Attention::forward."""
    d = small_dims(**over)
    announce(f"attention decode x12 small {over}")
    m = Mla(d, 101)
    try:
        x = tokens(102, 12, d.hidden)
        for t in range(12):
            y = m.forward(x[t:t + 1], t)
            want, n = m.oracle(x[t:t + 1], t)
            assert n == 1
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


@pytest.mark.parametrize("over", [dict(), dict(q_lora_rank=48, yarn=False)])
def test_prefill_batch_equals_sequential(over):
    """Twenty tokens in one call (causal attention inside the batch, queries in
    blocks of eight) give LiteMind's twenty sequential calls bit for bit; then
    three decode steps continue from the batched cache."""
    d = small_dims(**over)
    announce(f"attention prefill T=20 + decode x3 small {over}")
    m = Mla(d, 111)
    try:
        x = tokens(112, 23, d.hidden)
        y = m.forward(x[:20], 0)
        want, n = m.oracle(x[:20], 0)
        assert n == 20
        np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
        for t in range(20, 23):
            y = m.forward(x[t:t + 1], t)
            want, _ = m.oracle(x[t:t + 1], t)
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


@pytest.mark.parametrize("nope", [22, 21])
def test_odd_widths_and_dot_tails(nope):
    """Three heads, qk_nope 22 or 21 and qk_rope 6 (dots with fused tails past
    the last multiple of four; with 21 the rotary pairs do not fall on a row
    pair of the single-token query launch, which then runs the projection and
    the rotary step separately), v_head 24 (a partial wave in the context
    kernel), prefill of 5 then 4 tokens, then three single-token steps."""
    d = small_dims(heads=3, qk_nope=nope, qk_rope=6, v_head=24)
    announce(f"attention odd widths nope={nope}")
    m = Mla(d, 121)
    try:
        x = tokens(122, 12, d.hidden)
        for lo, hi in ((0, 5), (5, 9), (9, 10), (10, 11), (11, 12)):
            y = m.forward(x[lo:hi], lo)
            want, _ = m.oracle(x[lo:hi], lo)
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


def test_decode_positions_past_the_rotary_table():
    """Single-token steps at positions 20..25 with a 24-row rotary table (cache
    slots 4..9 after four tokens at positions 16..19): the query and key
    rotations of the single-token launches leave positions 24 and 25
    unrotated (and in place), as RotaryEmbedding::apply does."""
    d = small_dims(max_positions=24)
    announce("attention decode past table")
    m = Mla(d, 135)
    try:
        x = tokens(136, 10, d.hidden)
        y = m.forward(x[:4], 16)
        want, _ = m.oracle(x[:4], 16)
        np.testing.assert_array_equal(bits(y), bits(want))
        for t in range(4, 10):
            y = m.forward(x[t:t + 1], 16 + t)
            want, _ = m.oracle(x[t:t + 1], 16 + t)
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


def test_positions_past_the_rotary_table():
    """RotaryEmbedding::apply leaves positions at or past its table unrotated:
    positions 21..26 with a 24-row table, in one call."""
    d = small_dims()
    announce("attention positions past table")
    m = Mla(d, 131)
    try:
        x = tokens(132, 6, d.hidden)
        y = m.forward(x, 21)
        want, _ = m.oracle(x, 21)
        np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


def test_cache_full_processes_what_fits():
    """A 24-token cache holding 20: a call with 6 tokens processes 4, leaves the
    other rows untouched and reports LM_EFULL; a further call changes nothing."""
    from litemind_amd import LM_EFULL, LmError
    d = small_dims()
    announce("attention cache full")
    m = Mla(d, 141)
    try:
        x = tokens(142, 27, d.hidden)
        m.forward(x[:20], 0)
        m.oracle(x[:20], 0)
        dx = m.ctx.to_device(x[20:26])
        dout = m.ctx.to_device(np.full((6, d.hidden), np.nan, np.float32))
        with pytest.raises(LmError) as err:
            m.ctx.attention_forward(0, dx, 6, 20, dout)
        assert err.value.status == LM_EFULL
        m.ctx.synchronize()
        y = dout.download()
        want, n = m.oracle(x[20:26], 20)
        assert n == 4 and m.ctx.kv_cache_tokens(0) == 24
        np.testing.assert_array_equal(bits(y[:4]), bits(want[:4]))
        assert np.isnan(y[4:]).all()
        with pytest.raises(LmError) as err:
            m.ctx.attention_forward(0, dx, 1, 24, dout)
        assert err.value.status == LM_EFULL and m.ctx.kv_cache_tokens(0) == 24
        m.check_cache()
        dx.free()
        dout.free()
        # KvCache::clear empties every layer; the next sequence starts at slot 0
        m.ctx.kv_cache_clear()
        assert m.ctx.kv_cache_tokens(0) == 0
        m.cache = ol.OracleKvCache(d, d.max_positions)
        y = m.forward(x[:3], 0)
        want, _ = m.oracle(x[:3], 0)
        np.testing.assert_array_equal(bits(y), bits(want))
    finally:
        m.close()


def test_accumulate_is_the_runners_residual_add():
    """accumulate = 1 gives h + attention(x), which is the runner's
    gemm::axpy(1, block_output, hidden_state) bit for bit."""
    d = small_dims()
    announce("attention accumulate")
    m = Mla(d, 151)
    try:
        x = tokens(152, 5, d.hidden)
        h = tokens(153, 5, d.hidden) * np.float32(3.0)
        y = m.forward(x, 0, accumulate_into=h)
        want, _ = m.oracle(x, 0)
        hh = h.copy()
        o = ol.oracle()
        for t in range(5):
            o.orc_axpy(1.0, ol.p(np.ascontiguousarray(want[t])), ol.p(hh[t]), d.hidden)
        np.testing.assert_array_equal(bits(y), bits(hh))
    finally:
        m.close()


@pytest.mark.parametrize("q_lora", [0, 1536])
def test_v2_lite_shapes_prefill_and_decode(q_lora):
    """DeepSeek-V2-Lite's attention (16 heads, kv_lora_rank 512, qk 128 + 64,
    v_head 128, hidden 2048, YaRN factor 40), and with a 1536-wide q_lora path
    as DeepSeek-V2 has: prefill of 40 tokens then 2 decode steps."""
    from litemind_amd import workload as wl
    d = dataclasses.replace(wl.V2_LITE_MLA, q_lora_rank=q_lora, max_positions=64)
    announce(f"attention V2-Lite shapes q_lora={q_lora}: prefill 40 + decode 2")
    m = Mla(d, 161)
    try:
        x = tokens(162, 42, d.hidden)
        y = m.forward(x[:40], 0)
        want, _ = m.oracle(x[:40], 0)
        np.testing.assert_array_equal(bits(y), bits(want))
        for t in (40, 41):
            y = m.forward(x[t:t + 1], t)
            want, _ = m.oracle(x[t:t + 1], t)
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


@pytest.mark.parametrize("prefill", [255, 2303, 8191])
def test_decode_across_value_chunks(prefill):
    """Decode steps whose cached lengths cross the single-token context
    kernel's 256-token chunks: n = 256, 257, 258 (one full chunk, then a
    partial one) and n = 2304, 2305, 2306 (nine chunks, more than its LDS
    ring holds, so slots are refilled), after a batched prefill; and n = 8192
    (the longest row whose softmax runs inside the context launch), 8193 and
    8194 (the softmax as its own launch, the context kernel with the
    probabilities in its ring)."""
    d = small_dims(max_positions=prefill + 8)
    announce(f"attention prefill T={prefill} + decode x3 small")
    m = Mla(d, 181)
    try:
        x = tokens(182, prefill + 3, d.hidden)
        y = m.forward(x[:prefill], 0)
        want, _ = m.oracle(x[:prefill], 0)
        np.testing.assert_array_equal(bits(y), bits(want))
        for t in range(prefill, prefill + 3):
            y = m.forward(x[t:t + 1], t)
            want, _ = m.oracle(x[t:t + 1], t)
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


def test_v2_lite_long_prefill_sampled():
    """A 600-token prefill in one call (two groups of query tokens in the
    attention core, three key tiles) at V2-Lite shapes: tokens 0..599 are
    processed by the oracle in order, and every 37th row plus the last is
    compared bit for bit, together with the whole cache."""
    from litemind_amd import workload as wl
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=640)
    announce("attention V2-Lite prefill T=600")
    m = Mla(d, 171)
    try:
        x = tokens(172, 600, d.hidden)
        y = m.forward(x, 0)
        want, _ = m.oracle(x, 0)
        rows = list(range(0, 600, 37)) + [599]
        np.testing.assert_array_equal(bits(y[rows]), bits(want[rows]))
        m.check_cache()
    finally:
        m.close()


def test_decoder_layers_match_oracle_chain():
    """lm_decoder_forward over a dense layer and a MoE layer of V2-Lite shapes:
    h += attention(rms_norm(h, input_norm)), h += FFN(rms_norm(h, post_norm))
    per layer, prefill of 5 tokens (FFN on the GEMV path) and one decode step
    (the single-token MoE kernel), against the oracle composed the same way
    (the attention is bit-exact; the fp32-activation FFN paths stay within
    1e-5 mean relative error)."""
    from litemind_amd import Context
    from litemind_amd import workload as wl
    dims = wl.V2_LITE
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=32)
    announce("decoder forward: dense + MoE layer with attention")
    ctx = Context(dims.moe_config(num_layers=2))
    try:
        ctx.attention_configure(wl.mla_config(d))
        gate, up, down = wl.dense_ffn(wl.MASTER_SEED, 0, dims)
        ctx.upload_dense(0, gate, up, down)
        ctx.finalize_layer(0)
        moe = wl.moe_layer(wl.MASTER_SEED, 1, dims)
        wl.upload_moe_layer(ctx, 1, moe)
        att = [wl.mla_layer(181, l, d) for l in range(2)]
        in_norm = [(1.0 + wl.normal_f32(182, l, 0.1, (dims.hidden,))).astype(np.float32) for l in range(2)]
        post_norm = [(1.0 + wl.normal_f32(183, l, 0.1, (dims.hidden,))).astype(np.float32) for l in range(2)]
        for l in range(2):
            wl.upload_mla_layer(ctx, l, att[l])
            ctx.upload_input_norm(l, in_norm[l])
            ctx.upload_norm(l, post_norm[l])
        h0 = tokens(184, 6, dims.hidden) * np.float32(4.0)

        caches = [ol.OracleKvCache(d, d.max_positions) for _ in range(2)]
        o = ol.oracle()

        def oracle_chain(h, pos0):
            h = h.copy()
            T = h.shape[0]
            for l in range(2):
                xn = h.copy()
                for t in range(T):
                    o.orc_rms_norm(ol.p(xn[t]), ol.p(in_norm[l]), dims.hidden, dims.rms_norm_eps)
                a, _ = ol.oracle_mla(att[l], xn, pos0, caches[l])
                for t in range(T):
                    o.orc_axpy(1.0, ol.p(np.ascontiguousarray(a[t])), ol.p(h[t]), dims.hidden)
                xn = h.copy()
                for t in range(T):
                    o.orc_rms_norm(ol.p(xn[t]), ol.p(post_norm[l]), dims.hidden, dims.rms_norm_eps)
                y = ol.oracle_dense(gate, up, down, xn) if l == 0 else ol.oracle_moe_layer(moe, xn)[0]
                y = np.ascontiguousarray(y, np.float32)
                for t in range(T):
                    o.orc_axpy(1.0, ol.p(y[t]), ol.p(h[t]), dims.hidden)
            return h

        from litemind_amd import PATH_AUTO, PATH_GEMV
        # 5 tokens: below the attention's MFMA crossover, so AUTO would be
        # bit-exact too; GEMV selects the fp32 FFN path as well
        for lo, hi, path in ((0, 5, PATH_GEMV), (5, 6, PATH_AUTO)):
            dh = ctx.to_device(h0[lo:hi])
            ctx.decoder_forward(0, 1, dh, hi - lo, lo, path)
            ctx.synchronize()
            got = dh.download()
            dh.free()
            want = oracle_chain(h0[lo:hi], lo)
            mx, rel = layer_error(got, want)
            assert mx <= MAX_ABS and rel <= MEAN_REL, (lo, mx, rel)
            assert rel <= 1e-5, (lo, rel)
        assert ctx.kv_cache_tokens(0) == 6 and ctx.kv_cache_tokens(1) == 6
    finally:
        ctx.close()


# ---- MFMA projections (tolerance-bounded) ----
# fp16 operands with fp32 accumulation in the four projections of a batch:
# every projection output carries the fp16 rounding of its input (~2^-12
# relative per element), which passes through the scores and the softmax into
# the context and o_proj.  Measured on V2-Lite shapes (512-token prefill):
# mean relative error ~1e-3 on the attention output; bar 5e-3 mean-rel and
# max-abs 5e-2 on outputs of magnitude ~1.  The KV cache entries (produced by
# kv_a / kv_b) are held to the same bar.
ATT_MEAN_REL = 5e-3
ATT_MAX_ABS = 5e-2


@pytest.mark.parametrize("q_lora", [0, 1536])
def test_mfma_projections_v2_lite_prefill_then_decode(q_lora):
    """A 512-token prefill on the MFMA projection path (LM_PATH_AUTO) at
    V2-Lite shapes with and without the q LoRA path, then two decode steps
    (single-token launches over the MFMA-filled cache), against the oracle."""
    from litemind_amd import PATH_AUTO
    from litemind_amd import workload as wl
    d = dataclasses.replace(wl.V2_LITE_MLA, q_lora_rank=q_lora, max_positions=520)
    announce(f"attention MFMA projections V2-Lite q_lora={q_lora}: prefill 512 + decode 2")
    m = Mla(d, 191, path=PATH_AUTO)
    try:
        x = tokens(192, 514, d.hidden)
        y = m.forward(x[:512], 0)
        want, _ = m.oracle(x[:512], 0)
        assert np.all(np.isfinite(y))
        mx, rel = layer_error(y, want)
        print(f"prefill 512 q_lora={q_lora}: max_abs={mx:.3e} mean_rel={rel:.3e} (|y| mean {np.abs(want).mean():.3f})")
        assert mx <= ATT_MAX_ABS and rel <= ATT_MEAN_REL
        n = 512
        kn, kr, v = m.ctx.kv_cache_read(0, n)
        for got, ref, name in ((kn, m.cache.key_nope[:n], "key_nope"), (kr, m.cache.key_rope[:n], "key_rope"),
                               (v, m.cache.value[:n], "value")):
            mx, rel = layer_error(got, ref)
            print(f"cache {name}: max_abs={mx:.3e} mean_rel={rel:.3e}")
            assert mx <= ATT_MAX_ABS and rel <= ATT_MEAN_REL, name
        for t in (512, 513):
            y = m.forward(x[t:t + 1], t)
            want, _ = m.oracle(x[t:t + 1], t)
            mx, rel = layer_error(y, want)
            print(f"decode {t}: max_abs={mx:.3e} mean_rel={rel:.3e}")
            assert mx <= ATT_MAX_ABS and rel <= ATT_MEAN_REL
    finally:
        m.close()


def test_mfma_path_selection():
    """LM_PATH_AUTO below 16 tokens keeps the bit-exact projections; LM_PATH_MFMA
    takes the MFMA projections from two tokens (within tolerance, and not bit
    for bit equal on these inputs); an unknown path is refused."""
    from litemind_amd import PATH_AUTO, PATH_MFMA, LmError
    from litemind_amd import workload as wl
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=32)
    announce("attention path selection: AUTO T=8 bit-exact, MFMA T=8 within tolerance")
    m = Mla(d, 201, path=PATH_AUTO)
    try:
        x = tokens(202, 16, d.hidden)
        y = m.forward(x[:8], 0)
        want, _ = m.oracle(x[:8], 0)
        np.testing.assert_array_equal(bits(y), bits(want))
        m.ctx.attention_set_path(PATH_MFMA)
        y = m.forward(x[8:16], 8)
        want, _ = m.oracle(x[8:16], 8)
        mx, rel = layer_error(y, want)
        print(f"MFMA T=8: max_abs={mx:.3e} mean_rel={rel:.3e}")
        assert mx <= ATT_MAX_ABS and rel <= ATT_MEAN_REL
        assert not np.array_equal(bits(y), bits(want))
        with pytest.raises(LmError):
            m.ctx.attention_set_path(7)
    finally:
        m.close()


# ---- query groups sized from the score budget ----

def test_small_score_budget_groups_bit_exact():
    """A score budget of five query tokens' scores: the 20-token call after 6
    cached tokens runs the attention core in four groups, still bit for bit
    LiteMind's sequential calls (bit-exact path)."""
    from litemind_amd import PATH_GEMV, attention_plan_core
    from litemind_amd import workload as wl
    d = small_dims(max_positions=32)
    budget = 5 * d.heads * 26 * 4  # five tokens of scores over 26 keys
    plan = attention_plan_core(wl.mla_config(d), 6, 20, PATH_GEMV, budget)
    assert plan.query_group == 5 and plan.mfma_core == 0
    announce("attention prefill 6 + 20 with a five-token score budget (bit-exact path)")
    m = Mla(d, 221)
    try:
        m.ctx.attention_set_score_budget(budget)
        x = tokens(222, 26, d.hidden)
        for lo, hi in ((0, 6), (6, 26)):
            y = m.forward(x[lo:hi], lo)
            want, n = m.oracle(x[lo:hi], lo)
            assert n == hi - lo
            np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()


def test_mfma_core_small_budget_two_groups():
    """V2-Lite on the MFMA core: 40 tokens, then 96 with a budget that holds 77
    query tokens (two core launches, the second of 19 rows per head on the
    narrow tile); the outputs equal those of one 96-token group bit for bit
    (every score and context element has the same K order either way) and meet
    the oracle within the MFMA tolerance."""
    from litemind_amd import PATH_AUTO, attention_plan_core
    from litemind_amd import workload as wl
    d = dataclasses.replace(wl.V2_LITE_MLA, max_positions=160)
    budget = 3_300_000
    plan = attention_plan_core(wl.mla_config(d), 40, 96, PATH_AUTO, budget)
    assert plan.mfma_core == 1 and plan.query_group == 77
    assert attention_plan_core(wl.mla_config(d), 40, 96, PATH_AUTO).query_group == 96
    announce("attention MFMA core V2-Lite 40 + 96 tokens, score budget of 77 query tokens vs default")
    x = tokens(232, 136, d.hidden)
    outs = []
    for b in (budget, 0):
        m = Mla(d, 231, path=PATH_AUTO)
        try:
            m.ctx.attention_set_score_budget(b)
            y0 = m.forward(x[:40], 0)
            y1 = m.forward(x[40:], 40)
            if b:
                for y, lo, hi in ((y0, 0, 40), (y1, 40, 136)):
                    want, _ = m.oracle(x[lo:hi], lo)
                    mx, rel = layer_error(y, want)
                    print(f"MFMA core {lo}..{hi}: max_abs={mx:.3e} mean_rel={rel:.3e}")
                    assert mx <= ATT_MAX_ABS and rel <= ATT_MEAN_REL
            outs.append((y0, y1))
        finally:
            m.close()
    for a, b in zip(outs[0], outs[1]):
        np.testing.assert_array_equal(bits(a), bits(b))


def test_kv_cache_write_read_range_truncate():
    """lm_kv_cache_write / read_range / truncate through the C ABI: entries
    written from KvCache's layout read back bit for bit (whole and by range),
    appended after a prefill, decoding continues over them as over entries the
    GPU made; a gap, a write past the capacity and a read past the count are
    refused; truncate keeps the first entries and the next call appends there."""
    from litemind_amd import LmError
    d = small_dims(max_positions=32)
    announce("KV cache write / read_range / truncate (small shapes)")
    m = Mla(d, 241)
    try:
        x = tokens(242, 12, d.hidden)
        m.forward(x[:6], 0)
        m.oracle(x[:6], 0)
        kn, kr, v = m.ctx.kv_cache_read(0, 6)
        # the same six entries written again, and four more from random data
        rng = np.random.default_rng(243)
        kn4 = rng.standard_normal((4, d.heads, d.qk_nope)).astype(np.float32)
        kr4 = rng.standard_normal((4, d.qk_rope)).astype(np.float32)
        v4 = rng.standard_normal((4, d.heads, d.v_head)).astype(np.float32)
        m.ctx.kv_cache_write(0, 6, kn4, kr4, v4)
        assert m.ctx.kv_cache_tokens(0) == 10
        rkn, rkr, rv = m.ctx.kv_cache_read_range(0, 6, 4)
        for a, b in ((rkn, kn4), (rkr, kr4), (rv, v4)):
            np.testing.assert_array_equal(bits(a), bits(b))
        rkn, rkr, rv = m.ctx.kv_cache_read_range(0, 2, 3)
        for a, b in ((rkn, kn[2:5]), (rkr, kr[2:5]), (rv, v[2:5])):
            np.testing.assert_array_equal(bits(a), bits(b))
        # the oracle's cache gets the same entries; decoding continues over them
        n = int(m.cache.count.value)
        m.cache.key_nope[n:n + 4], m.cache.key_rope[n:n + 4], m.cache.value[n:n + 4] = kn4, kr4, v4
        m.cache.count.value = n + 4
        y = m.forward(x[6:8], 10)
        want, _ = m.oracle(x[6:8], 10)
        np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
        with pytest.raises(LmError, match="write of entries"):
            m.ctx.kv_cache_write(0, 13, kn4, kr4, v4)  # gap after the 12 entries
        with pytest.raises(LmError, match="write of entries"):
            m.ctx.kv_cache_write(0, 30, kn4, kr4, v4)  # past the capacity of 32
        with pytest.raises(LmError, match="within the cache"):
            m.ctx.kv_cache_read_range(0, 10, 3)
        with pytest.raises(LmError, match="within the cache"):
            m.ctx.kv_cache_truncate(0, 13)
        # truncate to 6: the oracle's cache keeps its first 6 entries too
        m.ctx.kv_cache_truncate(0, 6)
        assert m.ctx.kv_cache_tokens(0) == 6
        m.cache.count.value = 6
        y = m.forward(x[8:12], 6)
        want, _ = m.oracle(x[8:12], 6)
        np.testing.assert_array_equal(bits(y), bits(want))
        m.check_cache()
    finally:
        m.close()
