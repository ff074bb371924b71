"""The LM head and greedy choice (lm_head_forward) against the oracle.

Logits must equal the oracle's gemm::rms_norm + gemm::matvec_bf16
(src/Gemm.cpp:46-82, :139-155, :197-207) bit for bit, and the token must be
Sampler::select_next's greedy choice (src/Sampler.cpp:117-126): std::max_element,
the first of equal maxima.  Hidden widths cover the 32-element chains alone,
the 8-wide remainder, and more than one staged chunk; token counts cross the
4-token group of a launch; V = 102400 is DeepSeek-V2-Lite's vocabulary.
"""
import numpy as np
import pytest

import oracle_lib as ol
from conftest import announce

pytestmark = pytest.mark.gpu

EPS = 1e-6


def _case(seed, V, H, T):
    from litemind_amd import workload as wl

    rng = np.random.default_rng(seed)
    head = wl.f32_to_bf16((0.02 * rng.standard_normal((V, H))).astype(np.float32))
    norm = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    hidden = (3.0 * rng.standard_normal((T, H))).astype(np.float32)
    return head, norm, hidden


def _oracle(head, norm, hidden):
    V, H = head.shape
    logits = np.zeros((hidden.shape[0], V), np.float32)
    for t in range(hidden.shape[0]):
        xn = np.ascontiguousarray(hidden[t]).copy()
        ol.oracle().orc_rms_norm(ol.p(xn), ol.p(norm), H, EPS)
        ol.oracle().orc_matvec_bf16(ol.p(head), ol.p(xn), ol.p(logits[t]), V, H)
    return logits


def _config(H):
    from litemind_amd import MoeConfig

    return MoeConfig(hidden_size=H, moe_intermediate_size=64, n_routed_experts=8, num_experts_per_tok=2,
                     n_shared_experts=0, intermediate_size=0, norm_topk_prob=0, routed_scaling_factor=1.0,
                     group_limited=0, n_group=1, topk_group=1, rms_norm_eps=EPS, num_layers=1)


def _gpu(ctx, hidden, V):
    T = hidden.shape[0]
    dh = ctx.to_device(hidden)
    dl, dt = ctx.empty((T, V)), ctx.empty((T,), np.int32)
    ctx.head_forward(dh, T, logits=dl, token=dt)
    dt2 = ctx.empty((T,), np.int32)
    ctx.head_forward(dh, T, token=dt2)  # without a logits buffer
    ctx.synchronize()
    out = dl.download(), dt.download(), dt2.download()
    for b in (dh, dl, dt, dt2):
        b.free()
    return out


@pytest.mark.parametrize("V,H,T", [(1003, 2048, 1), (1003, 2048, 3), (517, 2048, 9), (300, 2064, 2),
                                   (257, 528, 4), (64, 4112, 1), (102400, 2048, 1)])
def test_head_bit_exact(V, H, T):
    from litemind_amd import Context

    head, norm, hidden = _case(V * 31 + H + T, V, H, T)
    announce(f"head V={V} H={H} T={T}")
    with Context(_config(H)) as ctx:
        ctx.upload_head(norm, head)
        logits, token, token2 = _gpu(ctx, hidden, V)
    want = _oracle(head, norm, hidden)
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    assert token.tolist() == [int(np.argmax(want[t])) for t in range(T)]
    assert token2.tolist() == token.tolist()


def test_head_ties_pick_the_first():
    """Rows copied from the winning row make exact ties: the lowest index wins,
    wherever the copies sit relative to the original."""
    from litemind_amd import Context

    V, H, T = 2000, 2048, 2
    head, norm, hidden = _case(5, V, H, T)
    base = _oracle(head, norm, hidden)
    winners = [int(np.argmax(base[t])) for t in range(T)]
    head = head.copy()
    head[1500] = head[winners[0]]  # a later copy: the original still wins
    head[7] = head[winners[1]]     # an earlier copy: the copy wins
    announce("head ties V=2000")
    with Context(_config(H)) as ctx:
        ctx.upload_head(norm, head)
        logits, token, _ = _gpu(ctx, hidden, V)
    want = _oracle(head, norm, hidden)
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    assert logits[0, 1500] == logits[0, winners[0]] and logits[1, 7] == logits[1, winners[1]]
    assert token.tolist() == [int(np.argmax(want[t])) for t in range(T)]  # numpy: the first maximum
    assert token[0] == min(winners[0], 1500) and token[1] == min(winners[1], 7)


@pytest.mark.parametrize("tied", [False, True])
def test_head_from_checkpoint(tmp_path, tied):
    from litemind_amd import Checkpoint, Context
    from litemind_amd import workload as wl

    V, H, T = 777, 2048, 3
    head, norm, hidden = _case(11, V, H, T)
    name = "model.embed_tokens.weight" if tied else "lm_head.weight"
    wl.save_safetensors(tmp_path / "model.safetensors",
                        {"model.norm.weight": wl.f32_to_bf16(norm), name: head})
    widened = (wl.f32_to_bf16(norm).astype(np.uint32) << 16).view(np.float32)
    announce(f"head from checkpoint tied={tied}")
    with Checkpoint(tmp_path) as ck, Context(_config(H)) as ctx:
        ctx.load_head(ck, V)
        logits, token, _ = _gpu(ctx, hidden, V)
    want = _oracle(head, widened, hidden)
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    assert token.tolist() == [int(np.argmax(want[t])) for t in range(T)]
