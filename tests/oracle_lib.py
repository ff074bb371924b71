"""ctypes bindings of the CPU oracle (oracle/liboracle.so) and of LiteMind's own
sources compiled as a cross-check (oracle/_ref/libref.so).  Test infrastructure:
the checker, never the thing measured."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
REF_PATH = os.path.join(ROOT, "oracle", "_ref", "libref.so")

_P, _SZ, _F, _I32, _I64 = C.c_void_p, C.c_size_t, C.c_float, C.c_int32, C.c_int64


class RouterCfg(C.Structure):
    _fields_ = [("expert_count", C.c_int32), ("top_k", C.c_int32), ("n_group", C.c_int32),
                ("topk_group", C.c_int32), ("group_limited", C.c_int32), ("normalize", C.c_int32),
                ("routed_scaling_factor", C.c_float)]


class LayerDims(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("inter", C.c_int32), ("experts", C.c_int32), ("top_k", C.c_int32),
                ("shared_inter", C.c_int32)]


class LayerWeights(C.Structure):
    _fields_ = [("router", C.c_void_p), ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p),
                ("shared_gate", C.c_void_p), ("shared_up", C.c_void_p), ("shared_down", C.c_void_p)]


class MlaDims(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("heads", C.c_int32), ("q_lora_rank", C.c_int32), ("kv_lora_rank", C.c_int32),
                ("qk_nope", C.c_int32), ("qk_rope", C.c_int32), ("v_head", C.c_int32), ("softmax_scale", C.c_float),
                ("rms_norm_eps", C.c_float), ("max_positions", C.c_int32)]


class MlaWeights(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("q_proj", "q_a_proj", "q_a_layernorm", "q_b_proj", "kv_a_proj",
                                          "kv_a_layernorm", "kv_b_proj", "o_proj")]


def p(a):
    if a is None:
        return None
    return a.ctypes.data_as(C.c_void_p)


def _ptr_array(arrays):
    arr = (C.c_void_p * len(arrays))(*[a.ctypes.data for a in arrays])
    return arr


_oracle = None
_ref = None


def oracle() -> C.CDLL:
    global _oracle
    if _oracle is None:
        lib = C.CDLL(ORACLE_PATH)
        for name in ("orc_dot_bf16", "orc_dot_f32", "orc_widen", "orc_expf"):
            getattr(lib, name).restype = C.c_float
        lib.orc_dot_bf16.argtypes = [_P, _P, _SZ]
        lib.orc_dot_f32.argtypes = [_P, _P, _SZ]
        lib.orc_expf.argtypes = [_F]
        lib.orc_bf16_rne.argtypes = [_F]
        lib.orc_bf16_rne.restype = C.c_uint16
        lib.orc_matvec_bf16.argtypes = [_P, _P, _P, _SZ, _SZ]
        lib.orc_matvec_bf16_accumulate.argtypes = [_P, _P, _P, _SZ, _SZ, _F]
        lib.orc_matvec_f32.argtypes = [_P, _P, _P, _SZ, _SZ]
        lib.orc_softmax.argtypes = [_P, _SZ]
        lib.orc_silu_multiply.argtypes = [_P, _P, _P, _SZ]
        lib.orc_rms_norm.argtypes = [_P, _P, _SZ, _F]
        lib.orc_axpy.argtypes = [_F, _P, _P, _SZ]
        lib.orc_router_select.argtypes = [_P, _P, _I32, _P, _P]
        lib.orc_permute.argtypes = [_P, _I64, _I32, _I32, _P, _P, _P, _P]
        lib.orc_moe_layer.argtypes = [_P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _I32]
        lib.orc_dense_ffn.argtypes = [_P, _P, _P, _I32, _I32, _P, _I64, _P, _I32]
        lib.orc_softmax_scale.argtypes = [_I32, _I32, _I32, C.c_double, C.c_double]
        lib.orc_softmax_scale.restype = C.c_float
        lib.orc_rope_tables.argtypes = [_I32, _I32, C.c_double, _I32, C.c_double, C.c_double, C.c_double,
                                        C.c_double, C.c_double, _I64, _P, _P]
        lib.orc_rope_apply.argtypes = [_P, _I32, _P, _P]
        lib.orc_mla_forward.argtypes = [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _I64, _P]
        lib.orc_mla_forward.restype = C.c_int
        for name in ("orc_rope_tables", "orc_rope_apply"):
            getattr(lib, name).restype = None
        for name in ("orc_matvec_bf16", "orc_matvec_bf16_accumulate", "orc_matvec_f32", "orc_softmax",
                     "orc_silu_multiply", "orc_rms_norm", "orc_axpy", "orc_permute", "orc_dense_ffn"):
            getattr(lib, name).restype = None
        _oracle = lib
    return _oracle


def have_ref() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        lib = C.CDLL(REF_PATH)
        lib.ref_dot.restype = C.c_float
        lib.ref_dot.argtypes = [_P, _P, _SZ]
        lib.ref_matvec_bf16.argtypes = [_SZ, _P, _P, _P, _SZ, _SZ]
        lib.ref_matvec_bf16_serial.argtypes = [_P, _P, _P, _SZ, _SZ]
        lib.ref_matvec_bf16_accumulate.argtypes = [_SZ, _P, _P, _P, _SZ, _SZ, _F]
        lib.ref_matvec_f32.argtypes = [_P, _P, _P, _SZ, _SZ]
        lib.ref_axpy.argtypes = [_F, _P, _P, _SZ]
        lib.ref_rms_norm.argtypes = [_P, _P, _SZ, _F]
        lib.ref_softmax.argtypes = [_P, _SZ]
        lib.ref_silu_multiply.argtypes = [_P, _P, _P, _SZ]
        lib.ref_widen_bf16.argtypes = [_P, _P, _SZ]
        lib.ref_router_select.argtypes = [_I32, _I32, _I32, _I32, _I32, _I32, _F, _P, _I32, _P, _P]
        lib.ref_router_select_top_k.argtypes = [_P, _I32, _I32, _I32, _I32, _P, _P]
        lib.ref_parallel_for_visit.argtypes = [_SZ, _SZ, _P]
        lib.ref_kerneltest_inputs.argtypes = [_P, _P, _SZ, _SZ]
        lib.ref_cache_create.argtypes = [C.c_uint64]
        lib.ref_cache_create.restype = C.c_void_p
        lib.ref_cache_destroy.argtypes = [_P]
        lib.ref_cache_configure.argtypes = [_P, C.c_uint64]
        lib.ref_cache_clear.argtypes = [_P]
        lib.ref_cache_make_key.argtypes = [_SZ, _SZ]
        lib.ref_cache_make_key.restype = C.c_uint64
        lib.ref_cache_touch.argtypes = [_P, C.c_uint64, _SZ, _SZ]
        lib.ref_cache_counters.argtypes = [_P, _P]
        lib.ref_moe_layer.argtypes = [_I32, _I32, _I32, _I32, _I32, _I32, _F, _I32, _I32, _I32, _P, _P, _P, _P,
                                      _P, _P, _P, _P, _I64, _P, _P, _P, _P, _SZ]
        lib.ref_hardware_threads.restype = _SZ
        lib.ref_softmax_scale.argtypes = [_I32, _I32, _I32, C.c_double, C.c_double]
        lib.ref_softmax_scale.restype = C.c_float
        lib.ref_rope_tables.argtypes = [_I32, _I32, C.c_double, _I32, C.c_double, C.c_double, C.c_double,
                                        C.c_double, C.c_double, _I64, _P, _P]
        lib.ref_rope_apply.argtypes = [_I32, _I32, C.c_double, _I32, C.c_double, C.c_double, C.c_double, C.c_double,
                                       C.c_double, _I64, _P, _I64]
        lib.ref_mla_sequence.argtypes = [_I32, _I32, _I32, _I32, _I32, _I32, _I32, C.c_float, C.c_double, _I32,
                                         C.c_double, C.c_double, C.c_double, C.c_double, C.c_double, _I64, _I64,
                                         _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _P, _P]
        lib.ref_mla_sequence.restype = _I64
        lib.ref_kernel_description.argtypes = [_P, _SZ]
        _ref = lib
    return _ref


def router_cfg(experts, top_k, normalize=False, scale=1.0, group_limited=False, n_group=1, topk_group=1):
    return RouterCfg(experts, top_k, n_group, topk_group, 1 if group_limited else 0, 1 if normalize else 0, scale)


def oracle_select(logits: np.ndarray, cfg: RouterCfg):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(max(cfg.top_k, 1), np.int32)
    w = np.zeros(max(cfg.top_k, 1), np.float32)
    n = oracle().orc_router_select(C.byref(cfg), p(logits), logits.size, p(idx), p(w))
    return idx[:n], w[:n]


def ref_select(logits: np.ndarray, cfg: RouterCfg):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(max(cfg.top_k, 1), np.int32)
    w = np.zeros(max(cfg.top_k, 1), np.float32)
    n = ref().ref_router_select(cfg.expert_count, cfg.top_k, cfg.n_group, cfg.topk_group, cfg.group_limited,
                                cfg.normalize, cfg.routed_scaling_factor, p(logits), logits.size, p(idx), p(w))
    return idx[:n], w[:n]


def oracle_moe_layer(layer, x: np.ndarray, bias=None, threads: int = 0):
    """Runs the oracle MoE block on x [T, H]; returns (y, idx, weights, logits)."""
    d = layer.dims
    T = x.shape[0]
    dims = LayerDims(d.hidden, d.inter, d.experts, d.top_k, d.shared_inter if layer.shared_gate is not None else 0)
    cfg = router_cfg(d.experts, d.top_k, d.norm_topk_prob, d.routed_scaling_factor, d.group_limited, d.n_group,
                     d.topk_group)
    gate, up, down = _ptr_array(layer.gate), _ptr_array(layer.up), _ptr_array(layer.down)
    w = LayerWeights(layer.router.ctypes.data, C.cast(gate, C.c_void_p), C.cast(up, C.c_void_p),
                     C.cast(down, C.c_void_p),
                     layer.shared_gate.ctypes.data if layer.shared_gate is not None else None,
                     layer.shared_up.ctypes.data if layer.shared_up is not None else None,
                     layer.shared_down.ctypes.data if layer.shared_down is not None else None)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros((T, d.hidden), np.float32)
    idx = np.zeros((T, d.top_k), np.int32)
    wt = np.zeros((T, d.top_k), np.float32)
    logits = np.zeros((T, d.experts), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    rc = oracle().orc_moe_layer(C.byref(dims), C.byref(cfg), C.byref(w), p(x), T, p(b), p(y), p(logits), p(idx),
                                p(wt), threads)
    if rc != 0:
        raise RuntimeError(f"orc_moe_layer failed: {rc}")
    return y, idx, wt, logits


def ref_moe_layer(layer, x: np.ndarray, bias=None, workers: int = 0):
    """LiteMind's own kernels composed as its runner does, per token (compiled reference)."""
    d = layer.dims
    T = x.shape[0]
    gate, up, down = _ptr_array(layer.gate), _ptr_array(layer.up), _ptr_array(layer.down)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros((T, d.hidden), np.float32)
    idx = np.zeros((T, d.top_k), np.int32)
    wt = np.zeros((T, d.top_k), np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    S = d.shared_inter if layer.shared_gate is not None else 0
    rc = ref().ref_moe_layer(d.hidden, d.inter, d.experts, d.top_k, S, 1 if d.norm_topk_prob else 0,
                             d.routed_scaling_factor, d.n_group, d.topk_group, 1 if d.group_limited else 0,
                             p(layer.router), gate, up, down,
                             p(layer.shared_gate), p(layer.shared_up), p(layer.shared_down), p(x), T, p(b), p(y),
                             p(idx), p(wt), workers)
    if rc != 0:
        raise RuntimeError(f"ref_moe_layer failed: {rc}")
    return y, idx, wt


def oracle_permute(idx: np.ndarray, experts: int):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, K = idx.shape
    counts = np.zeros(experts, np.int32)
    offsets = np.zeros(experts + 1, np.int32)
    perm = np.zeros(T * K, np.int32)
    slot_of = np.zeros(T * K, np.int32)
    oracle().orc_permute(p(idx), T, K, experts, p(counts), p(offsets), p(perm), p(slot_of))
    return counts, offsets, perm, slot_of


def oracle_dense(gate, up, down, x: np.ndarray, threads: int = 0):
    D, H = gate.shape
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros((x.shape[0], H), np.float32)
    oracle().orc_dense_ffn(p(gate), p(up), p(down), H, D, p(x), x.shape[0], p(y), threads)
    return y


def oracle_stack(layers, h: np.ndarray, eps: float, every_layer: bool = False, norms=None):
    """The FFN chain of LiteMind's runner with attention omitted
    (src/DeepSeekRunner.cpp:264-290): for each layer, xn = rms_norm(h, w_l)
    (src/Gemm.cpp:197-207; w_l = 1 unless ``norms`` gives the weights), then
    h += 1 * FFN(xn) with gemm::axpy (src/Gemm.cpp:191-195).  ``layers`` is a
    list of ("dense", (gate, up, down)) or ("moe", MoeLayer); h [T, H] is not
    modified.  Returns the final h, or with every_layer the hidden state after
    each layer."""
    h = np.array(h, dtype=np.float32, copy=True)
    T, H = h.shape
    ones = np.ones(H, np.float32)
    o = oracle()
    states = []
    for l, (kind, data) in enumerate(layers):
        xn = h.copy()
        w = ones if norms is None else np.ascontiguousarray(norms[l], dtype=np.float32)
        for t in range(T):
            o.orc_rms_norm(p(xn[t]), p(w), H, eps)
        y = oracle_dense(*data, xn) if kind == "dense" else oracle_moe_layer(data, xn)[0]
        y = np.ascontiguousarray(y, dtype=np.float32)
        for t in range(T):
            o.orc_axpy(1.0, p(y[t]), p(h[t]), H)
        states.append(h.copy())
    return states if every_layer else h


# ---- multi-head latent attention ----

def _rope_args(d):
    return (d.qk_rope, d.max_positions, float(d.rope_theta), 1 if d.yarn else 0, float(d.factor), float(d.beta_fast),
            float(d.beta_slow), float(d.mscale), float(d.mscale_all_dim), int(d.original_max))


def softmax_scale(d) -> float:
    return float(oracle().orc_softmax_scale(d.qk_nope, d.qk_rope, 1 if d.yarn else 0, float(d.factor),
                                            float(d.mscale_all_dim)))


def oracle_rope_tables(d):
    half = d.qk_rope // 2
    cos = np.zeros((d.max_positions, half), np.float32)
    sin = np.zeros((d.max_positions, half), np.float32)
    oracle().orc_rope_tables(*_rope_args(d), p(cos), p(sin))
    return cos, sin


def ref_rope_tables(d):
    half = d.qk_rope // 2
    cos = np.zeros((d.max_positions, half), np.float32)
    sin = np.zeros((d.max_positions, half), np.float32)
    ref().ref_rope_tables(*_rope_args(d), p(cos), p(sin))
    return cos, sin


def _mla_structs(layer, scale=None):
    d = layer.dims
    dims = MlaDims(d.hidden, d.heads, d.q_lora_rank, d.kv_lora_rank, d.qk_nope, d.qk_rope, d.v_head,
                   softmax_scale(d) if scale is None else scale, d.rms_norm_eps, d.max_positions)
    keep = [a for a in (layer.q_proj, layer.q_a_proj, layer.q_a_layernorm, layer.q_b_proj, layer.kv_a_proj,
                        layer.kv_a_layernorm, layer.kv_b_proj, layer.o_proj)]
    w = MlaWeights(*[None if a is None else a.ctypes.data for a in keep])
    return dims, w, keep


class OracleKvCache:
    """KvCache (include/KvCache.hpp) for the oracle: [capacity, heads, qk_nope],
    [capacity, qk_rope], [capacity, heads, v_head] and the filled count."""

    def __init__(self, d, capacity):
        self.key_nope = np.zeros((capacity, d.heads, d.qk_nope), np.float32)
        self.key_rope = np.zeros((capacity, d.qk_rope), np.float32)
        self.value = np.zeros((capacity, d.heads, d.v_head), np.float32)
        self.capacity = capacity
        self.count = C.c_int64(0)


def oracle_mla(layer, x: np.ndarray, position0: int, cache: OracleKvCache, tables=None):
    """Attention::forward for every row of x [T, hidden] in turn (positions
    position0 + t), appending to cache; returns out [T, hidden] and how many
    tokens fit in the cache."""
    d = layer.dims
    dims, w, keep = _mla_structs(layer)
    cos, sin = tables if tables is not None else oracle_rope_tables(d)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    done = 0
    for t in range(x.shape[0]):
        rc = oracle().orc_mla_forward(C.byref(dims), C.byref(w), p(cos), p(sin), p(cache.key_nope), p(cache.key_rope),
                                      p(cache.value), cache.capacity, C.byref(cache.count), p(x[t]), position0 + t,
                                      p(out[t]))
        if rc != 0:
            break
        done += 1
    return out, done


def ref_mla(layer, x: np.ndarray, position0: int, capacity: int):
    """LiteMind's Attention::forward (compiled) over the rows of x; returns
    (out, tokens done, key_nope, key_rope, value) with a fresh cache."""
    d = layer.dims
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros_like(x)
    kn = np.zeros((capacity, d.heads, d.qk_nope), np.float32)
    kr = np.zeros((capacity, d.qk_rope), np.float32)
    v = np.zeros((capacity, d.heads, d.v_head), np.float32)
    done = ref().ref_mla_sequence(d.hidden, d.heads, d.q_lora_rank, d.kv_lora_rank, d.qk_nope, d.qk_rope, d.v_head,
                                  d.rms_norm_eps, float(d.rope_theta), 1 if d.yarn else 0, float(d.factor),
                                  float(d.beta_fast), float(d.beta_slow), float(d.mscale), float(d.mscale_all_dim),
                                  int(d.original_max), capacity, p(layer.q_proj), p(layer.q_a_proj),
                                  p(layer.q_a_layernorm), p(layer.q_b_proj), p(layer.kv_a_proj),
                                  p(layer.kv_a_layernorm), p(layer.kv_b_proj), p(layer.o_proj), p(x), x.shape[0],
                                  position0, p(out), p(kn), p(kr), p(v))
    return out, int(done), kn, kr, v
