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


def oracle_stack(layers, h: np.ndarray, eps: float, every_layer: bool = False):
    """The FFN chain of LiteMind's runner with attention omitted
    (src/DeepSeekRunner.cpp:264-290): for each layer, xn = rms_norm(h, 1)
    (src/Gemm.cpp:197-207), then h += 1 * FFN(xn) with gemm::axpy
    (src/Gemm.cpp:191-195).  ``layers`` is a list of ("dense", (gate, up, down))
    or ("moe", MoeLayer); h [T, H] is not modified.  Returns the final h, or
    with every_layer the hidden state after each layer."""
    h = np.array(h, dtype=np.float32, copy=True)
    T, H = h.shape
    ones = np.ones(H, np.float32)
    o = oracle()
    states = []
    for kind, data in layers:
        xn = h.copy()
        for t in range(T):
            o.orc_rms_norm(p(xn[t]), p(ones), H, eps)
        y = oracle_dense(*data, xn) if kind == "dense" else oracle_moe_layer(data, xn)[0]
        y = np.ascontiguousarray(y, dtype=np.float32)
        for t in range(T):
            o.orc_axpy(1.0, p(y[t]), p(h[t]), H)
        states.append(h.copy())
    return states if every_layer else h
