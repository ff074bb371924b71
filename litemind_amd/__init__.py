"""litemind_amd -- MI355X (gfx950) mixture-of-experts feed-forward path for LiteMind.

The product is the native library ``liblitemind_moe.so`` (HIP kernels + the C ABI
declared in ``include/litemind_moe.h``).  This module binds that ABI with ctypes
for Python callers (tests, the benchmark); it never falls back to a CPU path:
if the library is missing or a GPU call fails, it raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblitemind_moe.so")

LM_OK = 0
PATH_AUTO, PATH_GEMV, PATH_MFMA = 0, 1, 2
MFMA_CROSSOVER = 2  # LM_MFMA_CROSSOVER: PATH_AUTO takes the MFMA path above this many tokens
DECODE_TOKENS = 3  # LM_DECODE_TOKENS: LM_PATH_AUTO runs up to this many tokens one at a time on the single-token kernel
OP_DOT, OP_AXPY, OP_SOFTMAX, OP_SILU_MUL, OP_RMS_NORM, OP_WIDEN = range(6)
STAGES = ("router", "permute", "gate_up", "down", "combine")


LM_EFULL = -6  # the KV cache had no free slot (include/litemind_attention.h)


class LmError(RuntimeError):
    """A litemind_amd C ABI call returned a non-zero status (``status``)."""

    def __init__(self, message: str, status: int = 0):
        super().__init__(message)
        self.status = status


class MoeConfig(C.Structure):
    """lm_moe_config: the MoE subset of LiteMind's Config (include/Config.hpp:48, :58-71, :101-103)."""

    _fields_ = [
        ("hidden_size", C.c_int32),
        ("moe_intermediate_size", C.c_int32),
        ("n_routed_experts", C.c_int32),
        ("num_experts_per_tok", C.c_int32),
        ("n_shared_experts", C.c_int32),
        ("intermediate_size", C.c_int32),
        ("norm_topk_prob", C.c_int32),
        ("routed_scaling_factor", C.c_float),
        ("group_limited", C.c_int32),
        ("n_group", C.c_int32),
        ("topk_group", C.c_int32),
        ("rms_norm_eps", C.c_float),
        ("num_layers", C.c_int32),
    ]


class MlaConfig(C.Structure):
    """lm_mla_config: the attention subset of LiteMind's Config (include/Config.hpp) and
    the context length sizing RotaryEmbedding::build and KvCache::configure."""

    _fields_ = [
        ("hidden_size", C.c_int32),
        ("num_heads", C.c_int32),
        ("q_lora_rank", C.c_int32),
        ("kv_lora_rank", C.c_int32),
        ("qk_nope_head_dim", C.c_int32),
        ("qk_rope_head_dim", C.c_int32),
        ("v_head_dim", C.c_int32),
        ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_double),
        ("yarn", C.c_int32),
        ("factor", C.c_double),
        ("beta_fast", C.c_double),
        ("beta_slow", C.c_double),
        ("mscale", C.c_double),
        ("mscale_all_dim", C.c_double),
        ("original_max_positions", C.c_int64),
        ("context_length", C.c_int64),
    ]


_P = C.c_void_p
_I32 = C.c_int32
_I64 = C.c_int64
_SZ = C.c_size_t
_F = C.c_float

# name -> argtypes (all return int status unless listed in _RESTYPE)
PROTOTYPES = {
    "lm_last_error": [],
    "lm_version": [_P, _P],
    "lm_context_create": [_I32, _P, _P],
    "lm_context_destroy": [_P],
    "lm_synchronize": [_P],
    "lm_alloc": [_P, _SZ, _P],
    "lm_free": [_P, _P],
    "lm_copy_h2d": [_P, _P, _P, _SZ],
    "lm_copy_d2h": [_P, _P, _P, _SZ],
    "lm_memset": [_P, _P, _I32, _SZ],
    "lm_upload_router": [_P, _I32, _P],
    "lm_upload_expert": [_P, _I32, _I32, _P, _P, _P],
    "lm_upload_shared": [_P, _I32, _P, _P, _P],
    "lm_upload_dense": [_P, _I32, _P, _P, _P],
    "lm_upload_norm": [_P, _I32, _P],
    "lm_finalize_layer": [_P, _I32],
    "lm_layer_fp16_inexact": [_P, _I32, _P],
    "lm_resident_bytes": [_P, _P],
    "lm_moe_forward": [_P, _I32, _P, _I64, _P, _P, _P, _P, _P, _I32],
    "lm_moe_forward_noalloc": [_P, _I32, _P, _I64, _P, _P, _P, _P, _P],
    "lm_router": [_P, _I32, _P, _I64, _P, _P, _P, _P],
    "lm_router_select": [_P, _P, _I64, _P, _P],
    "lm_permute": [_P, _P, _I64, _P, _P, _P, _P],
    "lm_grouped_swiglu": [_P, _I32, _P, _I64, _P, _P, _I32],
    "lm_context_stream": [_P, _P],
    "lm_stack_forward": [_P, _I32, _I32, _P, _I64, _I32],
    "lm_stack_graph_create": [_P, _I32, _I32, _P, _I64, _I32, C.POINTER(C.c_void_p)],
    "lm_stack_graph_launch": [_P],
    "lm_stack_graph_destroy": [_P],
    "lm_rms_norm": [_P, _P, _P, _P, _I64, _I32, _F],
    "lm_dense_forward": [_P, _I32, _P, _I64, _P, _I32],
    "lm_gemm_matvec_bf16": [_P, _P, _P, _P, _SZ, _SZ, _F, _I32],
    "lm_gemm_matvec_f32": [_P, _P, _P, _P, _SZ, _SZ],
    "lm_vector_op": [_P, _I32, _P, _P, _P, _SZ, _F],
    "lm_weight_prefetch": [_P, _P, _SZ],
    "lm_weight_release": [_P, _P],
    "lm_weight_resident": [_P, _P, _P],
    "lm_decode_speculation_test": [_P, _I32],
    "lm_decode_wait_test": [_P, _I32],
    "lm_router_speculation": [_P, _I32],
    "lm_event_create": [_P, _P],
    "lm_event_destroy": [_P, _P],
    "lm_event_record": [_P, _P],
    "lm_event_elapsed_ms": [_P, _P, _P, _P],
    "lm_stage_timing": [_P, _I32],
    "lm_stage_times": [_P, _P, _P, _I32],
    "lm_clock_probe_start": [_P, C.c_double],
    "lm_clock_probe_finish": [_P, _P, _P, _P, _P],
    "lm_context_config": [_P, _P],
    "lm_checkpoint_open": [C.c_char_p, _P],
    "lm_checkpoint_close": [_P],
    "lm_checkpoint_count": [_P, _P, _P],
    "lm_checkpoint_find": [_P, C.c_char_p, _P, _P, _P, _P, _P],
    "lm_checkpoint_require": [_P, C.c_char_p, _I32, _P, _I32, _P],
    "lm_checkpoint_read_f32": [_P, C.c_char_p, _I32, _P, _P, C.c_uint64],
    "lm_load_layer": [_P, _P, _I32, _I32],
    "lm_upload_head": [_P, _P, _P, _I64],
    "lm_head_forward": [_P, _P, _I64, _P, _P],
    "lm_load_head": [_P, _P, _I64],
    "lm_mla_softmax_scale": [_P, _P],
    "lm_rope_tables": [_P, _I64, _P, _P],
    "lm_attention_configure": [_P, _P],
    "lm_upload_attention": [_P, _I32, _P, _P, _P, _P, _P, _P, _P, _P],
    "lm_upload_input_norm": [_P, _I32, _P],
    "lm_attention_forward": [_P, _I32, _P, _I64, _I64, _P, _I32],
    "lm_kv_cache_clear": [_P],
    "lm_attention_set_path": [_P, _I32],
    "lm_attention_set_score_budget": [_P, _I64],
    "lm_attention_plan_core": [_P, _I64, _I64, _I32, _I64, _P],
    "lm_kv_cache_tokens": [_P, _I32, _P],
    "lm_kv_cache_read": [_P, _I32, _I64, _P, _P, _P],
    "lm_kv_cache_read_range": [_P, _I32, _I64, _I64, _P, _P, _P],
    "lm_kv_cache_write": [_P, _I32, _I64, _I64, _P, _P, _P],
    "lm_kv_cache_truncate": [_P, _I32, _I64],
    "lm_decoder_forward": [_P, _I32, _I32, _P, _I64, _I64, _I32],
}
_RESTYPE = {"lm_last_error": C.c_char_p}

_lib = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Loads liblitemind_moe.so, raising if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise LmError(f"{path} is missing: build it with `python -m litemind_amd.build`")
    lib = C.CDLL(path)
    for name, args in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RESTYPE.get(name, C.c_int)
    _lib = lib
    return lib


def _ptr(a) -> C.c_void_p:
    if a is None:
        return None
    if isinstance(a, DeviceBuffer):
        return C.c_void_p(a.ptr)
    if isinstance(a, np.ndarray):
        if not a.flags["C_CONTIGUOUS"]:
            raise ValueError("array must be C-contiguous")
        return a.ctypes.data_as(C.c_void_p)
    if isinstance(a, int):
        return C.c_void_p(a)
    raise TypeError(f"cannot pass {type(a)} as a pointer")


class DeviceBuffer:
    """An HBM allocation owned by a Context (freed on close or context destroy)."""

    def __init__(self, ctx: "Context", nbytes: int, dtype=np.float32, shape=None):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        self.dtype = np.dtype(dtype)
        self.shape = shape if shape is not None else (self.nbytes // self.dtype.itemsize,)
        out = C.c_void_p()
        ctx._check(ctx.lib.lm_alloc(ctx.handle, max(self.nbytes, 1), C.byref(out)))
        self.ptr = out.value

    def upload(self, host: np.ndarray) -> "DeviceBuffer":
        host = np.ascontiguousarray(host)
        if host.nbytes > self.nbytes:
            raise ValueError("host array larger than the device buffer")
        self.ctx._check(self.ctx.lib.lm_copy_h2d(self.ctx.handle, C.c_void_p(self.ptr), _ptr(host), host.nbytes))
        return self

    def download(self, shape=None, dtype=None) -> np.ndarray:
        dtype = np.dtype(dtype) if dtype is not None else self.dtype
        shape = shape if shape is not None else self.shape
        out = np.empty(shape, dtype=dtype)
        self.ctx._check(self.ctx.lib.lm_copy_d2h(self.ctx.handle, _ptr(out), C.c_void_p(self.ptr), out.nbytes))
        return out

    def zero(self) -> "DeviceBuffer":
        self.ctx._check(self.ctx.lib.lm_memset(self.ctx.handle, C.c_void_p(self.ptr), 0, self.nbytes))
        return self

    def free(self) -> None:
        if self.ptr:
            self.ctx._check(self.ctx.lib.lm_free(self.ctx.handle, C.c_void_p(self.ptr)))
            self.ptr = 0


# SafeTensors element types (LM_DT_*) and the numpy type of their raw payload
# (BF16 as its uint16 bit patterns).
DT_BF16, DT_F16, DT_F32, DT_F64, DT_I8, DT_I16, DT_I32, DT_I64, DT_U8, DT_BOOL = range(1, 11)
_DT_NUMPY = {DT_BF16: np.uint16, DT_F16: np.float16, DT_F32: np.float32, DT_F64: np.float64, DT_I8: np.int8,
             DT_I16: np.int16, DT_I32: np.int32, DT_I64: np.int64, DT_U8: np.uint8, DT_BOOL: np.bool_}


def _check_status(lib, status: int) -> None:
    if status != LM_OK:
        msg = lib.lm_last_error().decode(errors="replace")
        raise LmError(f"litemind_amd status {status}: {msg}", status)


def rope_tables(config: MlaConfig, positions: int):
    """RotaryEmbedding::build's cos / sin tables [positions, qk_rope / 2] (lm_rope_tables, host only)."""
    lib = load_library()
    half = config.qk_rope_head_dim // 2
    cos = np.zeros((positions, half), np.float32)
    sin = np.zeros((positions, half), np.float32)
    _check_status(lib, lib.lm_rope_tables(C.byref(config), positions, _ptr(cos), _ptr(sin)))
    return cos, sin


class AttentionCorePlan(C.Structure):
    """lm_attention_core_plan: the attention core's query group and scratch for one call."""

    _fields_ = [
        ("query_group", C.c_int64),
        ("scratch_bytes", C.c_int64),
        ("mfma_core", C.c_int32),
        ("reserved", C.c_int32),
    ]


def attention_plan_core(config: MlaConfig, cached: int, tokens: int, path: int = 0,
                        budget_bytes: int = 0) -> AttentionCorePlan:
    """The query grouping lm_attention_forward takes after `cached` tokens (lm_attention_plan_core,
    host only)."""
    lib = load_library()
    out = AttentionCorePlan()
    _check_status(lib, lib.lm_attention_plan_core(C.byref(config), cached, tokens, path, budget_bytes,
                                                  C.byref(out)))
    return out


def mla_softmax_scale(config: MlaConfig) -> float:
    """Config::softmax_scale (lm_mla_softmax_scale, host only)."""
    lib = load_library()
    out = C.c_float()
    _check_status(lib, lib.lm_mla_softmax_scale(C.byref(config), C.byref(out)))
    return out.value


class Checkpoint:
    """A directory of SafeTensors shards mapped read-only (lm_checkpoint_open); the
    counterpart of LiteMind's WeightStore (src/WeightStore.cpp:52-185).  Needs no GPU."""

    def __init__(self, model_dir):
        self.lib = load_library()
        handle = C.c_void_p()
        _check_status(self.lib, self.lib.lm_checkpoint_open(os.fsencode(str(model_dir)), C.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if self.handle:
            self.lib.lm_checkpoint_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def count(self) -> tuple[int, int]:
        """(distinct tensor names, shards)."""
        t, sh = C.c_int64(), C.c_int64()
        _check_status(self.lib, self.lib.lm_checkpoint_count(self.handle, C.byref(t), C.byref(sh)))
        return t.value, sh.value

    def find(self, name: str):
        """(dtype code, shape, payload bytes, payload address) of a tensor."""
        dt, rank, nbytes, payload = C.c_int32(), C.c_int32(), C.c_uint64(), C.c_void_p()
        shape = (C.c_int64 * 8)()
        _check_status(self.lib, self.lib.lm_checkpoint_find(self.handle, name.encode(), C.byref(dt), C.byref(rank),
                                                            shape, C.byref(payload), C.byref(nbytes)))
        return dt.value, tuple(shape[i] for i in range(rank.value)), nbytes.value, payload.value or 0

    def array(self, name: str) -> np.ndarray:
        """A copy of the tensor's payload as numpy (BF16 as uint16 bit patterns)."""
        dt, shape, nbytes, payload = self.find(name)
        raw = C.string_at(payload, nbytes) if nbytes else b""
        return np.frombuffer(raw, dtype=_DT_NUMPY[dt]).reshape(shape).copy()

    def require(self, name: str, shape, dtype: int) -> int:
        """Payload address of a tensor that must have exactly this shape and dtype."""
        dims = (C.c_int64 * max(len(shape), 1))(*[int(d) for d in shape])
        payload = C.c_void_p()
        _check_status(self.lib, self.lib.lm_checkpoint_require(self.handle, name.encode(), len(shape), dims, dtype,
                                                               C.byref(payload)))
        return payload.value or 0

    def read_f32(self, name: str, shape) -> np.ndarray:
        """WeightStore::read_float32: F32, BF16 or F16 as float32."""
        dims = (C.c_int64 * max(len(shape), 1))(*[int(d) for d in shape])
        out = np.empty([int(d) for d in shape], np.float32)
        _check_status(self.lib, self.lib.lm_checkpoint_read_f32(self.handle, name.encode(), len(shape), dims,
                                                                _ptr(out), out.size))
        return out


class Context:
    """One GPU's resident MoE weights and stream (lm_context)."""

    def __init__(self, config: MoeConfig, device: int = 0):
        self.lib = load_library()
        self.config = config
        handle = C.c_void_p()
        self._check(self.lib.lm_context_create(device, C.byref(config), C.byref(handle)))
        self.handle = handle
        self._buffers: list[DeviceBuffer] = []

    def _check(self, status: int) -> None:
        _check_status(self.lib, status)

    def upload_head(self, norm: np.ndarray, head: np.ndarray) -> None:
        """Final norm [H] fp32 and LM head [V, H] BF16 bits (lm_upload_head)."""
        norm = np.ascontiguousarray(norm, np.float32)
        head = np.ascontiguousarray(head, np.uint16)
        self._check(self.lib.lm_upload_head(self.handle, _ptr(norm), _ptr(head), head.shape[0]))

    def head_forward(self, hidden, tokens: int, logits=None, token=None) -> None:
        """logits = head . rms_norm(hidden) and the greedy next token (lm_head_forward)."""
        self._check(self.lib.lm_head_forward(self.handle, _ptr(hidden), tokens, _ptr(logits), _ptr(token)))

    def load_head(self, checkpoint: "Checkpoint", vocab: int) -> None:
        """model.norm.weight and lm_head.weight (or the tied embedding) from a checkpoint."""
        self._check(self.lib.lm_load_head(self.handle, checkpoint.handle, vocab))

    def load_layer(self, checkpoint: "Checkpoint", layer: int, moe: int = -1) -> None:
        """Uploads a layer's FFN from a checkpoint (lm_load_layer): moe 1, 0, or -1 to
        decide by whether the checkpoint holds the layer's router."""
        self._check(self.lib.lm_load_layer(self.handle, checkpoint.handle, layer, moe))

    def close(self) -> None:
        if self.handle:
            self._check(self.lib.lm_context_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- memory ----
    def empty(self, shape, dtype=np.float32) -> DeviceBuffer:
        shape = tuple(int(s) for s in np.atleast_1d(shape))
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        return DeviceBuffer(self, n, dtype, shape)

    def to_device(self, host: np.ndarray) -> DeviceBuffer:
        host = np.ascontiguousarray(host)
        return DeviceBuffer(self, host.nbytes, host.dtype, host.shape).upload(host)

    def synchronize(self) -> None:
        self._check(self.lib.lm_synchronize(self.handle))

    # ---- residency ----
    def upload_router(self, layer: int, gate: np.ndarray) -> None:
        gate = np.ascontiguousarray(gate, dtype=np.float32)
        self._check(self.lib.lm_upload_router(self.handle, layer, _ptr(gate)))

    def upload_expert(self, layer: int, expert: int, gate, up, down) -> None:
        self._check(self.lib.lm_upload_expert(self.handle, layer, expert, _ptr(gate), _ptr(up), _ptr(down)))

    def upload_shared(self, layer: int, gate, up, down) -> None:
        self._check(self.lib.lm_upload_shared(self.handle, layer, _ptr(gate), _ptr(up), _ptr(down)))

    def upload_dense(self, layer: int, gate, up, down) -> None:
        self._check(self.lib.lm_upload_dense(self.handle, layer, _ptr(gate), _ptr(up), _ptr(down)))

    def upload_norm(self, layer: int, weight: np.ndarray) -> None:
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        self._check(self.lib.lm_upload_norm(self.handle, layer, _ptr(weight)))

    def finalize_layer(self, layer: int) -> None:
        self._check(self.lib.lm_finalize_layer(self.handle, layer))

    def layer_fp16_inexact(self, layer: int) -> int:
        """lm_layer_fp16_inexact: weights of a finalized layer whose fp16 copy
        (the MFMA path's operands) rounds: BF16 magnitudes below 2^-17."""
        n = C.c_int64()
        self._check(self.lib.lm_layer_fp16_inexact(self.handle, layer, C.byref(n)))
        return n.value

    def resident_bytes(self) -> int:
        out = C.c_uint64()
        self._check(self.lib.lm_resident_bytes(self.handle, C.byref(out)))
        return out.value

    # ---- compute (device buffers; asynchronous) ----
    def moe_forward(self, layer, x, tokens, y, bias=None, idx=None, w=None, logits=None, path=PATH_AUTO) -> None:
        self._check(self.lib.lm_moe_forward(self.handle, layer, _ptr(x), tokens, _ptr(y), _ptr(bias), _ptr(idx),
                                            _ptr(w), _ptr(logits), path))

    # ---- multi-head latent attention (include/litemind_attention.h) ----
    def attention_configure(self, config: MlaConfig) -> None:
        self.mla_config = config
        self._check(self.lib.lm_attention_configure(self.handle, C.byref(config)))

    def upload_attention(self, layer: int, q_proj=None, q_a_proj=None, q_a_layernorm=None, q_b_proj=None,
                         kv_a_proj=None, kv_a_layernorm=None, kv_b_proj=None, o_proj=None) -> None:
        keep = [None if a is None else np.ascontiguousarray(a) for a in
                (q_proj, q_a_proj, q_a_layernorm, q_b_proj, kv_a_proj, kv_a_layernorm, kv_b_proj, o_proj)]
        self._check(self.lib.lm_upload_attention(self.handle, layer, *[_ptr(a) for a in keep]))

    def upload_input_norm(self, layer: int, weight: np.ndarray) -> None:
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        self._check(self.lib.lm_upload_input_norm(self.handle, layer, _ptr(weight)))

    def attention_forward(self, layer, x, tokens, position0, out, accumulate=False) -> None:
        self._check(self.lib.lm_attention_forward(self.handle, layer, _ptr(x), tokens, position0, _ptr(out),
                                                  1 if accumulate else 0))

    def attention_set_path(self, path: int) -> None:
        """Projection path of attention_forward (lm_attention_set_path)."""
        self._check(self.lib.lm_attention_set_path(self.handle, path))

    def attention_set_score_budget(self, nbytes: int) -> None:
        """Byte budget of the attention core's scratch (lm_attention_set_score_budget; 0: default)."""
        self._check(self.lib.lm_attention_set_score_budget(self.handle, nbytes))

    def kv_cache_clear(self) -> None:
        self._check(self.lib.lm_kv_cache_clear(self.handle))

    def kv_cache_tokens(self, layer: int) -> int:
        out = C.c_int64()
        self._check(self.lib.lm_kv_cache_tokens(self.handle, layer, C.byref(out)))
        return out.value

    def kv_cache_read(self, layer: int, tokens: int):
        """The cache's first `tokens` entries in KvCache's layout: key_nope [T, heads, nope],
        key_rope [T, rope], value [T, heads, v_head]."""
        c = self.mla_config
        kn = np.zeros((tokens, c.num_heads, c.qk_nope_head_dim), np.float32)
        kr = np.zeros((tokens, c.qk_rope_head_dim), np.float32)
        v = np.zeros((tokens, c.num_heads, c.v_head_dim), np.float32)
        self._check(self.lib.lm_kv_cache_read(self.handle, layer, tokens, _ptr(kn), _ptr(kr), _ptr(v)))
        return kn, kr, v

    def kv_cache_read_range(self, layer: int, token0: int, tokens: int):
        """Entries [token0, token0 + tokens) in KvCache's layout (lm_kv_cache_read_range)."""
        c = self.mla_config
        kn = np.zeros((tokens, c.num_heads, c.qk_nope_head_dim), np.float32)
        kr = np.zeros((tokens, c.qk_rope_head_dim), np.float32)
        v = np.zeros((tokens, c.num_heads, c.v_head_dim), np.float32)
        self._check(self.lib.lm_kv_cache_read_range(self.handle, layer, token0, tokens, _ptr(kn), _ptr(kr), _ptr(v)))
        return kn, kr, v

    def kv_cache_write(self, layer: int, token0: int, key_nope, key_rope, value) -> None:
        """Stores entries token0 .. token0 + len - 1 from KvCache-layout arrays (lm_kv_cache_write)."""
        kn = np.ascontiguousarray(key_nope, np.float32)
        kr = np.ascontiguousarray(key_rope, np.float32)
        v = np.ascontiguousarray(value, np.float32)
        self._check(self.lib.lm_kv_cache_write(self.handle, layer, token0, kn.shape[0], _ptr(kn), _ptr(kr), _ptr(v)))

    def kv_cache_truncate(self, layer: int, tokens: int) -> None:
        self._check(self.lib.lm_kv_cache_truncate(self.handle, layer, tokens))

    def decoder_forward(self, first, last, hidden, tokens, position0, path=PATH_AUTO) -> None:
        self._check(self.lib.lm_decoder_forward(self.handle, first, last, _ptr(hidden), tokens, position0, path))

    def moe_forward_noalloc(self, layer, x, tokens, y, bias=None, idx=None, w=None, logits=None) -> None:
        """lm_moe_forward_noalloc: the single-token kernel per token, scratch in a fixed device array."""
        self._check(self.lib.lm_moe_forward_noalloc(self.handle, layer, _ptr(x), tokens, _ptr(y), _ptr(bias),
                                                    _ptr(idx), _ptr(w), _ptr(logits)))

    def router(self, layer, x, tokens, idx, w, bias=None, logits=None) -> None:
        self._check(self.lib.lm_router(self.handle, layer, _ptr(x), tokens, _ptr(bias), _ptr(logits), _ptr(idx),
                                       _ptr(w)))

    def router_select(self, logits, tokens, idx, w) -> None:
        self._check(self.lib.lm_router_select(self.handle, _ptr(logits), tokens, _ptr(idx), _ptr(w)))

    def permute(self, idx, tokens, counts, offsets, perm, slot_of) -> None:
        self._check(self.lib.lm_permute(self.handle, _ptr(idx), tokens, _ptr(counts), _ptr(offsets), _ptr(perm),
                                        _ptr(slot_of)))

    def grouped_swiglu(self, layer, x, tokens, idx, out, path=PATH_AUTO) -> None:
        """lm_grouped_swiglu: per-assignment FFN outputs [T*k + T, H] (routed rows in
        assignment order, then the shared rows) for the routing idx [T, k]."""
        self._check(self.lib.lm_grouped_swiglu(self.handle, layer, _ptr(x), tokens, _ptr(idx), _ptr(out), path))

    def stream(self) -> int:
        """The context's hipStream_t (lm_context_stream)."""
        out = C.c_void_p()
        self._check(self.lib.lm_context_stream(self.handle, C.byref(out)))
        return out.value or 0

    def stack_forward(self, first, last, hidden, tokens, path=PATH_AUTO) -> None:
        self._check(self.lib.lm_stack_forward(self.handle, first, last, _ptr(hidden), tokens, path))

    def router_speculation(self, mode: int) -> None:
        """lm_router_speculation: one token over more than 64 experts runs the
        router and gate/up as one speculative launch (1, the default), the router
        then gate/up (0), or the speculative launch with its repair forced (2)."""
        self._check(self.lib.lm_router_speculation(self.handle, mode))

    def stack_graph_create(self, first, last, hidden, tokens, path=PATH_AUTO) -> int:
        """lm_stack_graph_create: the stack pass recorded as a HIP graph (a handle for
        stack_graph_launch / stack_graph_destroy)."""
        out = C.c_void_p()
        self._check(self.lib.lm_stack_graph_create(self.handle, first, last, _ptr(hidden), tokens, path,
                                                   C.byref(out)))
        return out.value

    def stack_graph_launch(self, graph: int) -> None:
        self._check(self.lib.lm_stack_graph_launch(C.c_void_p(graph)))

    def stack_graph_destroy(self, graph: int) -> None:
        self._check(self.lib.lm_stack_graph_destroy(C.c_void_p(graph)))

    def rms_norm(self, x, weight, out, tokens, hidden, eps) -> None:
        self._check(self.lib.lm_rms_norm(self.handle, _ptr(x), _ptr(weight), _ptr(out), tokens, hidden, eps))

    def dense_forward(self, layer, x, tokens, y, path=PATH_AUTO) -> None:
        self._check(self.lib.lm_dense_forward(self.handle, layer, _ptr(x), tokens, _ptr(y), path))

    def gemm_matvec_bf16(self, w: np.ndarray, x: np.ndarray, out: np.ndarray, scale=1.0, accumulate=False) -> None:
        out_dim, in_dim = w.shape
        self._check(self.lib.lm_gemm_matvec_bf16(self.handle, _ptr(w), _ptr(x), _ptr(out), out_dim, in_dim,
                                                 scale, 1 if accumulate else 0))

    def gemm_matvec_f32(self, w: np.ndarray, x: np.ndarray, out: np.ndarray) -> None:
        out_dim, in_dim = w.shape
        self._check(self.lib.lm_gemm_matvec_f32(self.handle, _ptr(w), _ptr(x), _ptr(out), out_dim, in_dim))

    def vector_op(self, op: int, a: np.ndarray, b, out: np.ndarray, scalar: float = 0.0) -> None:
        self._check(self.lib.lm_vector_op(self.handle, op, _ptr(a), _ptr(b), _ptr(out), a.size, scalar))

    # ---- timing ----
    def event(self):
        out = C.c_void_p()
        self._check(self.lib.lm_event_create(self.handle, C.byref(out)))
        return out

    def record(self, event) -> None:
        self._check(self.lib.lm_event_record(self.handle, event))

    def elapsed_ms(self, start, stop) -> float:
        out = C.c_float()
        self._check(self.lib.lm_event_elapsed_ms(self.handle, start, stop, C.byref(out)))
        return out.value

    def stage_timing(self, enable: bool) -> None:
        self._check(self.lib.lm_stage_timing(self.handle, 1 if enable else 0))

    def stage_times(self) -> dict:
        ms = (C.c_double * len(STAGES))()
        calls = (C.c_int32 * len(STAGES))()
        self._check(self.lib.lm_stage_times(self.handle, ms, calls, len(STAGES)))
        return {name: (ms[i], calls[i]) for i, name in enumerate(STAGES)}

    def clock_probe_start(self, seconds: float) -> None:
        """lm_clock_probe_start: sample the core clock for `seconds` (<= 2) on a
        stream of its own while work is enqueued on the context stream."""
        self._check(self.lib.lm_clock_probe_start(self.handle, float(seconds)))

    def clock_probe_finish(self) -> dict:
        med, lo, hi = C.c_double(), C.c_double(), C.c_double()
        n = C.c_int32()
        self._check(self.lib.lm_clock_probe_finish(self.handle, C.byref(med), C.byref(lo), C.byref(hi), C.byref(n)))
        return {"mhz": round(med.value, 1), "min_mhz": round(lo.value, 1), "max_mhz": round(hi.value, 1),
                "intervals": n.value}
