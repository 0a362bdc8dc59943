"""ctypes binding of libtqattn.so (include/tq/tq_attn.h, tq_model.h), the C host interface.

Mirrors the reference's kv_cache / attention entry points for the device Q8
cache (model/model_ops.h:95-97,124; model/attention_layer.c:66-90,125-150,
169-194,200-236).  Loading fails loudly when the library is missing; every
compute call runs on the GPU through libtqhip.so.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import native

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtqattn.so")

TQ_KV_F32, TQ_KV_Q8, TQ_KV_Q8_DEVICE = 0, 1, 2

_vp, _i, _f = C.c_void_p, C.c_int, C.c_float


class AttnConfig(C.Structure):
    """tq_attn_config (model/model_ops.h:12-19)."""
    _fields_ = [("n_q_heads", _i), ("n_kv_heads", _i), ("head_dim", _i), ("hidden_size", _i),
                ("rope_theta", _f), ("rms_eps", _f)]


class KVCache(C.Structure):
    """tq_kv_cache (model/model_ops.h:41-48) with the trailing device handle."""
    _fields_ = [("type", _i), ("k_f32", _vp), ("v_f32", _vp), ("k_q8", _vp), ("v_q8", _vp),
                ("max_tokens", _i), ("dev", _vp)]


class DevLayerWeights(C.Structure):
    """tq_dev_layer_weights (include/tq/tq_model.h): tq_layer_weights with device pointers."""
    _fields_ = [("input_norm", _vp), ("attn", native.AttnWeights), ("post_norm", _vp), ("mlp", native.MlpWeights)]


class DevModel(C.Structure):
    """tq_dev_model: tq_model (model/model_ops.h:50-73) with device weights."""
    _fields_ = [("attn", AttnConfig), ("n_layers", _i), ("intermediate_size", _i), ("vocab_size", _i),
                ("embed", _vp), ("final_norm", _vp), ("layers", C.POINTER(DevLayerWeights)), ("embed_format", _i)]


class DevBatchWs(C.Structure):
    """tq_dev_batch_ws: tq_batch_ws (model/model_ops.h:146-154) for the device."""
    _fields_ = [("cap", _i), ("x", _vp), ("xn", _vp), ("y", _vp), ("tokens", _vp), ("ws", _vp),
                ("ws_bytes", C.c_size_t)]


class DevCtx(C.Structure):
    """tq_dev_ctx: tq_ctx (model/model_ops.h:75-95) for the device."""
    _fields_ = [("model", _vp), ("caches", _vp), ("pos", _i), ("max_tokens", _i), ("stream", _vp),
                ("x", _vp), ("xn", _vp), ("y", _vp), ("logits", _vp), ("cos_t", _vp), ("sin_t", _vp),
                ("positions", _vp), ("ws", _vp), ("ws_bytes", C.c_size_t), ("sampled", _vp)]


_PC, _PK = C.POINTER(AttnConfig), C.POINTER(KVCache)
_PM, _PX = C.POINTER(DevModel), C.POINTER(DevCtx)
_PB = C.POINTER(DevBatchWs)

_PROTOS = {
    "tq_kv_cache_init": (_i, [_PK, _i, _PC, _i]),
    "tq_kv_cache_free": (None, [_PK]),
    "tq_attn_validate_cache": (_i, [_PK]),
    "tq_attn_rope_table": (None, [_vp, _vp, _i, _i, _f]),
    "tq_store_kv_device": (_i, [_PK, _PC, _i, _vp, _vp]),
    "tq_attend_device": (_i, [_PK, _PC, _vp, _i, _vp]),
    "tq_attention_core": (_i, [_PC, _PK, _i, _vp, _vp, _vp, _vp]),
    "tq_attention_core_batch": (_i, [_PC, _PK, _i, _i, _vp, _vp, _vp, _vp]),
    "tq_kv_cache_upload": (_i, [_PK, _vp, _vp]),
    "tq_kv_cache_download": (_i, [_PK, _vp, _vp]),
    "tq_dev_ctx_init": (_i, [_PX, _PM, _i]),
    "tq_dev_ctx_free": (None, [_PX]),
    "tq_dev_forward_token": (_i, [_PX, _i]),
    "tq_dev_batch_ws_init": (_i, [_PB, _PM, _i]),
    "tq_dev_batch_ws_free": (None, [_PB]),
    "tq_dev_forward_batch": (_i, [_PX, _PB, _vp, _i, _i]),
    "tq_dev_prefill": (_i, [_PX, _vp, _i]),
    "tq_dev_logits": (_i, [_PX, _vp]),
    "tq_dev_sample_greedy": (_i, [_PX]),
}

EXPORTS = tuple(_PROTOS)

_lib: C.CDLL | None = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libtqattn.so (once; it pulls in libtqhip.so).  Raises if unbuilt."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C tailorquantkernel_amd/host` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
    native.load()
    lib = C.CDLL(path)
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def rope_table(head_dim: int, pos: int, theta: float):
    """tq_attn_rope_table: (cos, sin), head_dim/2 each."""
    c = np.empty(head_dim // 2, np.float32)
    s = np.empty(head_dim // 2, np.float32)
    load().tq_attn_rope_table(c.ctypes.data, s.ctypes.data, head_dim, pos, theta)
    return c, s


class Cache:
    """A tq_kv_cache made by tq_kv_cache_init, with the attention calls on it.

    Methods return the C return code; outputs come back as numpy arrays.
    """

    def __init__(self, kv_type: int, cfg: AttnConfig, max_tokens: int):
        self.lib = load()
        self.cfg = cfg
        self.c = KVCache()
        self.rc = self.lib.tq_kv_cache_init(C.byref(self.c), kv_type, C.byref(cfg), max_tokens)

    def free(self) -> None:
        self.lib.tq_kv_cache_free(C.byref(self.c))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def validate(self) -> int:
        return self.lib.tq_attn_validate_cache(C.byref(self.c))

    def upload(self, k_q8: np.ndarray | None, v_q8: np.ndarray | None) -> int:
        k = None if k_q8 is None else np.ascontiguousarray(k_q8)
        v = None if v_q8 is None else np.ascontiguousarray(v_q8)
        return self.lib.tq_kv_cache_upload(C.byref(self.c), None if k is None else k.ctypes.data,
                                           None if v is None else v.ctypes.data)

    def download(self):
        cfg = self.cfg
        shape = (cfg.n_kv_heads, self.c.max_tokens, cfg.head_dim // native.QK)
        k = np.zeros(shape, native.BLOCK_Q8)
        v = np.zeros(shape, native.BLOCK_Q8)
        rc = self.lib.tq_kv_cache_download(C.byref(self.c), k.ctypes.data, v.ctypes.data)
        return rc, k, v

    def store_kv(self, pos: int, k, v) -> int:
        k, v = _f32(k), _f32(v)
        return self.lib.tq_store_kv_device(C.byref(self.c), C.byref(self.cfg), pos, k.ctypes.data,
                                           v.ctypes.data)

    def attend(self, pos: int, q):
        q = _f32(q)
        out = np.zeros(self.cfg.n_q_heads * self.cfg.head_dim, np.float32)
        rc = self.lib.tq_attend_device(C.byref(self.c), C.byref(self.cfg), q.ctypes.data, pos,
                                       out.ctypes.data)
        return rc, out

    def attention_core(self, pos: int, q, k, v):
        q, k, v = _f32(q), _f32(k), _f32(v)
        out = np.zeros(self.cfg.n_q_heads * self.cfg.head_dim, np.float32)
        rc = self.lib.tq_attention_core(C.byref(self.cfg), C.byref(self.c), pos, q.ctypes.data,
                                        k.ctypes.data, v.ctypes.data, out.ctypes.data)
        return rc, out

    def attention_core_batch(self, pos0: int, n: int, q, k, v):
        q, k, v = _f32(q), _f32(k), _f32(v)
        out = np.zeros((max(n, 0), self.cfg.n_q_heads * self.cfg.head_dim), np.float32)
        rc = self.lib.tq_attention_core_batch(C.byref(self.cfg), C.byref(self.c), pos0, n,
                                              q.ctypes.data, k.ctypes.data, v.ctypes.data,
                                              out.ctypes.data)
        return rc, out
