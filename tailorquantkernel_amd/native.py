"""ctypes binding of libtqhip.so (include/tq/tq_hip.h).

The library is built in-tree (``make -C tailorquantkernel_amd/csrc``).  Loading
fails loudly when it is missing: there is no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtqhip.so")

QK = 32
PAGE_TOKENS = 16
BLOCK_Q8 = np.dtype([("d", "<f4"), ("q", "i1", (QK,))])

OK, EINVAL, ENOMEM, ETYPE, ENODEV, ENOTREADY, ESCRATCH = 0, -1, -2, -3, -4, -5, -6
EHIP_BASE = -1000

_vp, _i, _f, _sz = C.c_void_p, C.c_int, C.c_float, C.c_size_t
_vpp = C.POINTER(C.c_void_p)


class TqHipError(RuntimeError):
    def __init__(self, code: int, what: str, msg: str):
        super().__init__(f"{what} failed: {code} ({msg})")
        self.code = code


class KVDesc(C.Structure):
    _fields_ = [("n_q_heads", _i), ("n_kv_heads", _i), ("head_dim", _i), ("n_pages", _i),
                ("max_seqs", _i), ("max_pages_per_seq", _i)]


# name -> (restype, argtypes)
_PROTOS = {
    "tq_hip_init": (_i, [_i]),
    "tq_hip_strerror": (C.c_char_p, [_i]),
    "tq_hip_device_arch": (_i, [C.c_char_p, _sz]),
    "tq_hip_malloc": (_i, [_vpp, _sz]),
    "tq_hip_free": (_i, [_vp]),
    "tq_hip_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "tq_hip_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "tq_hip_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "tq_hip_stream_synchronize": (_i, [_vp]),
    "tq_hip_device_synchronize": (_i, []),
    "tq_hip_quantize_row_q8": (_i, [_vp, _vp, _i, _vp]),
    "tq_hip_rope_apply": (_i, [_vp, _i, _i, _vp, _vp, _vp]),
    "tq_hip_attn_scores_q8": (_i, [_vp, _i, _vp, _i, _i, _f, _vp, _sz, _vp]),
    "tq_hip_attn_accum_q8": (_i, [_vp, _sz, _i, _vp, _i, _i, _vp, _sz, _vp]),
    "tq_hip_softmax": (_i, [_vp, _i, _i, _sz, _vp]),
    "tq_hip_attention_head_q8": (_i, [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp]),
    "tq_hip_kv_create": (_i, [_vpp, C.POINTER(KVDesc)]),
    "tq_hip_kv_destroy": (None, [_vp]),
    "tq_hip_kv_set_pages": (_i, [_vp, _i, _vp, _i]),
    "tq_hip_kv_capacity": (_i, [_vp, _i]),
    "tq_hip_kv_get_desc": (_i, [_vp, C.POINTER(KVDesc)]),
    "tq_hip_kv_stream": (_vp, [_vp]),
    "tq_hip_kv_pool": (_i, [_vp, _vpp, C.POINTER(_sz), _vpp]),
    "tq_hip_kv_write": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "tq_hip_kv_read": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "tq_hip_kv_append": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "tq_hip_kv_append_async": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_attend": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "tq_hip_decode_async": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_decode_step_async": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_prefill": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_prefill_async": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_membw_sink_bytes": (_sz, []),
    "tq_hip_membw_read": (_i, [_vp, _sz, _vp, C.c_uint, _vp]),
    "tq_hip_decode_step_noalloc": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_decode_step_norm_async": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _vp,
                                          _vp, _vp]),
    "tq_hip_attention_layer_ws_bytes": (_sz, [_vp, _vp, _i]),
    "tq_hip_attention_layer_async": (_i, [_vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tq_hip_rmsnorm_rows": (_i, [_vp, _vp, _vp, _i, _i, C.c_float, _vp]),
    "tq_hip_attention_layer_batch_async": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "tq_hip_mlp_ws_bytes": (_sz, [_vp, _i]),
    "tq_hip_mlp_layer_async": (_i, [_vp, _i, _vp, _vp, _vp, _sz, _vp]),
    "tq_hip_add_rmsnorm": (_i, [_vp, _vp, _vp, _vp, _i, _i, C.c_float, _vp]),
    "tq_hip_embed_lookup_q8": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "tq_hip_embed_lookup_q8_batch": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp]),
    "tq_hip_sample_greedy": (_i, [_vp, _i, _vp, _vp]),
    "tq_hip_q8_matrix_bytes": (_sz, [_i, _i]),
    "tq_hip_q8_pack": (_i, [_vp, _vp, _i, _i, _vp]),
    "tq_hip_q8_unpack": (_i, [_vp, _vp, _i, _i, _vp]),
    "tq_hip_matmul_q8": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "tq_hip_matmul_q8_batch": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tq_hip_project_qkv": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_project_output": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp, _vp]),
    "tq_hip_q4_matrix_bytes": (_sz, [_i, _i]),
    "tq_hip_q4_pack": (_i, [_vp, _vp, _i, _i, _vp]),
    "tq_hip_q4_unpack": (_i, [_vp, _vp, _i, _i, _vp]),
    "tq_hip_matmul_q4": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "tq_hip_matmul_q4_batch": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "tq_hip_project_qkv_q4": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp, _vp, _vp, _vp, _vp]),
    "tq_hip_project_output_q4": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp, _vp]),
    "tq_hip_embed_lookup_q4": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "tq_hip_embed_lookup_q4_batch": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp]),
}

EXPORTS = tuple(_PROTOS)

_lib: C.CDLL | None = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load libtqhip.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `make -C tailorquantkernel_amd/csrc` "
                           "(or __graft_entry__.build()); there is no CPU fallback")
    lib = C.CDLL(path)
    for name, (res, args) in _PROTOS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def strerror(code: int) -> str:
    return load().tq_hip_strerror(code).decode()


def check(code: int, what: str) -> int:
    if code < 0:
        raise TqHipError(code, what, strerror(code))
    return code


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def init(device: int = 0) -> None:
    check(load().tq_hip_init(device), "tq_hip_init")


def device_arch() -> str:
    buf = C.create_string_buffer(256)
    check(load().tq_hip_device_arch(buf, 256), "tq_hip_device_arch")
    return buf.value.decode()


FORMAT_Q8, FORMAT_Q4 = 0, 1   # TQ_HIP_FORMAT_Q8 / TQ_HIP_FORMAT_Q4


class MlpWeights(C.Structure):
    """tq_hip_mlp_weights: device gate/up/down matrices (tiled Q8, or tiled Q4
    with format FORMAT_Q4)."""
    _fields_ = [("wgate", C.c_void_p), ("wup", C.c_void_p), ("wdown", C.c_void_p), ("hidden", C.c_int),
                ("inter", C.c_int), ("format", C.c_int)]


class AttnWeights(C.Structure):
    """tq_hip_attn_weights: device projection matrices (tiled Q8, or tiled Q4
    with format FORMAT_Q4) and norm weights."""
    _fields_ = [("wq", C.c_void_p), ("wk", C.c_void_p), ("wv", C.c_void_p), ("wo", C.c_void_p),
                ("q_norm", C.c_void_p), ("k_norm", C.c_void_p), ("hidden", C.c_int), ("rms_eps", C.c_float),
                ("format", C.c_int)]


class DeviceBuffer:
    """A device allocation made through the C-ABI."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(load().tq_hip_malloc(C.byref(p), self.nbytes), "tq_hip_malloc")
        self.ptr = p.value

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(max(a.nbytes, 1))
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(load().tq_hip_memcpy_h2d(self.ptr, _ptr(a), a.nbytes, stream), "tq_hip_memcpy_h2d")

    def download(self, shape, dtype, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(load().tq_hip_memcpy_d2h(_ptr(out), self.ptr, out.nbytes, stream), "tq_hip_memcpy_d2h")
        return out

    def free(self) -> None:
        if self.ptr:
            load().tq_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class PagedKV:
    """The HBM-resident paged Q8 cache (tq_hip_kv)."""

    def __init__(self, n_q_heads: int, n_kv_heads: int, head_dim: int, n_pages: int,
                 max_seqs: int = 1, max_pages_per_seq: int | None = None):
        self.lib = load()
        self.desc = KVDesc(n_q_heads, n_kv_heads, head_dim, n_pages, max_seqs,
                           max_pages_per_seq if max_pages_per_seq is not None else n_pages)
        h = C.c_void_p()
        check(self.lib.tq_hip_kv_create(C.byref(h), C.byref(self.desc)), "tq_hip_kv_create")
        self.h = h.value
        self.nq, self.nkv, self.hd = n_q_heads, n_kv_heads, head_dim
        self.nb = head_dim // QK

    @classmethod
    def single(cls, n_q_heads, n_kv_heads, head_dim, max_tokens):
        """One sequence with an identity page table, like a flat cache of max_tokens."""
        n_pages = (max_tokens + PAGE_TOKENS - 1) // PAGE_TOKENS
        kv = cls(n_q_heads, n_kv_heads, head_dim, n_pages, 1, n_pages)
        kv.set_pages(0, np.arange(n_pages, dtype=np.int32))
        return kv

    def close(self) -> None:
        if self.h:
            self.lib.tq_hip_kv_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def stream(self):
        return self.lib.tq_hip_kv_stream(self.h)

    def set_pages(self, seq: int, pages) -> None:
        p = np.ascontiguousarray(pages, dtype=np.int32)
        check(self.lib.tq_hip_kv_set_pages(self.h, seq, _ptr(p), p.size), "tq_hip_kv_set_pages")

    def capacity(self, seq: int) -> int:
        return self.lib.tq_hip_kv_capacity(self.h, seq)

    def pool(self):
        base, nbytes, pt = C.c_void_p(), C.c_size_t(), C.c_void_p()
        check(self.lib.tq_hip_kv_pool(self.h, C.byref(base), C.byref(nbytes), C.byref(pt)), "tq_hip_kv_pool")
        return base.value, nbytes.value, pt.value

    def write(self, seq, pos0, k_blocks, v_blocks) -> None:
        """k/v: block_q8 arrays [nkv][n][nb]."""
        n = k_blocks.shape[1]
        check(self.lib.tq_hip_kv_write(self.h, seq, pos0, n, _ptr(np.ascontiguousarray(k_blocks)),
                                       _ptr(np.ascontiguousarray(v_blocks))), "tq_hip_kv_write")

    def read(self, seq, pos0, n):
        k = np.zeros((self.nkv, n, self.nb), BLOCK_Q8)
        v = np.zeros((self.nkv, n, self.nb), BLOCK_Q8)
        check(self.lib.tq_hip_kv_read(self.h, seq, pos0, n, _ptr(k), _ptr(v)), "tq_hip_kv_read")
        return k, v

    # ---- synchronous host-buffer entry points -------------------------------
    def append(self, seq, pos, k, v, cos_t=None, sin_t=None) -> int:
        f = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
        k, v, cos_t, sin_t = f(k), f(v), f(cos_t), f(sin_t)
        return self.lib.tq_hip_kv_append(self.h, seq, pos, _ptr(k), _ptr(v), _ptr(cos_t), _ptr(sin_t))

    def attend(self, seq, pos, q, cos_t=None, sin_t=None):
        f = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
        q, cos_t, sin_t = f(q), f(cos_t), f(sin_t)
        out = np.zeros(self.nq * self.hd, np.float32)
        rc = self.lib.tq_hip_attend(self.h, seq, pos, _ptr(q), _ptr(cos_t), _ptr(sin_t), _ptr(out))
        return rc, out

    def prefill(self, seq, pos0, n, q, k, v, cos_t=None, sin_t=None):
        f = lambda a: None if a is None else np.ascontiguousarray(a, np.float32)
        q, k, v, cos_t, sin_t = f(q), f(k), f(v), f(cos_t), f(sin_t)
        out = np.zeros((max(n, 0), self.nq * self.hd), np.float32)
        rc = self.lib.tq_hip_prefill(self.h, seq, pos0, n, _ptr(q), _ptr(k), _ptr(v), _ptr(cos_t),
                                     _ptr(sin_t), _ptr(out))
        return rc, out
