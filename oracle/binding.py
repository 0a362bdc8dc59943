"""ctypes binding for the CPU oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg.  The product package (tailorquantkernel_amd) never
imports it.

* ``Oracle``  — liboracle.so, the C restatement of the reference's scalar Q8
  attention path (oracle/tq_oracle.c).
* ``Ref``     — oracle/_ref/libtqref{,_scalar}.so, the reference's own C sources
  compiled by oracle/Makefile plus oracle/ref_driver.c.  Present only where it
  was built; ``Ref.available()`` says whether it is.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
QK = 32
BLOCK_Q8 = np.dtype([("d", "<f4"), ("q", "i1", (QK,))])
BLOCK_Q4 = np.dtype([("d", "<f4"), ("q", "u1", (QK // 2,))])
assert BLOCK_Q8.itemsize == 36

_f32p = C.POINTER(C.c_float)
_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t


def ptr(a: np.ndarray | None):
    """Data pointer of a C-contiguous array (None -> NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to C must be contiguous"
    return a.ctypes.data


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def blocks(n: int) -> np.ndarray:
    return np.zeros(n, dtype=BLOCK_Q8)


def blocks4(n: int) -> np.ndarray:
    return np.zeros(n, dtype=BLOCK_Q4)


def dequant(b: np.ndarray) -> np.ndarray:
    """block_q8 rows -> fp32 values (d * q), shape (..., nb*32)."""
    vals = b["q"].astype(np.float32) * b["d"][..., None]
    return vals.reshape(*b.shape[:-1], b.shape[-1] * QK) if b.ndim > 1 else vals.reshape(-1)


def _load(path: str) -> C.CDLL:
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} is not built (run `make -C oracle` / `make -C oracle ref`)")
    return C.CDLL(path)


class Oracle:
    """The C restatement (liboracle.so)."""

    def __init__(self, path: str | None = None):
        self.lib = _load(path or os.path.join(HERE, "liboracle.so"))
        L = self.lib
        L.oracle_quantize_row_q8.argtypes = [_vp, _vp, _i]
        L.oracle_rope_table.argtypes = [_vp, _vp, _i, _i, _f]
        L.oracle_rope_apply.argtypes = [_vp, _i, _vp, _vp]
        L.oracle_softmax.argtypes = [_vp, _i]
        L.oracle_attn_scores_q8.argtypes = [_vp, _i, _vp, _i, _i, _f, _vp, _sz]
        L.oracle_attn_accum_q8.argtypes = [_vp, _sz, _i, _vp, _i, _i, _vp, _sz]
        L.oracle_attention_head_q8.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp]
        L.oracle_store_kv_q8.argtypes = [_vp, _vp, _i, _i, _i, _i, _vp, _vp]
        L.oracle_store_kv_q8.restype = _i
        L.oracle_attend_q8.argtypes = [_vp, _vp, _i, _i, _i, _i, _vp, _i, _vp, _vp]
        L.oracle_attend_q8.restype = _i
        L.oracle_attention_qkv.argtypes = [_vp, _vp, _i, _i, _i, _i, _f, _i, _vp, _vp, _vp, _vp, _vp]
        L.oracle_attention_qkv.restype = _i
        L.oracle_prefill_qkv.argtypes = [_vp, _vp, _i, _i, _i, _i, _f, _i, _i, _vp, _vp, _vp, _vp, _vp]
        L.oracle_prefill_qkv.restype = _i
        L.oracle_rmsnorm.argtypes = [_vp, _vp, _vp, _i, _f]
        L.oracle_attention_layer.argtypes = [_vp] * 6 + [_i, _i, _i, _i, _f, _f, _vp, _vp, _i, _i, _vp, _vp, _vp]
        L.oracle_attention_layer.restype = _i
        L.oracle_silu_mul.argtypes = [_vp, _vp, _vp, _i]
        L.oracle_mlp_layer.argtypes = [_vp, _vp, _vp, _i, _i, _vp, _vp]
        L.oracle_mlp_layer.restype = _i
        L.oracle_embed_lookup_q8.argtypes = [_vp, _i, _i, _i, _vp]
        L.oracle_embed_lookup_q8.restype = _i
        L.oracle_sample_greedy.argtypes = [_vp, _i]
        L.oracle_sample_greedy.restype = _i
        L.oracle_forward_token.argtypes = [_vp, _vp, _vp, _i, _i, _i, _vp]
        L.oracle_forward_token.restype = _i
        L.oracle_pack_matrix_q8.argtypes = [_vp, _i, _i, _vp]
        L.oracle_matmul_q8.argtypes = [_vp, _vp, _vp, _i, _i]
        L.oracle_matmul_q8_batch.argtypes = [_vp, _vp, _vp, _i, _i, _i]
        L.oracle_project_q8.argtypes = [_vp, _i, _i, _vp, _i, _vp]
        L.oracle_pack_matrix_q4.argtypes = [_vp, _i, _i, _vp]
        L.oracle_unpack_matrix_q4.argtypes = [_vp, _i, _i, _vp]
        L.oracle_matmul_q4_batch.argtypes = [_vp, _vp, _vp, _i, _i, _i]
        L.oracle_embed_lookup_q4.argtypes = [_vp, _i, _i, _i, _vp]
        L.oracle_embed_lookup_q4.restype = _i

    # --- element ops -------------------------------------------------------
    def quantize_row_q8(self, x) -> np.ndarray:
        x = f32(x).reshape(-1)
        out = blocks(x.size // QK)
        self.lib.oracle_quantize_row_q8(ptr(x), ptr(out), x.size)
        return out

    def rope_table(self, head_dim: int, pos: int, theta: float):
        c = np.zeros(head_dim // 2, np.float32)
        s = np.zeros(head_dim // 2, np.float32)
        self.lib.oracle_rope_table(ptr(c), ptr(s), head_dim, pos, theta)
        return c, s

    def rope_apply(self, x, cos_t, sin_t) -> np.ndarray:
        x = f32(x).copy()
        c, sn = f32(cos_t), f32(sin_t)   # held across the call (ptr of a temporary dangles)
        self.lib.oracle_rope_apply(ptr(x), x.size, ptr(c), ptr(sn))
        return x

    def softmax(self, x) -> np.ndarray:
        x = f32(x).copy()
        self.lib.oracle_softmax(ptr(x), x.size)
        return x

    def attn_scores_q8(self, q, g, k, n, nb, scale, scores, stride):
        self.lib.oracle_attn_scores_q8(ptr(q), g, ptr(k), n, nb, scale, ptr(scores), stride)

    def attn_accum_q8(self, w, w_stride, g, v, n, nb, out, out_stride):
        self.lib.oracle_attn_accum_q8(ptr(w), w_stride, g, ptr(v), n, nb, ptr(out), out_stride)

    def attention_head_q8(self, q, k, v, n, head_dim):
        q = f32(q)
        qq = blocks(head_dim // QK)
        scores = np.zeros(max(n, 1), np.float32)
        out = np.zeros(head_dim, np.float32)
        self.lib.oracle_attention_head_q8(ptr(q), ptr(qq), ptr(k), ptr(v), n, head_dim,
                                          ptr(scores), ptr(out))
        return out, qq, scores

    # --- layer-level -------------------------------------------------------
    def attention_qkv(self, kc, vc, nq, nkv, hd, max_tokens, theta, pos, q, k, v):
        """RoPE + store_kv + attend_q8 on flat caches (modified in place)."""
        q = f32(q).copy()
        k = f32(k).copy()
        v = f32(v)
        scores = np.zeros(nq * max_tokens, np.float32)
        out = np.zeros(nq * hd, np.float32)
        rc = self.lib.oracle_attention_qkv(ptr(kc), ptr(vc), nq, nkv, hd, max_tokens, theta, pos,
                                           ptr(q), ptr(k), ptr(v), ptr(scores), ptr(out))
        return rc, out

    def prefill_qkv(self, kc, vc, nq, nkv, hd, max_tokens, theta, pos0, n, q, k, v):
        q = f32(q).copy()
        k = f32(k).copy()
        v = f32(v)
        scores = np.zeros(nq * max_tokens, np.float32)
        out = np.zeros((max(n, 0), nq * hd), np.float32)
        rc = self.lib.oracle_prefill_qkv(ptr(kc), ptr(vc), nq, nkv, hd, max_tokens, theta, pos0, n,
                                         ptr(q), ptr(k), ptr(v), ptr(scores), ptr(out))
        return rc, out

    def rmsnorm(self, x, weight, eps: float) -> np.ndarray:
        """model/rmsnorm.c on each row of x (rows of len(weight))."""
        w = f32(weight)
        x = f32(x).reshape(-1, w.size).copy()
        for r in range(x.shape[0]):
            row = x[r]
            self.lib.oracle_rmsnorm(ptr(row), ptr(w), ptr(row), w.size, eps)
        return x.reshape(-1)

    def attention_layer(self, w, nq, nkv, hd, hidden, theta, eps, kc, vc, max_tokens, pos, xn):
        """attention_layer for one token; w = (wq, wk, wv, wo, q_norm, k_norm); caches in place."""
        wq, wk, wv, wo, qn, kn = (np.ascontiguousarray(a) for a in w)
        scores = np.zeros(nq * max_tokens, np.float32)
        out = np.zeros(hidden, np.float32)
        qn, kn, xn = f32(qn), f32(kn), f32(xn)
        rc = self.lib.oracle_attention_layer(ptr(wq), ptr(wk), ptr(wv), ptr(wo), ptr(qn), ptr(kn),
                                             nq, nkv, hd, hidden, theta, eps, ptr(kc), ptr(vc), max_tokens,
                                             pos, ptr(xn), ptr(scores), ptr(out))
        return rc, out

    # --- the rest of the block ----------------------------------------------
    def silu_mul(self, g, u) -> np.ndarray:
        g, u = f32(g), f32(u)
        out = np.zeros_like(g)
        self.lib.oracle_silu_mul(ptr(g), ptr(u), ptr(out), g.size)
        return out

    def mlp_layer(self, wgate, wup, wdown, hidden, inter, xn) -> np.ndarray:
        out = np.zeros(hidden, np.float32)
        wgate, wup, wdown, xn = (np.ascontiguousarray(wgate), np.ascontiguousarray(wup), np.ascontiguousarray(wdown),
                                 f32(xn))
        rc = self.lib.oracle_mlp_layer(ptr(wgate), ptr(wup), ptr(wdown), hidden, inter, ptr(xn), ptr(out))
        assert rc == 0
        return out

    def forward(self, model, tokens, max_tokens):
        """tq_forward_token over `tokens` on fresh caches; logits [len(tokens)][vocab]."""
        nb = model.hd // QK
        kc = [blocks(model.nkv * max_tokens * nb) for _ in range(model.n_layers)]
        vc = [blocks(model.nkv * max_tokens * nb) for _ in range(model.n_layers)]
        karr = (C.c_void_p * model.n_layers)(*[ptr(c) for c in kc])
        varr = (C.c_void_p * model.n_layers)(*[ptr(c) for c in vc])
        st, keep = model.struct()
        out = np.zeros((len(tokens), model.vocab), np.float32)
        for i, t in enumerate(tokens):
            rc = self.lib.oracle_forward_token(C.byref(st), karr, varr, max_tokens, i, int(t), ptr(out[i]))
            assert rc == 0, rc
        return out, kc, vc

    # --- weight side ---------------------------------------------------------
    def pack_matrix_q8(self, W) -> np.ndarray:
        """rows x cols floats -> rows x cols/32 block_q8 (packer/packer.c)."""
        W = f32(W)
        rows, cols = W.shape
        out = blocks(rows * (cols // QK)).reshape(rows, cols // QK)
        self.lib.oracle_pack_matrix_q8(ptr(W), rows, cols, ptr(out))
        return out

    def pack_matrix_q4(self, W) -> np.ndarray:
        """rows x cols floats -> rows x cols/32 block_q4 (packer/packer.c:40-52)."""
        W = f32(W)
        rows, cols = W.shape
        out = blocks4(rows * (cols // QK)).reshape(rows, cols // QK)
        self.lib.oracle_pack_matrix_q4(ptr(W), rows, cols, ptr(out))
        return out

    def unpack_matrix_q4(self, Wq, rows: int, cols: int) -> np.ndarray:
        out = np.zeros((rows, cols), np.float32)
        Wq = np.ascontiguousarray(Wq)
        assert Wq.size == rows * (cols // QK)
        self.lib.oracle_unpack_matrix_q4(ptr(Wq), rows, cols, ptr(out))
        return out

    def matmul_q4(self, Wq, xq, rows: int, cols: int, n_tok: int = 1) -> np.ndarray:
        """y[n_tok, rows] from block_q4 weights and n_tok block_q8 rows."""
        y = np.zeros((n_tok, rows), np.float32)
        Wq = np.ascontiguousarray(Wq)
        xq = np.ascontiguousarray(xq)
        assert Wq.size == rows * (cols // QK) and xq.size == n_tok * (cols // QK)
        self.lib.oracle_matmul_q4_batch(ptr(Wq), ptr(xq), ptr(y), rows, cols, n_tok)
        return y

    def embed_lookup_q4(self, E, rows: int, cols: int, token: int):
        out = np.zeros(cols, np.float32)
        E = np.ascontiguousarray(E)
        rc = self.lib.oracle_embed_lookup_q4(ptr(E), rows, cols, token, ptr(out))
        return rc, out

    def matmul_q8(self, Wq, xq, rows: int, cols: int, n_tok: int = 1) -> np.ndarray:
        """y[n_tok, rows] from block_q8 weights and n_tok block_q8 rows."""
        y = np.zeros((n_tok, rows), np.float32)
        Wq = np.ascontiguousarray(Wq)
        xq = np.ascontiguousarray(xq)
        assert Wq.size == rows * (cols // QK) and xq.size == n_tok * (cols // QK)
        self.lib.oracle_matmul_q8_batch(ptr(Wq), ptr(xq), ptr(y), rows, cols, n_tok)
        return y

    def project_q8(self, Wq, rows: int, cols: int, x) -> np.ndarray:
        """quantize_row_q8 of each row of x, then the Q8 matmul: y[n_tok, rows]."""
        x = f32(x).reshape(-1, cols)
        y = np.zeros((x.shape[0], rows), np.float32)
        Wq = np.ascontiguousarray(Wq)
        assert Wq.size == rows * (cols // QK)
        self.lib.oracle_project_q8(ptr(Wq), rows, cols, ptr(x), x.shape[0], ptr(y))
        return y

    def attend_q8(self, kc, vc, nq, nkv, hd, max_tokens, q, pos):
        scores = np.zeros(nq * max_tokens, np.float32)
        out = np.zeros(nq * hd, np.float32)
        q = f32(q)
        rc = self.lib.oracle_attend_q8(ptr(kc), ptr(vc), nq, nkv, hd, max_tokens, ptr(q), pos,
                                       ptr(scores), ptr(out))
        return rc, out


class OracleModel(C.Structure):
    """struct oracle_model (oracle/tq_oracle.h): a Q8 or Q4 model as flat per-layer pointer arrays."""
    _fields_ = [("n_layers", _i), ("n_q_heads", _i), ("n_kv_heads", _i), ("head_dim", _i), ("hidden", _i),
                ("inter", _i), ("vocab", _i), ("rope_theta", _f), ("rms_eps", _f), ("embed", _vp),
                ("final_norm", _vp), ("input_norm", _vp), ("post_norm", _vp), ("wq", _vp), ("wk", _vp),
                ("wv", _vp), ("wo", _vp), ("q_norm", _vp), ("k_norm", _vp), ("wgate", _vp), ("wup", _vp),
                ("wdown", _vp), ("format", _i), ("embed_format", _i)]


class Model:
    """A random model held as numpy arrays, in the shapes tq_model uses: layer
    matrices in `fmt` ("q8" or "q4"), the embedding in `embed_fmt`."""

    def __init__(self, oracle, n_layers, nq, nkv, hd, hidden, inter, vocab, theta=5e5, eps=1e-6, seed=0,
                 fmt="q8", embed_fmt="q8"):
        rng = np.random.default_rng(seed)
        self.n_layers, self.nq, self.nkv, self.hd = n_layers, nq, nkv, hd
        self.hidden, self.inter, self.vocab, self.theta, self.eps = hidden, inter, vocab, theta, eps
        self.format, self.embed_format = int(fmt == "q4"), int(embed_fmt == "q4")

        def mat(r, c, scale, f=fmt):
            pack = oracle.pack_matrix_q4 if f == "q4" else oracle.pack_matrix_q8
            return pack((rng.standard_normal((r, c)) * scale).astype(np.float32)).reshape(-1)

        def norm(n):
            return rng.uniform(0.6, 1.4, n).astype(np.float32)

        self.embed = mat(vocab, hidden, 1.0, embed_fmt)
        self.final_norm = norm(hidden)
        self.layers = []
        for _ in range(n_layers):
            self.layers.append(dict(
                input_norm=norm(hidden), post_norm=norm(hidden),
                wq=mat(nq * hd, hidden, 0.05), wk=mat(nkv * hd, hidden, 0.05), wv=mat(nkv * hd, hidden, 0.05),
                wo=mat(hidden, nq * hd, 0.05), q_norm=norm(hd), k_norm=norm(hd),
                wgate=mat(inter, hidden, 0.05), wup=mat(inter, hidden, 0.05), wdown=mat(hidden, inter, 0.05)))

    def ptr_array(self, key):
        arr = (C.c_void_p * self.n_layers)(*[ptr(l[key]) for l in self.layers])
        return arr

    def struct(self):
        keep = {k: self.ptr_array(k) for k in ("input_norm", "post_norm", "wq", "wk", "wv", "wo", "q_norm",
                                              "k_norm", "wgate", "wup", "wdown")}
        st = OracleModel(self.n_layers, self.nq, self.nkv, self.hd, self.hidden, self.inter, self.vocab,
                         self.theta, self.eps, ptr(self.embed), ptr(self.final_norm),
                         *[C.cast(keep[k], C.c_void_p) for k in ("input_norm", "post_norm", "wq", "wk", "wv",
                                                                  "wo", "q_norm", "k_norm", "wgate", "wup",
                                                                  "wdown")],
                         getattr(self, "format", 0), getattr(self, "embed_format", 0))
        return st, keep


class Ref:
    """The reference compiled from its own sources (oracle/_ref).

    dropin="fused" / "route" loads the scalar build whose attention_layer.c,
    context.c and model_ops.h carry the MI355X library's drop-in edits
    (oracle/dropin_patch.sh) and which links libtqattn.so: its entry points
    take TQ_KV_Q8_DEVICE caches after set_kv_type(TQ_KV_Q8_DEVICE)."""

    TQ_KV_Q8, TQ_KV_Q8_DEVICE = 1, 2

    @staticmethod
    def _name(scalar: bool, dropin: str | None) -> str:
        if dropin == "fused":
            return "libtqref_dropin.so"
        if dropin == "route":
            return "libtqref_dropin_route.so"
        return "libtqref_scalar.so" if scalar else "libtqref.so"

    def __init__(self, scalar: bool = False, dropin: str | None = None):
        self.lib = _load(os.path.join(HERE, "_ref", self._name(scalar, dropin)))
        self.dropin = dropin
        scalar = scalar or dropin is not None
        L = self.lib
        L.tqref_capture_attn.argtypes = [_vp]
        if dropin is not None:
            L.tqref_set_kv_type.argtypes = [_i]
            L.tqref_set_cache_q_heads.argtypes = [_i]
            L.tqref_layer_steps.argtypes = [_i, _i, _i, _i, _f, _f] + [_vp] * 6 + [_vp, _vp, _i, _i, _i, _vp, _vp,
                                                                                   _vp]
            L.tqref_layer_steps.restype = _i
            L.tqref_forward_devmodel_run.argtypes = [_i] * 7 + [_f, _f] + [_vp] * 13 + [_i, _i] + [_i, _i, _vp, _vp]
            L.tqref_forward_devmodel_run.restype = _i
        L.quantize_row_q8.argtypes = [_vp, _vp, _i]
        L.rope_table.argtypes = [_vp, _vp, _i, _i, _f]
        L.rope_apply.argtypes = [_vp, _i, _vp, _vp]
        L.softmax.argtypes = [_vp, _i]
        L.attn_scores_q8_scalar.argtypes = [_vp, _i, _vp, _i, _i, _f, _vp, _sz]
        L.attn_accum_q8_scalar.argtypes = [_vp, _sz, _i, _vp, _i, _i, _vp, _sz]
        L.attn_scores_q8.argtypes = [_vp, _i, _vp, _i, _i, _f, _vp, _sz]
        L.attn_accum_q8.argtypes = [_vp, _sz, _i, _vp, _i, _i, _vp, _sz]
        L.attention_head_q8.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp]
        L.tqref_layer_run.argtypes = [_i, _i, _i, _i, _f, _f] + [_vp] * 6 + [_vp, _vp, _i, _i, _vp, _vp, _vp]
        L.tqref_layer_run.restype = _i
        L.tqref_layer_batch_run.argtypes = [_i, _i, _i, _i, _f, _f] + [_vp] * 6 + [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]
        L.tqref_layer_batch_run.restype = _i
        L.tqref_project_qkv.argtypes = [_i, _i, _i, _i, _f] + [_vp] * 5 + [_vp, _vp, _vp, _vp]
        L.tqref_project_qkv.restype = _i
        L.tqref_project_out.argtypes = [_i, _i, _i, _vp, _vp, _vp]
        L.tqref_project_out.restype = _i
        L.tqref_attention_qkv.argtypes = [_i, _i, _i, _i, _f, _vp, _vp, _i, _vp, _vp, _vp, _vp, _vp]
        L.tqref_attention_qkv.restype = _i
        L.tqref_isa.restype = C.c_char_p
        L.rmsnorm.argtypes = [_vp, _vp, _vp, _i, _f]
        L.silu_mul.argtypes = [_vp, _vp, _vp, _i]
        L.sample_greedy.argtypes = [_vp, _i]
        L.sample_greedy.restype = _i
        L.tqref_mlp_run.argtypes = [_i, _i, _vp, _vp, _vp, _vp, _vp]
        L.tqref_mlp_run.restype = _i
        L.tqref_forward_run.argtypes = [_i] * 7 + [_f, _f] + [_vp] * 13 + [_i, _i] + [_i, _i, _vp, _vp]
        L.tqref_forward_run.restype = _i
        L.tqref_prefill_run.argtypes = [_i] * 7 + [_f, _f] + [_vp] * 13 + [_i, _i] + [_i, _i, _vp, _vp, _vp, _vp]
        L.tqref_prefill_run.restype = _i
        L.pack_matrix.argtypes = [_vp, _i, _i, _vp, C.c_char]
        L.pack_matrix.restype = _i
        L.unpack_matrix.argtypes = [_vp, _i, _i, _vp, C.c_char]
        L.unpack_matrix.restype = _i
        simd = ("matmul_q8_avx2", "matmul_q4_avx2") if not scalar else ()
        for fn in ("matmul_q8_scalar", "matmul_q4_scalar") + simd:
            getattr(L, fn).argtypes = [_vp, _vp, _vp, _i, _i]
            getattr(L, fn + "_batch").argtypes = [_vp, _vp, _vp, _i, _i, _i]

    @staticmethod
    def available(scalar: bool = False, dropin: str | None = None) -> bool:
        return os.path.exists(os.path.join(HERE, "_ref", Ref._name(scalar, dropin)))

    def set_kv_type(self, kv_type: int) -> None:
        self.lib.tqref_set_kv_type(kv_type)

    def forward_devmodel(self, model, tokens, max_tokens):
        """tq_forward_token with ctx.dev set: each token on the device model
        built from the same weights (the edited context.c's branch)."""
        st, keep = model.struct()
        toks = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros((len(toks), model.vocab), np.float32)
        rc = self.lib.tqref_forward_devmodel_run(
            model.n_layers, model.nq, model.nkv, model.hd, model.hidden, model.inter, model.vocab, model.theta,
            model.eps, ptr(model.embed), ptr(model.final_norm),
            *[keep[k] for k in ("input_norm", "post_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm", "wgate",
                                "wup", "wdown")],
            getattr(model, "format", 0), getattr(model, "embed_format", 0), max_tokens, len(toks), ptr(toks),
            ptr(out))
        assert rc == 0, rc
        return out

    def isa(self) -> str:
        return self.lib.tqref_isa().decode()

    def forward(self, model, tokens, max_tokens):
        """The reference's tq_forward_token over `tokens` (tq_ctx with TQ_KV_Q8 caches)."""
        st, keep = model.struct()
        toks = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros((len(toks), model.vocab), np.float32)
        rc = self.lib.tqref_forward_run(model.n_layers, model.nq, model.nkv, model.hd, model.hidden, model.inter,
                                        model.vocab, model.theta, model.eps, ptr(model.embed),
                                        ptr(model.final_norm), *[keep[k] for k in (
                                            "input_norm", "post_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm",
                                            "wgate", "wup", "wdown")], getattr(model, "format", 0),
                                        getattr(model, "embed_format", 0), max_tokens, len(toks), ptr(toks),
                                        ptr(out))
        assert rc == 0, rc
        return out

    def prefill(self, model, tokens, max_tokens):
        """The reference's tq_prefill over `tokens` on fresh TQ_KV_Q8 caches: the last
        token's logits [vocab] and per-layer K and V caches."""
        st, keep = model.struct()
        toks = np.ascontiguousarray(tokens, np.int32)
        out = np.zeros(model.vocab, np.float32)
        nb = model.hd // QK
        kc = [blocks(model.nkv * max_tokens * nb) for _ in range(model.n_layers)]
        vc = [blocks(model.nkv * max_tokens * nb) for _ in range(model.n_layers)]
        karr = (C.c_void_p * model.n_layers)(*[ptr(c) for c in kc])
        varr = (C.c_void_p * model.n_layers)(*[ptr(c) for c in vc])
        rc = self.lib.tqref_prefill_run(model.n_layers, model.nq, model.nkv, model.hd, model.hidden, model.inter,
                                        model.vocab, model.theta, model.eps, ptr(model.embed),
                                        ptr(model.final_norm), *[keep[k] for k in (
                                            "input_norm", "post_norm", "wq", "wk", "wv", "wo", "q_norm", "k_norm",
                                            "wgate", "wup", "wdown")], getattr(model, "format", 0),
                                        getattr(model, "embed_format", 0), max_tokens, len(toks), ptr(toks),
                                        ptr(out), karr, varr)
        assert rc == 0, rc
        return out, kc, vc

    def rmsnorm(self, x, weight, eps: float) -> np.ndarray:
        w = f32(weight)
        x = f32(x).reshape(-1, w.size)
        out = np.zeros_like(x)
        for r in range(x.shape[0]):
            xr = np.ascontiguousarray(x[r])
            o = out[r]
            self.lib.rmsnorm(ptr(xr), ptr(w), ptr(o), w.size, eps)
        return out.reshape(-1)

    def pack_matrix_q8(self, W) -> np.ndarray:
        W = f32(W)
        rows, cols = W.shape
        out = blocks(rows * (cols // QK)).reshape(rows, cols // QK)
        rc = self.lib.pack_matrix(ptr(W), rows, cols, ptr(out), b"8")
        assert rc == 0
        return out

    def pack_matrix_q4(self, W) -> np.ndarray:
        W = f32(W)
        rows, cols = W.shape
        out = blocks4(rows * (cols // QK)).reshape(rows, cols // QK)
        rc = self.lib.pack_matrix(ptr(W), rows, cols, ptr(out), b"4")
        assert rc == 0
        return out

    def unpack_matrix_q4(self, Wq, rows: int, cols: int) -> np.ndarray:
        out = np.zeros((rows, cols), np.float32)
        Wq = np.ascontiguousarray(Wq)
        rc = self.lib.unpack_matrix(ptr(Wq), rows, cols, ptr(out), b"4")
        assert rc == 0
        return out

    def matmul_q4(self, Wq, xq, rows: int, cols: int, n_tok: int = 1, simd: bool = False):
        """matmul_q4_scalar / matmul_q4_avx2 (their _batch forms for n_tok > 1)."""
        return self.matmul_q8(Wq, xq, rows, cols, n_tok, simd, fmt="q4")

    def matmul_q8(self, Wq, xq, rows: int, cols: int, n_tok: int = 1, simd: bool = False, fmt: str = "q8"):
        """matmul_q8_scalar / matmul_q8_avx2 (their _batch forms for n_tok > 1)."""
        y = np.zeros((n_tok, rows), np.float32)
        Wq = np.ascontiguousarray(Wq)
        xq = np.ascontiguousarray(xq)
        name = f"matmul_{fmt}_avx2" if simd else f"matmul_{fmt}_scalar"
        if n_tok == 1:
            getattr(self.lib, name)(ptr(Wq), ptr(xq), ptr(y), rows, cols)
        else:
            getattr(self.lib, name + "_batch")(ptr(Wq), ptr(xq), ptr(y), rows, cols, n_tok)
        return y
