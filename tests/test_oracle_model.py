"""Pins the oracle's rest of the transformer block and the token forward:
oracle_silu_mul (model/silu.c:6-18), oracle_mlp_layer (model/mlp.c:3-17),
oracle_embed_lookup_q8 (model/embedding.c:4-17), oracle_sample_greedy
(model/sampler.c:3-13) and oracle_forward_token (model/context.c:104-126).

Anchors: bit-exact against the compiled reference (its silu_mul, mlp_layer,
sample_greedy, and tq_ctx_init + tq_forward_token through oracle/_ref's
tqref_forward_run: logits of every token equal bit for bit); and closed forms:
silu(0) = 0, silu(x) - silu(-x) = x, the MLP against an fp64 evaluation of the
quantized product chain, greedy ties to the first index.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import Model, QK, ptr


def test_silu_mul_vs_reference_and_identities(oracle, ref_scalar):
    rng = np.random.default_rng(1)
    g = (rng.standard_normal(5000) * 6).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    out_o = oracle.silu_mul(g, u)
    out_r = np.zeros_like(g)
    ref_scalar.lib.silu_mul(ptr(g), ptr(u), ptr(out_r), g.size)
    assert out_o.tobytes() == out_r.tobytes()
    ones = np.ones(5, np.float32)
    assert oracle.silu_mul(np.zeros(5, np.float32), ones).tolist() == [0.0] * 5
    x = np.linspace(-8, 8, 101).astype(np.float32)
    d = oracle.silu_mul(x, np.ones_like(x)).astype(np.float64) - oracle.silu_mul(-x, np.ones_like(x))
    np.testing.assert_allclose(d, x, rtol=0, atol=2e-6)


def test_mlp_vs_reference_and_fp64(oracle, ref_scalar):
    rng = np.random.default_rng(2)
    for hidden, inter in ((128, 320), (256, 512), (64, 96)):
        wg = oracle.pack_matrix_q8(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
        wu = oracle.pack_matrix_q8(rng.standard_normal((inter, hidden)).astype(np.float32) * 0.1)
        wd = oracle.pack_matrix_q8(rng.standard_normal((hidden, inter)).astype(np.float32) * 0.1)
        xn = rng.standard_normal(hidden).astype(np.float32)
        out_o = oracle.mlp_layer(wg, wu, wd, hidden, inter, xn)
        out_r = np.zeros(hidden, np.float32)
        assert ref_scalar.lib.tqref_mlp_run(hidden, inter, ptr(wg), ptr(wu), ptr(wd), ptr(xn), ptr(out_r)) == 0
        assert out_o.tobytes() == out_r.tobytes()
        # fp64 chain on the same quantized operands (gate/up from quantized xn, h re-quantized)
        xq = oracle.quantize_row_q8(xn)
        deq = lambda b: (b["q"].astype(np.float64) * b["d"][..., None]).reshape(-1)
        W = lambda m, r, c: (m["q"].astype(np.float64) * m["d"][..., None]).reshape(r, c)
        g = W(wg, inter, hidden) @ deq(xq)
        u = W(wu, inter, hidden) @ deq(xq)
        h = g / (1 + np.exp(-g)) * u
        ref64 = W(wd, hidden, inter) @ deq(oracle.quantize_row_q8(h.astype(np.float32)))
        assert np.sqrt(((out_o - ref64) ** 2).sum() / (ref64 ** 2).sum()) < 2e-2


def test_sample_greedy(oracle, ref_scalar):
    L = oracle.lib
    for logits in (np.array([0.5, 2.0, 2.0, -1.0], np.float32), np.array([-3.0], np.float32),
                   np.array([1.0, np.nan, 3.0], np.float32), np.array([-np.inf, -np.inf], np.float32)):
        a = L.oracle_sample_greedy(ptr(logits), logits.size)
        b = ref_scalar.lib.sample_greedy(ptr(logits), logits.size)
        assert a == b
    tie = np.array([0.5, 2.0, 2.0], np.float32)
    assert L.oracle_sample_greedy(ptr(tie), 3) == 1
    assert L.oracle_sample_greedy(None, 0) == -1


def test_embed_lookup(oracle):
    rng = np.random.default_rng(3)
    E = oracle.pack_matrix_q8(rng.standard_normal((50, 96)).astype(np.float32))
    out = np.zeros(96, np.float32)
    assert oracle.lib.oracle_embed_lookup_q8(ptr(E), 50, 96, 7, ptr(out)) == 0
    exp = (E[7]["q"].astype(np.float32) * E[7]["d"][:, None]).reshape(-1)
    assert out.tobytes() == exp.astype(np.float32).tobytes()
    assert oracle.lib.oracle_embed_lookup_q8(ptr(E), 50, 96, 50, ptr(out)) == -1


def test_forward_token_vs_reference(oracle, ref_scalar):
    for shape in ((2, 4, 2, 32, 128, 256, 300), (1, 8, 2, 64, 256, 512, 97)):
        m = Model(oracle, *shape, seed=shape[0])
        tokens = [3, 77, 12, 3, 96, 0]
        lo, kc, vc = oracle.forward(m, tokens, 8)
        lr = ref_scalar.forward(m, tokens, 8)
        assert lo.tobytes() == lr.tobytes()
        assert [oracle.lib.oracle_sample_greedy(ptr(lo[i]), m.vocab) for i in range(len(tokens))] == \
               [int(np.argmax(lr[i])) for i in range(len(tokens))]


@pytest.mark.parametrize("fmt,embed_fmt", [("q4", "q4"), ("q4", "q8"), ("q8", "q4")])
def test_forward_token_q4_vs_reference(oracle, ref_scalar, fmt, embed_fmt):
    """The forward with Q4 layer matrices and/or a Q4 embedding (get_matmul and
    embed_lookup on TQ_FORMAT_Q4, kernel/q4_scalar.c, model/embedding.c:20-27):
    bit-exact against the reference's scalar build, and its own prefill."""
    m = Model(oracle, 2, 4, 2, 32, 128, 256, 300, seed=5, fmt=fmt, embed_fmt=embed_fmt)
    tokens = [3, 77, 12, 3, 96, 0]
    lo, kc, vc = oracle.forward(m, tokens, 8)
    lr = ref_scalar.forward(m, tokens, 8)
    assert lo.tobytes() == lr.tobytes()
    lp, rk, rv = ref_scalar.prefill(m, tokens, 8)
    assert lp.tobytes() == lr[-1].tobytes()
    for l in range(m.n_layers):
        n = len(tokens)
        own = kc[l].reshape(m.nkv, 8, -1)[:, :n]
        assert own.tobytes() == rk[l].reshape(m.nkv, 8, -1)[:, :n].tobytes()
