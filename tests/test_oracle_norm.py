"""Pins oracle_rmsnorm (model/rmsnorm.c:4-19) and oracle_attention_layer
(model/attention_layer.c:169-194), the whole layer composed from the oracle's
own projections, norm and attention core.

Anchors: bit-exact against the compiled reference (its rmsnorm, and its real
attention_layer through oracle/_ref's tqref_layer_run); and what the
mathematics fixes for the norm: the fp64 value x*w/sqrt(eps + mean(x^2))
within a few ulp, unit RMS with unit weights, a zero row giving zero, the
weights applied per element (a transposed or missing weight fails).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle.binding import QK, blocks, ptr
from tests.golden.gen import fill_random


def test_rmsnorm_vs_reference(oracle, ref_scalar):
    rng = np.random.default_rng(3)
    for n, scale, eps in ((128, 1.0, 1e-6), (64, 40.0, 1e-5), (32, 1e-3, 1e-6), (256, 3.0, 0.0), (128, 1e-20, 1e-6)):
        x = (rng.standard_normal(4 * n) * scale).astype(np.float32)
        w = (1.0 + 0.5 * rng.standard_normal(n)).astype(np.float32)
        assert oracle.rmsnorm(x, w, eps).tobytes() == ref_scalar.rmsnorm(x, w, eps).tobytes()


def test_rmsnorm_closed_forms(oracle):
    rng = np.random.default_rng(5)
    n, eps = 128, 1e-6
    x = rng.standard_normal(n).astype(np.float32) * 2
    w = rng.uniform(0.5, 2.0, n).astype(np.float32)
    got = oracle.rmsnorm(x, w, eps).astype(np.float64)
    x64 = x.astype(np.float64)
    exact = x64 * w / np.sqrt(eps + (x64 * x64).mean())
    # n serial adds, a divide, a sqrt, a reciprocal and two products
    assert (np.abs(got - exact) <= (n + 8) * 2.0 ** -24 * np.abs(exact) + 1e-30).all()
    ones = np.ones(n, np.float32)
    u = oracle.rmsnorm(x, ones, 0.0).astype(np.float64)
    assert abs(np.sqrt((u * u).mean()) - 1.0) < 1e-5
    assert (oracle.rmsnorm(np.zeros(n, np.float32), w, eps) == 0.0).all()
    # the weight is per element: permuting it permutes the output's scaling
    perm = rng.permutation(n)
    a = oracle.rmsnorm(x, w, eps)
    b = oracle.rmsnorm(x, w[perm], eps)
    np.testing.assert_allclose(a / w, b / w[perm], rtol=1e-6)


@pytest.mark.parametrize("shape", [(4, 2, 32, 64, 1e6), (8, 2, 64, 128, 1e4), (32, 8, 128, 256, 5e5)])
def test_attention_layer_vs_reference(oracle, ref_scalar, shape):
    nq, nkv, hd, hidden, theta = shape
    eps, T = 1e-6, 20
    nb = hd // QK

    def mat(rows, cols, s):
        return oracle.quantize_row_q8(fill_random(rows * cols, s, 0.5))

    wq, wk, wv, wo = mat(nq * hd, hidden, 1), mat(nkv * hd, hidden, 2), mat(nkv * hd, hidden, 3), mat(hidden, nq * hd, 4)
    qn = (1.25 + 0.75 * fill_random(hd, 5)).astype(np.float32)
    kn = (1.25 + 0.75 * fill_random(hd, 6)).astype(np.float32)
    kc_r, vc_r, kc_o, vc_o = (blocks(nkv * T * nb) for _ in range(4))
    L = ref_scalar.lib
    for pos in range(T):
        xn = fill_random(hidden, 900 + pos)
        out_r = np.zeros(hidden, np.float32)
        sc = np.zeros(nq * T, np.float32)
        assert L.tqref_layer_run(nq, nkv, hd, hidden, theta, eps, ptr(wq), ptr(wk), ptr(wv), ptr(wo), ptr(qn),
                                 ptr(kn), ptr(kc_r), ptr(vc_r), T, pos, ptr(xn), ptr(sc), ptr(out_r)) == 0
        rc, out_o = oracle.attention_layer((wq, wk, wv, wo, qn, kn), nq, nkv, hd, hidden, theta, eps,
                                           kc_o, vc_o, T, pos, xn)
        assert rc == 0
        assert out_o.tobytes() == out_r.tobytes(), pos
    assert kc_o.tobytes() == kc_r.tobytes() and vc_o.tobytes() == vc_r.tobytes()
    rc, _ = oracle.attention_layer((wq, wk, wv, wo, qn, kn), nq, nkv, hd, hidden, theta, eps, kc_o, vc_o, T, T,
                                   fill_random(hidden, 1))
    assert rc == -1
