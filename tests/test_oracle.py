"""Pins the CPU oracle (oracle/tq_oracle.c) before the HIP path is compared against it.

Three independent anchors:

1. the committed golden vectors (tests/golden/golden_q8.npz), made by running
   the reference compiled from its own sources — bit-exact;
2. the compiled reference itself (oracle/_ref), when it is built here — bit-exact
   for the scalar build, within 1e-5 for the AVX2 dispatch (the reference's own
   SIMD-vs-scalar tolerance, tools/test_kernel.c:15,104);
3. what the mathematics fixes, chosen so that a plausible slip fails: fp64 brute
   force on dequantized data (tools/test_model.c:1623-1677), RoPE identities
   (:294-397), softmax known values (:200-292), quantizer invariants and
   ties-to-even, the GQA head mapping, untouched unused slots, bad positions.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest

from oracle.binding import BLOCK_Q8, QK, blocks, dequant, f32, ptr
from tests.golden.gen import checksum, fill_random

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden_q8.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def is_close(actual, expected, tol):
    """tools/test_model.c:12-14: |a - e| <= tol * (1 + |e|)."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    return np.abs(a - e) <= tol * (1.0 + np.abs(e))


def quantize_rows(oracle, x, rows, hd):
    return oracle.quantize_row_q8(f32(x).reshape(rows * hd)).reshape(rows, hd // QK)


# --------------------------------------------------------------------------
# 1. golden vectors
# --------------------------------------------------------------------------

def test_golden_quantize(oracle, golden):
    seed, n = golden["quant_x_seed"]
    x = np.concatenate([fill_random(int(n), int(seed), 3.0), golden["quant_edges"].reshape(-1)])
    assert checksum(x) == int(golden["quant_x_sum"][0])
    qb = oracle.quantize_row_q8(x)
    np.testing.assert_array_equal(qb["d"].view(np.uint32), golden["quant_d"].view(np.uint32))
    np.testing.assert_array_equal(qb["q"], golden["quant_q"])


def test_golden_rope_table(oracle, golden):
    for i, (hd, pos, th) in enumerate(golden["rope_cases"]):
        c, s = oracle.rope_table(int(hd), int(pos), float(th))
        np.testing.assert_array_equal(c.view(np.uint32), golden[f"rope_cos_{i}"].view(np.uint32))
        np.testing.assert_array_equal(s.view(np.uint32), golden[f"rope_sin_{i}"].view(np.uint32))


def _kernel_inputs(oracle, i, g, n, hd):
    nb = hd // QK
    seed = 900 + 7 * i
    qb = oracle.quantize_row_q8(fill_random(g * hd, seed))
    kb = oracle.quantize_row_q8(fill_random(n * hd, seed + 1))
    vb = oracle.quantize_row_q8(fill_random(n * hd, seed + 2))
    w = fill_random(g * n, seed + 3)
    return nb, qb, kb, vb, w


def test_golden_kernels(oracle, golden):
    for i, (g, n, hd) in enumerate(golden["kern_cases"]):
        g, n, hd = int(g), int(n), int(hd)
        nb, qb, kb, vb, w = _kernel_inputs(oracle, i, g, n, hd)
        assert [checksum(qb), checksum(kb), checksum(vb), checksum(w)] == list(golden[f"kern_in_sum_{i}"])
        scale = np.float32(1.0) / np.sqrt(np.float32(hd))
        sc = np.zeros(g * n, np.float32)
        oracle.attn_scores_q8(qb, g, kb, n, nb, float(scale), sc, n)
        np.testing.assert_array_equal(sc.view(np.uint32), golden[f"kern_scores_{i}"].view(np.uint32))
        sm = np.concatenate([oracle.softmax(sc[h * n:(h + 1) * n]) for h in range(g)])
        np.testing.assert_array_equal(sm.view(np.uint32), golden[f"kern_softmax_{i}"].view(np.uint32))
        out = np.zeros(g * hd, np.float32)
        oracle.attn_accum_q8(w, n, g, vb, n, nb, out, hd)
        np.testing.assert_array_equal(out.view(np.uint32), golden[f"kern_accum_{i}"].view(np.uint32))


def test_golden_attention_head(oracle, golden):
    for i, (hd, n) in enumerate(golden["head_cases"]):
        hd, n = int(hd), int(n)
        seed = 70 + 11 * i
        q = fill_random(hd, seed)
        kb = oracle.quantize_row_q8(fill_random(n * hd, seed + 1000))
        vb = oracle.quantize_row_q8(fill_random(n * hd, seed + 2000))
        out, qq, _ = oracle.attention_head_q8(q, kb, vb, n, hd)
        np.testing.assert_array_equal(out.view(np.uint32), golden[f"head_out_{i}"].view(np.uint32))
        np.testing.assert_array_equal(qq["d"], golden[f"head_qd_{i}"])
        np.testing.assert_array_equal(qq["q"], golden[f"head_qq_{i}"])


def test_golden_attention_core_c1(oracle, golden):
    nq, nkv, hd, T, theta = 8, 2, 64, 256, 10000.0
    nb = hd // QK
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc["d"] = 999.0
    vc["d"] = 999.0
    keep = set(int(p) for p in golden["core1_keep"])
    for pos in range(T):
        q = fill_random(nq * hd, 5000 + pos)
        k = fill_random(nkv * hd, 6000 + pos)
        v = fill_random(nkv * hd, 7000 + pos)
        rc, out = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0
        if pos in keep:
            np.testing.assert_array_equal(out.view(np.uint32), golden[f"core1_out_{pos}"].view(np.uint32))
    np.testing.assert_array_equal(kc.view(np.uint8).reshape(-1), golden["core1_kc"])
    np.testing.assert_array_equal(vc.view(np.uint8).reshape(-1), golden["core1_vc"])


def test_golden_attention_core_c2_step(oracle, golden):
    nq, nkv, hd, T, theta = 32, 8, 128, 4096, 500000.0
    nb = hd // QK
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    pos = T - 1
    rc, out = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, fill_random(nq * hd, 8100),
                                   fill_random(nkv * hd, 8200), fill_random(nkv * hd, 8300))
    assert rc == 0
    rows_k = np.stack([kc[(h * T + pos) * nb:(h * T + pos + 1) * nb] for h in range(nkv)])
    rows_v = np.stack([vc[(h * T + pos) * nb:(h * T + pos + 1) * nb] for h in range(nkv)])
    np.testing.assert_array_equal(rows_k.view(np.uint8).reshape(-1), golden["core2_k_rows"])
    np.testing.assert_array_equal(rows_v.view(np.uint8).reshape(-1), golden["core2_v_rows"])
    np.testing.assert_array_equal(out.view(np.uint32), golden["core2_out"].view(np.uint32))


# --------------------------------------------------------------------------
# 2. against the compiled reference (when built here)
# --------------------------------------------------------------------------

def test_ref_quantize_bitexact(oracle, ref_scalar):
    rng = np.random.default_rng(1)
    for scale in (1e-30, 1e-3, 1.0, 8.0, 1e30):
        x = (rng.standard_normal(4096) * scale).astype(np.float32)
        mine = oracle.quantize_row_q8(x)
        theirs = blocks(x.size // QK)
        ref_scalar.lib.quantize_row_q8(ptr(x), ptr(theirs), x.size)
        assert mine.tobytes() == theirs.tobytes()


def test_ref_rope_softmax_bitexact(oracle, ref_scalar):
    L = ref_scalar.lib
    for hd in (2, 8, 32, 64, 128, 256):
        for pos in (0, 1, 7, 100, 4095, 32767):
            for th in (10000.0, 500000.0, 1000000.0):
                c, s = oracle.rope_table(hd, pos, th)
                c2, s2 = np.zeros(hd // 2, np.float32), np.zeros(hd // 2, np.float32)
                L.rope_table(ptr(c2), ptr(s2), hd, pos, th)
                assert c.tobytes() == c2.tobytes() and s.tobytes() == s2.tobytes()
                x = fill_random(hd, 13 + pos, 3.0)
                mine = oracle.rope_apply(x, c, s)
                theirs = x.copy()
                L.rope_apply(ptr(theirs), hd, ptr(c2), ptr(s2))
                assert mine.tobytes() == theirs.tobytes()
    for n in (1, 2, 3, 100, 1024, 5000):
        x = fill_random(n, 10 + n, 20.0)
        theirs = x.copy()
        L.softmax(ptr(theirs), n)
        assert oracle.softmax(x).tobytes() == theirs.tobytes()


@pytest.mark.parametrize("g", [1, 2, 3, 4, 5, 8])
def test_ref_scores_accum_bitexact(oracle, ref_scalar, ref_avx2, g):
    """Scalar kernels bit for bit; the AVX2 dispatch within 1e-5."""
    for n in (1, 7, 100, 129, 300):
        for hd in (32, 64, 128):
            nb = hd // QK
            seed = 900 + g * 100 + n + hd
            qb = oracle.quantize_row_q8(fill_random(g * hd, seed))
            kb = oracle.quantize_row_q8(fill_random(n * hd, seed + 1))
            vb = oracle.quantize_row_q8(fill_random(n * hd, seed + 2))
            stride = n + 4
            w = fill_random(g * stride, seed + 3)
            scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
            outs = {}
            for name, fn_s, fn_a in (("oracle", oracle.lib.oracle_attn_scores_q8, oracle.lib.oracle_attn_accum_q8),
                                     ("scalar", ref_scalar.lib.attn_scores_q8_scalar, ref_scalar.lib.attn_accum_q8_scalar),
                                     ("avx2", ref_avx2.lib.attn_scores_q8, ref_avx2.lib.attn_accum_q8)):
                sc = np.full(g * stride, 12345.0, np.float32)
                fn_s(ptr(qb), g, ptr(kb), n, nb, scale, ptr(sc), stride)
                out = np.full(g * (hd + 8), 12345.0, np.float32)
                fn_a(ptr(w), stride, g, ptr(vb), n, nb, ptr(out), hd + 8)
                outs[name] = (sc, out)
            assert outs["oracle"][0].tobytes() == outs["scalar"][0].tobytes()
            assert outs["oracle"][1].tobytes() == outs["scalar"][1].tobytes()
            assert is_close(outs["avx2"][0], outs["oracle"][0], 1e-5).all()
            assert is_close(outs["avx2"][1], outs["oracle"][1], 1e-5).all()


def _layer_weights(oracle, nq, nkv, hd, hidden, seed):
    def mat(rows, cols, s):
        return quantize_rows(oracle, fill_random(rows * cols, s, 0.5), rows, cols).reshape(-1)
    wq = mat(nq * hd, hidden, seed + 1)
    wk = mat(nkv * hd, hidden, seed + 2)
    wv = mat(nkv * hd, hidden, seed + 3)
    wo = mat(hidden, nq * hd, seed + 4)
    qn = (1.25 + 0.75 * fill_random(hd, seed + 5)).astype(np.float32)
    kn = (1.25 + 0.75 * fill_random(hd, seed + 6)).astype(np.float32)
    return wq, wk, wv, wo, qn, kn


@pytest.mark.parametrize("shape", [(4, 2, 32, 64, 1000000.0), (8, 2, 64, 128, 10000.0),
                                   (32, 8, 128, 256, 500000.0), (6, 2, 32, 64, 10000.0)])
def test_ref_attention_layer_bitexact(oracle, ref_scalar, shape):
    """The reference's own attention_layer (its static store_kv + attend_q8)
    against the oracle's attention core placed between the reference's
    projections: caches and layer outputs equal bit for bit."""
    nq, nkv, hd, hidden, theta = shape
    eps = 1e-6
    T = 24
    nb = hd // QK
    L = ref_scalar.lib
    wq, wk, wv, wo, qn, kn = _layer_weights(oracle, nq, nkv, hd, hidden, 100)
    kc_r, vc_r = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc_o, vc_o = blocks(nkv * T * nb), blocks(nkv * T * nb)
    for c in (kc_r, vc_r, kc_o, vc_o):
        c["d"] = 999.0
        c["q"] = 127
    for pos in range(T - 4):
        xn = fill_random(hidden, 500 + pos)
        out_r = np.zeros(hidden, np.float32)
        sc = np.zeros(nq * T, np.float32)
        rc = L.tqref_layer_run(nq, nkv, hd, hidden, theta, eps, ptr(wq), ptr(wk), ptr(wv), ptr(wo),
                               ptr(qn), ptr(kn), ptr(kc_r), ptr(vc_r), T, pos, ptr(xn), ptr(sc), ptr(out_r))
        assert rc == 0
        q = np.zeros(nq * hd, np.float32)
        k = np.zeros(nkv * hd, np.float32)
        v = np.zeros(nkv * hd, np.float32)
        assert L.tqref_project_qkv(nq, nkv, hd, hidden, eps, ptr(wq), ptr(wk), ptr(wv), ptr(qn), ptr(kn),
                                   ptr(xn), ptr(q), ptr(k), ptr(v)) == 0
        rc, attn = oracle.attention_qkv(kc_o, vc_o, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0
        out_o = np.zeros(hidden, np.float32)
        assert L.tqref_project_out(nq, hd, hidden, ptr(wo), ptr(attn), ptr(out_o)) == 0
        assert out_o.tobytes() == out_r.tobytes(), f"layer output differs at pos {pos}"
        assert kc_o.tobytes() == kc_r.tobytes() and vc_o.tobytes() == vc_r.tobytes()
    # slots past the last position are untouched (d stays 999)
    for h in range(nkv):
        tail = kc_o[(h * T + T - 4) * nb:(h * T + T) * nb]
        assert (tail["d"] == 999.0).all()


def test_ref_attention_layer_batch_bitexact(oracle, ref_scalar):
    """attention_layer_batch (prefill) in the reference == the oracle's prefill."""
    nq, nkv, hd, hidden, theta, eps = 8, 2, 64, 128, 10000.0, 1e-6
    T, pos0, n = 40, 3, 17
    nb = hd // QK
    L = ref_scalar.lib
    wq, wk, wv, wo, qn, kn = _layer_weights(oracle, nq, nkv, hd, hidden, 300)
    kc_r, vc_r = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc_o, vc_o = blocks(nkv * T * nb), blocks(nkv * T * nb)
    xn = fill_random(n * hidden, 77)
    out_r = np.zeros(n * hidden, np.float32)
    sc = np.zeros(nq * T, np.float32)
    rc = L.tqref_layer_batch_run(nq, nkv, hd, hidden, theta, eps, ptr(wq), ptr(wk), ptr(wv), ptr(wo),
                                 ptr(qn), ptr(kn), ptr(kc_r), ptr(vc_r), T, pos0, n, ptr(xn), ptr(sc),
                                 ptr(out_r))
    assert rc == 0
    qs = np.zeros((n, nq * hd), np.float32)
    ks = np.zeros((n, nkv * hd), np.float32)
    vs = np.zeros((n, nkv * hd), np.float32)
    for i in range(n):
        assert L.tqref_project_qkv(nq, nkv, hd, hidden, eps, ptr(wq), ptr(wk), ptr(wv), ptr(qn), ptr(kn),
                                   ptr(np.ascontiguousarray(xn[i * hidden:(i + 1) * hidden])),
                                   ptr(qs[i]), ptr(ks[i]), ptr(vs[i])) == 0
    rc, attn = oracle.prefill_qkv(kc_o, vc_o, nq, nkv, hd, T, theta, pos0, n, qs, ks, vs)
    assert rc == 0
    for i in range(n):
        out_o = np.zeros(hidden, np.float32)
        assert L.tqref_project_out(nq, hd, hidden, ptr(wo), ptr(np.ascontiguousarray(attn[i])), ptr(out_o)) == 0
        assert out_o.tobytes() == out_r[i * hidden:(i + 1) * hidden].tobytes()
    assert kc_o.tobytes() == kc_r.tobytes() and vc_o.tobytes() == vc_r.tobytes()


def test_ref_attention_core_avx2_close(oracle, ref_avx2):
    """The CPU baseline composition (reference kernels, AVX2 dispatch, OpenMP
    over kv heads) agrees with the scalar oracle within 1e-5."""
    nq, nkv, hd, T, theta = 32, 8, 128, 300, 500000.0
    nb = hd // QK
    kc_a, vc_a = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc_o, vc_o = blocks(nkv * T * nb), blocks(nkv * T * nb)
    L = ref_avx2.lib
    for pos in range(T):
        q = fill_random(nq * hd, 40 + pos)
        k = fill_random(nkv * hd, 41 + pos)
        v = fill_random(nkv * hd, 42 + pos)
        qa, ka = q.copy(), k.copy()
        sc = np.zeros(nq * T, np.float32)
        out_a = np.zeros(nq * hd, np.float32)
        assert L.tqref_attention_qkv(nq, nkv, hd, T, theta, ptr(kc_a), ptr(vc_a), pos, ptr(qa), ptr(ka),
                                     ptr(v), ptr(sc), ptr(out_a)) == 0
        rc, out_o = oracle.attention_qkv(kc_o, vc_o, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0
        assert is_close(out_a, out_o, 1e-5).all()
    assert kc_a.tobytes() == kc_o.tobytes() and vc_a.tobytes() == vc_o.tobytes()


# --------------------------------------------------------------------------
# 3. closed forms and invariants
# --------------------------------------------------------------------------

def test_quantize_invariants(oracle):
    x = fill_random(32 * 200, 5, 4.0)
    qb = oracle.quantize_row_q8(x)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert (np.abs(qb["q"].astype(np.int32)).max(axis=1) == 127).all()
    np.testing.assert_array_equal(qb["d"], (amax / np.float32(127.0)).astype(np.float32))
    err = np.abs(dequant(qb.reshape(200, 1)).reshape(-1, 32) - x.reshape(-1, 32))
    assert (err <= qb["d"][:, None] * 0.5 * (1 + 1e-6)).all()
    # tools/test_kernel.c:139-142: relative round-trip error <= 0.6 %
    rt = dequant(qb.reshape(200, 1)).reshape(-1)
    assert np.linalg.norm(rt - x) / np.linalg.norm(x) <= 6e-3
    z = oracle.quantize_row_q8(np.zeros(64, np.float32))
    assert (z["d"] == 0).all() and (z["q"] == 0).all()


def test_quantize_ties_to_even(oracle):
    # amax = 127 gives d = 1 and inverse 1, so x*inv = x: exact .5 ties.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    ties = np.array([0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, 126.5], np.float32)
    x[1:9] = ties
    qb = oracle.quantize_row_q8(x)
    assert qb["d"][0] == 1.0
    np.testing.assert_array_equal(qb["q"][0, 1:9], [0, 2, 2, 4, 0, -2, -2, 126])
    # round-half-away-from-zero (lroundf, packer/packer.c:5) would give these:
    away = np.sign(ties) * np.floor(np.abs(ties) + 0.5)
    assert (qb["q"][0, 1:9] != away).any()


def test_rope_known_values_and_identities(oracle):
    # tools/test_model.c:316-326
    c, s = oracle.rope_table(2, 1, 10000.0)
    x = oracle.rope_apply(np.array([1.0, 0.0], np.float32), c, s)
    assert is_close(x, [math.cos(1.0), math.sin(1.0)], 1e-5).all()
    # position 0 is the identity
    x = fill_random(128, 11, 3.0)
    c, s = oracle.rope_table(128, 0, 1e6)
    assert oracle.rope_apply(x, c, s).tobytes() == x.tobytes()
    # norm preserved
    c, s = oracle.rope_table(128, 100, 1e6)
    y = oracle.rope_apply(x, c, s)
    assert is_close(np.dot(y.astype(np.float64), y), np.dot(x.astype(np.float64), x), 1e-5)
    # dot products depend on relative position only
    q = fill_random(128, 20)
    k = fill_random(128, 21)
    def rot(v, p):
        c, s = oracle.rope_table(128, p, 1e6)
        return oracle.rope_apply(v, c, s).astype(np.float64)
    assert is_close(np.dot(rot(q, 5), rot(k, 3)), np.dot(rot(q, 12), rot(k, 10)), 1e-4)
    # fp64 reference (tools/test_model.c:296-306) with the pairing i <-> i + hd/2
    for hd in (8, 128):
        for pos in (1, 7, 100):
            x = fill_random(hd, 13 + pos, 3.0)
            c, s = oracle.rope_table(hd, pos, 1e6)
            y = oracle.rope_apply(x, c, s)
            half = hd // 2
            i = np.arange(half)
            ang = pos * np.power(1e6, -2.0 * i / hd)
            x64 = x.astype(np.float64)
            exp = np.concatenate([x64[:half] * np.cos(ang) - x64[half:] * np.sin(ang),
                                  x64[:half] * np.sin(ang) + x64[half:] * np.cos(ang)])
            assert is_close(y, exp, 1e-4).all()


def test_softmax_known_values(oracle):
    # tools/test_model.c:216-226
    assert is_close(oracle.softmax([1.0, 2.0, 3.0]), [0.0900, 0.2447, 0.6652], 1e-3).all()
    x = fill_random(1024, 9, 10.0)
    assert is_close(oracle.softmax(x).astype(np.float64).sum(), 1.0, 1e-5)
    assert is_close(oracle.softmax([1000, 1001, 1002]), oracle.softmax([0, 1, 2]), 1e-6).all()
    assert is_close(oracle.softmax(np.full(8, 5.0)), np.full(8, 1 / 8), 1e-6).all()
    x = fill_random(1024, 10, 20.0)
    e = np.exp(x.astype(np.float64) - x.max())
    assert is_close(oracle.softmax(x), e / e.sum(), 1e-5).all()


@pytest.mark.parametrize("g", [1, 2, 3, 4, 5, 8])
def test_scores_accum_vs_fp64(oracle, g):
    """tools/test_model.c:1623-1677: fp64 on dequantized data, 1e-4; guard
    values past n and past hd stay untouched."""
    GUARD = 12345.0
    for n in (1, 7, 100, 129, 300):
        for hd in (32, 64, 128):
            nb = hd // QK
            seed = 900 + g * 100 + n * 10 + hd
            qb = oracle.quantize_row_q8(fill_random(g * hd, seed))
            kb = oracle.quantize_row_q8(fill_random(n * hd, seed + 1))
            vb = oracle.quantize_row_q8(fill_random(n * hd, seed + 2))
            qd = dequant(qb.reshape(g, nb)).astype(np.float64)
            kd = dequant(kb.reshape(n, nb)).astype(np.float64)
            vd = dequant(vb.reshape(n, nb)).astype(np.float64)
            sstride, ostride = n + 4, hd + 8
            scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
            sc = np.full(g * sstride, GUARD, np.float32)
            oracle.attn_scores_q8(qb, g, kb, n, nb, scale, sc, sstride)
            sc2 = sc.reshape(g, sstride)
            assert is_close(sc2[:, :n], (qd @ kd.T) * scale, 1e-4).all()
            assert (sc2[:, n:] == GUARD).all()
            w = fill_random(g * sstride, seed + 3)
            out = np.full(g * ostride, GUARD, np.float32)
            oracle.attn_accum_q8(w, sstride, g, vb, n, nb, out, ostride)
            out2 = out.reshape(g, ostride)
            exp = w.reshape(g, sstride)[:, :n].astype(np.float64) @ vd
            assert is_close(out2[:, :hd], exp, 1e-4).all()
            assert (out2[:, hd:] == GUARD).all()


def _attention_fp64(q, kd, vd):
    s = kd @ q / math.sqrt(q.size)
    p = np.exp(s - s.max())
    return (p / p.sum()) @ vd


def test_attention_head_q8_vs_fp64(oracle):
    """tools/test_model.c:666-699: n = 1 returns the dequantized v; otherwise
    equals fp64 attention on the dequantized q, k, v within 1e-4."""
    q = fill_random(32, 60)
    kb = oracle.quantize_row_q8(fill_random(32, 61))
    vb = oracle.quantize_row_q8(fill_random(32, 62))
    out, _, _ = oracle.attention_head_q8(q, kb, vb, 1, 32)
    assert is_close(out, dequant(vb), 1e-5).all()
    for hd in (32, 128):
        for n in (1, 7, 100):
            nb = hd // QK
            q = fill_random(hd, 70 + hd + n)
            kb = oracle.quantize_row_q8(fill_random(n * hd, 1070 + hd + n))
            vb = oracle.quantize_row_q8(fill_random(n * hd, 2070 + hd + n))
            out, qq, _ = oracle.attention_head_q8(q, kb, vb, n, hd)
            exp = _attention_fp64(dequant(qq).astype(np.float64), dequant(kb.reshape(n, nb)).astype(np.float64),
                                  dequant(vb.reshape(n, nb)).astype(np.float64))
            assert is_close(out, exp, 1e-4).all()


@pytest.mark.parametrize("nq,nkv", [(8, 2), (6, 3), (4, 4), (8, 1)])
def test_attend_gqa_mapping(oracle, nq, nkv):
    """q head h reads kv head h // (nq/nkv): checked head by head against fp64
    attention over that kv head's dequantized rows."""
    hd, T, pos = 64, 50, 37
    nb = hd // QK
    n = pos + 1
    kc = oracle.quantize_row_q8(fill_random(nkv * T * hd, 3))
    vc = oracle.quantize_row_q8(fill_random(nkv * T * hd, 4))
    q = fill_random(nq * hd, 5)
    rc, out = oracle.attend_q8(kc, vc, nq, nkv, hd, T, q, pos)
    assert rc == 0
    g = nq // nkv
    for h in range(nq):
        kvh = h // g
        qq = oracle.quantize_row_q8(q[h * hd:(h + 1) * hd])
        kd = dequant(kc.reshape(nkv, T, nb)[kvh, :n]).astype(np.float64)
        vd = dequant(vc.reshape(nkv, T, nb)[kvh, :n]).astype(np.float64)
        exp = _attention_fp64(dequant(qq).astype(np.float64), kd, vd)
        assert is_close(out[h * hd:(h + 1) * hd], exp, 1e-4).all(), f"head {h}"


def test_store_kv_slots_and_bad_pos(oracle):
    nq, nkv, hd, T, theta = 8, 2, 64, 16, 1e4
    nb = hd // QK
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc["d"] = 999.0
    vc["d"] = 999.0
    before = (kc.tobytes(), vc.tobytes())
    for bad in (-1, T, T + 5):
        rc, out = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, bad, fill_random(nq * hd, 1),
                                       fill_random(nkv * hd, 2), fill_random(nkv * hd, 3))
        assert rc == -1
        assert (kc.tobytes(), vc.tobytes()) == before
    pos = 5
    k = fill_random(nkv * hd, 2)
    v = fill_random(nkv * hd, 3)
    rc, _ = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, fill_random(nq * hd, 1), k, v)
    assert rc == 0
    c, s = oracle.rope_table(hd, pos, theta)
    for h in range(nkv):
        kr = oracle.quantize_row_q8(oracle.rope_apply(k[h * hd:(h + 1) * hd], c, s))
        vr = oracle.quantize_row_q8(v[h * hd:(h + 1) * hd])
        assert kc[(h * T + pos) * nb:(h * T + pos + 1) * nb].tobytes() == kr.tobytes()
        assert vc[(h * T + pos) * nb:(h * T + pos + 1) * nb].tobytes() == vr.tobytes()
    touched = np.zeros(nkv * T * nb, bool)
    for h in range(nkv):
        touched[(h * T + pos) * nb:(h * T + pos + 1) * nb] = True
    assert (kc["d"][~touched] == 999.0).all() and (vc["d"][~touched] == 999.0).all()


def test_prefill_equals_sequential(oracle):
    nq, nkv, hd, T, theta = 8, 2, 64, 64, 1e4
    nb = hd // QK
    n, pos0 = 20, 4
    q = fill_random(n * nq * hd, 1)
    k = fill_random(n * nkv * hd, 2)
    v = fill_random(n * nkv * hd, 3)
    kc1, vc1 = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kc2, vc2 = blocks(nkv * T * nb), blocks(nkv * T * nb)
    rc, outp = oracle.prefill_qkv(kc1, vc1, nq, nkv, hd, T, theta, pos0, n, q, k, v)
    assert rc == 0
    for i in range(n):
        rc, o = oracle.attention_qkv(kc2, vc2, nq, nkv, hd, T, theta, pos0 + i, q[i * nq * hd:(i + 1) * nq * hd],
                                     k[i * nkv * hd:(i + 1) * nkv * hd], v[i * nkv * hd:(i + 1) * nkv * hd])
        assert o.tobytes() == outp[i].tobytes()
    assert kc1.tobytes() == kc2.tobytes()
    for bad in ((0, 0), (-1, 3), (T - 2, 3)):
        rc, _ = oracle.prefill_qkv(kc1, vc1, nq, nkv, hd, T, theta, bad[0], bad[1], q, k, v)
        assert rc == -1
