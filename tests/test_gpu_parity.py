"""GPU parity: the HIP path (through libtqhip.so's C-ABI) against the oracle.

Bar: KV codes and scales, quantize_row_q8, RoPE, attn_scores_q8 and
attn_accum_q8 bit-exact; attention outputs |gpu - oracle| <= 1e-4 + 1e-3*|oracle|
(fp32), as the north-star tolerance states.  Edge cases follow the
reference's tests: g in {1,2,3,4,5,8} x n in {1,7,100,129,300} x hd in
{32,64,128} with guard values past n / hd (tools/test_model.c:1612-1697),
n = 1, unused slots untouched (:1093-1135), bad positions write nothing
(:1015-1049).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from oracle.binding import BLOCK_Q8, QK, blocks, dequant
from tests.golden.gen import fill_random, normal

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-3
GUARD = 12345.0
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "golden_q8.npz")


def assert_close(gpu, ref, what=""):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref)
    bad = err > ATOL + RTOL * np.abs(ref)
    if bad.any():
        i = int(np.argmax(err - (ATOL + RTOL * np.abs(ref))))
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside 1e-4 + 1e-3|ref|; "
                             f"worst at {i}: gpu {gpu.flat[i]!r} ref {ref.flat[i]!r}")


@pytest.fixture(scope="module")
def nat():
    from tailorquantkernel_amd import native
    native.init(0)
    assert native.device_arch().startswith("gfx950")
    return native


def dev(nat, a):
    return nat.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def sync(nat):
    nat.check(nat.load().tq_hip_device_synchronize(), "sync")


# ---------------------------------------------------------------------------
# element ops
# ---------------------------------------------------------------------------

def gpu_quantize(nat, x):
    x = np.ascontiguousarray(x, np.float32)
    nbk = x.size // QK
    dx = dev(nat, x)
    dq = nat.DeviceBuffer(max(nbk * 36, 1))
    nat.check(nat.load().tq_hip_quantize_row_q8(dx.ptr, dq.ptr, x.size, None), "quantize")
    sync(nat)
    return dq.download((nbk,), BLOCK_Q8)


def test_quantize_bitexact_golden(nat):
    g = np.load(GOLDEN, allow_pickle=False)
    seed, n = g["quant_x_seed"]
    x = np.concatenate([fill_random(int(n), int(seed), 3.0), g["quant_edges"].reshape(-1)])
    qb = gpu_quantize(nat, x)
    np.testing.assert_array_equal(qb["d"].view(np.uint32), g["quant_d"].view(np.uint32))
    np.testing.assert_array_equal(qb["q"], g["quant_q"])


def gpu_quantize_skewed(nat, x, skew_x, skew_out):
    """quantize_row_q8 with x and out `skew_*` bytes past a 16-byte boundary
    (multiples of 4): x off a 16-byte boundary takes the one-value-per-lane
    kernel, the rest the 8-lane one."""
    x = np.ascontiguousarray(x, np.float32)
    nbk = x.size // QK
    dx = dev(nat, np.concatenate([np.zeros(skew_x // 4, np.float32), x]))
    dq = nat.DeviceBuffer(nbk * 36 + 16)
    nat.check(nat.load().tq_hip_quantize_row_q8(dx.ptr + skew_x, dq.ptr + skew_out, x.size, None), "quantize")
    sync(nat)
    raw = dq.download((nbk * 36 + skew_out,), np.uint8)
    return raw[skew_out:].view(BLOCK_Q8)


def test_quantize_bitexact_oracle(nat, oracle):
    rng = np.random.default_rng(7)
    for scale in (1e-38, 1e-20, 1e-3, 1.0, 8.0, 1e20):
        x = (rng.standard_normal(32 * 997) * scale).astype(np.float32)
        ref = oracle.quantize_row_q8(x).tobytes()
        assert gpu_quantize(nat, x).tobytes() == ref
        for skew_x, skew_out in ((4, 0), (8, 0), (12, 4), (0, 8)):
            assert gpu_quantize_skewed(nat, x, skew_x, skew_out).tobytes() == ref, (scale, skew_x, skew_out)
    # x and out must be 4-byte aligned (the kernels store dwords)
    dx, dq = dev(nat, np.zeros(64, np.float32)), nat.DeviceBuffer(2 * 36 + 16)
    assert nat.load().tq_hip_quantize_row_q8(dx.ptr, dq.ptr + 1, 32, None) == nat.EINVAL
    assert nat.load().tq_hip_quantize_row_q8(dx.ptr + 2, dq.ptr, 32, None) == nat.EINVAL
    # trailing values past the last whole block are ignored, as n / QK drops them
    x = fill_random(100, 3)
    assert gpu_quantize(nat, x).tobytes() == oracle.quantize_row_q8(x).tobytes()


def test_rope_bitexact(nat, oracle):
    for hd, pos, th in ((64, 255, 1e4), (128, 4095, 5e5), (128, 7, 1e6), (32, 100, 1e4), (256, 31, 5e5)):
        x = fill_random(8 * hd, 11 + pos, 3.0)
        c, s = oracle.rope_table(hd, pos, th)
        dx, dc, ds = dev(nat, x), dev(nat, c), dev(nat, s)
        nat.check(nat.load().tq_hip_rope_apply(dx.ptr, 8, hd, dc.ptr, ds.ptr, None), "rope")
        sync(nat)
        got = dx.download((8 * hd,), np.float32)
        exp = np.concatenate([oracle.rope_apply(x[h * hd:(h + 1) * hd], c, s) for h in range(8)])
        assert got.tobytes() == exp.tobytes()


@pytest.mark.parametrize("g", [1, 2, 3, 4, 5, 8])
def test_scores_accum_bitexact(nat, oracle, g):
    lib = nat.load()
    for n in (1, 7, 100, 129, 300):
        for hd in (32, 64, 128):
            nb = hd // QK
            seed = 900 + g * 100 + n * 10 + hd
            qb = oracle.quantize_row_q8(fill_random(g * hd, seed))
            kb = oracle.quantize_row_q8(fill_random(n * hd, seed + 1))
            vb = oracle.quantize_row_q8(fill_random(n * hd, seed + 2))
            sstride, ostride = n + 4, hd + 8
            scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
            sc_ref = np.full(g * sstride, GUARD, np.float32)
            oracle.attn_scores_q8(qb, g, kb, n, nb, scale, sc_ref, sstride)
            dq, dk = dev(nat, qb), dev(nat, kb)
            dsc = dev(nat, np.full(g * sstride, GUARD, np.float32))
            nat.check(lib.tq_hip_attn_scores_q8(dq.ptr, g, dk.ptr, n, nb, scale, dsc.ptr, sstride, None), "scores")
            sync(nat)
            assert dsc.download((g * sstride,), np.float32).tobytes() == sc_ref.tobytes(), (g, n, hd)

            w = fill_random(g * sstride, seed + 3)
            out_ref = np.full(g * ostride, GUARD, np.float32)
            oracle.attn_accum_q8(w, sstride, g, vb, n, nb, out_ref, ostride)
            dw, dv = dev(nat, w), dev(nat, vb)
            dout = dev(nat, np.full(g * ostride, GUARD, np.float32))
            nat.check(lib.tq_hip_attn_accum_q8(dw.ptr, sstride, g, dv.ptr, n, nb, dout.ptr, ostride, None), "accum")
            sync(nat)
            assert dout.download((g * ostride,), np.float32).tobytes() == out_ref.tobytes(), (g, n, hd)


def test_softmax_close(nat, oracle):
    lib = nat.load()
    for n, scale in ((1, 1.0), (3, 1.0), (1024, 20.0), (4096, 5.0), (5000, 50.0)):
        rows, stride = 3, n + 5
        x = np.full(rows * stride, GUARD, np.float32)
        for r in range(rows):
            x[r * stride:r * stride + n] = fill_random(n, 10 + n + r, scale)
        dx = dev(nat, x)
        nat.check(lib.tq_hip_softmax(dx.ptr, n, rows, stride, None), "softmax")
        sync(nat)
        got = dx.download((rows * stride,), np.float32).reshape(rows, stride)
        for r in range(rows):
            exp = oracle.softmax(x[r * stride:r * stride + n])
            np.testing.assert_allclose(got[r, :n], exp, rtol=2e-6, atol=1e-9)
            assert (got[r, n:] == GUARD).all()


def test_attention_head_q8(nat, oracle):
    lib = nat.load()
    for hd, n in ((32, 1), (32, 7), (128, 100), (128, 16), (64, 300), (128, 4096)):
        nb = hd // QK
        q = fill_random(hd, 70 + n)
        kb = oracle.quantize_row_q8(fill_random(n * hd, 1070 + n))
        vb = oracle.quantize_row_q8(fill_random(n * hd, 2070 + n))
        out_ref, qq_ref, sc_ref = oracle.attention_head_q8(q, kb, vb, n, hd)
        dq, dk, dv = dev(nat, q), dev(nat, kb), dev(nat, vb)
        dqq, dsc, dout = nat.DeviceBuffer(nb * 36), nat.DeviceBuffer(n * 4), nat.DeviceBuffer(hd * 4)
        nat.check(lib.tq_hip_attention_head_q8(dq.ptr, dqq.ptr, dk.ptr, dv.ptr, n, hd, dsc.ptr, dout.ptr, None),
                  "attention_head_q8")
        sync(nat)
        assert dqq.download((nb,), BLOCK_Q8).tobytes() == qq_ref.tobytes()
        assert_close(dout.download((hd,), np.float32), out_ref, f"head hd={hd} n={n}")
        if n == 1:
            np.testing.assert_array_equal(dout.download((hd,), np.float32), dequant(vb))


def test_golden_kernels_on_gpu(nat, oracle):
    """The reference's own scores/softmax/accum outputs (golden) reproduced on the GPU."""
    g_ = np.load(GOLDEN, allow_pickle=False)
    lib = nat.load()
    for i, (g, n, hd) in enumerate(g_["kern_cases"]):
        g, n, hd = int(g), int(n), int(hd)
        nb = hd // QK
        seed = 900 + 7 * i
        qb = oracle.quantize_row_q8(fill_random(g * hd, seed))
        kb = oracle.quantize_row_q8(fill_random(n * hd, seed + 1))
        vb = oracle.quantize_row_q8(fill_random(n * hd, seed + 2))
        w = fill_random(g * n, seed + 3)
        scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
        dq, dk, dv, dw = dev(nat, qb), dev(nat, kb), dev(nat, vb), dev(nat, w)
        dsc, dout = nat.DeviceBuffer(g * n * 4), nat.DeviceBuffer(g * hd * 4)
        nat.check(lib.tq_hip_attn_scores_q8(dq.ptr, g, dk.ptr, n, nb, scale, dsc.ptr, n, None), "scores")
        nat.check(lib.tq_hip_attn_accum_q8(dw.ptr, n, g, dv.ptr, n, nb, dout.ptr, hd, None), "accum")
        nat.check(lib.tq_hip_softmax(dsc.ptr, n, g, n, None), "softmax")
        sync(nat)
        np.testing.assert_array_equal(dout.download((g * hd,), np.float32).view(np.uint32),
                                      g_[f"kern_accum_{i}"].view(np.uint32))
        np.testing.assert_allclose(dsc.download((g * n,), np.float32), g_[f"kern_softmax_{i}"], rtol=2e-6, atol=1e-9)


# ---------------------------------------------------------------------------
# paged cache: append / attend / step / batch / prefill
# ---------------------------------------------------------------------------

def flat_from_paged(kv, seq, n):
    """Device cache rows [0, n) as the reference's flat arrays [nkv][n][nb]."""
    k, v = kv.read(seq, 0, n)
    return k.reshape(-1), v.reshape(-1)


@pytest.mark.parametrize("shape", [(8, 2, 64, 256, 1e4), (32, 8, 128, 4096, 5e5), (4, 2, 32, 40, 1e6),
                                   (6, 2, 256, 48, 1e4), (5, 1, 64, 70, 1e4)])
def test_append_bitexact_and_untouched(nat, oracle, shape):
    nq, nkv, hd, T, theta = shape
    nb = hd // QK
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    sent_k = blocks(nkv * T * nb).reshape(nkv, T, nb)
    sent_k["d"] = 999.0
    sent_k["q"] = 127
    kv.write(0, 0, sent_k, sent_k)
    kc, vc = sent_k.reshape(-1).copy(), sent_k.reshape(-1).copy()
    for pos in sorted({0, 1, T // 2, T - 1}):
        k = fill_random(nkv * hd, 100 + pos)
        v = fill_random(nkv * hd, 200 + pos)
        c, s = oracle.rope_table(hd, pos, theta)
        assert kv.append(0, pos, k, v, c, s) == 0
        kr = np.concatenate([oracle.rope_apply(k[h * hd:(h + 1) * hd], c, s) for h in range(nkv)])
        assert oracle.lib.oracle_store_kv_q8(kc.ctypes.data, vc.ctypes.data, nkv, hd, T, pos,
                                             kr.ctypes.data, v.ctypes.data) == 0
    gk, gv = flat_from_paged(kv, 0, T)
    assert gk.tobytes() == kc.tobytes() and gv.tobytes() == vc.tobytes()
    # bad positions return -1 and write nothing
    for bad in (-1, kv.capacity(0), kv.capacity(0) + 5):
        assert kv.append(0, bad, fill_random(nkv * hd, 1), fill_random(nkv * hd, 2)) == -1
    gk2, gv2 = flat_from_paged(kv, 0, T)
    assert gk2.tobytes() == gk.tobytes() and gv2.tobytes() == gv.tobytes()
    kv.close()


def _step_compare(nat, oracle, nq, nkv, hd, T, theta, positions, seed):
    """Device append + attend per position vs the oracle's attention core."""
    nb = hd // QK
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    for pos in positions:
        q = fill_random(nq * hd, seed + 3 * pos)
        k = fill_random(nkv * hd, seed + 3 * pos + 1)
        v = fill_random(nkv * hd, seed + 3 * pos + 2)
        c, s = oracle.rope_table(hd, pos, theta)
        rc, out_ref = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0
        assert kv.append(0, pos, k, v, c, s) == 0
        rc, out = kv.attend(0, pos, q, c, s)
        assert rc == 0
        assert_close(out, out_ref, f"attend nq={nq} nkv={nkv} hd={hd} pos={pos}")
    return kv, kc, vc


def test_attend_c1_every_position(nat, oracle):
    """8q/2kv/hd64, theta 1e4: every step of a 256-token context."""
    kv, kc, vc = _step_compare(nat, oracle, 8, 2, 64, 256, 1e4, range(256), 5000)
    gk, gv = flat_from_paged(kv, 0, 256)
    assert gk.tobytes() == kc.tobytes() and gv.tobytes() == vc.tobytes()
    kv.close()


@pytest.mark.parametrize("g", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("hd", [32, 64, 128, 256])
def test_attend_group_sizes(nat, oracle, g, hd):
    nkv = 2
    positions = [0, 1, 15, 16, 63, 64, 100, 255, 299]
    kv, kc, vc = _step_compare(nat, oracle, g * nkv, nkv, hd, 300, 1e4, positions, 700 + g + hd)
    kv.close()


def test_attend_c2_full_context(nat, oracle):
    """32q/8kv/hd128, theta 5e5, context 4096: cache filled, then the last steps."""
    nq, nkv, hd, T, theta = 32, 8, 128, 4096, 5e5
    nb = hd // QK
    kc = oracle.quantize_row_q8(normal(nkv * T * hd, 1))
    vc = oracle.quantize_row_q8(normal(nkv * T * hd, 2))
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    kv.write(0, 0, kc.reshape(nkv, T, nb), vc.reshape(nkv, T, nb))
    for pos in (0, 1000, 4094, 4095):
        q = normal(nq * hd, 10 + pos)
        k = normal(nkv * hd, 20 + pos)
        v = normal(nkv * hd, 30 + pos)
        c, s = oracle.rope_table(hd, pos, theta)
        rc, out_ref = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, pos, q, k, v)
        assert rc == 0
        assert kv.append(0, pos, k, v, c, s) == 0
        rc, out = kv.attend(0, pos, q, c, s)
        assert rc == 0
        assert_close(out, out_ref, f"C2 pos={pos}")
    gk, gv = flat_from_paged(kv, 0, T)
    assert gk.tobytes() == kc.tobytes() and gv.tobytes() == vc.tobytes()
    # deterministic: the same call twice gives the same bits
    q = normal(nq * hd, 99)
    _, o1 = kv.attend(0, T - 1, q)
    _, o2 = kv.attend(0, T - 1, q)
    assert o1.tobytes() == o2.tobytes()
    kv.close()


def test_split_combine_first_call_and_repeats(nat, oracle):
    """Split-K combine: a fresh cache whose very first call uses several splits
    (arrival counters allocated and zeroed on that call), many times over, then
    a run of consecutive multi-split steps — every output against the oracle."""
    nq, nkv, hd, T, theta = 32, 8, 128, 1200, 5e5
    nb = hd // QK
    kc = oracle.quantize_row_q8(normal(nkv * T * hd, 31))
    vc = oracle.quantize_row_q8(normal(nkv * T * hd, 32))
    for rep in range(8):
        kv = nat.PagedKV.single(nq, nkv, hd, T)
        kv.write(0, 0, kc.reshape(nkv, T, nb), vc.reshape(nkv, T, nb))
        q = normal(nq * hd, 40 + rep)
        pos = T - 1 - 37 * rep
        rc, out = kv.attend(0, pos, q)
        assert rc == 0
        rc, ref = oracle.attend_q8(kc, vc, nq, nkv, hd, T, q, pos)
        assert_close(out, ref, f"fresh cache rep {rep} pos {pos}")
        kv.close()
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    kv.write(0, 0, kc.reshape(nkv, T, nb), vc.reshape(nkv, T, nb))
    for i, pos in enumerate(range(300, T, 29)):
        q = normal(nq * hd, 100 + i)
        rc, out = kv.attend(0, pos, q)
        assert rc == 0
        rc, ref = oracle.attend_q8(kc, vc, nq, nkv, hd, T, q, pos)
        assert_close(out, ref, f"consecutive step pos {pos}")
    kv.close()


def test_attend_single_token_is_dequantized_v(nat, oracle):
    nq, nkv, hd = 8, 2, 64
    kv = nat.PagedKV.single(nq, nkv, hd, 16)
    k = fill_random(nkv * hd, 61)
    v = fill_random(nkv * hd, 62)
    assert kv.append(0, 0, k, v) == 0
    rc, out = kv.attend(0, 0, fill_random(nq * hd, 60))
    assert rc == 0
    vq = [dequant(oracle.quantize_row_q8(v[h * hd:(h + 1) * hd])) for h in range(nkv)]
    g = nq // nkv
    # the reference's bar for this case: |out - v_deq| <= 1e-5 * (1 + |v_deq|)
    # (tools/test_model.c:12-14, 681); the P.V weight w = p*vd goes through the
    # matrix cores as bf16 hi + lo, exact to 2^-18 relative
    for h in range(nq):
        got = out[h * hd:(h + 1) * hd].astype(np.float64)
        want = vq[h // g].astype(np.float64)
        assert (np.abs(got - want) <= 1e-5 * (1.0 + np.abs(want))).all(), f"head {h}"
        assert (np.abs(got - want) <= 2.0 ** -17 * np.abs(want)).all(), f"head {h}: beyond the hi/lo split's bound"
    # bad positions: -1, out untouched
    for bad in (-1, 16, 100):
        rc, _ = kv.attend(0, bad, fill_random(nq * hd, 60))
        assert rc == -1
    kv.close()


def test_decode_step_fused(nat, oracle):
    """tq_hip_decode_step_async: append + attend in one launch, 2 sequences."""
    lib = nat.load()
    nq, nkv, hd, T, theta = 32, 8, 128, 700, 5e5
    nb = hd // QK
    pages = (T + 15) // 16
    kv = nat.PagedKV(nq, nkv, hd, n_pages=2 * pages, max_seqs=2, max_pages_per_seq=pages)
    perm = np.random.default_rng(3).permutation(2 * pages).astype(np.int32)
    kv.set_pages(0, perm[:pages])
    kv.set_pages(1, perm[pages:])
    caches = [(blocks(nkv * T * nb), blocks(nkv * T * nb)) for _ in range(2)]
    dseq = dev(nat, np.array([0, 1], np.int32))
    for step in range(0, T, 37):
        pos = np.array([step, min(T - 1, step + 5)], np.int32)
        q = normal(2 * nq * hd, step)
        k = normal(2 * nkv * hd, step + 1)
        v = normal(2 * nkv * hd, step + 2)
        cs = [oracle.rope_table(hd, int(p), theta) for p in pos]
        cos = np.concatenate([c for c, _ in cs])
        sin = np.concatenate([s for _, s in cs])
        dq, dk, dv, dc, ds = dev(nat, q), dev(nat, k), dev(nat, v), dev(nat, cos), dev(nat, sin)
        dpos, dout = dev(nat, pos), nat.DeviceBuffer(2 * nq * hd * 4)
        nat.check(lib.tq_hip_decode_step_async(kv.h, 2, dseq.ptr, dpos.ptr, int(pos.max()), dq.ptr, dk.ptr,
                                               dv.ptr, dc.ptr, ds.ptr, dout.ptr, None), "decode_step")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        out = dout.download((2, nq * hd), np.float32)
        for i in range(2):
            kc, vc = caches[i]
            rc, ref = oracle.attention_qkv(kc, vc, nq, nkv, hd, T, theta, int(pos[i]), q[i * nq * hd:(i + 1) * nq * hd],
                                           k[i * nkv * hd:(i + 1) * nkv * hd], v[i * nkv * hd:(i + 1) * nkv * hd])
            assert rc == 0
            assert_close(out[i], ref, f"step seq {i} pos {pos[i]}")
    for i in range(2):
        gk, gv = flat_from_paged(kv, i, T)
        kc, vc = caches[i]
        assert gk.tobytes() == kc.tobytes() and gv.tobytes() == vc.tobytes()
    kv.close()


@pytest.mark.parametrize("nseq", [40, 160])
def test_batched_decode_order(nat, oracle, nseq):
    """Ragged batches with repeated lengths: up to 128 queries are served
    longest first (ties by index), larger batches in order; either way every
    query matches the oracle on its own rows and launches repeat bit for bit."""
    lib = nat.load()
    nq, nkv, hd = 8, 2, 64
    nb = hd // QK
    rng = np.random.default_rng(nseq)
    lens = rng.choice(np.array([1, 16, 17, 64, 129, 300], np.int32), size=nseq)
    pages_per = (lens + 15) // 16
    maxp = int(pages_per.max())
    total = int(pages_per.sum())
    kv = nat.PagedKV(nq, nkv, hd, n_pages=total, max_seqs=nseq, max_pages_per_seq=maxp)
    perm = rng.permutation(total).astype(np.int32)
    at = 0
    flats = []
    for i, L in enumerate(lens):
        kv.set_pages(i, perm[at:at + pages_per[i]])
        at += pages_per[i]
        kc = oracle.quantize_row_q8(normal(nkv * int(L) * hd, 300 + i))
        vc = oracle.quantize_row_q8(normal(nkv * int(L) * hd, 700 + i))
        kv.write(i, 0, kc.reshape(nkv, L, nb), vc.reshape(nkv, L, nb))
        flats.append((kc, vc))
    q = normal(nseq * nq * hd, 9)
    dseq, dlen = dev(nat, np.arange(nseq, dtype=np.int32)), dev(nat, lens)
    dq, dout = dev(nat, q), nat.DeviceBuffer(nseq * nq * hd * 4)
    outs = []
    for _ in range(2):
        nat.check(lib.tq_hip_decode_async(kv.h, nseq, dseq.ptr, dlen.ptr, int(lens.max()), dq.ptr, None, None,
                                          dout.ptr, None), "decode_async")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        outs.append(dout.download((nseq, nq * hd), np.float32))
    assert outs[0].tobytes() == outs[1].tobytes()
    for qi in range(nseq):
        L = int(lens[qi])
        kc, vc = flats[qi]
        rc, ref = oracle.attend_q8(kc, vc, nq, nkv, hd, L, q[qi * nq * hd:(qi + 1) * nq * hd], L - 1)
        assert rc == 0
        assert_close(outs[0][qi], ref, f"query {qi} len {L} of {nseq}")
    kv.close()


def test_batched_decode_paged(nat, oracle):
    """Many sequences of ragged lengths on shuffled pages (the batched-decode
    shape at reduced count); each checked against the oracle on its own rows."""
    lib = nat.load()
    nq, nkv, hd = 32, 8, 128
    nb = hd // QK
    rng = np.random.default_rng(11)
    lens = np.array([1, 2, 15, 16, 17, 100, 512, 1000, 2047, 3000, 513, 64], np.int32)
    nseq = lens.size
    pages_per = (lens + 15) // 16
    maxp = int(pages_per.max())
    total = int(pages_per.sum())
    kv = nat.PagedKV(nq, nkv, hd, n_pages=total + 3, max_seqs=nseq, max_pages_per_seq=maxp)
    perm = rng.permutation(total + 3).astype(np.int32)
    at = 0
    flats = []
    for i, L in enumerate(lens):
        kv.set_pages(i, perm[at:at + pages_per[i]])
        at += pages_per[i]
        kc = oracle.quantize_row_q8(normal(nkv * int(L) * hd, 100 + i))
        vc = oracle.quantize_row_q8(normal(nkv * int(L) * hd, 200 + i))
        kv.write(i, 0, kc.reshape(nkv, L, nb), vc.reshape(nkv, L, nb))
        flats.append((kc, vc))
    q = normal(nseq * nq * hd, 5)
    order = rng.permutation(nseq).astype(np.int32)          # queries in shuffled sequence order
    dseq, dlen = dev(nat, order), dev(nat, lens[order])
    dq, dout = dev(nat, q), nat.DeviceBuffer(nseq * nq * hd * 4)
    outs = []
    for _ in range(3):  # repeated launches: split counters reset, results identical
        nat.check(lib.tq_hip_decode_async(kv.h, nseq, dseq.ptr, dlen.ptr, int(lens.max()), dq.ptr, None, None,
                                          dout.ptr, None), "decode_async")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        outs.append(dout.download((nseq, nq * hd), np.float32))
    assert outs[0].tobytes() == outs[1].tobytes() == outs[2].tobytes()
    out = outs[0]
    for qi, s in enumerate(order):
        L = int(lens[s])
        kc, vc = flats[s]
        rc, ref = oracle.attend_q8(kc, vc, nq, nkv, hd, L, q[qi * nq * hd:(qi + 1) * nq * hd], L - 1)
        assert rc == 0
        assert_close(out[qi], ref, f"batch query {qi} seq {s} len {L}")
    kv.close()


def test_long_context_outliers(nat, oracle):
    """64q/8kv/hd128 at 32,768 tokens (two sequences), 1 % of K/V values at
    +-8 sigma, split-K over the context."""
    lib = nat.load()
    nq, nkv, hd, T = 64, 8, 128, 32768
    nb = hd // QK
    nseq = 2
    pages = T // 16
    kv = nat.PagedKV(nq, nkv, hd, n_pages=nseq * pages, max_seqs=nseq, max_pages_per_seq=pages)
    flats = []
    rng = np.random.default_rng(21)
    for i in range(nseq):
        kv.set_pages(i, np.arange(i * pages, (i + 1) * pages, dtype=np.int32))
        kf = normal(nkv * T * hd, 300 + i)
        vf = normal(nkv * T * hd, 400 + i)
        for a in (kf, vf):
            idx = rng.choice(a.size, a.size // 100, replace=False)
            a[idx] = np.where(rng.random(idx.size) < 0.5, -8.0, 8.0).astype(np.float32)
        kc, vc = oracle.quantize_row_q8(kf), oracle.quantize_row_q8(vf)
        kv.write(i, 0, kc.reshape(nkv, T, nb), vc.reshape(nkv, T, nb))
        flats.append((kc, vc))
    q = normal(nseq * nq * hd, 9)
    dseq, dlen = dev(nat, np.arange(nseq, dtype=np.int32)), dev(nat, np.full(nseq, T, np.int32))
    dq, dout = dev(nat, q), nat.DeviceBuffer(nseq * nq * hd * 4)
    nat.check(lib.tq_hip_decode_async(kv.h, nseq, dseq.ptr, dlen.ptr, T, dq.ptr, None, None, dout.ptr, None),
              "decode_async")
    nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
    out = dout.download((nseq, nq * hd), np.float32)
    for i in range(nseq):
        kc, vc = flats[i]
        rc, ref = oracle.attend_q8(kc, vc, nq, nkv, hd, T, q[i * nq * hd:(i + 1) * nq * hd], T - 1)
        assert rc == 0
        assert_close(out[i], ref, f"long context seq {i}")
    kv.close()


PREFILL_SHAPES = [
    # nq, nkv, hd, T, theta, pos0, n — dense MFMA kernel: hd 64/128, g 1/2/4/8
    (8, 2, 64, 300, 1e4, 0, 300), (32, 8, 128, 1100, 5e5, 37, 1000), (4, 4, 64, 200, 1e4, 0, 200),
    (16, 8, 128, 300, 5e5, 0, 257), (64, 8, 128, 400, 1e6, 16, 333), (8, 2, 64, 1200, 1e4, 0, 1100),
    (8, 2, 64, 120, 1e4, 70, 40), (2, 1, 128, 80, 1e4, 0, 33),
    # one token: the fused decode step; fewer than 32: the decode form
    (2, 1, 128, 40, 1e4, 0, 1), (8, 2, 64, 90, 1e4, 70, 17), (32, 8, 128, 300, 5e5, 255, 1),
    # shapes the dense kernel does not cover run the decode form per token
    (6, 3, 32, 80, 1e6, 5, 70), (8, 2, 256, 100, 1e4, 3, 90), (12, 4, 128, 120, 1e4, 0, 100)]


@pytest.mark.parametrize("shape", PREFILL_SHAPES)
def test_prefill(nat, oracle, shape):
    """attention_layer_batch semantics: n tokens stored then attending
    causally; equal to n sequential oracle steps."""
    check_prefill(nat, oracle, shape)


@pytest.mark.parametrize("whole", ["1", "0"])
@pytest.mark.parametrize("shape", PREFILL_SHAPES[:8])
def test_prefill_both_plans(nat, oracle, shape, whole, monkeypatch):
    """The dense shapes through each of the two attention kernels, forced:
    whole query blocks (one 8-wave work-group per block, its two halves merged
    in LDS) and the paired, split blocks (partials merged by the last
    segment).  Both against the oracle's sequential steps, cache bytes
    bit-exact."""
    monkeypatch.setenv("TQ_HIP_PREFILL_WHOLE", whole)
    check_prefill(nat, oracle, shape)


def check_prefill(nat, oracle, shape):
    nq, nkv, hd, T, theta, pos0, n = shape
    nb = hd // QK
    kc, vc = blocks(nkv * T * nb), blocks(nkv * T * nb)
    kv = nat.PagedKV.single(nq, nkv, hd, T)
    if pos0:
        pre_k = oracle.quantize_row_q8(normal(nkv * T * hd, 1)).reshape(nkv, T, nb)
        pre_v = oracle.quantize_row_q8(normal(nkv * T * hd, 2)).reshape(nkv, T, nb)
        pre_k[:, pos0:] = np.zeros(1, BLOCK_Q8)
        pre_v[:, pos0:] = np.zeros(1, BLOCK_Q8)
        kv.write(0, 0, pre_k, pre_v)
        kc[:], vc[:] = pre_k.reshape(-1), pre_v.reshape(-1)
    q = normal(n * nq * hd, 3)
    k = normal(n * nkv * hd, 4)
    v = normal(n * nkv * hd, 5)
    cos = np.zeros((n, hd // 2), np.float32)
    sin = np.zeros((n, hd // 2), np.float32)
    for i in range(n):
        cos[i], sin[i] = oracle.rope_table(hd, pos0 + i, theta)
    rc, out_ref = oracle.prefill_qkv(kc, vc, nq, nkv, hd, T, theta, pos0, n, q, k, v)
    assert rc == 0
    rc, out = kv.prefill(0, pos0, n, q, k, v, cos, sin)
    assert rc == 0
    assert_close(out, out_ref, f"prefill {shape}")
    gk, gv = flat_from_paged(kv, 0, T)
    assert gk.tobytes() == kc.tobytes() and gv.tobytes() == vc.tobytes()
    for bad_pos0, bad_n in ((0, 0), (-1, 3), (kv.capacity(0) - 2, 3)):
        rc, _ = kv.prefill(0, bad_pos0, bad_n, q, k, v, cos, sin)
        assert rc == -1
    kv.close()


def test_prefill_scattered_pages(nat, oracle):
    """Prefill of a sequence whose pages are scattered over the pool, after
    earlier context, next to another sequence that must stay untouched."""
    nq, nkv, hd, theta, pos0, n = 16, 4, 128, 5e5, 45, 150
    nb = hd // QK
    T = 208   # 13 pages
    n_pages = 32
    kv = nat.PagedKV(nq, nkv, hd, n_pages=n_pages, max_seqs=2, max_pages_per_seq=13)
    rng = np.random.default_rng(11)
    perm = rng.permutation(n_pages).astype(np.int32)
    kv.set_pages(1, perm[:13])
    kv.set_pages(0, perm[13:26])
    other_k = oracle.quantize_row_q8(normal(nkv * T * hd, 21)).reshape(nkv, T, nb)
    kv.write(0, 0, other_k, other_k)
    pre_k = oracle.quantize_row_q8(normal(nkv * T * hd, 22)).reshape(nkv, T, nb)
    pre_v = oracle.quantize_row_q8(normal(nkv * T * hd, 23)).reshape(nkv, T, nb)
    pre_k[:, pos0:] = np.zeros(1, BLOCK_Q8)
    pre_v[:, pos0:] = np.zeros(1, BLOCK_Q8)
    kv.write(1, 0, pre_k, pre_v)
    kc, vc = pre_k.reshape(-1).copy(), pre_v.reshape(-1).copy()
    q, k, v = normal(n * nq * hd, 24), normal(n * nkv * hd, 25), normal(n * nkv * hd, 26)
    cos = np.zeros((n, hd // 2), np.float32)
    sin = np.zeros((n, hd // 2), np.float32)
    for i in range(n):
        cos[i], sin[i] = oracle.rope_table(hd, pos0 + i, theta)
    rc, out_ref = oracle.prefill_qkv(kc, vc, nq, nkv, hd, T, theta, pos0, n, q, k, v)
    assert rc == 0
    rc, out = kv.prefill(1, pos0, n, q, k, v, cos, sin)
    assert rc == 0
    assert_close(out, out_ref, "prefill on scattered pages")
    gk, gv = kv.read(1, 0, T)
    assert gk.reshape(-1).tobytes() == kc.tobytes() and gv.reshape(-1).tobytes() == vc.tobytes()
    ok_, ov_ = kv.read(0, 0, T)
    assert ok_.tobytes() == other_k.tobytes() and ov_.tobytes() == other_k.tobytes()
    kv.close()


def test_prefill_unaligned_kv(nat, oracle):
    """k and v 4 bytes off 16-byte alignment: the dense prefill then appends
    the new rows in a launch of their own and stages them from the cache, so
    the cache bytes and the outputs equal those of the aligned call (whose
    staging launch appends them itself)."""
    nq, nkv, hd, theta, pos0, n = 16, 4, 128, 5e5, 37, 250
    nb = hd // QK
    T = 320
    lib = nat.load()
    pre_k = oracle.quantize_row_q8(normal(nkv * T * hd, 41)).reshape(nkv, T, nb)
    pre_v = oracle.quantize_row_q8(normal(nkv * T * hd, 42)).reshape(nkv, T, nb)
    q, k, v = normal(n * nq * hd, 43), normal(n * nkv * hd, 44), normal(n * nkv * hd, 45)
    cos = np.zeros((n, hd // 2), np.float32)
    sin = np.zeros((n, hd // 2), np.float32)
    for i in range(n):
        cos[i], sin[i] = oracle.rope_table(hd, pos0 + i, theta)
    D = nat.DeviceBuffer.from_numpy
    pad = np.zeros(1, np.float32)
    dq, dc, ds = D(q), D(cos), D(sin)
    results = []
    for off in (0, 4):
        kv = nat.PagedKV.single(nq, nkv, hd, T)
        kv.write(0, 0, pre_k, pre_v)
        dk = D(np.concatenate([pad, k]) if off else k)
        dv = D(np.concatenate([pad, v]) if off else v)
        out = nat.DeviceBuffer(n * nq * hd * 4)
        nat.check(lib.tq_hip_prefill_async(kv.h, 0, pos0, n, dq.ptr, dk.ptr + off, dv.ptr + off, dc.ptr, ds.ptr,
                                           out.ptr, kv.stream), "prefill")
        nat.check(lib.tq_hip_stream_synchronize(kv.stream), "sync")
        gk, gv = kv.read(0, 0, T)
        results.append((gk.tobytes(), gv.tobytes(), out.download((n, nq * hd), np.float32)))
        for b in (dk, dv, out):
            b.free()
        kv.close()
    (ka, va, oa), (kb, vb, ob) = results
    assert ka == kb and va == vb, "cache bytes of the unaligned call"
    assert ob.tobytes() == oa.tobytes(), "outputs of the unaligned call"
    kc, vc = pre_k.reshape(-1).copy(), pre_v.reshape(-1).copy()
    rc, out_ref = oracle.prefill_qkv(kc, vc, nq, nkv, hd, T, theta, pos0, n, q, k, v)
    assert rc == 0
    assert_close(oa, out_ref, "prefill, aligned k/v")
    assert ka == kc.tobytes() and va == vc.tobytes()
    for b in (dq, dc, ds):
        b.free()


def test_prefill_c4_sampled(nat, oracle):
    """The 8B-shape causal prefill of 2048 tokens: outputs of sampled tokens
    against attend_q8 of the oracle on the cache the prefill left (token i
    reads rows [0, i] only), and a repeat of the call is bit-identical."""
    nq, nkv, hd, n, theta = 32, 8, 128, 2048, 5e5
    nb = hd // QK
    kv = nat.PagedKV.single(nq, nkv, hd, n)
    q, k, v = normal(n * nq * hd, 31), normal(n * nkv * hd, 32), normal(n * nkv * hd, 33)
    cos = np.zeros((n, hd // 2), np.float32)
    sin = np.zeros((n, hd // 2), np.float32)
    for i in range(n):
        cos[i], sin[i] = oracle.rope_table(hd, i, theta)
    rc, out = kv.prefill(0, 0, n, q, k, v, cos, sin)
    assert rc == 0
    gk, gv = kv.read(0, 0, n)
    for i in (0, 1, 31, 32, 100, 511, 1024, 1500, 2046, 2047):
        qi = q[i * nq * hd:(i + 1) * nq * hd]
        qr = np.concatenate([oracle.rope_apply(qi[h * hd:(h + 1) * hd], cos[i], sin[i]) for h in range(nq)])
        rc, ref = oracle.attend_q8(gk.reshape(-1), gv.reshape(-1), nq, nkv, hd, n, qr, i)
        assert rc == 0
        assert_close(out[i], ref, f"C4 token {i}")
    # K rows are the quantized, rotated k (spot-check token 1999 of every head)
    t = 1999
    for h in range(nkv):
        kr = oracle.rope_apply(k[(t * nkv + h) * hd:(t * nkv + h + 1) * hd], cos[t], sin[t])
        assert gk[h, t].tobytes() == oracle.quantize_row_q8(kr).tobytes()
    rc, out2 = kv.prefill(0, 0, n, q, k, v, cos, sin)
    assert rc == 0 and out2.tobytes() == out.tobytes()
    kv.close()


def test_error_codes(nat):
    lib = nat.load()
    import ctypes as C
    h = C.c_void_p()
    for desc, code in (((0, 2, 64, 4, 1, 4), nat.EINVAL), ((8, 3, 64, 4, 1, 4), nat.EINVAL),
                       ((8, 2, 48, 4, 1, 4), nat.EINVAL), ((8, 2, 96, 4, 1, 4), nat.ETYPE),
                       ((36, 2, 64, 4, 1, 4), nat.ETYPE), ((8, 2, 64, 0, 1, 4), nat.EINVAL)):
        d = nat.KVDesc(*desc)
        assert lib.tq_hip_kv_create(C.byref(h), C.byref(d)) == code, desc
    kv = nat.PagedKV(8, 2, 64, n_pages=4, max_seqs=2, max_pages_per_seq=4)
    assert lib.tq_hip_kv_set_pages(kv.h, 2, None, 0) == nat.EINVAL
    assert lib.tq_hip_kv_set_pages(kv.h, 0, np.array([0, 9], np.int32).ctypes.data, 2) == nat.EINVAL
    assert kv.capacity(0) == 0 and kv.capacity(5) == nat.EINVAL
    assert kv.append(0, 0, np.zeros(128, np.float32), np.zeros(128, np.float32)) == nat.EINVAL  # no pages
    kv.close()
